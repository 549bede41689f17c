"""Seeded synthetic workloads for the five benchmark configurations (C1-C5).

Recipe (the same for tests and bench):
  * generator torch.Generator("cpu").manual_seed(42 + c) for config Cc
    (42 is the seed of the reference's bench, bench/run_suite.py:38);
  * context lengths drawn first: uniform via torch.randint, or log-uniform
    floor(exp(U(ln lo, ln hi))) for C3;
  * pages per row ceil(len / 16); block tables are slices of one
    torch.randperm over the pool, unused columns are 0; in C4 every row's first
    512 entries are the same 512 pages (a radix-shared prefix, refcount 8);
  * then q, then every layer's K pool and V pool ~ N(0, 1) in fp32, cast to
    the config dtype. With ``values_device`` set to a GPU the values are drawn
    there by a generator with the same seed (faster, different numbers); the
    lengths and tables are always drawn on the CPU and so never change.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

BLOCK = 16


@dataclass
class Workload:
    name: str
    cfg: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    dtype: torch.dtype
    batch: int
    q_len: int
    lens: list[int]
    table: torch.Tensor          # int64 [batch, width], CPU
    num_blocks: int
    layers: int
    query: torch.Tensor          # [batch, q_len, H, D]
    k_caches: list[torch.Tensor] = field(default_factory=list)
    v_caches: list[torch.Tensor] = field(default_factory=list)
    shared_prefix_pages: int = 0
    block_size: int = BLOCK
    causal: bool = True

    @property
    def group(self) -> int:
        return self.num_heads // self.num_kv_heads

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)

    def kv_bytes_per_token(self) -> int:
        return 2 * self.num_kv_heads * self.head_dim * self.k_caches[0].element_size()

    def unique_pages(self) -> int:
        """Distinct physical pages the batch reads (shared prefix counted once)."""
        pages = set()
        for b, L in enumerate(self.lens):
            pages.update(self.table[b, : math.ceil(L / self.block_size)].tolist())
        return len(pages)

    def algorithmic_bytes(self, unique: bool = True) -> int:
        """HBM bytes one layer must move: K+V rows read (shared pages once when
        `unique`), q and out, int32 table entries, int32 lens."""
        tokens = sum(self.lens)
        if unique and self.shared_prefix_pages:
            # every row's context covers the whole shared prefix
            tokens -= (self.batch - 1) * self.shared_prefix_pages * self.block_size
        kv = tokens * self.kv_bytes_per_token()
        pages = sum(math.ceil(L / self.block_size) for L in self.lens)
        qo = 2 * self.batch * self.q_len * self.num_heads * self.head_dim * self.query.element_size()
        return kv + qo + 4 * pages + 4 * self.batch


def _lens_uniform(g, lo, hi, n):
    return [int(x) for x in torch.randint(lo, hi + 1, (n,), generator=g)]


def _lens_loguniform(g, lo, hi, n):
    u = torch.rand(n, generator=g, dtype=torch.float64)
    vals = torch.floor(torch.exp(math.log(lo) + u * (math.log(hi) - math.log(lo))))
    return [int(min(hi, max(lo, v))) for v in vals]


def _tables(g, lens, pool, width, shared=0):
    perm = torch.randperm(pool, generator=g)
    table = torch.zeros(len(lens), width, dtype=torch.long)
    if shared:
        prefix = perm[:shared]
        cursor = shared
    else:
        cursor = 0
    for b, L in enumerate(lens):
        n = math.ceil(L / BLOCK)
        if shared:
            table[b, :shared] = prefix
            own = n - shared
            table[b, shared:n] = perm[cursor:cursor + own]
            cursor += own
        else:
            table[b, :n] = perm[cursor:cursor + n]
            cursor += n
    assert cursor <= pool
    return table


def _values(shape, dtype, gen, device):
    x = torch.randn(shape, generator=gen, dtype=torch.float32, device=device)
    return x.to(dtype)


GEOMETRY = {
    # cfg: (H, KVH, D, dtype)
    1: (14, 2, 64, torch.float32),
    2: (14, 2, 64, torch.bfloat16),
    3: (32, 8, 128, torch.bfloat16),
    4: (32, 8, 128, torch.bfloat16),
    5: (28, 4, 128, torch.bfloat16),
}


def make_workload(cfg: int, *, device="cpu", values_device=None, layers: int | None = None,
                  part: str = "decode") -> Workload:
    """Build config C`cfg` (1-5). For C5 `part` is "decode" or "prefill"; both
    parts share one pool and one seeded draw (so they describe one batch)."""
    H, KVH, D, dtype = GEOMETRY[cfg]
    g = torch.Generator("cpu").manual_seed(42 + cfg)
    shared = 0
    q_len = 1
    if cfg == 1:
        lens = _lens_uniform(g, 128, 512, 4)
        pool, width = 256, 512 // BLOCK
        nlayers = 1
    elif cfg == 2:
        lens = _lens_uniform(g, 512, 2048, 32)
        pool, width = 8192, 2048 // BLOCK
        nlayers = 24
    elif cfg == 3:
        lens = _lens_loguniform(g, 1024, 8192, 64)
        need = sum(math.ceil(L / BLOCK) for L in lens)
        pool, width = math.ceil(1.25 * need), 8192 // BLOCK
        nlayers = 1
    elif cfg == 4:
        lens = _lens_uniform(g, 32768, 131072, 8)
        shared = 512
        unique = sum(math.ceil(L / BLOCK) - shared for L in lens)
        pool, width = unique + shared, 131072 // BLOCK
        nlayers = 1
    elif cfg == 5:
        dec = _lens_uniform(g, 1024, 4096, 16)
        pre = [4096 + 512, 4096 + 512]
        all_lens = dec + pre
        need = sum(math.ceil(L / BLOCK) for L in all_lens)
        pool, width = math.ceil(1.25 * need), 4608 // BLOCK
        nlayers = 1
    else:
        raise ValueError(f"unknown config C{cfg}")
    if cfg == 5:
        table_all = _tables(g, all_lens, pool, width)
    else:
        table = _tables(g, lens, pool, width, shared)
    if layers is not None:
        nlayers = layers
    vdev = torch.device(values_device) if values_device is not None else torch.device("cpu")
    vgen = g if vdev.type == "cpu" else torch.Generator(vdev).manual_seed(42 + cfg)
    if cfg == 5:
        q_dec = _values((16, 1, H, D), dtype, vgen, vdev)
        q_pre = _values((2, 512, H, D), dtype, vgen, vdev)
        if part == "decode":
            lens, table, query = dec, table_all[:16].clone(), q_dec
        elif part == "prefill":
            lens, table, query, q_len = pre, table_all[16:].clone(), q_pre, 512
        else:
            raise ValueError("part must be 'decode' or 'prefill'")
    else:
        query = _values((len(lens), 1, H, D), dtype, vgen, vdev)
    kcs, vcs = [], []
    for _ in range(nlayers):
        kcs.append(_values((pool, BLOCK, KVH, D), dtype, vgen, vdev).to(device))
        vcs.append(_values((pool, BLOCK, KVH, D), dtype, vgen, vdev).to(device))
    return Workload(
        name=f"C{cfg}" + (f"-{part}" if cfg == 5 else ""), cfg=cfg, num_heads=H,
        num_kv_heads=KVH, head_dim=D, dtype=dtype, batch=len(lens), q_len=q_len, lens=lens,
        table=table, num_blocks=pool, layers=nlayers, query=query.to(device), k_caches=kcs,
        v_caches=vcs, shared_prefix_pages=shared)
