"""Bucketed hipGraph decode over the paged-attention path.

Restates GraphedDecodeRunner (miniserve/model_runner.py:224-336) for the attention
path alone. A decode step over L layers is, per layer:
    write_kv(new k, v at position ctx[b])    (miniserve/attention.py:111-133)
    forward(q, caches, table, ctx + 1)       (miniserve/attention.py:205-250)
captured once per (bucket, input set) as a hipGraph through torch.cuda.CUDAGraph. The two
calls go through one msattn_paged_attention_append per layer (one launch where the
partition kernel takes the decode; `fused_append=False` keeps them apart).
Batches that are not a bucket size replay the next larger bucket with pad rows.

Kept from the reference: sorted buckets starting at 1 (ValueError otherwise), two
alternating static input sets (double buffering) with a `replay_log`, a shared graph
memory pool, static buffers sized for the largest bucket, `memory_report()`.

Differences, deliberate:
  * buckets go up to 64 by default (the bs-64 decode configuration);
  * every input the step reads lives in device buffers (int32 block tables, context
    lengths, write positions): the captured step never reads the host, which the
    reference's `.tolist()` and `int(...)` reads (model_runner.py:273,
    attention.py:131, :236) would;
  * pad rows (table -1, ctx 0) are true no-ops: write_kv skips hole pages and a
    row with no key gets zeros, where the reference's pad rows write into and read
    from the cache's last page: their context length becomes 1 through
    `row_starts = ctx` (model_runner.py:70-76, 273) and page id -1 wraps to
    num_blocks - 1 (attention.py:131-133, 171).
"""
from __future__ import annotations

from itertools import chain
from typing import List, Sequence

import numpy as np
import torch

from . import _native as nat
from .attention import PagedAttention, paged_attention, paged_attention_append


def fill_table(tab: np.ndarray, tables, batch: int) -> None:
    """Write the page ids of `batch` rows into the int32 array tab [rows >= batch, width]:
    row b's pages from column 0, every other entry -1 (a hole). `tables` is a sequence of
    per-row page-id sequences, or a 2-D array / tensor of page ids padded with -1. Ragged
    lists are placed with one scatter (no per-row arrays)."""
    width = tab.shape[1]
    tab.fill(-1)
    if isinstance(tables, (torch.Tensor, np.ndarray)):
        arr = tables.cpu().numpy() if isinstance(tables, torch.Tensor) else tables
        if arr.ndim != 2 or arr.shape[0] != batch or arr.shape[1] > width:
            raise ValueError(f"tables must be [{batch}, <= {width}] page ids")
        tab[:batch, : arr.shape[1]] = arr
        return
    rows = [r if isinstance(r, (list, tuple)) else list(r) for r in tables]
    if len(rows) != batch:
        raise ValueError(f"{len(rows)} table rows for a batch of {batch}")
    counts = np.fromiter((len(r) for r in rows), dtype=np.int64, count=batch)
    if batch and int(counts.max()) > width:
        b = int(counts.argmax())
        raise ValueError(f"row {b}: {int(counts[b])} pages > table width {width}")
    total = int(counts.sum())
    flat = np.fromiter(chain.from_iterable(rows), dtype=np.int32, count=total)
    row_of = np.repeat(np.arange(batch), counts)
    first = np.repeat(np.cumsum(counts) - counts, counts)
    tab[row_of, np.arange(total) - first] = flat


class DecodeLayer:
    """One layer's paged-attention state: the reference's _LayerState
    (miniserve/model_runner.py:88-95) without a block table of its own."""

    __slots__ = ("pa", "k_cache", "v_cache")

    def __init__(self, pa: PagedAttention, k_cache: torch.Tensor, v_cache: torch.Tensor):
        self.pa, self.k_cache, self.v_cache = pa, k_cache, v_cache


class GraphedDecodeRunner:
    """Bucketed hipGraph decode: one graph per bucket and input set, shared pool."""

    def __init__(self, layers: Sequence[DecodeLayer], table_width: int,
                 buckets: Sequence[int] = (1, 2, 4, 8, 16, 32, 64),
                 dtype: torch.dtype | None = None, fused_append: bool = True) -> None:
        """fused_append: each layer's write_kv and decode through one
        msattn_paged_attention_append call (one launch where the partition kernel takes
        it, the same caches and output bit for bit); False keeps the two calls."""
        buckets = list(buckets)
        if not buckets or sorted(buckets) != buckets or buckets[0] < 1:
            raise ValueError("buckets must be sorted, start at 1")
        if not layers:
            raise ValueError("at least one layer is needed")
        self.layers = list(layers)
        self.fused_append = bool(fused_append)
        self.buckets = tuple(buckets)
        self.max_batch = self.buckets[-1]
        self.table_width = int(table_width)
        self.replay_log: List[tuple[int, int]] = []
        self._buf_idx = 0
        self._graphs: dict[int, list] = {}
        self._pool = None
        pa0 = self.layers[0].pa
        kc0 = self.layers[0].k_cache
        if kc0.device.type != "cuda":
            raise RuntimeError("GraphedDecodeRunner needs caches on a ROCm GPU device")
        self._device = kc0.device
        self.block_size = kc0.shape[1]
        self.num_heads = pa0.num_heads
        self.num_kv_heads = kc0.shape[2]
        self.head_dim = kc0.shape[3]
        self.dtype = dtype or pa0.dtype
        L, Bm, H, KVH, D = (len(self.layers), self.max_batch, self.num_heads,
                            self.num_kv_heads, self.head_dim)
        dev = self._device

        Wt = self.table_width

        def input_set():
            # table, write positions and lengths share one int32 buffer, so a step's
            # integer inputs go to the device in one copy from one pinned staging buffer
            ints = torch.zeros(Bm * Wt + 2 * Bm, dtype=torch.int32, device=dev)
            ints[: Bm * Wt].fill_(-1)
            return {
                "q": torch.zeros((L, Bm, 1, H, D), dtype=self.dtype, device=dev),
                "k": torch.zeros((L, Bm, 1, KVH, D), dtype=self.dtype, device=dev),
                "v": torch.zeros((L, Bm, 1, KVH, D), dtype=self.dtype, device=dev),
                "ints": ints,
                "table": ints[: Bm * Wt].view(Bm, Wt),
                "start": ints[Bm * Wt: Bm * Wt + Bm],
                "lens": ints[Bm * Wt + Bm:],
            }

        self._in = [input_set() for _ in range(2)]
        # Host staging per input set (pinned; refilled only once that set's previous copy
        # has run, which its event records).
        self._stage = [torch.empty(Bm * Wt + 2 * Bm, dtype=torch.int32, pin_memory=True)
                       for _ in range(2)]
        self._stage_np = [t.numpy() for t in self._stage]
        self._stage_ev: list = [None, None]
        self._out = torch.zeros((L, Bm, 1, H, D), dtype=self.dtype, device=dev)
        self.max_context = self.table_width * self.block_size
        ws_bytes = max(nat.lib().msattn_workspace_bytes(b, 1, H, KVH, D, self.max_context)
                       for b in self.buckets)
        self._ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)

    # ---------------------------------------------------------------- step
    def _run_static(self, buf: dict, bucket: int) -> None:
        """One decode step over every layer, on static buffers only (captured)."""
        table = buf["table"][:bucket]
        start = buf["start"][:bucket]
        lens = buf["lens"][:bucket]
        for li, layer in enumerate(self.layers):
            if self.fused_append and buf["k"].dtype == buf["q"].dtype:
                # write_kv at lens - 1 (= start for real rows; pad rows have lens 0 and
                # write nothing) and the decode, in one launch where the partition
                # kernel takes the call
                paged_attention_append(buf["q"][li, :bucket], buf["k"][li, :bucket],
                                       buf["v"][li, :bucket], layer.k_cache, layer.v_cache,
                                       table, lens, window=layer.pa.window,
                                       max_context=self.max_context, workspace=self._ws,
                                       out=self._out[li, :bucket])
                continue
            layer.pa.write_kv(layer.k_cache, layer.v_cache, buf["k"][li, :bucket],
                              buf["v"][li, :bucket], table, start=start)
            paged_attention(buf["q"][li, :bucket], layer.k_cache, layer.v_cache, table, lens,
                            window=layer.pa.window, max_context=self.max_context,
                            workspace=self._ws, out=self._out[li, :bucket])

    def _bucket_fn(self, bucket: int, set_idx: int):
        """Capture the step for (bucket, input set); returns its replay callable."""
        dev = self._device
        buf = self._in[set_idx]
        # The warm-up below really runs the step on this set, which may still hold an
        # earlier decode's rows: their pages may since belong to other sequences, and
        # write_kv would overwrite those. Every row becomes a pad row first (all pages
        # holes, no context), so the warm-up writes and reads nothing; decode() fills the
        # set before any replay.
        buf["table"].fill_(-1)
        buf["start"].zero_()
        buf["lens"].zero_()
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):  # warm-up outside capture
            self._run_static(buf, bucket)
        torch.cuda.current_stream(dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        self._pool = self._pool or torch.cuda.graph_pool_handle()
        with torch.cuda.graph(graph, pool=self._pool):
            self._run_static(buf, bucket)
        return graph.replay

    # ---------------------------------------------------------------- API
    def decode(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
               tables: Sequence[Sequence[int]], ctx: Sequence[int],
               use_graph: bool = True) -> torch.Tensor:
        """One decode step for len(ctx) real rows.

        q [L, B, 1, H, D], k/v [L, B, 1, KVH, D]: the new token of every row and layer;
        tables: page ids per row (lists, or a 2-D int array / tensor whose rows are padded
        with -1); ctx: tokens already cached per row. Row b's new k/v land at position
        ctx[b] and it attends over ctx[b] + 1 tokens. Returns the attention output
        [L, B, 1, H, D]. Pad rows are padded to the bucket with table -1 and ctx 0 and
        produce nothing.
        """
        B = len(ctx)
        if B > self.max_batch:
            raise ValueError(f"batch {B} > max bucket {self.max_batch}")
        if B == 0:
            raise ValueError("empty batch")
        bucket = next(b for b in self.buckets if b >= B)
        if use_graph and bucket not in self._graphs:  # capture both sets lazily
            self._graphs[bucket] = [self._bucket_fn(bucket, i) for i in range(2)]
        idx = self._buf_idx
        self._buf_idx = 1 - self._buf_idx
        buf = self._in[idx]
        self._stage_inputs(idx, tables, ctx)
        buf["q"][:, :B].copy_(q)
        buf["k"][:, :B].copy_(k)
        buf["v"][:, :B].copy_(v)
        if use_graph:
            self._graphs[bucket][idx]()
        else:
            self._run_static(buf, bucket)  # eager reference on the same buffers
        self.replay_log.append((len(self.replay_log), idx))
        return self._out[:, :B].clone()

    def _stage_inputs(self, idx: int, tables, ctx: Sequence[int]) -> None:
        """Block tables, write positions and lengths of a step into input set idx: filled
        in its pinned staging buffer (vectorised, no per-row tensors) and sent in one
        asynchronous copy on the current stream."""
        Bm, Wt = self.max_batch, self.table_width
        B = len(ctx)
        ev = self._stage_ev[idx]
        if ev is not None:
            ev.synchronize()  # the staging buffer's previous copy has run
        st = self._stage_np[idx]
        fill_table(st[: Bm * Wt].reshape(Bm, Wt), tables, B)
        start = st[Bm * Wt: Bm * Wt + Bm]
        lens = st[Bm * Wt + Bm:]
        start.fill(0)
        start[:B] = np.fromiter((int(c) for c in ctx), dtype=np.int32, count=B)
        lens.fill(0)
        lens[:B] = start[:B] + 1
        top = int(lens[:B].max())
        if top > self.max_context:
            raise ValueError(f"context {top} > table capacity {self.max_context}")
        self._in[idx]["ints"].copy_(self._stage[idx], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        self._stage_ev[idx] = ev

    def memory_report(self) -> dict:
        """Static footprint: inputs are max-bucket-sized and shared by every bucket's
        graphs, so the total tracks the largest bucket, not the number of buckets."""
        nb = lambda t: t.element_size() * t.numel()
        per_set = sum(nb(self._in[0][name]) for name in ("q", "k", "v", "ints"))
        out_b = nb(self._out) + nb(self._ws)
        max_fp = per_set + out_b
        total = 2 * per_set + out_b
        return {"per_input_set_bytes": per_set, "output_bytes": out_b,
                "max_bucket_footprint_bytes": max_fp, "total_static_bytes": total,
                "total_over_max": total / max_fp, "buckets_captured": sorted(self._graphs),
                "shared_pool": self._pool is not None}
