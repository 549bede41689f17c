"""GPU parity for a query and a KV cache of different types.

The reference's forward casts the gathered K/V to the query dtype before attending
(miniserve/attention.py:240-241), so any (query, cache) pair is a valid call; its own
runner allocates fp32 caches (miniserve/model_runner.py:122-123) and is loaded with bf16
weights (bench/cuda_graph_tradeoff.py:60), which gives a bf16 query over an fp32 cache.

Bars (as in test_gpu_parity.py): fp32 query -> max-abs 1e-4, bf16/fp16 query -> max-rel
2e-2, both against the float64 oracle run on K/V cast to the query dtype first
(dense.paged_attention_f64(kv_cast=True)). On the MFMA kernels an fp32 cache is rounded to
the query type as it is loaded, so the result must also equal, bit for bit, the same call
over the cache converted to the query type beforehand.
"""
import numpy as np
import pytest
import torch

from miniserve_amd import PagedAttention, kernel_route, paged_attention
from oracle import dense, paged_sdpa

pytestmark = pytest.mark.gpu

FP32_ATOL = 1e-4
BF16_REL = 2e-2
Q_DTYPES = [torch.float32, torch.float16, torch.bfloat16]
KV_DTYPES = [torch.float32, torch.float16, torch.bfloat16, torch.float8_e4m3fn]
PAIRS = [(q, kv) for q in Q_DTYPES for kv in KV_DTYPES]


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def name(dt) -> str:
    return str(dt).replace("torch.", "")


def case(H, KVH, D, lens, q_dtype, kv_dtype, q_len=1, bs=16, width=None, seed=0):
    """Seeded q [B, q_len, H, D] in q_dtype; fp32 N(0, 1) K/V pools stored as kv_dtype;
    scattered block tables `width` pages wide."""
    g = torch.Generator().manual_seed(seed)
    need = sum((L + bs - 1) // bs for L in lens)
    pool = max(need, 1) + 5
    width = width or max(1, max((L + bs - 1) // bs for L in lens))
    q = torch.randn(len(lens), q_len, H, D, generator=g).to(q_dtype)
    kc = torch.randn(pool, bs, KVH, D, generator=g).to(kv_dtype)
    vc = torch.randn(pool, bs, KVH, D, generator=g).to(kv_dtype)
    perm = torch.randperm(pool, generator=g)
    table = torch.zeros(len(lens), width, dtype=torch.long)
    cur = 0
    for b, L in enumerate(lens):
        n = (L + bs - 1) // bs
        table[b, :n] = perm[cur:cur + n]
        cur += n
    return q, kc, vc, table


def check(out: torch.Tensor, ref: np.ndarray, q_dtype) -> float:
    o = out.double().cpu().numpy()
    if q_dtype == torch.float32:
        err = float(np.abs(o - ref).max())
        note(f"max-abs {err:.3e}")
        assert err < FP32_ATOL
    else:
        err = float(np.abs(o - ref).max() / max(np.abs(ref).max(), 1e-30))
        note(f"max-rel {err:.3e}")
        assert err < BF16_REL
    return err


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("q_dtype,kv_dtype", PAIRS)
def test_decode_every_pair(device, q_dtype, kv_dtype, D):
    """Decode (partition kernels: MFMA for a bf16/fp16 query over its own type, fp8 or
    fp32 and for an fp32 query over any cache, the generic kernel for fp16 over bf16 and
    bf16 over fp16) against the oracle with the cast; a row of
    context 1 returns exactly V[0] as the query type holds it."""
    H, KVH = 8, 2
    lens = [1, 17, 300, 1000, 0, 64]
    note(f"decode q={name(q_dtype)} kv={name(kv_dtype)} D={D}")
    q, kc, vc, table = case(H, KVH, D, lens, q_dtype, kv_dtype, seed=D)
    out = paged_attention(q.to(device), kc.to(device), vc.to(device), table, lens)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens, kv_cast=True)
    check(out, ref, q_dtype)
    v0 = vc[table[0, 0], 0].to(q_dtype)
    for h in range(H):
        assert torch.equal(out[0, 0, h].cpu(), v0[h // (H // KVH)])
    assert not out[4].any()


@pytest.mark.parametrize("q_dtype,kv_dtype", PAIRS)
def test_prefill_every_pair(device, q_dtype, kv_dtype):
    """Chunked prefill (q_len 24 x group 4 = 96 rows per KV head: the MFMA prefill kernel
    for a bf16/fp16 query over its own type, fp8 or fp32; the generic kernel otherwise),
    causal, against the oracle with the cast."""
    H, KVH, D, q_len = 16, 4, 128, 24
    lens = [24, 500, 131]
    note(f"prefill q={name(q_dtype)} kv={name(kv_dtype)}")
    q, kc, vc, table = case(H, KVH, D, lens, q_dtype, kv_dtype, q_len=q_len, seed=3)
    on_prefill_kernel = q_dtype != torch.float32 and kv_dtype in (q_dtype, torch.float32,
                                                                   torch.float8_e4m3fn)
    # an fp32 query over any cache: the fp32 MFMA partition kernel at 16 rows per tile
    want = ("prefill" if on_prefill_kernel else
            "partition-fused" if q_dtype == torch.float32 else "generic")
    route = kernel_route(q.to(device), kc.to(device), table, max_context=max(lens))
    assert route == want, (route, want)
    out = paged_attention(q.to(device), kc.to(device), vc.to(device), table, lens)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens, kv_cast=True)
    check(out, ref, q_dtype)


ROUTES = {  # name -> (H, KVH, D, lens, q_len, width in pages, prefix pages)
    "partition": (14, 2, 64, [5, 100, 1000, 333], 1, None, 0),
    "stream-K": (32, 8, 128, [3000, 17, 5000, 0, 800, 4096, 1, 2500], 1, 4096, 0),
    "prefill": (28, 4, 128, [512, 700], 64, None, 0),
    "cascade": (32, 8, 128, [5, 100, 1000, 333, 2000, 160, 161, 0], 1, 130, 10),
}


@pytest.mark.parametrize("route", list(ROUTES))
@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float16])
def test_fp32_cache_equals_converted_cache(device, route, q_dtype):
    """On every MFMA route an fp32 cache gives, bit for bit, the result of the same call
    over the cache converted to the query type first (the rounding happens in registers as
    the rows load), and that result is within the bar of the oracle."""
    H, KVH, D, lens, q_len, width, prefix = ROUTES[route]
    note(f"fp32 cache, {route}, q={name(q_dtype)}")
    q, kc, vc, table = case(H, KVH, D, lens, q_dtype, torch.float32, q_len=q_len,
                            width=width, seed=11)
    if prefix:
        table[:, :prefix] = table[0, :prefix]  # every row shares its first pages
    cap = table.shape[1] * 16
    kw = dict(max_context=cap, prefix_pages=prefix or None)
    qd = q.to(device)
    out32 = paged_attention(qd, kc.to(device), vc.to(device), table, lens, **kw)
    outc = paged_attention(qd, kc.to(q_dtype).to(device), vc.to(q_dtype).to(device), table,
                           lens, **kw)
    torch.cuda.synchronize()
    assert torch.equal(out32, outc)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens, kv_cast=True)
    check(out32, ref, q_dtype)


def _views(x: torch.Tensor, H: int, KVH: int, D: int):
    """q/k/v as the reference's runner makes them (model_runner.py:62-67): projections
    viewed [batch, seq, heads, D] and transposed to [batch, heads, seq, D]; `x` is one
    [batch, seq, (H + 2 KVH) * D] tensor, so every view is non-contiguous."""
    b, s, _ = x.shape
    parts = x.view(b, s, H + 2 * KVH, D)
    q = parts[:, :, :H].transpose(1, 2)
    k = parts[:, :, H:H + KVH].transpose(1, 2)
    v = parts[:, :, H + KVH:].transpose(1, 2)
    return q, k, v


@pytest.mark.parametrize("q_dtype,kv_dtype", [(torch.bfloat16, torch.float32),
                                              (torch.float32, torch.float32),
                                              (torch.bfloat16, torch.bfloat16)])
def test_model_runner_attention_lines(device, q_dtype, kv_dtype):
    """The attention lines of _paged_attention_forward (miniserve/model_runner.py:62-85) run
    unchanged over this PagedAttention, built as the runner builds it
    (model_runner.py:120-123: dtype=fp32, kv_dtype=fp32, allocate_kv_cache) and fed by a
    model of another dtype: first the prefill branch (write_kv of a 512-token chunk at
    `start`, forward over start + 512), then the batched-decode branch (write_kv at each
    row's start, forward over start + 1). Caches must equal the oracle's write_kv bit for
    bit, outputs the float64 oracle (K/V cast to the query dtype) within the bar."""
    H, KVH, D, bs, pool, W = 14, 2, 64, 16, 256, 64   # Qwen2.5-0.5B attention
    window = None
    g = torch.Generator().manual_seed(21)
    pa = PagedAttention(H, KVH, D, num_blocks=pool, block_size=bs, dtype=torch.float32,
                        kv_dtype=kv_dtype, device=device)
    k_cache, v_cache = pa.allocate_kv_cache()
    kc_ref = torch.zeros(k_cache.shape, dtype=kv_dtype)
    vc_ref = torch.zeros(v_cache.shape, dtype=kv_dtype)
    tables = torch.randperm(pool, generator=g)[: 4 * W].view(4, W)

    # --- prefill branch (model_runner.py:79-85), batch 1, a chunk after `start` tokens
    start, seq = 100, 512
    note(f"runner prefill q={name(q_dtype)} kv={name(kv_dtype)} start={start} seq={seq}")
    block_table = tables[:1].to(device)
    for chunk_start in (0, start):  # the first 100 tokens, then the 512-token chunk
        n = start if chunk_start == 0 else seq
        x = torch.randn(1, n, (H + 2 * KVH) * D, generator=g).to(q_dtype)
        q, k, v = _views(x.to(device), H, KVH, D)
        assert not q.transpose(1, 2).is_contiguous()
        pa.write_kv(k_cache, v_cache, k.transpose(1, 2), v.transpose(1, 2), block_table,
                    start=chunk_start)
        ctx_len = chunk_start + n
        out = pa.forward(q.transpose(1, 2), k_cache, v_cache, block_table, [ctx_len],
                         window=window)
        out = out.reshape(1, n, -1).contiguous()
        qc, kcpu, vcpu = _views(x, H, KVH, D)
        paged_sdpa.write_kv(kc_ref, vc_ref, kcpu.transpose(1, 2), vcpu.transpose(1, 2),
                            tables[:1], start=chunk_start)
        assert torch.equal(k_cache.cpu(), kc_ref) and torch.equal(v_cache.cpu(), vc_ref)
        ref = dense.paged_attention_f64(qc.transpose(1, 2), kc_ref, vc_ref, tables[:1],
                                        [ctx_len], kv_cast=True)
        check(out.view(1, n, H, D), ref, q_dtype)

    # --- batched-decode branch (model_runner.py:70-78): four rows, ragged starts
    row_starts = [start + seq, 37, 250, 1]
    block_table = tables.to(device)
    for step in range(3):
        note(f"runner decode step {step} starts={row_starts}")
        x = torch.randn(4, 1, (H + 2 * KVH) * D, generator=g).to(q_dtype)
        q, k, v = _views(x.to(device), H, KVH, D)
        pa.write_kv(k_cache, v_cache, k.transpose(1, 2), v.transpose(1, 2), block_table,
                    start=row_starts)
        out = pa.forward(q.transpose(1, 2), k_cache, v_cache, block_table,
                         [s + 1 for s in row_starts], window=window)
        out = out.reshape(4, 1, -1).contiguous()
        qc, kcpu, vcpu = _views(x, H, KVH, D)
        paged_sdpa.write_kv(kc_ref, vc_ref, kcpu.transpose(1, 2), vcpu.transpose(1, 2), tables,
                            start=row_starts)
        assert torch.equal(k_cache.cpu(), kc_ref) and torch.equal(v_cache.cpu(), vc_ref)
        ref = dense.paged_attention_f64(qc.transpose(1, 2), kc_ref, vc_ref, tables,
                                        [s + 1 for s in row_starts], kv_cast=True)
        check(out.view(4, 1, H, D), ref, q_dtype)
        row_starts = [s + 1 for s in row_starts]


@pytest.mark.parametrize("route", ["partition", "stream-K"])
@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float16, torch.float8_e4m3fn])
def test_fp32_query_narrow_cache_equals_widened(device, route, kv_dtype):
    """An fp32 query over a bf16/fp16/fp8 cache runs the fp32 MFMA decode kernels on the
    cache's rows widened exactly in registers (the reference's .to(query.dtype),
    miniserve/attention.py:240-241). The same call over the cache converted to fp32
    beforehand gives the same result: bit for bit for a 2-byte cache, whose head-dim split
    across the MFMA steps is the fp32 cache's; within 1e-6 relative for fp8, whose split
    differs (so the fp32 sums run in another order). Both are within max-abs 1e-4 of the
    float64 oracle."""
    H, KVH, D, lens, q_len, width, _ = ROUTES[route]
    note(f"fp32 query over {name(kv_dtype)}, {route}")
    q, kc, vc, table = case(H, KVH, D, lens, torch.float32, kv_dtype, q_len=q_len,
                            width=width, seed=13)
    cap = table.shape[1] * 16
    qd = q.to(device)
    out_n = paged_attention(qd, kc.to(device), vc.to(device), table, lens, max_context=cap)
    out_w = paged_attention(qd, kc.float().to(device), vc.float().to(device), table, lens,
                            max_context=cap)
    torch.cuda.synchronize()
    if kv_dtype == torch.float8_e4m3fn:
        diff = float((out_n - out_w).abs().max() / out_w.abs().max())
        note(f"fp8 against widened: {diff:.3e}")
        assert diff < 1e-6
    else:
        assert torch.equal(out_n, out_w)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens, kv_cast=True)
    check(out_n, ref, torch.float32)
