"""GPU parity: the HIP path (libmsattn.so through PagedAttention) against the oracle.

Bars (written into each test):
  * gather / write_kv addressing: bit-exact (torch.equal);
  * fp32: max-abs error <= 1e-4 against the float64 oracle;
  * bf16 / fp16: max|out - ref| / max|ref| <= 2e-2 against the float64 oracle
    on the same (already rounded) inputs;
  * the reference's own gates where it states them (tests/test_parity.py:120-192,
    tests/test_triton_parity.py:55-123).
"""
import math

import numpy as np
import pytest
import torch

from miniserve_amd import PagedAttention, gather_kv, kernel_route, paged_attention
from miniserve_amd import _native as nat
from miniserve_amd.workloads import make_workload
from oracle import dense, paged_sdpa, split_k

# Decodes whose table capacity (batch x KV heads x table tiles) reaches this run on the
# stream-K kernel (MSATTN_STREAMK_MIN_TILES in csrc/abi.hip); smaller ones on the partition
# kernel. Tests that mean to reach stream-K size their tables from it.
SK_MIN_TILES = 1 << 18

pytestmark = pytest.mark.gpu

FP32_ATOL = 1e-4
BF16_REL = 2e-2


def rel_err(out: torch.Tensor, ref: np.ndarray) -> float:
    o = out.double().cpu().numpy()
    return float(np.abs(o - ref).max() / max(np.abs(ref).max(), 1e-30))


def abs_err(out: torch.Tensor, ref: np.ndarray) -> float:
    return float(np.abs(out.double().cpu().numpy() - ref).max())


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def scenario(h, kv_heads, d, lens, q_len=1, block_size=8, dtype=torch.float32, seed=0,
             scale=1.0, kv_dtype=None, scatter=True):
    """CPU inputs: seeded q + dense k/v written into a paged cache by the oracle."""
    g = torch.Generator().manual_seed(seed)
    kv_dtype = dtype if kv_dtype is None else kv_dtype
    batch, max_l = len(lens), max(lens)
    nblocks = max(1, (max_l + block_size - 1) // block_size)
    q = (torch.randn(batch, q_len, h, d, generator=g) * scale).to(dtype)
    k = torch.randn(batch, max_l, kv_heads, d, generator=g) * scale
    v = torch.randn(batch, max_l, kv_heads, d, generator=g) * scale
    pool = batch * nblocks
    kc = torch.zeros(pool, block_size, kv_heads, d, dtype=kv_dtype)
    vc = torch.zeros(pool, block_size, kv_heads, d, dtype=kv_dtype)
    order = torch.randperm(pool, generator=g) if scatter else torch.arange(pool)
    table = order.view(batch, nblocks).clone()
    for i, length in enumerate(lens):
        paged_sdpa.write_kv(kc, vc, k[i:i + 1, :length], v[i:i + 1, :length], table[i:i + 1], 0)
    return q, kc, vc, table, lens


def run_hip(device, q, kc, vc, table, lens, **kw):
    return paged_attention(q.to(device), kc.to(device), vc.to(device), table, lens, **kw)


# Workspace header word 0 after a call: the layout the partials kernel recorded (0 the
# partition kernels, 1 stream-K, 2 the partition kernel merging in-kernel); the prefill
# kernel leaves it untouched (its stream-K schedule uses only the tickets and partials).
_SENTINEL = 0x5EED
_SK = "prefill stream-K"
_KIND_OF_ROUTE = {"prefill": _SENTINEL, "prefill stream-K": _SENTINEL, "partition-fused": 2,
                  "partition": 0, "generic": 0, "stream-K": 1}


def run_routed(device, want, q, kc, vc, table, lens, **kw):
    """run_hip, after checking that the call takes kernel route `want` (as the library
    reports it for this shape, and as the workspace header shows after the call)."""
    qd, kcd, vcd = q.to(device), kc.to(device), vc.to(device)
    B, q_len, H, D = q.shape
    max_ctx = kw.get("max_context") or max(lens)
    got = kernel_route(qd, kcd, table, max_context=max_ctx)
    assert got == want, f"route {got}, expected {want}"
    ws_bytes = nat.lib().msattn_workspace_bytes(B, q_len, H, kc.shape[2], D, max_ctx)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=device)
    ws[:4].view(torch.int32).fill_(_SENTINEL)
    out = paged_attention(qd, kcd, vcd, table, lens, workspace=ws, **kw)
    kind = int(ws[:4].view(torch.int32).item())
    assert kind == _KIND_OF_ROUTE[want], f"header kind {kind} after route {want}"
    return out


# ------------------------------------------------------------------ addressing

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float8_e4m3fn])
def test_gather_bit_exact(device, dtype):
    note(f"gather {dtype}")
    g = torch.Generator().manual_seed(21)
    nb, bs, kvh, d = 40, 16, 2, 64
    bits = {torch.float32: torch.int32, torch.bfloat16: torch.int16,
            torch.float8_e4m3fn: torch.uint8}[dtype]
    if bits == torch.uint8:
        raw = torch.randint(0, 256, (nb, bs, kvh, d), generator=g, dtype=torch.uint8)
    else:
        info = torch.iinfo(bits)
        raw = torch.randint(info.min, info.max, (nb, bs, kvh, d), generator=g, dtype=bits)
    cache = raw.view(dtype)
    table = torch.randperm(nb, generator=g)[:36].view(3, 12)
    lens = [190, 17, 1]
    got = gather_kv(cache.to(device), table, lens, max_context=190)
    want = paged_sdpa.gather(cache, table, torch.tensor(lens), 190)
    assert torch.equal(got.cpu().view(bits), want.view(bits))


@pytest.mark.parametrize("src,dst", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.float32, torch.bfloat16), (torch.float32, torch.float16),
                                     (torch.float16, torch.float32)])
def test_write_kv_bit_exact(device, src, dst):
    note(f"write_kv {src}->{dst}")
    g = torch.Generator().manual_seed(22)
    nb, bs, kvh, d = 30, 16, 2, 32
    pa = PagedAttention(4, kvh, d, num_blocks=nb, block_size=bs, kv_dtype=dst, device=device)
    kc, vc = pa.allocate_kv_cache()
    k = (torch.randn(3, 20, kvh, d, generator=g) * 3).to(src)
    v = (torch.randn(3, 20, kvh, d, generator=g) * 3).to(src)
    table = torch.randperm(nb, generator=g)[:9].view(3, 3)
    starts = [0, 5, 27]
    pa.write_kv(kc, vc, k.to(device), v.to(device), table.to(device), start=starts)
    kc_ref = torch.zeros(nb, bs, kvh, d, dtype=dst)
    vc_ref = torch.zeros(nb, bs, kvh, d, dtype=dst)
    paged_sdpa.write_kv(kc_ref, vc_ref, k, v, table, start=starts)
    assert torch.equal(kc.cpu(), kc_ref) and torch.equal(vc.cpu(), vc_ref)


def test_write_kv_skips_holes(device):
    """Pad rows (table -1) write nothing -- unlike the reference's wraparound."""
    note("write_kv holes")
    pa = PagedAttention(2, 2, 16, num_blocks=4, block_size=16, kv_dtype=torch.float32,
                        device=device)
    kc, vc = pa.allocate_kv_cache()
    k = torch.ones(2, 1, 2, 16, device=device)
    table = torch.tensor([[1], [-1]], device=device)
    pa.write_kv(kc, vc, k, k, table, start=[3, 0])
    assert kc[1, 3].eq(1).all() and kc.sum().item() == 32 and vc.sum().item() == 32


# ------------------------------------------------------------------ reference gates

def test_mha_ragged_q_len3(device):
    """tests/test_parity.py:120-128 (MHA, ragged, q_len 3, block 8) at 1e-4."""
    note("mha q_len=3")
    q, kc, vc, table, lens = scenario(8, 8, 16, [8, 13, 21], q_len=3)
    out = run_hip(device, q, kc, vc, table, lens)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens)
    assert abs_err(out, ref) < FP32_ATOL


def test_gqa_32_8(device):
    """tests/test_parity.py:131-141 (GQA 32q/8kv, D 64): gate 1e-3, checked at 1e-4."""
    note("gqa 32/8")
    q, kc, vc, table, lens = scenario(32, 8, 64, [32, 47])
    out = run_hip(device, q, kc, vc, table, lens)
    assert abs_err(out, dense.paged_attention_f64(q, kc, vc, table, lens)) < FP32_ATOL


def test_mqa(device):
    """tests/test_parity.py:144-153 (MQA 8q/1kv, D 32)."""
    note("mqa")
    q, kc, vc, table, lens = scenario(8, 1, 32, [16, 23])
    out = run_hip(device, q, kc, vc, table, lens)
    assert abs_err(out, dense.paged_attention_f64(q, kc, vc, table, lens)) < FP32_ATOL


def test_sliding_window(device):
    """tests/test_parity.py:156-171: window 64 over ctx 512, q_len 2, block 16."""
    note("window")
    q, kc, vc, table, lens = scenario(4, 4, 16, [512, 300], q_len=2, block_size=16)
    pa = PagedAttention(4, 4, 16, num_blocks=kc.shape[0], block_size=16, window=64,
                        dtype=torch.float32, kv_dtype=torch.float32, device=device)
    out = pa.forward(q.to(device), kc.to(device), vc.to(device), table, lens)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens, window=64)
    assert abs_err(out, ref) < FP32_ATOL


def test_fp8_kv_vs_fp16(device):
    """tests/test_parity.py:174-192: FP8 e4m3 cache within 5e-2 of the FP16 cache."""
    note("fp8")
    kw = dict(q_len=1, block_size=8, dtype=torch.float16, seed=3, scale=0.25, scatter=False)
    q, kc16, vc16, table, lens = scenario(4, 2, 32, [16, 24], kv_dtype=torch.float16, **kw)
    q8, kc8, vc8, _, _ = scenario(4, 2, 32, [16, 24], kv_dtype=torch.float8_e4m3fn, **kw)
    assert torch.equal(q, q8)
    out16 = run_hip(device, q, kc16, vc16, table, lens)
    out8 = run_hip(device, q8, kc8, vc8, table, lens)
    assert (out16.float() - out8.float()).abs().max().item() < 5e-2
    # and the fp8 path itself matches the float64 oracle on the fp8 values
    ref8 = dense.paged_attention_f64(q8, kc8, vc8, table, lens)
    assert rel_err(out8, ref8) < BF16_REL


def test_triton_flash_backend_and_rope(device):
    """backend="triton_flash" keeps the reference contract and its fused-RoPE result
    (tests/test_triton_parity.py:71-81, :165-177)."""
    note("triton_flash rope")
    ctx, D = 300, 64
    q, kc, vc, table, _ = scenario(4, 2, D, [ctx], block_size=16)
    inv = 1.0 / (10000 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    emb = torch.outer(torch.arange(ctx + 1, dtype=torch.float32), inv)
    emb = torch.cat([emb, emb], dim=-1)
    cos, sin = torch.cos(emb), torch.sin(emb)
    pos = torch.tensor([ctx - 1])
    pa = PagedAttention(4, 2, D, num_blocks=kc.shape[0], block_size=16, dtype=torch.float32,
                        kv_dtype=torch.float32, device=device)
    got = pa.forward(q.to(device), kc.to(device), vc.to(device), table, [ctx],
                     backend="triton_flash", cos=cos.to(device), sin=sin.to(device),
                     position=pos.to(device))
    ref = split_k.split_k_decode(q, kc, vc, table, [ctx], cos=cos, sin=sin, position=pos)
    assert (got.cpu() - ref).abs().max().item() < 1e-4


@pytest.mark.parametrize("H,KVH,D,dtype,wide,window", [
    (32, 8, 128, torch.bfloat16, True, None),    # stream-K kernel
    (32, 8, 128, torch.bfloat16, True, 200),     # stream-K kernel, sliding window
    (14, 2, 64, torch.bfloat16, False, None),    # partition kernel
    (28, 4, 128, torch.float16, False, None),    # partition kernel, fp16 query
    (28, 4, 128, torch.float16, True, None),     # stream-K kernel, fp16 query
])
def test_fp8_kv_mfma_equals_dequantized(device, H, KVH, D, dtype, wide, window):
    """An fp8 (e4m3fn) cache on the MFMA decode kernels, widened in registers, gives the
    result of the same kernels on the cache converted to the query type first
    (miniserve/attention.py:168-170 then .to(q.dtype)) to summation order, and the float64
    oracle's within tolerance. The two runs differ in summation order only: for an fp8 cache
    the score MFMAs group the head dims differently (each lane's chunks contiguous in the
    row), and stream-K splits the work over 8 waves per CU instead of 4; so they agree
    within two output ulps. (The widening itself is checked bit for bit on the prefill
    kernel, test_fp8_kv_prefill_equals_dequantized, which shares it.)"""
    note(f"fp8 MFMA H={H} KVH={KVH} D={D} {dtype} wide={wide} window={window}")
    lens = [0, 1, 17, 300, 1234, 77, 4096, 999]
    width = SK_MIN_TILES // (len(lens) * KVH) + 1 if wide else (max(lens) + 15) // 16
    q, kc, vc, table = wide_table_case(H, KVH, D, lens, dtype, width, seed=D + KVH)
    kc8, vc8 = kc.to(torch.float8_e4m3fn), vc.to(torch.float8_e4m3fn)
    kd, vd = kc8.to(dtype), vc8.to(dtype)
    cap = width * 16
    qd = q.to(device)
    got = paged_attention(qd, kc8.to(device), vc8.to(device), table, lens, window=window,
                          max_context=cap)
    want = paged_attention(qd, kd.to(device), vd.to(device), table, lens, window=window,
                           max_context=cap)
    assert rel_err(got, want.double().cpu().numpy()) < 2.0 ** -7
    ref = dense.paged_attention_f64(q, kc8, vc8, table, lens, window=window)
    assert rel_err(got, ref) < BF16_REL
    assert not got[0].any()


@pytest.mark.parametrize("B,H,KVH,D,q_len,kv_dtype", [
    (8, 28, 4, 128, 4, torch.bfloat16),      # 28 rows per KV head, 32 (sequence, KV head)s
    (4, 32, 8, 128, 16, torch.bfloat16),     # 64 rows: four 16-row tiles
    (32, 14, 2, 64, 3, torch.bfloat16),      # head_dim 64
    (16, 32, 8, 128, 5, torch.float8_e4m3fn),
])
def test_speculative_rows_on_partition_kernel(device, B, H, KVH, D, q_len, kv_dtype):
    """Multi-token queries (speculative decoding: q_len 3-16, more than 16 rows per KV head)
    over few (sequence, KV head) pairs take the partition kernel's 16-row tiles, which
    split the keys over many workgroups, rather than the prefill kernel's one workgroup per
    128-row block: the header must name the in-kernel-merge route, and the causal result
    must meet the float64 oracle's bar."""
    g = torch.Generator().manual_seed(B * q_len)
    lens = [int(x) for x in torch.randint(max(q_len, 900), 6001, (B,), generator=g)]
    bs = 16
    width = (max(lens) + bs - 1) // bs + 1
    note(f"speculative rows B={B} H={H} KVH={KVH} D={D} q_len={q_len} kv={kv_dtype}")
    q, kc, vc, table = paged_case(H, KVH, D, lens, torch.bfloat16, bs, width, seed=B + q_len,
                                  q_len=q_len)
    kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=device)
    out = paged_attention(q.to(device), kc.to(device), vc.to(device), table, lens,
                          max_context=width * bs, workspace=ws)
    torch.cuda.synchronize()
    assert int(ws[:4].view(torch.int32).item()) == 2  # partition kernel, merged in-kernel
    ref = dense.paged_attention_f64(q, kc, vc, table, lens)
    err = rel_err(out, ref)
    note(f"speculative rows max-rel {err:.3e}")
    assert err < BF16_REL


@pytest.mark.parametrize("H,KVH,D,q_len,dtype,causal,window,prefix", [
    (28, 4, 128, 512, torch.bfloat16, True, None, 0),     # chunked prefill (C5 shape)
    (32, 8, 128, 100, torch.float16, True, 64, 0),        # fp16 query, sliding window
    (16, 2, 128, 96, torch.bfloat16, False, None, 0),     # non-causal
    (14, 2, 64, 200, torch.bfloat16, True, None, 0),      # head_dim 64
    (32, 8, 128, 1, torch.bfloat16, True, None, 12),      # cascade decode: the prefix pass
])
def test_fp8_kv_prefill_equals_dequantized(device, H, KVH, D, q_len, dtype, causal, window,
                                           prefix):
    """The MFMA prefill kernel (and the cascade's shared-prefix pass, which runs on it) over
    an fp8 cache widens the chunks exactly as it stages them: bit-exact against the same
    kernel on the cache converted to the query type, and within tolerance of the oracle.
    A cascade decode's suffix pass runs on the decode kernels, whose fp8 split of the head
    dims over the score MFMAs differs from the 2-byte one: there the whole result agrees to
    summation order (two output ulps)."""
    note(f"fp8 prefill H={H} KVH={KVH} D={D} q_len={q_len} {dtype} causal={causal} "
         f"window={window} prefix={prefix}")
    bs = 16
    lens = [max(q_len, L) for L in (700, 2048, 1031, 4096)]
    if prefix:
        q, kc, vc, table = shared_prefix_case(H, KVH, D, lens, dtype, bs, prefix, 260, seed=21)
    else:
        q, kc, vc, table = paged_case(H, KVH, D, lens, dtype, bs, (max(lens) + bs - 1) // bs + 1,
                                      seed=20, q_len=q_len)
    kc8, vc8 = kc.to(torch.float8_e4m3fn), vc.to(torch.float8_e4m3fn)
    kd, vd = kc8.to(dtype), vc8.to(dtype)
    cap = table.shape[1] * bs
    kw = dict(causal=causal, window=window, max_context=cap)
    if prefix:
        kw["prefix_pages"] = prefix
    qd = q.to(device)
    got = paged_attention(qd, kc8.to(device), vc8.to(device), table, lens, **kw)
    want = paged_attention(qd, kd.to(device), vd.to(device), table, lens, **kw)
    if prefix:
        assert rel_err(got, want.double().cpu().numpy()) < 2.0 ** -7
    else:
        assert torch.equal(got, want)
    ref = dense.paged_attention_f64(q, kc8, vc8, table, lens, causal=causal, window=window)
    assert rel_err(got, ref) < BF16_REL


def rope_tables(max_pos, D, base=10000.0):
    inv = 1.0 / (base ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    emb = torch.outer(torch.arange(max_pos, dtype=torch.float32), inv)
    emb = torch.cat([emb, emb], dim=-1)
    return torch.cos(emb), torch.sin(emb)


def rope_unfused(q, cos, sin, pos):
    """(q * cos + rotate_half(q) * sin).to(q.dtype) per row, every op rounded in fp32
    (miniserve/attention.py:41-62)."""
    D = q.shape[-1]
    qf = q.float()
    rot = torch.cat([-qf[..., D // 2:], qf[..., : D // 2]], dim=-1)
    cs = cos[pos][:, None, None, :]
    sn = sin[pos][:, None, None, :]
    return (qf * cs + rot * sn).to(q.dtype)


@pytest.mark.parametrize("H,KVH,D,dtype,kv_dtype,wide", [
    (32, 8, 128, torch.bfloat16, torch.bfloat16, True),    # stream-K MFMA kernel
    (14, 2, 64, torch.bfloat16, torch.bfloat16, False),    # partition MFMA kernel
    (28, 4, 128, torch.float16, torch.float16, False),     # partition MFMA kernel, fp16
    (4, 2, 64, torch.float32, torch.float32, False),       # partition MFMA kernel, fp32
    (32, 8, 128, torch.float32, torch.float32, True),      # stream-K MFMA kernel, fp32
    (4, 2, 96, torch.float32, torch.float32, False),       # generic kernel, fp32
    (8, 2, 96, torch.bfloat16, torch.float8_e4m3fn, False),  # generic kernel, fp8 KV
    # fp8 KV on the MFMA kernels: the query's chunks follow the fp8 split of the head dims,
    # so the rotate-half partner comes from the other half-wave
    (32, 8, 128, torch.bfloat16, torch.float8_e4m3fn, True),   # stream-K
    (14, 2, 64, torch.bfloat16, torch.float8_e4m3fn, False),   # partition, head_dim 64
    (28, 4, 128, torch.float16, torch.float8_e4m3fn, False),   # partition, fp16 query
    (14, 2, 64, torch.float32, torch.float8_e4m3fn, False),    # fp32 query over fp8
    (32, 8, 128, torch.float32, torch.bfloat16, True),         # stream-K, fp32 over bf16
])
def test_rope_in_kernel_matches_unfused(device, H, KVH, D, dtype, kv_dtype, wide):
    """RoPE applied inside the decode kernels equals attention over the query rotated
    beforehand (tests/test_triton_parity.py:71-81 asks 1e-4; here bit-exact), and the
    float64 oracle over the rotated query."""
    note(f"rope H={H} KVH={KVH} D={D} {dtype} kv={kv_dtype} wide={wide}")
    lens = [1, 300, 77, 1234, 16, 999]
    width = SK_MIN_TILES // (len(lens) * KVH) + 1 if wide else (max(lens) + 15) // 16
    q, kc, vc, table = wide_table_case(H, KVH, D, lens, dtype, width, seed=D + H)
    if kv_dtype != dtype:
        kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
    cos, sin = rope_tables(max(lens) + 8, D)
    pos = torch.tensor([L - 1 for L in lens])
    cap = width * 16
    fused = paged_attention(q.to(device), kc.to(device), vc.to(device), table, lens,
                            max_context=cap, rope=(cos.to(device), sin.to(device), pos.to(device)))
    qr = rope_unfused(q, cos, sin, pos)
    unfused = paged_attention(qr.to(device), kc.to(device), vc.to(device), table, lens,
                              max_context=cap)
    assert torch.equal(fused, unfused)
    ref = dense.paged_attention_f64(qr, kc, vc, table, lens)
    assert rel_err(fused, ref) < (1e-4 if dtype == torch.float32 else BF16_REL)


@pytest.mark.parametrize("D", [6, 40, 80, 112, 200, 256])
@pytest.mark.parametrize("dtype,kv_dtype", [
    (torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
    (torch.float16, torch.float8_e4m3fn)])
def test_any_even_head_dim(device, D, dtype, kv_dtype):
    """Head sizes outside the MFMA kernels' 64 / 128 (miniserve/attention.py:87-88 accepts
    any even head_dim): decode, chunked prefill (causal, windowed) and fused RoPE on the
    generic kernel's element mode (a capacity of 16, 64, 128 or 256 dims with the dims
    past head_dim masked), each against the float64 oracle."""
    H, KVH = 8, 2
    bar = 1e-4 if dtype == torch.float32 else BF16_REL
    err = abs_err if dtype == torch.float32 else rel_err
    for q_len, lens, window in ((1, [1, 17, 300, 1000, 0, 64], None), (24, [24, 300, 90], None),
                                (20, [500, 33], 64)):
        note(f"head_dim {D}: {dtype} over {kv_dtype}, q_len={q_len} lens={lens} "
             f"window={window}")
        width = max((L + 15) // 16 for L in lens) + 2
        q, kc, vc, table = paged_case(H, KVH, D, lens, dtype, 16, width, seed=D + q_len,
                                      q_len=q_len)
        kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
        out = run_routed(device, "generic", q, kc, vc, table, lens, window=window)
        ref = dense.paged_attention_f64(q, kc.to(dtype), vc.to(dtype), table, lens,
                                        window=window)
        assert err(out, ref) < bar
        if q_len == 1:
            assert not out[4].any()  # context 0
            v0 = vc[table[0, 0], 0].to(dtype)
            for h in range(H):       # context 1: exactly V[0]
                assert torch.equal(out[0, 0, h].cpu(), v0[h // (H // KVH)])
    # fused RoPE on the element mode: the partner of dim d is d +- D / 2
    lens = [1, 300, 77]
    q, kc, vc, table = paged_case(H, KVH, D, lens, dtype, 16, 20, seed=D)
    kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
    cos, sin = rope_tables(max(lens) + 8, D)
    pos = torch.tensor([L - 1 for L in lens])
    fused = paged_attention(q.to(device), kc.to(device), vc.to(device), table, lens,
                            rope=(cos.to(device), sin.to(device), pos.to(device)))
    qr = rope_unfused(q, cos, sin, pos)
    unfused = paged_attention(qr.to(device), kc.to(device), vc.to(device), table, lens)
    assert torch.equal(fused, unfused)


def test_generic_kernel_rows_off_16_byte_boundaries(device):
    """Cache views whose rows do not start on 16-byte boundaries (a bf16 pool padded to
    head_dim + 3 per head, viewed as [.., KVH, 64]: 134-byte head stride) are accepted, as
    the reference's indexing accepts any strided cache, and read element by element on
    the generic kernel; decode and prefill against the float64 oracle."""
    H, KVH, D, pad = 8, 2, 64, 3
    lens = [5, 300, 1000]
    for q_len in (1, 24):
        note(f"padded cache rows: q_len={q_len}")
        q, kc, vc, table = paged_case(H, KVH, D, lens, torch.bfloat16, 16, 70, seed=q_len)
        kpad = torch.zeros(kc.shape[0], 16, KVH, D + pad, dtype=torch.bfloat16)
        vpad = torch.zeros_like(kpad)
        kpad[..., :D], vpad[..., :D] = kc, vc
        kd, vd = kpad.to(device)[..., :D], vpad.to(device)[..., :D]
        assert kd.stride(2) * 2 % 16 != 0
        assert kernel_route(q.to(device), kd, table) == "generic"
        out = paged_attention(q.to(device), kd, vd, table, lens)
        ref = dense.paged_attention_f64(q, kc, vc, table, lens)
        assert rel_err(out, ref) < BF16_REL


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_rope_in_kernel_wide_partition_shape(device, kv_dtype):
    """Fused RoPE on the partition kernel's wide shape (8 waves over 1024-token partitions:
    few (sequence, KV head) pairs over a long table), bit-exact against the query rotated
    beforehand, and the workspace header naming that shape."""
    H, KVH, D, dtype = 28, 4, 128, torch.bfloat16
    lens = [1, 3000, 77, 9000, 1025, 10240]
    width = 640  # 10240 tokens: 24 (sequence, KV head) pairs, ten 1024-token partitions
    note(f"rope wide partition shape kv={kv_dtype}")
    q, kc, vc, table = wide_table_case(H, KVH, D, lens, dtype, width, seed=77)
    kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
    cos, sin = rope_tables(max(lens) + 8, D)
    pos = torch.tensor([L - 1 for L in lens])
    cap = width * 16
    ws = torch.zeros(64 << 20, dtype=torch.uint8, device=device)
    fused = paged_attention(q.to(device), kc.to(device), vc.to(device), table, lens,
                            max_context=cap, workspace=ws,
                            rope=(cos.to(device), sin.to(device), pos.to(device)))
    torch.cuda.synchronize()
    hdr = ws[:64].view(torch.int32).cpu()
    assert (int(hdr[0]), int(hdr[8]), int(hdr[9])) == (2, 1024, 8), hdr[:10].tolist()
    qr = rope_unfused(q, cos, sin, pos)
    unfused = paged_attention(qr.to(device), kc.to(device), vc.to(device), table, lens,
                              max_context=cap)
    assert torch.equal(fused, unfused)
    ref = dense.paged_attention_f64(qr, kc, vc, table, lens)
    assert rel_err(fused, ref) < BF16_REL


@pytest.mark.parametrize("H,KVH,D,dtype,wide", [
    (32, 8, 128, torch.bfloat16, True),     # stream-K MFMA kernel
    (14, 2, 64, torch.bfloat16, False),     # partition MFMA kernel
    (28, 4, 128, torch.float16, False),     # partition MFMA kernel, fp16
])
def test_rope_low_precision_against_fp32_rotation(device, H, KVH, D, dtype, wide):
    """The reference's fused RoPE keeps the rotated query in fp32
    (kernels/paged_attn_triton.py:211-220; flash_decode_reference :134-138), while the
    MFMA kernels round it to the query type to feed the bf16/fp16 matrix cores: one
    rounding of the rotated query (relative 2^-9 for bf16). Against the oracle's split-K
    decode with the fp32 rotation (split_k.split_k_decode) the result stays within the
    2e-2 max-rel bar."""
    note(f"rope vs fp32 rotation H={H} KVH={KVH} D={D} {dtype} wide={wide}")
    lens = [1, 300, 77, 1234, 16, 999]
    width = SK_MIN_TILES // (len(lens) * KVH) + 1 if wide else (max(lens) + 15) // 16
    q, kc, vc, table = wide_table_case(H, KVH, D, lens, dtype, width, seed=D + H + 1)
    cos, sin = rope_tables(max(lens) + 8, D)
    pos = torch.tensor([L - 1 for L in lens])
    fused = paged_attention(q.to(device), kc.to(device), vc.to(device), table, lens,
                            max_context=width * 16,
                            rope=(cos.to(device), sin.to(device), pos.to(device)))
    ref = split_k.split_k_decode(q, kc, vc, table, lens, cos=cos, sin=sin, position=pos)
    err = rel_err(fused, ref.double().numpy())
    note(f"max-rel {err:.3e}")
    assert err < BF16_REL


def test_rope_contract(device):
    """Decode-only, as the reference's fused path; malformed tables are rejected."""
    q, kc, vc, table, _ = scenario(4, 2, 64, [40], block_size=16)
    cos, sin = rope_tables(64, 64)
    args = (q.to(device), kc.to(device), vc.to(device), table, [40])
    pos = torch.tensor([39], device=device)
    q2 = torch.zeros(1, 2, 4, 64, device=device)
    with pytest.raises(ValueError, match="decode-only"):
        paged_attention(q2, *args[1:], rope=(cos.to(device), sin.to(device), pos))
    with pytest.raises(ValueError, match="max_pos"):
        paged_attention(*args, rope=(cos[:, :32].to(device), sin[:, :32].to(device), pos))


def test_shape_fuzz_50(device):
    """Seeds 1000+i as tests/test_triton_parity.py:110-123, HIP vs float64 oracle."""
    for i in range(50):
        gen = torch.Generator().manual_seed(1000 + i)
        B = int(torch.randint(1, 4, (1,), generator=gen))
        KVH = int(torch.randint(1, 3, (1,), generator=gen))
        factor = int(torch.randint(1, 5, (1,), generator=gen))
        H, D = KVH * factor, int(torch.randint(2, 5, (1,), generator=gen)) * 8
        ctx = int(torch.randint(1, 65, (1,), generator=gen))
        bs = (8, 16, 32)[int(torch.randint(0, 3, (1,), generator=gen))]
        note(f"fuzz #{i} B={B} H={H} KVH={KVH} D={D} ctx={ctx} bs={bs}")
        q, kc, vc, table, lens = scenario(H, KVH, D, [ctx] * B, block_size=bs, seed=i)
        out = run_hip(device, q, kc, vc, table, lens)
        err = abs_err(out, dense.paged_attention_f64(q, kc, vc, table, lens))
        assert err < FP32_ATOL, f"shape #{i}: err {err}"


def test_mfma_routes_fuzz(device):
    """Seeded shapes over every MFMA route (partition and stream-K decode, short q_len on
    the decode kernel, chunked prefill, cascade decode), bf16/fp16 queries over caches of
    their type or fp8, head_dim 64/128, pages of 16..64 tokens, windows, non-causal rows
    and contexts shorter than the chunk: each against the float64 oracle."""
    for i in range(40):
        gen = torch.Generator().manual_seed(5000 + i)
        pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=gen))]
        D = pick((64, 128))
        KVH = pick((1, 2, 4, 8))
        G = pick((1, 2, 4, 5, 7, 8, 16))
        H = KVH * G
        dtype = pick((torch.bfloat16, torch.float16))
        kv_dtype = pick((dtype, dtype, torch.float8_e4m3fn))
        bs = pick((16, 32, 48, 64))
        B = int(torch.randint(1, 5, (1,), generator=gen))
        route = pick(("decode", "decode", "wide", "short", "prefill", "prefill", "cascade"))
        q_len = {"short": int(torch.randint(2, 4, (1,), generator=gen)),
                 "prefill": int(torch.randint(8, 41, (1,), generator=gen))}.get(route, 1)
        lens = [int(torch.randint(1, 1500, (1,), generator=gen)) for _ in range(B)]
        if route == "prefill":
            lens = [max(L, 1) for L in lens]
        causal = route != "prefill" or bool(torch.randint(0, 4, (1,), generator=gen))
        window = (pick((None, None, 64, 300)) if route in ("decode", "wide", "prefill")
                  and causal else None)
        pages = max((L + bs - 1) // bs for L in lens)
        width = pages + 2
        if route == "wide":
            width = max(width, -(-SK_MIN_TILES * 16 // (B * KVH * bs)))
        prefix = 0
        if route == "cascade":
            prefix = int(torch.randint(1, max(2, min(lens) // bs + 2), (1,), generator=gen))
            width = max(width, prefix + 1)
        note(f"fuzz #{i} {route} B={B} H={H} KVH={KVH} D={D} q_len={q_len} {dtype} "
             f"kv={kv_dtype} bs={bs} width={width} causal={causal} window={window} "
             f"prefix={prefix} lens={lens}")
        if prefix:
            q, kc, vc, table = shared_prefix_case(H, KVH, D, lens, dtype, bs, prefix, width,
                                                  seed=i)
        else:
            q, kc, vc, table = paged_case(H, KVH, D, lens, dtype, bs, width, seed=i, q_len=q_len)
        kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
        kw = dict(causal=causal, window=window, max_context=width * bs)
        if prefix:
            kw["prefix_pages"] = prefix
        out = run_hip(device, q, kc, vc, table, lens, **kw)
        ref = dense.paged_attention_f64(q, kc, vc, table, lens, causal=causal, window=window)
        err = rel_err(out, ref)
        assert err < BF16_REL, f"fuzz #{i}: max-rel {err}"


def test_mfma_fp32_routes_fuzz(device):
    """Seeded shapes for an fp32 query over an fp32 cache (the reference runner's types,
    miniserve/model_runner.py:120-123): partition and stream-K decode and short q_len on
    the fp32 MFMA decode kernels, chunked prefill and cascade decode on the generic kernel;
    head_dim 64/128, pages of 16..64 tokens, windows; each within max-abs 1e-4 of the
    float64 oracle."""
    for i in range(24):
        gen = torch.Generator().manual_seed(7000 + i)
        pick = lambda seq: seq[int(torch.randint(0, len(seq), (1,), generator=gen))]
        D = pick((64, 128))
        KVH = pick((1, 2, 4, 8))
        G = pick((1, 2, 4, 5, 7, 8, 16))
        H = KVH * G
        bs = pick((16, 32, 48, 64))
        B = int(torch.randint(1, 5, (1,), generator=gen))
        route = pick(("decode", "decode", "wide", "wide", "short", "prefill", "cascade"))
        q_len = {"short": int(torch.randint(2, 4, (1,), generator=gen)),
                 "prefill": int(torch.randint(8, 41, (1,), generator=gen))}.get(route, 1)
        lens = [int(torch.randint(1, 1500, (1,), generator=gen)) for _ in range(B)]
        window = pick((None, None, 64, 300)) if route != "cascade" else None
        pages = max((L + bs - 1) // bs for L in lens)
        width = pages + 2
        if route == "wide":
            width = max(width, -(-SK_MIN_TILES * 16 // (B * KVH * bs)))
        prefix = 0
        if route == "cascade":
            prefix = int(torch.randint(1, max(2, min(lens) // bs + 2), (1,), generator=gen))
            width = max(width, prefix + 1)
        note(f"fp32 fuzz #{i} {route} B={B} H={H} KVH={KVH} D={D} q_len={q_len} bs={bs} "
             f"width={width} window={window} prefix={prefix} lens={lens}")
        if prefix:
            q, kc, vc, table = shared_prefix_case(H, KVH, D, lens, torch.float32, bs, prefix,
                                                  width, seed=i)
        else:
            q, kc, vc, table = paged_case(H, KVH, D, lens, torch.float32, bs, width, seed=i,
                                          q_len=q_len)
        kw = dict(window=window, max_context=width * bs)
        if prefix:
            kw["prefix_pages"] = prefix
        out = run_hip(device, q, kc, vc, table, lens, **kw)
        ref = dense.paged_attention_f64(q, kc, vc, table, lens, window=window)
        err = abs_err(out, ref)
        assert err < FP32_ATOL, f"fp32 fuzz #{i}: max-abs {err}"


# ------------------------------------------------------------------ edge cases

def test_ragged_zero_and_one(device):
    """Ragged lens [64, 17, 33] (tests/test_triton_parity.py:99-107), plus context 0
    (zeros) and context 1 (exactly V[0])."""
    note("ragged 0/1")
    q, kc, vc, table, _ = scenario(4, 2, 16, [64, 64, 64, 64, 64], block_size=16)
    lens = [64, 17, 33, 0, 1]
    out = run_hip(device, q, kc, vc, table, lens).cpu()
    ref = dense.paged_attention_f64(q, kc, vc, table, lens)
    assert abs_err(out, ref) < FP32_ATOL
    assert not out[3].any()
    for h in range(4):
        assert torch.equal(out[4, 0, h], vc[table[4, 0], 0, h // 2])


def test_nan_poisoned_tail_is_never_read(device):
    """Slots past each row's length hold NaN; the output must stay finite and exact."""
    note("nan tail")
    q, kc, vc, table, lens = scenario(8, 2, 64, [37, 100, 16], block_size=16, seed=5)
    kc, vc = kc.clone(), vc.clone()
    for b, L in enumerate(lens):
        for pos in range(L, table.shape[1] * 16):
            kc[table[b, pos // 16], pos % 16] = float("nan")
            vc[table[b, pos // 16], pos % 16] = float("nan")
    out = run_hip(device, q, kc, vc, table, lens)
    assert torch.isfinite(out).all()
    ref = dense.paged_attention_f64(q, kc, vc, table, lens)
    assert abs_err(out, ref) < FP32_ATOL


def test_holes_are_masked(device):
    """A -1 page inside the context is a hole: its tokens drop out of the softmax."""
    note("holes")
    q, kc, vc, table, lens = scenario(4, 2, 32, [64], block_size=16, seed=12)
    holed = table.clone()
    holed[0, 1] = -1
    out = run_hip(device, q, kc, vc, holed, lens)
    keep_pages = [table[0, 0], table[0, 2], table[0, 3]]
    kc2 = torch.stack([kc[p] for p in keep_pages])
    vc2 = torch.stack([vc[p] for p in keep_pages])
    ref = dense.paged_attention_f64(q, kc2, vc2, torch.tensor([[0, 1, 2]]), [48])
    assert abs_err(out, ref) < FP32_ATOL


def test_query_and_output_not_16_byte_aligned(device):
    """The MFMA kernels read the query (and the prefill kernel writes the output) with
    16- and 8-byte vector accesses; a query or output aligned only to its element size
    takes the generic kernel (and a cascade decode the one-pass decode) instead, with the
    same result within the bar."""
    H, KVH, D = 32, 8, 128
    lens = [300, 1000, 64, 2000]
    for q_len, prefix in ((1, 0), (40, 0), (1, 2)):
        note(f"misaligned query/out: q_len={q_len} prefix={prefix}")
        q, kc, vc, table = paged_case(H, KVH, D, lens, torch.bfloat16, 16,
                                      (max(lens) + 15) // 16 + 1, seed=q_len + prefix,
                                      q_len=q_len)
        if prefix:
            table[:, :prefix] = table[0, :prefix]
        n = q.numel()
        qbuf = torch.empty(n + 1, dtype=torch.bfloat16, device=device)
        qm = qbuf[1:].view(q.shape)
        qm.copy_(q.to(device))
        obuf = torch.empty(n + 1, dtype=torch.bfloat16, device=device)
        om = obuf[1:].view(q.shape)
        assert qm.data_ptr() % 16 and om.data_ptr() % 16
        got = paged_attention(qm, kc.to(device), vc.to(device), table, lens, out=om,
                              prefix_pages=prefix or None)
        assert got.data_ptr() == om.data_ptr()
        ref = dense.paged_attention_f64(q, kc, vc, table, lens)
        assert rel_err(got, ref) < BF16_REL


def test_partition_invariance(device):
    """max_context changes the partition size; the result may not change beyond fp32 noise."""
    note("partition invariance")
    q, kc, vc, table, lens = scenario(8, 2, 64, [2000, 1500, 700], block_size=16, seed=13)
    a = run_hip(device, q, kc, vc, table, lens, max_context=2000)
    b = run_hip(device, q, kc, vc, table, lens, max_context=table.shape[1] * 16)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens)
    assert abs_err(a, ref) < FP32_ATOL and abs_err(b, ref) < FP32_ATOL
    assert (a - b).abs().max().item() < 1e-5


def test_deterministic(device):
    note("determinism")
    q, kc, vc, table, lens = scenario(32, 8, 128, [3000, 1000], block_size=16, seed=14,
                                      dtype=torch.bfloat16)
    a = run_hip(device, q, kc, vc, table, lens)
    b = run_hip(device, q, kc, vc, table, lens)
    assert torch.equal(a, b)


# ------------------------------------------------------------------ stream-K decode path

def wide_table_case(H, KVH, D, lens, dtype, width_pages, seed):
    """Scattered pages for `lens` inside a block table `width_pages` wide: a wide table
    (large capacity) routes bf16/fp16 decode to the stream-K kernel."""
    g = torch.Generator().manual_seed(seed)
    need = sum((L + 15) // 16 for L in lens)
    pool = max(need, 1) + 7
    q = torch.randn(len(lens), 1, H, D, generator=g).to(dtype)
    kc = torch.randn(pool, 16, KVH, D, generator=g).to(dtype)
    vc = torch.randn(pool, 16, KVH, D, generator=g).to(dtype)
    perm = torch.randperm(pool, generator=g)
    table = torch.zeros(len(lens), width_pages, dtype=torch.long)
    cur = 0
    for b, L in enumerate(lens):
        n = (L + 15) // 16
        table[b, :n] = perm[cur:cur + n]
        cur += n
    return q, kc, vc, table


@pytest.mark.parametrize("H,KVH,D,dtype,window", [
    (14, 2, 64, torch.bfloat16, None),     # Qwen2.5-0.5B geometry, G = 7
    (28, 4, 128, torch.bfloat16, None),    # Qwen2.5-7B geometry, G = 7
    (32, 8, 128, torch.float16, None),     # Llama-3-8B geometry in fp16
    (32, 8, 128, torch.bfloat16, 100),     # windowed decode
    (8, 8, 64, torch.bfloat16, None),      # MHA, G = 1
    (32, 1, 128, torch.bfloat16, None),    # MQA, G = 32: two row tiles per KV head
    (32, 8, 128, torch.float32, None),     # fp32 query over an fp32 cache
    (14, 2, 64, torch.float32, 100),       # fp32, head_dim 64, windowed
])
def test_streamk_decode(device, H, KVH, D, dtype, window):
    lens = [0, 1, 16, 17, 300, 1234, 77, 4096, 5, 2048, 999, 33]
    width = SK_MIN_TILES // (len(lens) * KVH) + 1  # capacity past the stream-K threshold
    note(f"stream-K H={H} KVH={KVH} D={D} {dtype} window={window}")
    q, kc, vc, table = wide_table_case(H, KVH, D, lens, dtype, width, seed=H + D)
    out = run_hip(device, q, kc, vc, table, lens, window=window, max_context=width * 16)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens, window=window)
    if dtype == torch.float32:
        err = abs_err(out, ref)
        note(f"stream-K max-abs {err:.3e}")
        assert err < FP32_ATOL
    else:
        err = rel_err(out, ref)
        note(f"stream-K max-rel {err:.3e}")
        assert err < BF16_REL
    assert not out[0].any()  # context 0 -> zeros
    for h in range(H):      # context 1 -> V[0] of the row's KV head (rounded to dtype)
        assert torch.equal(out[1, 0, h].cpu(), vc[table[1, 0], 0, h // (H // KVH)])


@pytest.mark.parametrize("batch,max_ctx,width", [
    (257, 300, 512),    # two slices of the in-kernel context-length scan
    (700, 300, 192),    # three slices
    (4096, 128, 32),    # the path's largest batch: sixteen slices
])
def test_streamk_large_batch(device, batch, max_ctx, width):
    """Stream-K decode over batches past one 256-sequence slice of its context-length scan
    (tables wide enough for the stream-K route: batch x KV heads x width >= SK_MIN_TILES),
    against the float64 oracle; empty and one-token contexts included."""
    H, KVH, D = 14, 2, 64
    g = torch.Generator().manual_seed(batch)
    lens = [int(x) for x in torch.randint(0, max_ctx + 1, (batch,), generator=g)]
    lens[0], lens[1] = 0, 1
    note(f"stream-K large batch B={batch} ctx<={max_ctx} width={width}")
    assert batch * KVH * width >= SK_MIN_TILES
    q, kc, vc, table = wide_table_case(H, KVH, D, lens, torch.bfloat16, width, seed=batch + 1)
    out = run_hip(device, q, kc, vc, table, lens, max_context=width * 16)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens)
    err = rel_err(out, ref)
    note(f"stream-K large batch max-rel {err:.3e}")
    assert err < BF16_REL
    assert not out[0].any()
    for h in range(H):
        assert torch.equal(out[1, 0, h].cpu(), vc[table[1, 0], 0, h // (H // KVH)])


@pytest.mark.parametrize("other", ["another batch", "same batch, other heads"])
def test_merge_reads_only_its_workspace_after_another_geometry(device, other):
    """msattn_merge_partials over a workspace last written by a stream-K call of another
    geometry: the header describes a layout that is not this call's. The merge checks every
    header word and clamps the slots it reads to the workspace (merge_slot_range), so the
    call returns MSATTN_OK with a finite output (zeros where the header names no slot of
    this row) and the next regular call on the workspace is correct again."""
    lib = nat.lib()
    H, KVH, D = 32, 8, 128
    lens = [3000, 17, 5000, 0, 800, 4096, 1, 2500] * 8
    width = SK_MIN_TILES // (len(lens) * KVH) + 1
    note(f"stale header ({other}): stream-K over {len(lens)} sequences")
    q, kc, vc, table = wide_table_case(H, KVH, D, lens, torch.bfloat16, width, seed=404)
    kd, vd = kc.to(device), vc.to(device)
    td = table.to(device=device, dtype=torch.int32)
    ld = torch.tensor(lens, dtype=torch.int32, device=device)
    cap = width * 16
    ws = torch.zeros(256 << 20, dtype=torch.uint8, device=device)
    stream = nat.stream_handle(device)
    st = lib.msattn_paged_attention_partials(
        q.to(device).data_ptr(), kd.data_ptr(), vd.data_ptr(), kd.stride(0), kd.stride(1),
        kd.stride(2), td.data_ptr(), ld.data_ptr(), ws.data_ptr(), ws.numel(), len(lens), 1, H,
        KVH, D, 16, kd.shape[0], width, cap, 1, 0, 1 / D ** 0.5, nat.BF16, nat.BF16, stream)
    assert st == nat.OK
    torch.cuda.synchronize()
    assert int(ws[:4].view(torch.int32).item()) == 1  # a stream-K header
    if other == "another batch":
        B2, H2, KVH2, D2, ctx2 = 5, 14, 2, 64, 1000
    else:  # the header's batch matches, so its stream-K words are used, for other heads
        B2, H2, KVH2, D2, ctx2 = len(lens), 8, 8, 64, 4096
    need = lib.msattn_workspace_bytes(B2, 1, H2, KVH2, D2, ctx2)
    assert need <= ws.numel()
    lens2 = torch.randint(0, ctx2 + 1, (B2,), dtype=torch.int32, device=device)
    out = torch.full((B2, 1, H2, D2), float("nan"), dtype=torch.bfloat16, device=device)
    st = lib.msattn_merge_partials(ws.data_ptr(), need, lens2.data_ptr(), out.data_ptr(), B2, 1,
                                   H2, KVH2, D2, ctx2, nat.BF16, stream)
    assert st == nat.OK
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    # the workspace still serves a regular call of the second geometry
    q2, kc2, vc2, table2 = wide_table_case(H2, KVH2, D2, [min(int(x), ctx2) for x in lens2],
                                           torch.bfloat16, ctx2 // 16, seed=405)
    lens2l = [int(x) for x in lens2]
    got = paged_attention(q2.to(device), kc2.to(device), vc2.to(device), table2, lens2l,
                          max_context=ctx2, workspace=ws)
    ref = dense.paged_attention_f64(q2, kc2, vc2, table2, lens2l)
    assert rel_err(got, ref) < BF16_REL


def test_streamk_graph_replays(device):
    """Stream-K decode captured in a graph: replays with new lengths match eager bit-exactly."""
    note("stream-K graph")
    H, KVH, D = 32, 8, 128
    lens = [3000, 17, 5000, 0, 800, 4096, 1, 2500]
    width = SK_MIN_TILES // (len(lens) * KVH)  # stream-K capacity; pages for 8192 tokens a row
    top = 8192
    q, kc, vc, table = wide_table_case(H, KVH, D, [top] * len(lens), torch.bfloat16, width,
                                       seed=5)
    kc, vc = kc.to(device), vc.to(device)
    sq = q.to(device)
    stable = table.to(device=device, dtype=torch.int32)
    slens = torch.tensor(lens, dtype=torch.int32, device=device)
    ws = torch.zeros(256 << 20, dtype=torch.uint8, device=device)
    out = torch.empty_like(sq)
    cap = width * 16

    def step():
        paged_attention(sq, kc, vc, stable, slens, max_context=cap, workspace=ws, out=out)

    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream(device).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    g = torch.Generator().manual_seed(6)
    for rep in range(4):
        new = [int(x) for x in torch.randint(0, top + 1, (len(lens),), generator=g)]
        slens.copy_(torch.tensor(new, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = paged_attention(sq, kc, vc, stable, new, max_context=cap)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay {rep}"


# ------------------------------------------------------------------ chunked prefill (MFMA)

# Chunked prefill (more than 16 query rows per KV head). "prefill": the MFMA prefill
# kernel; "partition-fused": the partition kernel at 16 rows per tile, which the cost
# model picks for at most 64 rows per KV head over few (sequence, KV head) pairs.
@pytest.mark.parametrize("H,KVH,D,q_len,lens,dtype,causal,window,route", [
    (28, 4, 128, 512, [4608, 4608], torch.bfloat16, True, None, "prefill"),   # C5 prefill shape
    (28, 4, 128, 100, [100, 1000, 357], torch.bfloat16, True, None, "prefill"),
    (32, 8, 128, 17, [17, 40, 3000], torch.bfloat16, True, None, "prefill stream-K"),  # 68 rows
    (32, 8, 128, 64, [64, 700], torch.float16, True, None, "prefill"),
    (8, 8, 128, 80, [80, 150], torch.bfloat16, False, None, "prefill"),       # non-causal
    (28, 4, 128, 200, [1200, 300], torch.bfloat16, True, 128, "prefill"),     # sliding window
    (16, 2, 128, 80, [50, 2000], torch.bfloat16, True, None, _SK),            # context shorter than the chunk
    # head_dim 64 (Qwen2.5-0.5B geometry): a staging pass spans two 16-token tiles
    (14, 2, 64, 512, [2560, 600], torch.bfloat16, True, None, _SK),
    (14, 2, 64, 37, [37, 1500, 90], torch.float16, True, 100, _SK),
    (8, 8, 64, 72, [72, 333], torch.bfloat16, False, None, "prefill"),        # non-causal
    (14, 2, 64, 37, [37, 1500, 90], torch.bfloat16, True, None, _SK),
    # few pairs, at most 64 rows per KV head: the partition kernel's 16-row tiles
    (8, 8, 128, 33, [33, 90], torch.bfloat16, False, None, "partition-fused"),
    (8, 8, 64, 40, [40, 333], torch.bfloat16, False, None, "partition-fused"),
    (32, 8, 128, 16, [16, 40, 3000], torch.float16, True, None, "partition-fused"),
    (16, 2, 128, 8, [5, 2000], torch.bfloat16, True, 100, "partition-fused"),  # ctx < chunk
])
def test_prefill_mfma(device, H, KVH, D, q_len, lens, dtype, causal, window, route):
    note(f"prefill H={H} KVH={KVH} D={D} q_len={q_len} lens={lens} {dtype} causal={causal} "
         f"window={window} route={route}")
    g = torch.Generator().manual_seed(q_len + H)
    width = max((L + 15) // 16 for L in lens) + 3
    q, kc, vc, table = wide_table_case(H, KVH, D, lens, dtype, width, seed=q_len)
    q = torch.randn(len(lens), q_len, H, D, generator=g).to(dtype)
    out = run_routed(device, route, q, kc, vc, table, lens, causal=causal, window=window)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens, causal=causal, window=window)
    err = rel_err(out, ref)
    note(f"prefill max-rel {err:.3e}")
    assert err < BF16_REL
    # rows whose key set is empty are zeros (first rows when the context is shorter)
    for b, L in enumerate(lens):
        if causal and L < q_len:
            assert not out[b, : q_len - L].any()



@pytest.mark.parametrize("B,H,KVH,D,q_len,lo,hi,dtype,kv_dtype,want", [
    # 16 tasks of ~94 key-step pairs over 256 workgroups: every task split over ~16 shares
    (1, 8, 8, 128, 200, 12000, 12000, torch.bfloat16, torch.bfloat16, _SK),
    # 96 tasks: ~2.7 shares each
    (2, 32, 8, 128, 192, 6000, 6144, torch.bfloat16, torch.bfloat16, _SK),
    # 300 tasks (two rounds of 256 otherwise): shares of 1.2 tasks, spanning two
    (75, 4, 4, 64, 32, 500, 4000, torch.bfloat16, torch.bfloat16, _SK),
    # head_dim 64, fp16, and fp8 and fp32 caches (register staging) in stream-K mode
    (2, 14, 2, 64, 200, 200, 5000, torch.float16, torch.float16, _SK),
    (3, 32, 8, 128, 100, 100, 6000, torch.bfloat16, torch.float8_e4m3fn, _SK),
    (2, 28, 4, 128, 160, 160, 7000, torch.bfloat16, torch.float32, _SK),
    # 256 short tasks: one per workgroup (the cost model keeps stream-K off)
    (16, 32, 8, 128, 64, 64, 1000, torch.bfloat16, torch.bfloat16, "prefill"),
])
def test_prefill_stream_k_schedule(device, B, H, KVH, D, q_len, lo, hi, dtype, kv_dtype,
                                   want):
    """The prefill kernel's stream-K schedule (one workgroup per CU, each an equal share of
    all tasks' key-step pairs; a task split between shares merged by the fold launch that
    follows), which the cost model picks for launches that would leave CUs idle, against
    the float64 oracle: tasks over many shares, shares over two tasks, the staged (fp8)
    path, and a launch of one task per CU (no stream-K); three calls in a row on one
    workspace (whose ticket area, which the decode kernels use, stays at zero)."""
    g = torch.Generator().manual_seed(B * q_len + H)
    lens = [int(x) for x in torch.randint(lo, hi + 1, (B,), generator=g)]
    lens = [max(L, q_len) for L in lens]
    width = (max(lens) + 15) // 16 + 1
    ws = None
    for call in range(3):
        note(f"prefill stream-K B={B} H={H}/{KVH} D={D} q_len={q_len} lens={lens[:6]} "
             f"{dtype}/{kv_dtype} call {call}")
        q, kc, vc, table = paged_case(H, KVH, D, lens, dtype, 16, width, seed=call + q_len,
                                      q_len=q_len)
        kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
        qd = q.to(device)
        assert kernel_route(qd, kc.to(device), table) == want
        if ws is None:
            nbytes = nat.lib().msattn_workspace_bytes(B, q_len, H, KVH, D, width * 16)
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        out = paged_attention(qd, kc.to(device), vc.to(device), table, lens,
                              max_context=width * 16, workspace=ws)
        torch.cuda.synchronize()
        assert not ws[:(64 + 4096) * 4].view(torch.int32)[64:].any(), "tickets not at zero"
        ref = dense.paged_attention_f64(q, kc, vc, table, lens, kv_cast=True)
        err = rel_err(out, ref)
        note(f"stream-K prefill max-rel {err:.3e}")
        assert err < BF16_REL
        lens = [max(q_len, L - 7 * (call + 1)) for L in lens]


def paged_case(H, KVH, D, lens, dtype, bs, width_pages, seed, q_len=1):
    """Scattered pages of `bs` tokens for `lens` in a table `width_pages` wide."""
    g = torch.Generator().manual_seed(seed)
    need = sum((L + bs - 1) // bs for L in lens)
    pool = max(need, 1) + 5
    q = torch.randn(len(lens), q_len, H, D, generator=g).to(dtype)
    kc = torch.randn(pool, bs, KVH, D, generator=g).to(dtype)
    vc = torch.randn(pool, bs, KVH, D, generator=g).to(dtype)
    perm = torch.randperm(pool, generator=g)
    table = torch.zeros(len(lens), width_pages, dtype=torch.long)
    cur = 0
    for b, L in enumerate(lens):
        n = (L + bs - 1) // bs
        table[b, :n] = perm[cur:cur + n]
        cur += n
    return q, kc, vc, table


@pytest.mark.parametrize("bs", [32, 48, 64])
def test_mfma_paths_other_page_sizes(device, bs):
    """Pages of 32, 48 (not a power of two) and 64 tokens on the MFMA kernels: chunked
    prefill, partition decode, stream-K decode (wide table) and an fp8 cache, each
    against the float64 oracle."""
    lens = [5, 100, 1000, 333]
    cases = [  # (H, KVH, D, q_len, table width in pages, kv dtype)
        (28, 4, 128, 64, (max(lens) + bs - 1) // bs + 2, torch.bfloat16),   # prefill
        (14, 2, 64, 1, (max(lens) + bs - 1) // bs + 2, torch.bfloat16),     # partition decode
        (32, 8, 128, 1, SK_MIN_TILES * 16 // (bs * len(lens) * 8) + 1, torch.bfloat16),  # stream-K
        (32, 8, 128, 1, (max(lens) + bs - 1) // bs + 2, torch.float8_e4m3fn),     # fp8
    ]
    for H, KVH, D, q_len, width, kv_dtype in cases:
        note(f"page size {bs}: H={H} KVH={KVH} D={D} q_len={q_len} width={width} kv={kv_dtype}")
        q, kc, vc, table = paged_case(H, KVH, D, [max(L, q_len) for L in lens], torch.bfloat16,
                                      bs, width, seed=bs + D + q_len)
        kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
        ctx = [max(L, q_len) for L in lens]
        out = run_hip(device, q, kc, vc, table, ctx, max_context=width * bs)
        ref = dense.paged_attention_f64(q, kc, vc, table, ctx)
        assert rel_err(out, ref) < BF16_REL


def test_slot_stride_past_32_bit_tile_span(device):
    """Caches stored [block_size, num_blocks, KVH, D] and passed as the permuted view
    [num_blocks, block_size, KVH, D]: the slot stride is num_blocks * KVH * D elements, so a
    16-token tile spans 15 * 70000 * 1024 * 2 B = 2.15 GB, past what a 32-bit buffer offset
    reaches. Decode, chunked prefill and cascade decode must still match the float64 oracle
    (within 2e-2 max-rel); the oracle sees compact copies of the same pages."""
    H, KVH, D, bs, nb = 32, 8, 128, 16, 70_000
    assert 15 * nb * KVH * D * 2 >= 2 ** 31
    g = torch.Generator().manual_seed(11)
    lens = [300, 40, 1000]
    need = [(L + bs - 1) // bs for L in lens]
    used = torch.randperm(nb, generator=g)[: sum(need)]
    table = torch.zeros(len(lens), max(need), dtype=torch.long)
    cur = 0
    for b, n in enumerate(need):
        table[b, :n] = used[cur:cur + n]
        cur += n
    kbig = torch.zeros(bs, nb, KVH, D, dtype=torch.bfloat16, device=device)
    vbig = torch.zeros_like(kbig)
    kc, vc = kbig.permute(1, 0, 2, 3), vbig.permute(1, 0, 2, 3)
    assert kc.stride(1) == nb * KVH * D
    kvals = torch.randn(len(used), bs, KVH, D, generator=g).to(torch.bfloat16)
    vvals = torch.randn(len(used), bs, KVH, D, generator=g).to(torch.bfloat16)
    kc[used.to(device)] = kvals.to(device)
    vc[used.to(device)] = vvals.to(device)
    remap = torch.zeros(nb, dtype=torch.long)
    remap[used] = torch.arange(len(used))
    try:
        for q_len in (1, 24):  # 24 x 4 rows per KV head: the chunked-prefill route
            note(f"slot stride {kc.stride(1)}: q_len={q_len} lens={lens}")
            q = torch.randn(len(lens), q_len, H, D, generator=g).to(torch.bfloat16)
            out = paged_attention(q.to(device), kc, vc, table, lens)
            ref = dense.paged_attention_f64(q, kvals, vvals, remap[table], lens)
            assert rel_err(out, ref) < BF16_REL
        shared = table.clone()
        shared[:, :2] = table[0, :2]  # two pages every row shares
        note(f"slot stride {kc.stride(1)}: cascade, 2 shared pages")
        q = torch.randn(len(lens), 1, H, D, generator=g).to(torch.bfloat16)
        out = paged_attention(q.to(device), kc, vc, shared, lens, prefix_pages=2)
        ref = dense.paged_attention_f64(q, kvals, vvals, remap[shared], lens)
        assert rel_err(out, ref) < BF16_REL
    finally:
        del kc, vc, kbig, vbig
        torch.cuda.empty_cache()


# ------------------------------------------------------------------ cascade decode

def shared_prefix_case(H, KVH, D, lens, dtype, bs, prefix_pages, width, seed):
    """Block tables whose first `prefix_pages` entries are the same physical pages in
    every row (a radix-cache hit); each row's later pages are its own, scattered."""
    g = torch.Generator().manual_seed(seed)
    own = [max(0, (L + bs - 1) // bs - prefix_pages) for L in lens]
    pool = prefix_pages + sum(own) + 3
    q = torch.randn(len(lens), 1, H, D, generator=g).to(dtype)
    kc = torch.randn(pool, bs, KVH, D, generator=g).to(dtype)
    vc = torch.randn(pool, bs, KVH, D, generator=g).to(dtype)
    perm = torch.randperm(pool, generator=g)
    table = torch.zeros(len(lens), width, dtype=torch.long)
    table[:, :prefix_pages] = perm[:prefix_pages]
    cur = prefix_pages
    for b, n in enumerate(own):
        table[b, prefix_pages:prefix_pages + n] = perm[cur:cur + n]
        cur += n
    return q, kc, vc, table


_g = torch.Generator().manual_seed(77)
CASCADE_CASES = [  # (H, KVH, D, dtype, bs, lens, prefix pages, table width in pages)
    # partition decode for the suffix; rows ending before, at and just after the prefix
    (32, 8, 128, torch.bfloat16, 16, [5, 100, 1000, 333, 2000, 160, 161, 0], 10, 130),
    # 20 x 7 = 140 query rows per KV head: two row blocks in the prefix pass
    (28, 4, 128, torch.float16, 16,
     [int(x) for x in torch.randint(1, 3000, (20,), generator=_g)], 37, 190),
    (32, 8, 128, torch.bfloat16, 32, [700, 64, 4000], 20, 126),     # 32-token pages
    (32, 8, 128, torch.bfloat16, 48, [700, 64, 4000], 9, 90),       # 48-token pages
    # stream-K decode for the suffix (batch x KV heads x table tiles >= SK_MIN_TILES)
    (32, 8, 128, torch.bfloat16, 16, [30000, 9000, 20000, 1000], 256, 8192),
    # every key in the prefix: the suffix pass has no work
    (32, 8, 128, torch.bfloat16, 16, [480, 480, 480], 30, 30),
    # head_dim 64 (the prefix pass on the head_dim-64 prefill kernel)
    (14, 2, 64, torch.bfloat16, 16, [300, 50, 900], 8, 60),
    # without cascade kernels (fp32): one pass over the whole context
    (4, 2, 64, torch.float32, 16, [300, 50, 900], 8, 60),
]


@pytest.mark.parametrize("case", range(len(CASCADE_CASES)))
def test_cascade_decode(device, case):
    """Cascade decode (shared prefix read once per KV head, then each row's own pages,
    then one merge) against the float64 oracle and against the one-pass decode."""
    H, KVH, D, dtype, bs, lens, pages, width = CASCADE_CASES[case]
    note(f"cascade case {case}: H={H} KVH={KVH} D={D} {dtype} bs={bs} B={len(lens)} "
         f"prefix={pages} pages width={width}")
    q, kc, vc, table = shared_prefix_case(H, KVH, D, lens, dtype, bs, pages, width, seed=case)
    cap = width * bs
    out = run_hip(device, q, kc, vc, table, lens, max_context=cap, prefix_pages=pages)
    one = run_hip(device, q, kc, vc, table, lens, max_context=cap)
    ref = dense.paged_attention_f64(q, kc, vc, table, lens)
    if dtype == torch.float32:
        assert abs_err(out, ref) < FP32_ATOL
        assert torch.equal(out, one)  # no cascade kernels: the same one-pass launch
    else:
        assert rel_err(out, ref) < BF16_REL
        assert rel_err(out, one.double().cpu().numpy()) < BF16_REL
    zero = [b for b, L in enumerate(lens) if L == 0]
    if zero:
        assert not out[zero].abs().any().item()


def test_cascade_graph_replays(device):
    """Cascade decode captured in a graph: replays with new lengths match eager bit-exactly."""
    note("cascade graph")
    H, KVH, D, bs, pages, width = 32, 8, 128, 16, 40, 200
    lens = [3000, 17, 640, 0, 800, 3200]
    q, kc, vc, table = shared_prefix_case(H, KVH, D, [width * bs] * len(lens), torch.bfloat16,
                                          bs, pages, width, seed=9)
    kc, vc = kc.to(device), vc.to(device)
    sq = q.to(device)
    stable = table.to(device=device, dtype=torch.int32)
    slens = torch.tensor(lens, dtype=torch.int32, device=device)
    ws = torch.zeros(256 << 20, dtype=torch.uint8, device=device)
    out = torch.empty_like(sq)
    cap = width * bs

    def step():
        paged_attention(sq, kc, vc, stable, slens, max_context=cap, workspace=ws, out=out,
                        prefix_pages=pages)

    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream(device).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    g = torch.Generator().manual_seed(10)
    for rep in range(4):
        new = [int(x) for x in torch.randint(0, cap + 1, (len(lens),), generator=g)]
        slens.copy_(torch.tensor(new, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = paged_attention(sq, kc, vc, stable, new, max_context=cap, prefix_pages=pages)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay {rep}"


def test_prefill_stream_k_graph_replays(device):
    """A chunked prefill on the stream-K schedule (32 tasks over a 16,384-token table)
    captured in a hipGraph: replays with new context lengths each time match eager calls
    bit for bit (the tickets come back to zero between replays, and the fold order is the
    shares' order whichever share arrives last)."""
    note("prefill stream-K graph")
    H, KVH, D, q_len, width = 32, 8, 128, 128, 1024
    cap = width * 16
    lens = [cap]
    q, kc, vc, table = paged_case(H, KVH, D, lens, torch.bfloat16, 16, width, seed=77,
                                  q_len=q_len)
    kc, vc = kc.to(device), vc.to(device)
    sq = q.to(device)
    stable = table.to(device=device, dtype=torch.int32)
    assert kernel_route(sq, kc, stable, max_context=cap) == "prefill stream-K"
    slens = torch.tensor(lens, dtype=torch.int32, device=device)
    nbytes = nat.lib().msattn_workspace_bytes(1, q_len, H, KVH, D, cap)
    ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    out = torch.empty_like(sq)

    def step():
        paged_attention(sq, kc, vc, stable, slens, max_context=cap, workspace=ws, out=out)

    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream(device).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    g = torch.Generator().manual_seed(78)
    for rep in range(4):
        new = [int(torch.randint(q_len, cap + 1, (1,), generator=g))]
        slens.copy_(torch.tensor(new, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        assert not ws[:(64 + 4096) * 4].view(torch.int32)[64:].any(), "tickets not back at zero"
        eager = paged_attention(sq, kc, vc, stable, new, max_context=cap)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay {rep}: lens {new}"


# ------------------------------------------------------------------ benchmark configs

@pytest.fixture(scope="module")
def c3():
    note("building C3 inputs")
    return make_workload(3)


def check_workload(device, w, rows=None):
    q = w.query
    kc, vc = w.k_caches[0], w.v_caches[0]
    note(f"{w.name}: B={w.batch} q_len={w.q_len} H={w.num_heads} KVH={w.num_kv_heads} "
         f"D={w.head_dim} max_ctx={max(w.lens)} dtype={w.dtype}")
    out = paged_attention(q.to(device), kc.to(device), vc.to(device), w.table, w.lens)
    ref = dense.paged_attention_f64(q, kc, vc, w.table, w.lens, rows=rows)
    sel = list(range(w.batch)) if rows is None else rows
    o = out.cpu()[sel]
    r = ref[sel]
    if w.dtype == torch.float32:
        err = abs_err(o, r)
        note(f"{w.name} max-abs {err:.3e}")
        assert err < FP32_ATOL
    else:
        err = rel_err(o, r)
        note(f"{w.name} max-rel {err:.3e}")
        assert err < BF16_REL
    return out


def test_c1_fp32(device):
    check_workload(device, make_workload(1))


def test_c2_layer0_bf16(device):
    check_workload(device, make_workload(2, layers=1))


def test_c3_bf16(device, c3):
    check_workload(device, c3)


def test_c3_batch_permutation(device, c3):
    """Size-independent property at full C3 size: a row's result depends only on its own
    query, table and length. Permuting the batch permutes the output up to summation
    order (the work split follows the batch order): within 2 bf16 ulps of the row's
    magnitude, and both results within the oracle bar."""
    kc, vc = c3.k_caches[0].to(device), c3.v_caches[0].to(device)
    full = paged_attention(c3.query.to(device), kc, vc, c3.table, c3.lens)
    perm = torch.randperm(c3.batch, generator=torch.Generator().manual_seed(3))
    permuted = paged_attention(c3.query[perm].to(device), kc, vc, c3.table[perm],
                               [c3.lens[i] for i in perm.tolist()])
    a = full[perm.to(device)].float()
    b = permuted.float()
    scale = a.abs().amax(dim=-1, keepdim=True).clamp_min(1e-30)
    assert ((a - b).abs() / scale).max().item() <= 2 * 2.0 ** -8


def test_c4_long_context_rows(device):
    w = make_workload(4, values_device=device)
    w.query = w.query.cpu()
    w.k_caches = [w.k_caches[0].cpu()]
    w.v_caches = [w.v_caches[0].cpu()]
    check_workload(device, w, rows=[0, 7])


def test_c5_decode(device):
    check_workload(device, make_workload(5, part="decode"))


def test_c5_prefill_chunk(device):
    check_workload(device, make_workload(5, part="prefill"))


# ------------------------------------------------------------------ graphs

def test_graph_capture_replay(device):
    """The call is capture-safe: replays with new inputs match eager every time."""
    note("graph capture")
    H, KVH, D, bs = 32, 8, 128, 16
    q, kc, vc, table, lens = scenario(H, KVH, D, [900, 1700, 33, 2048], block_size=bs, seed=15,
                                      dtype=torch.bfloat16)
    kc, vc = kc.to(device), vc.to(device)
    static_q = q.to(device)
    static_table = table.to(device=device, dtype=torch.int32)
    static_lens = torch.tensor(lens, dtype=torch.int32, device=device)
    cap = table.shape[1] * bs
    ws_bytes = 64 << 20
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=device)
    out = torch.empty_like(static_q)

    def step():
        paged_attention(static_q, kc, vc, static_table, static_lens, max_context=cap,
                        workspace=ws, out=out)

    s = torch.cuda.Stream(device)
    s.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream(device).wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    g = torch.Generator().manual_seed(16)
    for rep in range(4):
        new_lens = [int(x) for x in torch.randint(0, cap + 1, (4,), generator=g)]
        static_q.copy_(torch.randn(q.shape, generator=g).to(torch.bfloat16))
        static_lens.copy_(torch.tensor(new_lens, dtype=torch.int32))
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = paged_attention(static_q, kc, vc, static_table, new_lens, max_context=cap)
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"replay {rep}"


def test_stream_read_probe(device):
    """The streaming-read probe runs over a buffer that is not a whole number of its
    64 KiB chunks, and the sink keeps its contents unless the fold hits the sentinel."""
    from miniserve_amd import _native as nat
    nbytes = (3 << 20) + 4096
    buf = torch.ones(nbytes // 4, dtype=torch.float32, device=device)
    sink = torch.zeros((nbytes + 65535) // 65536, dtype=torch.int32, device=device)
    st = nat.lib().msattn_probe_stream_read(buf.data_ptr(), nbytes, sink.data_ptr(),
                                            nat.stream_handle(device))
    assert st == nat.OK
    torch.cuda.synchronize()
    assert not sink.any()
