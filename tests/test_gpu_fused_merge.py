"""GPU parity of the in-kernel merge of the partition decode kernel.

msattn_paged_attention runs small decodes (the partition MFMA kernel) as one launch: the
last partition workgroup of each (sequence, KV head, row tile) to arrive folds the
others' partials into the output, and a sequence of one partition writes its output
directly. The partials travel between workgroups (and XCDs) through device-coherent
stores and loads, and the arrival counters live in the workspace header.

Checked here, over several consecutive calls on one workspace (so stale partials and
counters of an earlier call would show): the output against the float64 oracle (fp32
max-abs 1e-4, bf16/fp16 max-rel 2e-2) and against the two-launch path of the same
partials (msattn_paged_attention_partials + msattn_merge_partials; the fold's summation
order differs, so fp32 within 1e-5 relative and bf16/fp16 within two units of the last
place of the output type), that the workspace's counters are all zero after each call,
and that the workspace header names the in-kernel route (kind 2).
"""
import numpy as np
import pytest
import torch

from miniserve_amd import _native as nat
from oracle import dense

pytestmark = pytest.mark.gpu

FP32_ATOL = 1e-4
BF16_REL = 2e-2
HDR_TICKETS, MAX_TICKETS = 64, 4096


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def make(H, KVH, D, lens, dtype, width, seed, q_len=1):
    g = torch.Generator().manual_seed(seed)
    pool = sum((L + 15) // 16 for L in lens) + 3
    q = torch.randn(len(lens), q_len, H, D, generator=g).to(dtype)
    kc = torch.randn(pool, 16, KVH, D, generator=g).to(dtype)
    vc = torch.randn(pool, 16, KVH, D, generator=g).to(dtype)
    perm = torch.randperm(pool, generator=g)
    table = torch.zeros(len(lens), width, dtype=torch.int32)
    cur = 0
    for b, L in enumerate(lens):
        n = (L + 15) // 16
        table[b, :n] = perm[cur:cur + n].to(torch.int32)
        cur += n
    return q, kc, vc, table


class Caller:
    """One workspace reused by every call (zeroed once), and a separate one for the
    two-launch path."""

    def __init__(self, device, nbytes):
        self.device = device
        self.ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        self.ws2 = torch.zeros(nbytes, dtype=torch.uint8, device=device)

    def run(self, q, kc, vc, table, lens, window=0):
        lib = nat.lib()
        dev = self.device
        B, q_len, H, D = q.shape
        nb, bs, KVH, _ = kc.shape
        max_ctx = table.shape[1] * bs
        ws_bytes = lib.msattn_workspace_bytes(B, q_len, H, KVH, D, max_ctx)
        assert 0 < ws_bytes <= self.ws.numel()
        qd, kcd, vcd = q.to(dev), kc.to(dev), vc.to(dev)
        td, ld = table.to(dev), torch.tensor(lens, dtype=torch.int32, device=dev)
        common = (qd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), kcd.stride(0), kcd.stride(1),
                  kcd.stride(2), td.data_ptr(), ld.data_ptr())
        qc, kvc = nat.dtype_code(q.dtype), nat.dtype_code(kc.dtype)
        tail = (B, q_len, H, KVH, D, bs, nb, table.shape[1], max_ctx, 1, window,
                1.0 / D ** 0.5, qc, kvc)
        stream = nat.stream_handle(dev)
        fused = torch.full_like(qd, float("nan"))
        st = lib.msattn_paged_attention(*common, fused.data_ptr(), self.ws.data_ptr(),
                                        ws_bytes, *tail, stream)
        assert st == nat.OK, st
        two = torch.full_like(qd, float("nan"))
        st = lib.msattn_paged_attention_partials(*common, self.ws2.data_ptr(), ws_bytes, *tail,
                                                 stream)
        assert st == nat.OK, st
        st = lib.msattn_merge_partials(self.ws2.data_ptr(), ws_bytes, ld.data_ptr(),
                                       two.data_ptr(), B, q_len, H, KVH, D, max_ctx, qc, stream)
        assert st == nat.OK, st
        torch.cuda.synchronize()
        hdr = self.ws[: 4 * (HDR_TICKETS + MAX_TICKETS)].view(torch.int32).cpu()
        hdr2 = self.ws2[: 4 * HDR_TICKETS].view(torch.int32).cpu()
        return fused, two, hdr, hdr2


def check(fused, two, hdr, q, kc, vc, table, lens, window=None, hdr2=None):
    assert int(hdr[0]) == 2, f"workspace kind {int(hdr[0])}: not the in-kernel merge"
    # The same partitions on both paths unless the fused call took the wide shape (longer
    # partitions): then the weights meet other running maxima before their rounding to
    # the cache type for v_dot2, and only the oracle's bar applies between the two.
    same_split = hdr2 is None or (int(hdr[8]), int(hdr[9])) == (int(hdr2[8]), int(hdr2[9]))
    assert not hdr[HDR_TICKETS:].any(), "merge counters not left at zero"
    assert not torch.isnan(fused).any()
    ref = dense.paged_attention_f64(q, kc, vc, table.long(), lens, window=window)
    f = fused.double().cpu().numpy()
    t = two.double().cpu().numpy()
    if q.dtype == torch.float32:
        err = float(np.abs(f - ref).max())
        assert err < FP32_ATOL, err
        diff = float(np.abs(f - t).max() / max(np.abs(t).max(), 1e-30))
        assert diff < 1e-5, diff
    else:
        err = float(np.abs(f - ref).max() / max(np.abs(ref).max(), 1e-30))
        assert err < BF16_REL, err
        ulp = 2.0 ** (-7 if q.dtype == torch.bfloat16 else -10)
        if same_split:
            assert np.all(np.abs(f - t) <= 2 * ulp * np.maximum(np.abs(t), 2.0 ** -14)), \
                float(np.abs(f - t).max())
        else:
            terr = float(np.abs(t - ref).max() / max(np.abs(ref).max(), 1e-30))
            assert terr < BF16_REL, terr
    note(f"oracle err {err:.3e}")


CASES = {  # name -> (H, KVH, D, dtype, width in pages)
    "C2 geometry bf16": (14, 2, 64, torch.bfloat16, 128),
    "C5 geometry bf16": (28, 4, 128, torch.bfloat16, 240),
    "fp32 (runner default)": (14, 2, 64, torch.float32, 64),
    "fp16 MHA": (8, 8, 128, torch.float16, 64),
    "MQA two row tiles": (32, 1, 128, torch.bfloat16, 64),
}


@pytest.mark.parametrize("name", list(CASES))
def test_fused_merge_consecutive_calls(device, name):
    """Five calls on one workspace with new data and lengths each time: empty, one-token
    and one-partition sequences (direct output) beside many-partition ones."""
    H, KVH, D, dtype, width = CASES[name]
    caller = Caller(device, 64 << 20)
    for i in range(5):
        g = torch.Generator().manual_seed(100 * i + H)
        B = int(torch.randint(3, 33, (1,), generator=g))
        cap = width * 16
        lens = [int(x) for x in torch.randint(0, cap + 1, (B,), generator=g)]
        lens[0], lens[1] = 0, 1
        lens[2] = int(torch.randint(2, 60, (1,), generator=g))  # one partition
        note(f"fused {name} call {i}: B={B} lens={lens}")
        q, kc, vc, table = make(H, KVH, D, lens, dtype, width, seed=i + 7 * H)
        fused, two, hdr, hdr2 = caller.run(q, kc, vc, table, lens)
        check(fused, two, hdr, q, kc, vc, table, lens, hdr2=hdr2)
        assert not fused[0].cpu().any()  # context 0 -> zeros


def test_fused_merge_window_and_short_q(device):
    """Windowed decode (partitions below the window hold no key and carry no weight) and
    q_len 2 (speculative rows, causal) through the in-kernel merge."""
    caller = Caller(device, 64 << 20)
    H, KVH, D, width = 14, 2, 64, 128
    lens = [2000, 700, 1, 1500, 33, 0, 1999]
    for window, q_len in ((100, 1), (600, 1), (0, 2)):
        note(f"fused window={window} q_len={q_len}")
        q, kc, vc, table = make(H, KVH, D, lens, torch.bfloat16, width, seed=window + q_len,
                                q_len=q_len)
        if q_len > 1:
            lens_q = [max(L, q_len) for L in lens]
            q, kc, vc, table = make(H, KVH, D, lens_q, torch.bfloat16, width, seed=5,
                                    q_len=q_len)
        else:
            lens_q = lens
        fused, two, hdr, hdr2 = caller.run(q, kc, vc, table, lens_q, window=window)
        check(fused, two, hdr, q, kc, vc, table, lens_q, window=window or None, hdr2=hdr2)


def test_stream_k_leaves_counters_alone(device):
    """A stream-K decode (wide table) on the same workspace neither uses nor disturbs the
    merge counters, and a partition decode after it still merges correctly."""
    lib = nat.lib()
    caller = Caller(device, 256 << 20)
    H, KVH, D = 32, 8, 128
    lens = [3000, 17, 5000, 0, 800, 4096, 1, 2500]
    q, kc, vc, table = make(H, KVH, D, lens, torch.bfloat16, 4096, seed=3)
    fused, two, hdr, hdr2 = caller.run(q, kc, vc, table, lens)
    assert int(hdr[0]) == 1  # stream-K: the merge kernel ran
    assert not hdr[HDR_TICKETS:].any()
    assert torch.equal(fused, two)
    lens = [300, 1200, 0, 64]
    q, kc, vc, table = make(14, 2, 64, lens, torch.bfloat16, 80, seed=4)
    fused, two, hdr, hdr2 = caller.run(q, kc, vc, table, lens)
    check(fused, two, hdr, q, kc, vc, table, lens, hdr2=hdr2)
    assert lib is nat.lib()


@pytest.mark.parametrize("D,window", [(128, 0), (64, 0), (128, 700)])
def test_fp32_prefill_long_partitions(device, D, window):
    """fp32 chunked prefill large enough (grid of >= 512 workgroups) for the fp32 16-row
    route's long partitions (up to 2048 tokens a workgroup, P.V on the matrix core, merged
    in-kernel): against the float64 oracle and the two-launch path, whose partitions are
    512 tokens, on two consecutive calls."""
    caller = Caller(device, 64 << 20)
    H, KVH, q_len, width = 16, 4, 200, 256  # 800 rows per KV head: 50 row tiles
    for i, lens in enumerate(([2500, 3100], [4096, 333])):
        note(f"fp32 long prefill D={D} window={window} call {i}: lens={lens}")
        q, kc, vc, table = make(H, KVH, D, lens, torch.float32, width, seed=D + i,
                                q_len=q_len)
        fused, two, hdr, hdr2 = caller.run(q, kc, vc, table, lens, window=window)
        check(fused, two, hdr, q, kc, vc, table, lens, window=window or None, hdr2=hdr2)


WIDE_CASES = {  # name -> (H, KVH, D, q dtype, cache dtype, batch, window)
    "C5 geometry bf16": (28, 4, 128, torch.bfloat16, torch.bfloat16, 16, 0),
    "C5 geometry fp8 cache": (28, 4, 128, torch.bfloat16, torch.float8_e4m3fn, 16, 0),
    "fp16 D64 G4": (16, 4, 64, torch.float16, torch.float16, 16, 0),
    "bf16 window 1500": (28, 4, 128, torch.bfloat16, torch.bfloat16, 16, 1500),
    # an fp8 cache at 4 rows per tile takes the wide shape past 1.5 workgroups per CU
    "fp8 cache G4, 512 workgroups": (32, 8, 128, torch.bfloat16, torch.float8_e4m3fn, 16, 0),
}


@pytest.mark.parametrize("name", list(WIDE_CASES))
def test_wide_shape_long_contexts(device, name):
    """Few (sequence, KV head) pairs over long contexts take the wide partition shape (8
    waves, partitions of more than 512 tokens, about one workgroup per CU): the header
    must name it, and the output must meet the float64 oracle's bar (K/V cast to the
    query type) on three consecutive calls, with empty, one-token, one-partition and
    full-table sequences among them."""
    H, KVH, D, q_dtype, kv_dtype, B, window = WIDE_CASES[name]
    width = 256  # 4096 tokens: a 1024-token partition for 64 (sequence, KV head) pairs
    caller = Caller(device, 64 << 20)
    for i in range(3):
        g = torch.Generator().manual_seed(300 + 10 * i + H)
        lens = [int(x) for x in torch.randint(1024, width * 16 + 1, (B,), generator=g)]
        lens[0], lens[1], lens[2], lens[3] = 0, 1, 700, width * 16
        note(f"wide {name} call {i}: lens={lens}")
        q, kc, vc, table = make(H, KVH, D, lens, q_dtype, width, seed=i + 11 * H)
        kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
        fused, two, hdr, hdr2 = caller.run(q, kc, vc, table, lens, window=window)
        assert (int(hdr[0]), int(hdr[9])) == (2, 8), f"kind {int(hdr[0])}, waves {int(hdr[9])}"
        assert int(hdr[8]) > 512, int(hdr[8])
        assert not hdr[HDR_TICKETS:].any(), "merge counters not left at zero"
        assert not torch.isnan(fused).any()
        assert not fused[0].cpu().any()  # context 0 -> zeros
        ref = dense.paged_attention_f64(q, kc, vc, table.long(), lens, window=window or None,
                                        kv_cast=True)
        for out in (fused, two):
            f = out.double().cpu().numpy()
            err = float(np.abs(f - ref).max() / max(np.abs(ref).max(), 1e-30))
            assert err < BF16_REL, err
        note(f"oracle err {err:.3e}, partition {int(hdr[8])}")


@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_deep_residency_head_dim_64(device, kv_dtype):
    """A head_dim-64 partition decode of many workgroups per CU (128 sequences x 2 KV heads
    of 1-3.8k tokens over 512-token partitions: eight per CU) holds three workgroups a CU
    instead of two: the header must name that residency, and the output must meet the
    float64 oracle's bar on two consecutive calls (the merge counters back at zero). The
    table (61,440 tiles of capacity) stays below the fp8 cache's stream-K threshold."""
    H, KVH, D, B, width = 14, 2, 64, 128, 240
    caller = Caller(device, 64 << 20)
    for i in range(2):
        g = torch.Generator().manual_seed(500 + i)
        lens = [int(x) for x in torch.randint(1024, width * 16 + 1, (B,), generator=g)]
        lens[0], lens[1] = 0, 1
        note(f"deep residency kv={kv_dtype} call {i}: sum {sum(lens)}")
        q, kc, vc, table = make(H, KVH, D, lens, torch.bfloat16, width, seed=600 + i)
        kc, vc = kc.to(kv_dtype), vc.to(kv_dtype)
        fused, two, hdr, hdr2 = caller.run(q, kc, vc, table, lens)
        assert (int(hdr[0]), int(hdr[9]), int(hdr[14])) == (2, 4, 3), hdr[:16].tolist()
        assert not hdr[HDR_TICKETS:].any(), "merge counters not left at zero"
        assert not fused[0].cpu().any()
        ref = dense.paged_attention_f64(q, kc, vc, table.long(), lens, kv_cast=True)
        for out in (fused, two):
            f = out.double().cpu().numpy()
            err = float(np.abs(f - ref).max() / max(np.abs(ref).max(), 1e-30))
            assert err < BF16_REL, err
        note(f"oracle err {err:.3e}")
