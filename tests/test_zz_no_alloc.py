"""msattn_paged_attention_noalloc: the workspace-free variant of msattn_paged_attention.

Called through the C ABI (ctypes) and compared with the workspace entry point on the
same inputs: two calls in a row, the second with a smaller batch and shorter contexts
(so the scratch still holds the first call's partials), on the stream-K decode, the
partition decode (bf16 and fp32), the generic kernel (fp32, head_dim 96) and the direct
prefill route; the results
must be bit-identical (the same kernels run) and within the float64 oracle's bar. A
geometry whose workspace exceeds the scratch is refused before any work.
"""
import numpy as np
import pytest
import torch

from miniserve_amd import _native as nat
from miniserve_amd import kernel_route
from oracle import dense

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20
FP32_ATOL = 1e-4
BF16_REL = 2e-2


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def make(H, KVH, D, lens, q_len, dtype, width, seed):
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


def call_both(device, q, kc, vc, table, lens, max_ctx):
    """(workspace entry's output, no-allocation entry's output) for one input."""
    lib = nat.lib()
    B, q_len, H, D = q.shape
    nb, bs, KVH, _ = kc.shape
    qd, kcd, vcd = q.to(device), kc.to(device), vc.to(device)
    td = table.to(device)
    ld = torch.tensor(lens, dtype=torch.int32, device=device)
    ws_bytes = lib.msattn_workspace_bytes(B, q_len, H, KVH, D, max_ctx)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=device)
    out_ws = torch.full_like(qd, float("nan"))
    out_na = torch.full_like(qd, float("nan"))
    scale = 1.0 / D ** 0.5
    common = (qd.data_ptr(), kcd.data_ptr(), vcd.data_ptr(), kcd.stride(0), kcd.stride(1),
              kcd.stride(2), td.data_ptr(), ld.data_ptr())
    tail = (B, q_len, H, KVH, D, bs, nb, table.shape[1], max_ctx, 1, 0, scale,
            nat.dtype_code(q.dtype), nat.dtype_code(kc.dtype))
    stream = nat.stream_handle(device)
    st = lib.msattn_paged_attention(*common, out_ws.data_ptr(), ws.data_ptr(), ws_bytes, *tail,
                                    stream)
    assert st == nat.OK, st
    st = lib.msattn_paged_attention_noalloc(*common, out_na.data_ptr(), *tail, stream)
    assert st == nat.OK, st
    torch.cuda.synchronize()
    return out_ws, out_na


def check_oracle(out, q, kc, vc, table, lens):
    ref = dense.paged_attention_f64(q, kc, vc, table.long(), lens)
    o = out.double().cpu().numpy()
    if q.dtype == torch.float32:
        assert np.abs(o - ref).max() < FP32_ATOL
    else:
        assert np.abs(o - ref).max() / np.abs(ref).max() < BF16_REL


CASES = {  # name -> (H, KVH, D, dtype, q_len, first lens, second lens, width in pages)
    "stream-K": (32, 8, 128, torch.bfloat16, 1, [3000, 17, 5000, 0, 800, 4096, 1, 2500],
                 [900, 33, 4000], 4096),
    "partition": (14, 2, 64, torch.bfloat16, 1, [1500, 300, 2048, 77, 1024, 640],
                  [100, 1800], 128),
    "partition fp32": (14, 2, 64, torch.float32, 1, [400, 130, 512, 9], [200, 35], 32),
    "generic fp32": (14, 2, 96, torch.float32, 1, [400, 130, 512, 9], [200, 35], 32),
    "prefill": (28, 4, 128, torch.bfloat16, 64, [512, 700], [64], 48),
    # 8 x 4 = 32 rows per KV head over 16 pairs: the partition kernel's 16-row tiles
    "partition prefill": (32, 8, 128, torch.bfloat16, 8, [900, 3000], [100], 256),
}


@pytest.mark.parametrize("name", list(CASES))
def test_noalloc_matches_workspace_entry(device, name):
    H, KVH, D, dtype, q_len, lens1, lens2, width = CASES[name]
    for i, lens in enumerate((lens1, lens2)):
        note(f"noalloc {name} call {i + 1}: B={len(lens)} lens={lens}")
        q, kc, vc, table = make(H, KVH, D, lens, q_len, dtype, width, seed=7 * i + len(name))
        max_ctx = width * 16
        out_ws, out_na = call_both(device, q, kc, vc, table, lens, max_ctx)
        assert torch.equal(out_ws, out_na)
        check_oracle(out_na, q, kc, vc, table, lens)


def test_noalloc_refuses_geometry_past_scratch(device):
    """A decode whose workspace would exceed the scratch returns MSATTN_ERR_WORKSPACE
    before launching anything."""
    lib = nat.lib()
    B, H, KVH, D, W = 512, 32, 8, 128, 1024
    assert lib.msattn_workspace_bytes(B, 1, H, KVH, D, W * 16) > SCRATCH
    q = torch.zeros(B, 1, H, D, dtype=torch.bfloat16, device=device)
    kc = torch.zeros(4, 16, KVH, D, dtype=torch.bfloat16, device=device)
    table = torch.zeros(B, W, dtype=torch.int32, device=device)
    lens = torch.ones(B, dtype=torch.int32, device=device)
    out = torch.empty_like(q)
    st = lib.msattn_paged_attention_noalloc(
        q.data_ptr(), kc.data_ptr(), kc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2),
        table.data_ptr(), lens.data_ptr(), out.data_ptr(), B, 1, H, KVH, D, 16, 4, W, W * 16, 1, 0,
        0.1, nat.BF16, nat.BF16, nat.stream_handle(device))
    assert st == nat.ERR_WORKSPACE


def test_noalloc_long_table_prefill_takes_the_prefill_kernel(device):
    """A short chunked prefill over a long-capacity table (131072 tokens): the workspace
    entry runs it on the partition kernel, whose layout at that capacity exceeds the
    scratch; the no-allocation entry runs it on the prefill kernel (whose stream-K
    tickets and partials fit the scratch) instead of refusing it. Both within the oracle's bar, and within two output ulps of
    each other (different kernels sum in different orders); two calls in a row, the
    second smaller."""
    H, KVH, D, q_len, width = 32, 8, 128, 8, 8192
    assert nat.lib().msattn_workspace_bytes(4, q_len, H, KVH, D, width * 16) > SCRATCH
    for i, lens in enumerate(([300, 2000, 9, 1200], [40, 700])):
        note(f"noalloc long table call {i + 1}: lens={lens}")
        q, kc, vc, table = make(H, KVH, D, lens, q_len, torch.bfloat16, width, seed=31 + i)
        qd, kcd, td = q.to(device), kc.to(device), table.to(device)
        assert kernel_route(qd, kcd, td) == "partition-fused"
        assert kernel_route(qd, kcd, td, workspace_bytes=SCRATCH) == "prefill stream-K"
        out_ws, out_na = call_both(device, q, kc, vc, table, lens, width * 16)
        check_oracle(out_ws, q, kc, vc, table, lens)
        check_oracle(out_na, q, kc, vc, table, lens)
        diff = (out_ws.float() - out_na.float()).abs().max().item()
        assert diff <= 2 * 2.0 ** -7 * out_ws.float().abs().max().item()
