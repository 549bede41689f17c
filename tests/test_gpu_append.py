"""GPU parity of msattn_paged_attention_append: write_kv of the new token at position
context_lens[b] - 1 followed by the decode, inside the decode launch where the partition
or stream-K kernel takes the call (bf16/fp16 query, at most 8 query rows per KV head), as
two launches elsewhere.

The reference pair is the library's own two calls on a copy of the caches:
msattn_write_kv at starts = context_lens - 1, then paged_attention. The fused call must
leave the caches and give the output equal to them bit for bit (the appended row is cast
as write_kv casts it, and the decode reads exactly those values), over several calls in
a row on one workspace, with pad rows (length 0), one-token rows (the new token is the
only key), rows whose new position falls on a hole in the table, and full tables. The
graphed runner is compared with and without the fused call over several decode steps.
"""
import pytest
import torch

from miniserve_amd import PagedAttention, _native as nat, kernel_route, paged_attention
from miniserve_amd import paged_attention_append
from miniserve_amd.graphs import DecodeLayer, GraphedDecodeRunner

pytestmark = pytest.mark.gpu


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def write_kv_ref(k_cache, v_cache, k_new, v_new, table, lens):
    """msattn_write_kv of k_new / v_new [B, 1, KVH, D] at starts = lens - 1."""
    B, _, KVH, D = k_new.shape
    nb, bs = k_cache.shape[:2]
    starts = (lens - 1).to(torch.int32).contiguous()
    st = nat.lib().msattn_write_kv(
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), k_cache.stride(1),
        k_cache.stride(2), k_new.contiguous().data_ptr(), v_new.contiguous().data_ptr(),
        table.data_ptr(), starts.data_ptr(), B, 1, KVH, D, bs, nb, table.shape[1],
        nat.dtype_code(k_new.dtype), nat.dtype_code(k_cache.dtype),
        nat.stream_handle(k_cache.device))
    assert st == nat.OK, st


# name -> (H, KVH, D, query dtype, cache dtype, batch, table pages, window, expected route)
CASES = {
    "C2 geometry bf16 (G7, RT8)": (14, 2, 64, torch.bfloat16, torch.bfloat16, 32, 128, 0,
                                   "partition-fused"),
    "C5 geometry bf16, wide shape": (28, 4, 128, torch.bfloat16, torch.bfloat16, 16, 288, 0,
                                     "partition-fused"),
    "fp16 G4 D128 window": (32, 8, 128, torch.float16, torch.float16, 8, 64, 300,
                            "partition-fused"),
    "bf16 over fp8": (28, 4, 128, torch.bfloat16, torch.float8_e4m3fn, 8, 96, 0,
                      "partition-fused"),
    "bf16 over fp32 (the runner's caches)": (14, 2, 64, torch.bfloat16, torch.float32, 16, 64, 0,
                                             "partition-fused"),
    "fp16 over fp8 D64 G8": (16, 2, 64, torch.float16, torch.float8_e4m3fn, 8, 64, 0,
                             "partition-fused"),
    # the two-launch forms
    "fp32 query (two launches)": (14, 2, 64, torch.float32, torch.float32, 8, 64, 0,
                                  "partition-fused"),
    "G16 (two launches)": (32, 2, 128, torch.bfloat16, torch.bfloat16, 8, 64, 0,
                           "partition-fused"),
    # stream-K (then the merge kernel): the append in the stream-K launch
    "stream-K table": (32, 8, 128, torch.bfloat16, torch.bfloat16, 16, 512, 0, "stream-K"),
    "stream-K table, fp8 cache (two launches)": (32, 8, 128, torch.bfloat16,
                                                 torch.float8_e4m3fn, 16, 512, 0, "stream-K"),
    "stream-K table, bf16 over fp32": (32, 8, 128, torch.bfloat16, torch.float32, 16, 512, 0,
                                       "stream-K"),
    "stream-K table, fp16 D64 G7 window": (14, 2, 64, torch.float16, torch.float16, 64, 1024,
                                           1000, "stream-K"),
    "head_dim 80, generic kernel (two launches)": (8, 2, 80, torch.bfloat16, torch.bfloat16, 8,
                                                   64, 0, "generic"),
}


@pytest.mark.parametrize("name", list(CASES))
def test_append_equals_write_kv_then_decode(device, name):
    H, KVH, D, q_dtype, kv_dtype, B, width, window, route = CASES[name]
    bs = 16
    cap = width * bs
    g = torch.Generator().manual_seed(width + H + D)
    gd = torch.Generator(device=device).manual_seed(width + H + D)
    pool = B * width + 8
    kc_a = torch.randn(pool, bs, KVH, D, generator=gd, device=device).to(kv_dtype)
    vc_a = torch.randn(pool, bs, KVH, D, generator=gd, device=device).to(kv_dtype)
    table = torch.randperm(pool, generator=g)[: B * width].view(B, width).to(torch.int32)
    kc_b, vc_b = kc_a.clone(), vc_a.clone()
    ws = torch.zeros(nat.lib().msattn_workspace_bytes(B, 1, H, KVH, D, cap), dtype=torch.uint8,
                     device=device)
    for call in range(3):
        lens = [int(x) for x in torch.randint(1, cap + 1, (B,), generator=g)]
        lens[0], lens[1], lens[2] = 0, 1, cap  # pad row, new token alone, full table
        tab = table.clone()
        tab[3, (lens[3] - 1) // bs] = -1  # row 3 appends onto a hole: nothing written or read
        note(f"append {name} call {call}: lens={lens[:6]}")
        q = torch.randn(B, 1, H, D, generator=gd, device=device).to(q_dtype)
        kn = torch.randn(B, 1, KVH, D, generator=gd, device=device).to(q_dtype)
        vn = torch.randn(B, 1, KVH, D, generator=gd, device=device).to(q_dtype)
        td = tab.to(device)
        ld = torch.tensor(lens, dtype=torch.int32, device=device)
        assert kernel_route(q, kc_a, td, max_context=cap) == route
        write_kv_ref(kc_b, vc_b, kn, vn, td, ld)
        ref = paged_attention(q, kc_b, vc_b, td, ld, max_context=cap,
                              window=window or None)
        out = paged_attention_append(q, kn, vn, kc_a, vc_a, td, ld, max_context=cap,
                                     window=window or None, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(kc_a.view(torch.uint8), kc_b.view(torch.uint8)), "K caches differ"
        assert torch.equal(vc_a.view(torch.uint8), vc_b.view(torch.uint8)), "V caches differ"
        assert not torch.isnan(out.float()).any()
        assert torch.equal(out, ref), float((out.float() - ref.float()).abs().max())
        assert not out[0].any()  # the pad row: no key, zeros
        assert not ws[:(64 + 4096) * 4].view(torch.int32)[64:].any(), "tickets not at zero"


def test_runner_fused_append_equals_two_calls(device):
    """The graphed runner with the fused call (default) and without it: the same outputs
    and caches over four decode steps of growing contexts, bucket padding included."""
    H_, KVH_, D_, BS, WIDTH, LAYERS, POOL = 14, 2, 64, 16, 32, 2, 2048

    def build(fused):
        g = torch.Generator().manual_seed(5)
        layers = []
        for _ in range(LAYERS):
            pa = PagedAttention(H_, KVH_, D_, num_blocks=POOL, block_size=BS,
                                dtype=torch.bfloat16, kv_dtype=torch.bfloat16, device=device)
            kc = torch.randn(POOL, BS, KVH_, D_, generator=g).to(torch.bfloat16).to(device)
            vc = torch.randn(POOL, BS, KVH_, D_, generator=g).to(torch.bfloat16).to(device)
            layers.append(DecodeLayer(pa, kc, vc))
        return GraphedDecodeRunner(layers, table_width=WIDTH, buckets=(1, 2, 4, 8),
                                   fused_append=fused), layers

    fused, lf = build(True)
    plain, lp = build(False)
    g = torch.Generator().manual_seed(6)
    B = 6  # bucket 8: two pad rows
    pages = torch.randperm(POOL, generator=g)[: B * WIDTH].view(B, WIDTH)
    ctx = [int(x) for x in torch.randint(1, 300, (B,), generator=g)]
    for step in range(4):
        note(f"runner fused append step {step}: ctx={ctx}")
        q = torch.randn(LAYERS, B, 1, H_, D_, generator=g).to(torch.bfloat16).to(device)
        k = torch.randn(LAYERS, B, 1, KVH_, D_, generator=g).to(torch.bfloat16).to(device)
        v = torch.randn(LAYERS, B, 1, KVH_, D_, generator=g).to(torch.bfloat16).to(device)
        tables = [row.tolist() for row in pages]
        a = fused.decode(q, k, v, tables, ctx).clone()
        b = plain.decode(q, k, v, tables, ctx).clone()
        torch.cuda.synchronize()
        assert torch.equal(a, b), f"step {step}"
        for x, y in zip(lf, lp):
            assert torch.equal(x.k_cache, y.k_cache) and torch.equal(x.v_cache, y.v_cache)
        ctx = [c + 1 for c in ctx]
