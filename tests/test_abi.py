"""CPU checks of the C ABI: the library loads, exports every symbol the header
declares, and rejects bad arguments with status codes before touching the GPU."""
import ctypes
import re
from pathlib import Path

import pytest

from miniserve_amd import _native as nat

HEADER = Path(__file__).resolve().parents[1] / "include" / "msattn.h"


def declared_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^[a-z][\w \*]*?\b(msattn_\w+)\(", text, flags=re.M)))


def test_header_declares_the_bound_api():
    names = declared_functions()
    assert names == sorted(nat.SIGNATURES), names


def test_library_exports_every_declared_symbol():
    lib = nat.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_abi_version_and_status_strings():
    lib = nat.lib()
    assert lib.msattn_abi_version() == 1
    for code, text in [(0, b"ok"), (1, b"invalid argument"), (3, b"workspace too small"),
                       (99, b"unknown status")]:
        assert lib.msattn_status_string(code) == text


@pytest.mark.parametrize("B,q_len,H,KVH,D,ctx,part", [
    (64, 1, 32, 8, 128, 8192, 512),     # C3
    (8, 1, 32, 8, 128, 131072, 512),    # C4
    (32, 1, 14, 2, 64, 2048, 256),      # C2: few (row, head) units -> smaller partitions
    (4, 1, 14, 2, 64, 512, 64),         # C1: the smallest partitions
    (16, 1, 28, 4, 128, 4608, 512),     # C5 decode
])
def test_partition_policy(B, q_len, H, KVH, D, ctx, part):
    lib = nat.lib()
    assert lib.msattn_partition_tokens(B, q_len, H, KVH, D, ctx) == part
    # header: 64 ints, 4096 merge tickets, B + 1 prefix sums; slots: rows x (partitions
    # + end marker),
    # or stream-K pieces x UG x RT if larger: pieces = chunks + NUG x B, chunks at
    # most 256 workgroups x waves / UG and at most tiles / 4, for the larger of the
    # two stream-K shapes (4 waves for a 2-byte cache, 8 for fp8)
    r256 = lambda x: -(-x // 256) * 256
    rows = B * q_len * H
    slots = rows * (-(-ctx // part) + 1)
    if q_len == 1:
        G = H // KVH
        RT = 16 if G >= 16 else 1 << (G - 1).bit_length()
        units = KVH * -(-G // RT)
        for waves in (4, 8):
            UG = max(u for u in (1, 2, 4, 8) if u <= waves and units % u == 0)
            segments = units // UG * B
            chunks = min(256 * waves // UG, -(-(segments * -(-ctx // 16)) // 4))
            slots = max(slots, (chunks + segments) * UG * RT)
    expect = r256(4 * (64 + 4096 + B + 1)) + r256(slots * 2 * 4) + slots * D * 4
    assert lib.msattn_workspace_bytes(B, q_len, H, KVH, D, ctx) == expect


def test_workspace_rejects_bad_geometry():
    lib = nat.lib()
    assert lib.msattn_workspace_bytes(1, 1, 6, 4, 64, 16) == 0     # H % KVH != 0
    assert lib.msattn_workspace_bytes(1, 1, 4, 4, 65, 16) == 0     # odd head_dim
    assert lib.msattn_workspace_bytes(1, 1, 4, 4, 258, 16) == 0    # head_dim past 256
    assert lib.msattn_partition_tokens(0, 1, 4, 4, 64, 16) == -1


@pytest.mark.parametrize("D", [2, 6, 40, 66, 80, 112, 200, 256])
def test_every_even_head_dim_up_to_256_is_a_valid_geometry(D):
    """miniserve/attention.py:87-88 accepts any positive even head_dim; the library takes
    every even size up to 256 (the generic kernel's element mode for sizes it does not
    compile exactly)."""
    lib = nat.lib()
    assert lib.msattn_workspace_bytes(3, 1, 8, 2, D, 1000) > 0
    assert lib.msattn_workspace_bytes(3, 5, 8, 2, D, 1000) > 0


def _attn_args(**over):
    buf = ctypes.create_string_buffer(1 << 16)
    p = ctypes.addressof(buf)
    p16 = (p + 15) // 16 * 16
    k_off = over.pop("k_off", 0)
    args = dict(query=p16, k=p16 + k_off, v=p16, bstride=16 * 2 * 64, sstride=2 * 64,
                hstride=64, table=p16, lens=p16, out=p16, ws=p16, ws_bytes=1 << 15, batch=1,
                q_len=1, H=4, KVH=2, D=64, bs=16, nb=4, W=1, max_ctx=16, causal=1, window=0,
                scale=0.125, qd=nat.F32, kvd=nat.F32, stream=None)
    args.update(over)
    return buf, list(args.values())


@pytest.mark.parametrize("over,status", [
    (dict(query=None), nat.ERR_INVALID_ARG),
    (dict(H=6, KVH=4), nat.ERR_INVALID_ARG),
    (dict(batch=0), nat.ERR_INVALID_ARG),
    (dict(qd=nat.FP8_E4M3), nat.ERR_INVALID_ARG),
    (dict(kvd=7), nat.ERR_INVALID_ARG),
    (dict(scale=float("nan")), nat.ERR_INVALID_ARG),
    (dict(k_off=2), nat.ERR_INVALID_ARG),                  # cache not aligned to its element
    (dict(sstride=-1), nat.ERR_INVALID_ARG),
    (dict(ws_bytes=16), nat.ERR_WORKSPACE),
    (dict(D=65, bstride=16 * 2 * 65, sstride=2 * 65, hstride=65), nat.ERR_INVALID_ARG),
    (dict(D=258, bstride=16 * 2 * 258, sstride=2 * 258, hstride=258), nat.ERR_INVALID_ARG),
    (dict(query=1), nat.ERR_INVALID_ARG),                  # query not aligned to its element
    (dict(out=2), nat.ERR_INVALID_ARG),                    # output not aligned to its element
])
def test_paged_attention_argument_errors(over, status):
    """Every error path returns before any HIP call, so it runs without a GPU."""
    buf, args = _attn_args(**over)
    assert nat.lib().msattn_paged_attention(*args) == status


@pytest.mark.parametrize("over,rope,status", [
    (dict(), (None, 1, 1, 8), nat.ERR_INVALID_ARG),         # no cos table
    (dict(), (1, 1, 1, 0), nat.ERR_INVALID_ARG),            # empty tables
    (dict(), (2, 1, 1, 8), nat.ERR_INVALID_ARG),            # cos not 16-byte aligned
    (dict(q_len=2), (1, 1, 1, 8), nat.ERR_UNSUPPORTED),     # decode-only
])
def test_rope_entry_argument_errors(over, rope, status):
    """msattn_paged_attention_rope rejects bad RoPE arguments before any HIP call."""
    buf, args = _attn_args(**over)
    base = (ctypes.addressof(buf) + 15) // 16 * 16
    ptr = lambda x: None if x is None else base + (0 if x == 1 else x)
    cos, sin, pos, max_pos = ptr(rope[0]), ptr(rope[1]), ptr(rope[2]), rope[3]
    assert nat.lib().msattn_paged_attention_rope(*args[:-1], cos, sin, pos, max_pos,
                                                 None) == status


@pytest.mark.parametrize("B,H,KVH,D,bs,ctx,pages", [
    (8, 32, 8, 128, 16, 131072, 512),   # C4: 8192 shared tokens
    (4, 14, 2, 64, 16, 512, 3),
    (64, 32, 8, 128, 32, 8192, 1),
    (3, 32, 8, 128, 16, 100, 40),       # prefix longer than max_context
])
def test_prefix_workspace_layout(B, H, KVH, D, bs, ctx, pages):
    """Cascade workspace = the decode workspace, then (m, l) and acc slots for
    rows x prefix partitions; partitions of >= 128 tokens (whole 64-token steps)
    sized so (row blocks x KV heads x partitions) about reaches 256 workgroups."""
    lib = nat.lib()
    r256 = lambda x: -(-x // 256) * 256
    base = lib.msattn_workspace_bytes(B, 1, H, KVH, D, ctx)
    prefix = min(pages * bs, ctx)
    per = -(-(B * (H // KVH)) // 128) * KVH
    want = max(1, min(-(-256 // per), -(-prefix // 128)))
    key_part = -(-(-(-prefix // want)) // 64) * 64
    npart = -(-prefix // key_part)
    slots = B * H * npart
    expect = r256(base) + r256(slots * 8) + slots * D * 4
    assert lib.msattn_prefix_workspace_bytes(B, H, KVH, D, bs, ctx, pages) == expect
    assert lib.msattn_prefix_workspace_bytes(B, H, KVH, D, bs, ctx, -1) == 0


def _prefix_args(pages=1, query_offset=0, **over):
    buf, args = _attn_args(**over)
    names = ["query", "k", "v", "bstride", "sstride", "hstride", "table", "lens", "out", "ws",
             "ws_bytes", "batch", "q_len", "H", "KVH", "D", "bs", "nb", "W", "max_ctx",
             "causal", "window", "scale", "qd", "kvd", "stream"]
    a = dict(zip(names, args))
    if a["query"] is not None:
        a["query"] += query_offset
    keep = names[:12] + ["H", "KVH", "D", "bs", "nb", "W", "max_ctx"]
    return buf, [a[n] for n in keep] + [pages, a["scale"], a["qd"], a["kvd"], None]


@pytest.mark.parametrize("over,status", [
    (dict(query=None), nat.ERR_INVALID_ARG),
    (dict(out=None), nat.ERR_INVALID_ARG),
    (dict(pages=-1), nat.ERR_INVALID_ARG),
    (dict(pages=2), nat.ERR_INVALID_ARG),                 # more pages than the table holds
    (dict(qd=nat.FP8_E4M3), nat.ERR_INVALID_ARG),
    (dict(scale=float("inf")), nat.ERR_INVALID_ARG),
    (dict(ws_bytes=16), nat.ERR_WORKSPACE),
    (dict(query_offset=2), nat.ERR_INVALID_ARG),          # fp32 query not 4-byte aligned
])
def test_prefix_entry_argument_errors(over, status):
    """msattn_paged_attention_prefix returns before any HIP call on a bad argument."""
    buf, args = _prefix_args(**over)
    assert nat.lib().msattn_paged_attention_prefix(*args) == status


def test_check_maps_status_to_exceptions():
    with pytest.raises(ValueError, match="workspace too small"):
        nat.check("f", nat.ERR_WORKSPACE)
    with pytest.raises(nat.MsattnError):
        nat.check("f", nat.ERR_HIP)
    nat.check("f", nat.OK)


def test_stream_read_probe_rejects_bad_arguments():
    """msattn_probe_stream_read returns before any HIP call on a bad argument: null or
    misaligned pointers, a size that is zero or not a multiple of 16."""
    lib = nat.lib()
    assert lib.msattn_probe_stream_read(None, 1 << 20, 256, None) == nat.ERR_INVALID_ARG
    assert lib.msattn_probe_stream_read(256, 1 << 20, None, None) == nat.ERR_INVALID_ARG
    assert lib.msattn_probe_stream_read(256, 0, 256, None) == nat.ERR_INVALID_ARG
    assert lib.msattn_probe_stream_read(256, (1 << 20) + 8, 256, None) == nat.ERR_INVALID_ARG
    assert lib.msattn_probe_stream_read(264, 1 << 20, 256, None) == nat.ERR_INVALID_ARG
    assert lib.msattn_probe_stream_read(256, 1 << 20, 258, None) == nat.ERR_INVALID_ARG


def test_noalloc_entry_checks_before_any_hip_call():
    """msattn_paged_attention_noalloc rejects bad arguments, and geometries whose
    workspace exceeds its scratch (MSATTN_NOALLOC_SCRATCH_BYTES, 64 MiB), before it
    looks up the scratch or launches anything."""
    lib = nat.lib()
    buf, args = _attn_args()
    a = args[:9] + args[11:]  # drop workspace and workspace_bytes
    bad_out = list(a)
    bad_out[8] = None
    assert lib.msattn_paged_attention_noalloc(*bad_out) == nat.ERR_INVALID_ARG
    bad_geom = list(a)
    bad_geom[11:13] = [6, 4]  # H % KVH != 0
    assert lib.msattn_paged_attention_noalloc(*bad_geom) == nat.ERR_INVALID_ARG
    big = list(a)
    # batch 512, H32/KVH8/D128, 16k context: a 276 MB workspace
    big[9], big[11], big[12], big[13], big[16], big[17] = 512, 32, 8, 128, 1024, 16384
    big[-3] = big[-2] = nat.BF16
    assert lib.msattn_workspace_bytes(512, 1, 32, 8, 128, 16384) > 64 << 20
    assert lib.msattn_paged_attention_noalloc(*big) == nat.ERR_WORKSPACE


# ------------------------------------------------------------------ kernel routes

def route(B, q_len, H, KVH, D, ctx, qd=nat.BF16, kvd=None, ws=None, slot_stride=None,
          bs=16, query=256, out=256):
    """msattn_paged_attention_route for a contiguous cache [.., bs, KVH, D] (or the given
    slot stride), with the call's own workspace size unless `ws` is given."""
    lib = nat.lib()
    kvd = qd if kvd is None else kvd
    ss = KVH * D if slot_stride is None else slot_stride
    ws = lib.msattn_workspace_bytes(B, q_len, H, KVH, D, ctx) if ws is None else ws
    r = ctypes.c_int(-1)
    st = lib.msattn_paged_attention_route(query, out, 256, 256, bs * ss, ss, D, B, q_len, H, KVH,
                                          D, bs, ctx, qd, kvd, ws, ctypes.byref(r))
    return st, r.value


@pytest.mark.parametrize("shape,want", [
    ((64, 1, 32, 8, 128, 8192), nat.ROUTE_STREAMK),            # C3
    ((32, 1, 14, 2, 64, 2048), nat.ROUTE_PARTITION_FUSED),     # C2
    ((16, 1, 28, 4, 128, 4608), nat.ROUTE_PARTITION_FUSED),    # C5 decode
    ((2, 512, 28, 4, 128, 4608), nat.ROUTE_PREFILL),           # C5 prefill
    ((8, 4, 28, 4, 128, 8192), nat.ROUTE_PARTITION_FUSED),     # speculative: 28 rows, 32 pairs
    ((64, 6, 32, 8, 128, 8192), nat.ROUTE_PREFILL),            # 24 rows over 512 pairs
    ((1, 512, 8, 1, 128, 8192), nat.ROUTE_PREFILL_STREAMK),    # 4096 rows: 32 tasks, stream-K
    ((4, 16, 32, 8, 128, 8192), nat.ROUTE_PARTITION_FUSED),    # 64 rows: the measured limit
    ((4, 17, 32, 8, 128, 8192), nat.ROUTE_PREFILL_STREAMK),    # 68 rows: past it (32 tasks)
    # prefill tasks scheduled stream-K where one task per CU leaves CUs idle long enough
    ((1, 128, 32, 8, 128, 8192), nat.ROUTE_PREFILL_STREAMK),   # 32 tasks of 64 key-step pairs
    ((2, 384, 32, 8, 128, 4096), nat.ROUTE_PREFILL),           # 192 tasks: one round
    ((4, 128, 32, 8, 128, 2048), nat.ROUTE_PREFILL_STREAMK),   # 128 tasks of 16 pairs
    ((2, 512, 28, 4, 128, 4608), nat.ROUTE_PREFILL),           # 224 tasks of 36 pairs
    # stream-K thresholds: 2^16 table tiles at head_dim 128, 2^17 at head_dim 64
    ((64, 1, 32, 8, 128, 8158), nat.ROUTE_STREAMK),            # C3 called with max(lens)
    ((16, 1, 32, 8, 128, 8192), nat.ROUTE_STREAMK),            # 65,536 tiles
    ((15, 1, 32, 8, 128, 8192), nat.ROUTE_PARTITION_FUSED),    # 61,440
    ((64, 1, 14, 2, 64, 8192), nat.ROUTE_PARTITION_FUSED),     # 65,536 at head_dim 64
    ((128, 1, 14, 2, 64, 8192), nat.ROUTE_STREAMK),            # 131,072 at head_dim 64
])
def test_route_policy(shape, want):
    """The routing rules in csrc/abi.hip: stream-K from 2^16 table tiles at head_dim 128
    (2^17 at head_dim 64), the partition kernel (merging in-kernel) below; chunked prefill
    on the prefill kernel unless at most 64 rows per KV head over too few (sequence, KV
    head) pairs to fill the device, stream-K scheduled where the cost model prefers it
    (sizes from the measured prefill sweep)."""
    st, r = route(*shape)
    assert st == nat.OK and r == want, (nat.ROUTE_NAMES.get(r), shape)


def test_route_generic_kernel_cases():
    """Pairs and layouts outside the MFMA kernels take the generic kernel."""
    assert route(4, 1, 8, 2, 40, 1000)[1] == nat.ROUTE_GENERIC            # head_dim 40
    assert route(4, 1, 8, 2, 6, 1000)[1] == nat.ROUTE_GENERIC             # head_dim 6
    assert route(4, 1, 8, 2, 128, 1000, qd=nat.F16, kvd=nat.BF16)[1] == nat.ROUTE_GENERIC
    assert route(4, 1, 8, 2, 64, 1000, slot_stride=2 * 64 + 1)[1] == nat.ROUTE_GENERIC
    assert route(4, 1, 8, 2, 64, 1000, bs=24)[1] == nat.ROUTE_GENERIC     # pages of 24 tokens
    assert route(4, 1, 8, 2, 64, 1000, query=258)[1] == nat.ROUTE_GENERIC  # query off 16 B
    # an fp32 query over any cache decodes on the MFMA partition kernel
    assert route(4, 1, 8, 2, 64, 1000, qd=nat.F32, kvd=nat.FP8_E4M3)[1] == \
        nat.ROUTE_PARTITION_FUSED


def test_noalloc_route_falls_back_to_the_prefill_kernel():
    """A chunked prefill the cost model sends to the partition kernel, whose partition
    layout at this table capacity exceeds the no-allocation scratch, runs on the prefill
    kernel (no scratch) instead of failing; a decode past the scratch still fails."""
    lib = nat.lib()
    B, q_len, H, KVH, D, ctx = 4, 8, 32, 8, 128, 131072
    assert lib.msattn_workspace_bytes(B, q_len, H, KVH, D, ctx) > nat.NOALLOC_SCRATCH_BYTES
    assert route(B, q_len, H, KVH, D, ctx) == (nat.OK, nat.ROUTE_PARTITION_FUSED)
    assert route(B, q_len, H, KVH, D, ctx, ws=nat.NOALLOC_SCRATCH_BYTES) == \
        (nat.OK, nat.ROUTE_PREFILL_STREAMK)
    # a 64-token chunk over a 131072-token table
    assert route(1, 64, 28, 4, 128, 131072, ws=nat.NOALLOC_SCRATCH_BYTES) == \
        (nat.OK, nat.ROUTE_PREFILL_STREAMK)
    # a workspace too small for the stream-K partials: one task per workgroup
    assert route(1, 64, 28, 4, 128, 131072, ws=4096) == (nat.OK, nat.ROUTE_PREFILL)
    # an fp32 query has no prefill kernel: past the scratch it is refused
    assert route(B, q_len, H, KVH, D, ctx, qd=nat.F32, ws=nat.NOALLOC_SCRATCH_BYTES)[0] == \
        nat.ERR_WORKSPACE
    assert route(512, 1, 32, 8, 128, 16384, ws=nat.NOALLOC_SCRATCH_BYTES)[0] == nat.ERR_WORKSPACE


def test_route_rejects_bad_arguments():
    lib = nat.lib()
    r = ctypes.c_int(0)
    args = [256, 256, 256, 256, 16 * 256, 256, 128, 2, 1, 4, 2, 128, 16, 100, nat.BF16,
            nat.BF16, 1 << 30]
    assert lib.msattn_paged_attention_route(*args, None) == nat.ERR_INVALID_ARG
    bad = list(args)
    bad[11] = 129  # odd head_dim
    assert lib.msattn_paged_attention_route(*bad, ctypes.byref(r)) == nat.ERR_INVALID_ARG
    bad = list(args)
    bad[14] = nat.FP8_E4M3  # fp8 query
    assert lib.msattn_paged_attention_route(*bad, ctypes.byref(r)) == nat.ERR_INVALID_ARG


def test_append_rejects_bad_arguments():
    """msattn_paged_attention_append checks its pointers, types and geometry before it
    launches anything (these calls never reach a device)."""
    lib = nat.lib()
    # query, k_new, v_new, k_cache, v_cache, strides x3, table, lens, out, ws, ws_bytes,
    # batch, H, KVH, D, bs, num_blocks, W, max_context, window, scale, q/kv dtype, stream
    args = [256, 512, 768, 1024, 2048, 16 * 256, 256, 128, 4096, 8192, 16384, 32768, 1 << 20,
            2, 4, 2, 128, 16, 100, 4, 64, 0, 0.1, nat.BF16, nat.BF16, None]
    for i in (1, 2, 3, 4, 9, 10):  # k_new, v_new, k_cache, v_cache, lens, out
        bad = list(args)
        bad[i] = None
        assert lib.msattn_paged_attention_append(*bad) == nat.ERR_INVALID_ARG, i
    bad = list(args)
    bad[23] = nat.FP8_E4M3  # fp8 query
    assert lib.msattn_paged_attention_append(*bad) == nat.ERR_INVALID_ARG
    bad = list(args)
    bad[16] = 129  # odd head_dim
    assert lib.msattn_paged_attention_append(*bad) == nat.ERR_INVALID_ARG
    bad = list(args)
    bad[14] = 3  # heads not a multiple of KV heads
    assert lib.msattn_paged_attention_append(*bad) == nat.ERR_INVALID_ARG
