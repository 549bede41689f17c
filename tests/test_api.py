"""CPU checks of the PagedAttention interface (constructor contract, mask, errors)."""
import pytest
import torch

from miniserve_amd import PagedAttention
from oracle import paged_sdpa


@pytest.mark.parametrize("kwargs,msg", [
    (dict(num_heads=0, num_kv_heads=1, head_dim=8), "num_heads must be positive"),
    (dict(num_heads=6, num_kv_heads=4, head_dim=8), "multiple of num_kv_heads"),
    (dict(num_heads=4, num_kv_heads=2, head_dim=7), "positive even integer"),
    (dict(num_heads=4, num_kv_heads=2, head_dim=None), "positive even integer"),
    (dict(num_heads=4, num_kv_heads=2, head_dim=8, window=0), "window must be positive"),
])
def test_constructor_contract(kwargs, msg):
    """The ValueErrors of miniserve/attention.py:81-92."""
    with pytest.raises(ValueError, match=msg):
        PagedAttention(**kwargs, num_blocks=4, block_size=16)


def test_constructor_blocks():
    with pytest.raises(ValueError, match="num_blocks and block_size"):
        PagedAttention(4, 2, 8, num_blocks=0, block_size=16)


def test_group_and_cache_layout():
    """GQA KAT of tests/test_parity.py:135-136."""
    pa = PagedAttention(32, 8, 64, num_blocks=12, block_size=8, kv_dtype=torch.float32)
    assert pa.group == 4
    kc, vc = pa.allocate_kv_cache()
    assert kc.shape == (12, 8, 8, 64) and vc.dtype == torch.float32 and not kc.any()


def test_fp8_cache_bytes():
    pa8 = PagedAttention(4, 2, 32, num_blocks=8, block_size=8, kv_dtype=torch.float8_e4m3fn)
    kc8, _ = pa8.allocate_kv_cache()
    assert kc8.dtype == torch.float8_e4m3fn and kc8.element_size() == 1


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("window", [None, 64, 5])
def test_build_mask_matches_oracle(causal, window):
    pa = PagedAttention(4, 4, 16, num_blocks=4, block_size=16)
    lens = torch.tensor([512, 300, 1])
    got = pa.build_mask(lens, 2, window, causal)
    assert torch.equal(got, paged_sdpa.build_mask(lens, 2, window, causal))


def test_build_mask_window_kat():
    pa = PagedAttention(4, 4, 16, num_blocks=4, block_size=16)
    mask = pa.build_mask(torch.tensor([512, 300]), 2, 64)
    assert not mask[0, 1, :448].any() and mask[0, 1, 448:512].all()


def test_backend_contract_errors():
    """The contract errors of attention.py:187-194, 231-232, raised before any device work."""
    pa = PagedAttention(4, 4, 16, num_blocks=4, block_size=16, dtype=torch.float32)
    kc, vc = pa.allocate_kv_cache()
    q = torch.zeros(1, 1, 4, 16)
    table = torch.zeros(1, 1, dtype=torch.long)
    with pytest.raises(ValueError, match="decode-only"):
        pa.forward(torch.zeros(1, 2, 4, 16), kc, vc, table, [8], backend="triton_flash")
    with pytest.raises(ValueError, match="sliding window"):
        pa.forward(q, kc, vc, table, [8], window=4, backend="triton_flash")
    with pytest.raises(ValueError, match="causal decode only"):
        pa.forward(q, kc, vc, table, [8], causal=False, backend="triton_flash")
    with pytest.raises(ValueError, match="unknown attention backend"):
        pa.forward(q, kc, vc, table, [8], backend="nope")
    with pytest.raises(RuntimeError, match="requires CUDA"):
        pa.forward(q, kc, vc, table, [8], backend="triton_flash")


def test_cpu_tensors_fail_loudly():
    """No CPU path: forward and write_kv on CPU tensors raise instead of falling back."""
    pa = PagedAttention(4, 2, 16, num_blocks=4, block_size=16)
    kc, vc = pa.allocate_kv_cache()
    with pytest.raises(RuntimeError, match="GPU"):
        pa.forward(torch.zeros(1, 1, 4, 16, dtype=torch.float16), kc, vc,
                   torch.zeros(1, 1, dtype=torch.long), [1])
    with pytest.raises(RuntimeError, match="GPU"):
        pa.write_kv(kc, vc, torch.zeros(1, 1, 2, 16), torch.zeros(1, 1, 2, 16),
                    torch.zeros(1, 1, dtype=torch.long))


def test_graph_runner_bucket_contract():
    """miniserve/model_runner.py:243-244: buckets must be sorted and start at 1."""
    from miniserve_amd.graphs import GraphedDecodeRunner
    with pytest.raises(ValueError, match="sorted, start at 1"):
        GraphedDecodeRunner([object()], table_width=4, buckets=(4, 2))
    with pytest.raises(ValueError, match="sorted, start at 1"):
        GraphedDecodeRunner([object()], table_width=4, buckets=(0, 2))


@pytest.mark.parametrize("pos_shape", ["seq", "batch_seq"])
@pytest.mark.parametrize("with_k", [True, False])
def test_apply_rope_closed_form(pos_shape, with_k):
    """apply_rope (miniserve/attention.py:41-62) against the rotation written out element
    by element: out[..., d] = x[d] cos[p, d] - x[d + D/2] sin[p, d] for d < D/2 and
    x[d] cos[p, d] + x[d - D/2] sin[p, d] above, with cos/sin cast to the input dtype."""
    from miniserve_amd import apply_rope

    g = torch.Generator().manual_seed(2)
    B, H, KVH, S, D = 2, 4, 2, 3, 8
    q = torch.randn(B, H, S, D, generator=g)
    k = torch.randn(B, KVH, S, D, generator=g) if with_k else None
    cos = torch.randn(16, D, generator=g)
    sin = torch.randn(16, D, generator=g)
    pos = torch.tensor([5, 0, 9]) if pos_shape == "seq" else torch.tensor([[5, 0, 9], [1, 15, 2]])
    q_rot, k_rot = apply_rope(q, k, cos, sin, pos)

    def closed(x):
        out = torch.empty_like(x)
        for b in range(x.shape[0]):
            for h in range(x.shape[1]):
                for s in range(S):
                    p = int(pos[s] if pos.ndim == 1 else pos[b, s])
                    for d in range(D):
                        partner = -x[b, h, s, d + D // 2] if d < D // 2 else x[b, h, s, d - D // 2]
                        out[b, h, s, d] = x[b, h, s, d] * cos[p, d] + partner * sin[p, d]
        return out

    assert torch.allclose(q_rot, closed(q), atol=1e-6)
    if with_k:
        assert torch.allclose(k_rot, closed(k), atol=1e-6)
    else:
        assert k_rot is None
    # a planted mistake (partner without the sign flip) fails the same comparison
    bad = q * cos[pos].unsqueeze(1 if pos.ndim == 2 else 0) + \
        torch.cat([q[..., D // 2:], q[..., :D // 2]], -1) * sin[pos].unsqueeze(1 if pos.ndim == 2 else 0)
    assert not torch.allclose(bad, closed(q), atol=1e-3)


def test_runner_table_fill_matches_row_by_row():
    """GraphedDecodeRunner's host staging places ragged per-row page lists with one
    scatter (graphs.fill_table); it must equal the row-by-row fill, for lists, tuples,
    generators, arrays and tensors, and refuse rows wider than the table."""
    import numpy as np

    from miniserve_amd.graphs import fill_table

    rng = np.random.default_rng(3)
    for trial in range(50):
        rows, width, batch = int(rng.integers(1, 70)), int(rng.integers(1, 40)), 0
        batch = int(rng.integers(1, rows + 1))
        lists = [list(rng.integers(0, 10_000, int(rng.integers(0, width + 1))))
                 for _ in range(batch)]
        want = np.full((rows, width), -1, dtype=np.int32)
        for b, r in enumerate(lists):
            want[b, : len(r)] = r
        got = np.zeros((rows, width), dtype=np.int32)
        fill_table(got, lists, batch)
        assert np.array_equal(got, want), trial
        got[:] = 7
        fill_table(got, [tuple(r) for r in lists], batch)
        assert np.array_equal(got, want)
        got[:] = 7
        fill_table(got, [iter(r) for r in lists], batch)
        assert np.array_equal(got, want)
        dense = want[:batch]
        got[:] = 7
        fill_table(got, torch.from_numpy(dense.copy()), batch)
        assert np.array_equal(got, want)
    with pytest.raises(ValueError):
        fill_table(np.zeros((2, 3), dtype=np.int32), [[1, 2, 3, 4]], 1)
    with pytest.raises(ValueError):
        fill_table(np.zeros((2, 3), dtype=np.int32), [[1]], 2)
