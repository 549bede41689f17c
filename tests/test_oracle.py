"""Pins the CPU oracle (oracle/) before it is trusted as the checker.

Each oracle function is checked against what fixes it independently:
  * known-answer tests from the reference's own tests
    (tests/test_parity.py:131-171, tests/test_triton_parity.py:62-107);
  * brute force with pure-Python loops on tiny inputs;
  * closed forms (context 1, zero query, equal keys, one dominant key);
  * invariants (split count, KV-head permutation, linearity in V);
  * mutation checks: a planted mistake in a copy of the oracle must fail.
"""
import math

import numpy as np
import pytest
import torch

from oracle import dense, paged_sdpa, split_k


def scenario(h, kv_heads, d, lens, q_len=1, block_size=8, dtype=torch.float32, seed=0,
             scale=1.0, scatter=False):
    """Seeded q + dense k/v mirrored into a paged cache (tests/test_parity.py:78-96)."""
    g = torch.Generator().manual_seed(seed)
    batch, max_l = len(lens), max(lens)
    nblocks = (max_l + block_size - 1) // block_size
    q = (torch.randn(batch, q_len, h, d, generator=g) * scale).to(dtype)
    k = torch.randn(batch, max_l, kv_heads, d, generator=g) * scale
    v = torch.randn(batch, max_l, kv_heads, d, generator=g) * scale
    pool = batch * nblocks
    kc = torch.zeros(pool, block_size, kv_heads, d, dtype=dtype)
    vc = torch.zeros(pool, block_size, kv_heads, d, dtype=dtype)
    order = torch.randperm(pool, generator=g) if scatter else torch.arange(pool)
    table = order.view(batch, nblocks).clone()
    for i, length in enumerate(lens):
        paged_sdpa.write_kv(kc, vc, k[i:i + 1, :length], v[i:i + 1, :length], table[i:i + 1], 0)
    return q, k, v, kc, vc, table, torch.tensor(lens)


def dense_closed_form(q, k, v, lens, window=None, causal=True):
    """Dense float32 reference of tests/test_parity.py:99-117 on unpaged k/v."""
    batch, q_len, heads, d = q.shape
    group = heads // k.shape[2]
    k = k.repeat_interleave(group, dim=2).float()
    v = v.repeat_interleave(group, dim=2).float()
    lens_t = torch.as_tensor(lens).reshape(-1)
    q_pos = lens_t[:, None] - q_len + torch.arange(q_len)[None, :]
    key_pos = torch.arange(k.shape[1])[None, None, :]
    mask = torch.ones(batch, q_len, k.shape[1], dtype=torch.bool)
    if causal:
        mask = key_pos <= q_pos[:, :, None]
    mask = mask & (key_pos < lens_t[:, None, None])
    if window is not None:
        mask = mask & (key_pos > (q_pos - window)[:, :, None])
    scores = torch.einsum("bqhd,bkhd->bhqk", q.float(), k) / math.sqrt(d)
    scores = scores.masked_fill(~mask[:, None], float("-inf"))
    return torch.einsum("bhqk,bkhd->bqhd", scores.softmax(-1), v)


# ---------------------------------------------------------------- build_mask

def test_mask_window_kat():
    """KAT of tests/test_parity.py:170-171."""
    mask = paged_sdpa.build_mask(torch.tensor([512, 300]), 2, 64)
    assert not mask[0, 1, :448].any() and mask[0, 1, 448:512].all()


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("window", [None, 1, 3])
def test_mask_brute_force(causal, window):
    lens, q_len = [5, 3, 7], 3
    mask = paged_sdpa.build_mask(lens, q_len, window, causal)
    for b, L in enumerate(lens):
        for i in range(q_len):
            qp = L - q_len + i
            for key in range(max(lens)):
                keep = key < L and (not causal or key <= qp) and (window is None or key > qp - window)
                assert bool(mask[b, i, key]) == keep, (b, i, key)


# ---------------------------------------------------------------- gather

def test_gather_address_encoded():
    """Every cache element holds its own address; the gather must return it."""
    nb, bs, kvh, d = 11, 4, 2, 3
    addr = torch.arange(nb * bs, dtype=torch.float32).view(nb, bs, 1, 1).expand(nb, bs, kvh, d)
    cache = addr.contiguous()
    g = torch.Generator().manual_seed(5)
    table = torch.randperm(nb, generator=g)[:8].view(2, 4)
    lens = torch.tensor([13, 6])
    out = paged_sdpa.gather(cache, table, lens, 13)
    for b in range(2):
        for p in range(13):
            want = table[b, p // bs] * bs + p % bs if p < lens[b] else p % bs  # page 0 past len
            assert torch.all(out[b, p] == float(want)), (b, p)


def test_gather_fp8_bytes():
    """The FP8 gather moves bytes unchanged (attention.py:168-170)."""
    g = torch.Generator().manual_seed(1)
    raw = torch.randint(0, 256, (6, 4, 1, 8), generator=g, dtype=torch.uint8)
    raw[raw == 0x7F] = 0
    raw[raw == 0xFF] = 0
    cache = raw.view(torch.float8_e4m3fn)
    table = torch.tensor([[3, 1, 5]])
    out = paged_sdpa.gather(cache, table, torch.tensor([10]), 10)
    for p in range(10):
        assert torch.equal(out[0, p].view(torch.uint8), raw[table[0, p // 4], p % 4])


# ---------------------------------------------------------------- write_kv

def test_write_kv_brute_force():
    g = torch.Generator().manual_seed(2)
    kc = torch.zeros(9, 4, 2, 3)
    vc = torch.zeros(9, 4, 2, 3)
    k = torch.randn(2, 5, 2, 3, generator=g)
    v = torch.randn(2, 5, 2, 3, generator=g)
    table = torch.tensor([[4, 0, 7], [2, 8, 1]])
    paged_sdpa.write_kv(kc, vc, k, v, table, start=[3, 6])
    written = set()
    for b, s in enumerate([3, 6]):
        for t in range(5):
            pos = s + t
            page, slot = int(table[b, pos // 4]), pos % 4
            assert torch.equal(kc[page, slot], k[b, t]) and torch.equal(vc[page, slot], v[b, t])
            written.add((page, slot))
    for page in range(9):
        for slot in range(4):
            if (page, slot) not in written:
                assert not kc[page, slot].any() and not vc[page, slot].any()


# ---------------------------------------------------------------- SDPA restatement

@pytest.mark.parametrize("case,tol", [
    (dict(h=8, kv=8, d=16, lens=[8, 13, 21], q_len=3), 1e-4),           # test_parity.py:120-128
    (dict(h=32, kv=8, d=64, lens=[32, 47], q_len=1), 1e-3),             # :131-141
    (dict(h=8, kv=1, d=32, lens=[16, 23], q_len=1), 1e-3),              # :144-153
])
def test_sdpa_restatement_matches_dense(case, tol):
    q, k, v, kc, vc, table, lens = scenario(case["h"], case["kv"], case["d"], case["lens"],
                                            q_len=case["q_len"])
    out = paged_sdpa.paged_attention_sdpa(q, kc, vc, table, lens)
    ref = dense_closed_form(q, k, v, lens)
    assert (out - ref).abs().max().item() < tol


def test_sdpa_restatement_window():
    """tests/test_parity.py:156-171: window 64 over ctx 512, block 16."""
    q, k, v, kc, vc, table, lens = scenario(4, 4, 16, [512, 300], q_len=2, block_size=16)
    out = paged_sdpa.paged_attention_sdpa(q, kc, vc, table, lens, window=64)
    ref = dense_closed_form(q, k, v, lens, window=64)
    assert (out - ref).abs().max().item() < 1e-4


def test_gqa_layout_kat():
    """Cache shape KAT of tests/test_parity.py:136."""
    _, _, _, kc, _, _, _ = scenario(32, 8, 64, [32, 47], q_len=1)
    assert kc.shape == (12, 8, 8, 64)


# ---------------------------------------------------------------- float64 oracle

def brute_force_attention(q, kc, vc, table, lens, causal=True, window=None):
    """Pure-Python loops over every (b, i, h, key, d)."""
    B, q_len, H, D = q.shape
    KVH, bs = kc.shape[2], kc.shape[1]
    group = H // KVH
    out = np.zeros((B, q_len, H, D))
    for b in range(B):
        L = int(lens[b])
        for i in range(q_len):
            qp = L - q_len + i
            for h in range(H):
                kvh = h // group
                keys = [key for key in range(L) if (not causal or key <= qp)
                        and (window is None or key > qp - window)]
                if not keys:
                    continue
                s = []
                for key in keys:
                    page, slot = int(table[b][key // bs]), key % bs
                    s.append(sum(float(q[b, i, h, d]) * float(kc[page, slot, kvh, d])
                                 for d in range(D)) / math.sqrt(D))
                m = max(s)
                w = [math.exp(x - m) for x in s]
                tot = sum(w)
                for d in range(D):
                    acc = 0.0
                    for wk, key in zip(w, keys):
                        page, slot = int(table[b][key // bs]), key % bs
                        acc += wk * float(vc[page, slot, kvh, d])
                    out[b, i, h, d] = acc / tot
    return out


@pytest.mark.parametrize("causal,window", [(True, None), (False, None), (True, 2)])
def test_dense_f64_brute_force(causal, window):
    q, _, _, kc, vc, table, lens = scenario(4, 2, 4, [5, 3], q_len=2, block_size=2,
                                            scatter=True, seed=7)
    got = dense.paged_attention_f64(q, kc, vc, table, lens, causal=causal, window=window)
    want = brute_force_attention(q, kc, vc, table, lens, causal, window)
    assert np.abs(got - want).max() < 1e-12


def test_dense_f64_special_cases():
    q, _, _, kc, vc, table, _ = scenario(4, 2, 8, [9, 9], q_len=1, scatter=True, seed=3)
    # context 1: output is exactly V[0] of the row's KV head
    out = dense.paged_attention_f64(q, kc, vc, table, [1, 1])
    for b in range(2):
        for h in range(4):
            v0 = vc[table[b, 0], 0, h // 2].double().numpy()
            assert np.array_equal(out[b, 0, h], v0)
    # zero query: uniform weights -> mean of V over the context
    out = dense.paged_attention_f64(torch.zeros_like(q), kc, vc, table, [9, 5])
    for b, L in enumerate([9, 5]):
        rows = dense.gather_rows(vc, table[b].numpy(), L)
        for h in range(4):
            assert np.allclose(out[b, 0, h], rows[:, h // 2].mean(axis=0), atol=1e-12)
    # one key with a dominant score: output is that V row
    kc2 = kc.clone()
    key = 4
    page, slot = table[1, key // 8], key % 8
    kc2[page, slot, 1] = q[1, 0, 2] * 1e3
    out = dense.paged_attention_f64(q, kc2, vc, table, [9, 9])
    assert np.allclose(out[1, 0, 2], vc[page, slot, 1].double().numpy(), atol=1e-9)
    # context 0: zeros by definition
    out = dense.paged_attention_f64(q, kc, vc, table, [0, 9])
    assert not out[0].any()


def test_dense_f64_kv_head_permutation():
    """Permuting KV heads permutes the output's head groups (h -> h // group)."""
    q, _, _, kc, vc, table, lens = scenario(6, 3, 8, [11, 7], scatter=True, seed=9)
    perm = torch.tensor([2, 0, 1])
    base = dense.paged_attention_f64(q, kc, vc, table, lens)
    # KV head j of the permuted cache is old head perm[j]; query group j must move with it
    qp = q.view(2, 1, 3, 2, 8)[:, :, perm].reshape(2, 1, 6, 8)
    got = dense.paged_attention_f64(qp, kc[:, :, perm], vc[:, :, perm], table, lens)
    want = base.reshape(2, 1, 3, 2, 8)[:, :, perm.numpy()].reshape(2, 1, 6, 8)
    assert np.allclose(got, want, atol=1e-12)


def test_dense_f64_linear_in_v():
    q, _, _, kc, vc, table, lens = scenario(4, 2, 8, [10, 6], scatter=True, seed=4)
    a = dense.paged_attention_f64(q, kc, vc, table, lens)
    b = dense.paged_attention_f64(q, kc, vc * 3.0, table, lens)
    c = dense.paged_attention_f64(q, kc, vc + 1.0, table, lens)
    assert np.allclose(b, 3 * a, atol=1e-9) and np.allclose(c, a + 1.0, atol=1e-9)


def test_dense_f64_matches_sdpa_restatement():
    """The two independent formulations agree (fp32 SDPA vs float64 einsum)."""
    q, _, _, kc, vc, table, lens = scenario(14, 2, 64, [130, 77, 300], scatter=True, seed=11)
    a = paged_sdpa.paged_attention_sdpa(q, kc, vc, table, lens).double().numpy()
    b = dense.paged_attention_f64(q, kc, vc, table, lens)
    assert np.abs(a - b).max() < 1e-5


# ---------------------------------------------------------------- split-K

def test_num_splits_kats():
    """tests/test_triton_parity.py:84-88 and :66-67."""
    assert split_k.num_splits_for(1) == 1
    assert split_k.num_splits_for(2048) == 1
    assert split_k.num_splits_for(2049) == 2
    assert split_k.num_splits_for(4096) == 2
    assert split_k.num_splits_for(16384) == split_k.MAX_SPLITS
    assert split_k.num_splits_for(100000) == split_k.MAX_SPLITS


@pytest.mark.parametrize("splits", [1, 2, 3, 8, 64])
def test_split_k_independent_of_split_count(splits):
    q, _, _, kc, vc, table, lens = scenario(8, 2, 32, [300, 64, 17, 33], scatter=True, seed=6)
    got = split_k.split_k_decode(q, kc, vc, table, lens, num_splits=splits).double().numpy()
    want = dense.paged_attention_f64(q, kc, vc, table, lens)
    assert np.abs(got - want).max() < 2e-6


def test_split_k_context_zero_and_rope():
    q, _, _, kc, vc, table, _ = scenario(4, 2, 16, [40, 40], scatter=True, seed=8)
    out = split_k.split_k_decode(q, kc, vc, table, [0, 40])
    assert not out[0].any()
    D = 16
    inv = 1.0 / (10000 ** (torch.arange(0, D, 2, dtype=torch.float32) / D))
    emb = torch.outer(torch.arange(41, dtype=torch.float32), inv)
    emb = torch.cat([emb, emb], dim=-1)
    cos, sin = emb.cos(), emb.sin()
    pos = torch.tensor([39, 39])
    fused = split_k.split_k_decode(q, kc, vc, table, [40, 40], cos=cos, sin=sin, position=pos)
    half = D // 2
    qr = q * cos[39] + torch.cat([-q[..., half:], q[..., :half]], -1) * sin[39]
    unfused = split_k.split_k_decode(qr, kc, vc, table, [40, 40])
    assert (fused - unfused).abs().max().item() < 1e-5


# ---------------------------------------------------------------- mutation checks

def test_planted_mistakes_are_caught():
    """A copy of the float64 oracle with one planted mistake fails the checks above."""
    q, _, _, kc, vc, table, lens = scenario(4, 2, 4, [5, 3], q_len=2, block_size=2,
                                            scatter=True, seed=7)
    want = brute_force_attention(q, kc, vc, table, lens)

    def off_by_one_qpos(length, q_len, causal, window):
        key = np.arange(length)[None, :]
        q_pos = length - q_len + np.arange(q_len)[:, None] + 1   # planted: +1
        keep = np.ones((q_len, length), dtype=bool)
        if causal:
            keep &= key <= q_pos
        return keep

    orig = dense.keep_mask
    dense.keep_mask = off_by_one_qpos
    try:
        bad = dense.paged_attention_f64(q, kc, vc, table, lens)
    finally:
        dense.keep_mask = orig
    assert np.abs(bad - want).max() > 1e-3

    # wrong GQA map (h % KVH instead of h // group) breaks the permutation invariant
    def wrong_map_attend(qq, k, v, keep, scale):
        q_len, H, D = qq.shape
        KVH = k.shape[1]
        out = np.zeros((q_len, H, D))
        for h in range(H):
            s = np.einsum("id,kd->ik", qq[:, h], k[:, h % KVH]) * scale
            s = np.where(keep, s, -np.inf)
            p = np.exp(s - s.max(-1, keepdims=True))
            out[:, h] = (p / p.sum(-1, keepdims=True)) @ v[:, h % KVH]
        return out

    q6, _, _, kc6, vc6, table6, lens6 = scenario(6, 3, 8, [11, 7], scatter=True, seed=9)
    good = dense.paged_attention_f64(q6, kc6, vc6, table6, lens6)
    orig = dense.attend_f64
    dense.attend_f64 = wrong_map_attend
    try:
        bad = dense.paged_attention_f64(q6, kc6, vc6, table6, lens6)
    finally:
        dense.attend_f64 = orig
    assert np.abs(bad - good).max() > 1e-3


# ---------------------------------------------------------------- K/V cast to the query dtype

@pytest.mark.parametrize("q_dtype,kv_dtype", [(torch.bfloat16, torch.float32),
                                              (torch.float16, torch.float32),
                                              (torch.float16, torch.bfloat16),
                                              (torch.bfloat16, torch.float16)])
def test_dense_kv_cast_context_one(q_dtype, kv_dtype):
    """Context 1: the output is V[0] as the query dtype holds it (attention.py:240-241
    casts the gathered rows to query.dtype). V values 1 + 2^-10 round to 1.0 in bf16 and
    stay in fp16, so dropping the cast, or casting to the wrong type, fails."""
    q, _, _, kc, vc, table, _ = scenario(4, 2, 8, [9, 9], q_len=1, scatter=True, seed=3)
    q = q.to(q_dtype)
    kc = kc.to(kv_dtype)
    vc = torch.full_like(vc, 1.0 + 2.0 ** -10, dtype=torch.float32).to(kv_dtype)
    vc[table[0, 0], 0] = 1.0e-8  # below half of fp16's smallest subnormal: fp16 rounds it to 0
    out = dense.paged_attention_f64(q, kc, vc, table, [1, 1], kv_cast=True)
    for b in range(2):
        v0 = vc[table[b, 0], 0].to(q_dtype).double().numpy()
        for h in range(4):
            assert np.array_equal(out[b, 0, h], v0[h // 2])
    uncast = dense.paged_attention_f64(q, kc, vc, table, [1, 1])
    assert not np.array_equal(out, uncast)


def test_dense_kv_cast_matches_sdpa_restatement():
    """The float64 oracle with the cast against the SDPA restatement (which casts the
    gathered rows itself, attention.py:240-241): a bf16 query over an fp32 cache."""
    q, _, _, kc, vc, table, lens = scenario(8, 2, 64, [130, 77, 300], scatter=True, seed=12)
    qb = q.to(torch.bfloat16)
    a = paged_sdpa.paged_attention_sdpa(qb, kc, vc, table, lens).double().numpy()
    b = dense.paged_attention_f64(qb, kc, vc, table, lens, kv_cast=True)
    assert np.abs(a - b).max() / np.abs(b).max() < 2e-2
    same = dense.paged_attention_f64(q, kc, vc, table, lens, kv_cast=True)
    assert np.array_equal(same, dense.paged_attention_f64(q, kc, vc, table, lens))
