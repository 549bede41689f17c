"""Bucketed hipGraph decode (miniserve_amd.graphs), restating the semantics of the
reference's tests/test_cuda_graph.py without HF weights: the step is every layer's
write_kv + paged attention, on random q/k/v."""
import numpy as np
import pytest
import torch

from miniserve_amd import PagedAttention
from miniserve_amd.graphs import DecodeLayer, GraphedDecodeRunner
from oracle import dense, paged_sdpa

pytestmark = pytest.mark.gpu

H, KVH, D, BS, WIDTH, LAYERS = 14, 2, 64, 16, 16, 2
POOL = 2048


def note(msg):
    print(f"[case] {msg}", flush=True)


@pytest.fixture(scope="module")
def graphed(device):
    g = torch.Generator().manual_seed(0)
    layers = []
    for _ in range(LAYERS):
        pa = PagedAttention(H, KVH, D, num_blocks=POOL, block_size=BS, dtype=torch.bfloat16,
                            kv_dtype=torch.bfloat16, device=device)
        kc = torch.randn(POOL, BS, KVH, D, generator=g).to(torch.bfloat16).to(device)
        vc = torch.randn(POOL, BS, KVH, D, generator=g).to(torch.bfloat16).to(device)
        layers.append(DecodeLayer(pa, kc, vc))
    return GraphedDecodeRunner(layers, table_width=WIDTH)


def make_batch(B, seed, prompt_len=None):
    """B rows: distinct pages per row (disjoint across calls by seed), ctx tokens cached."""
    g = torch.Generator().manual_seed(seed)
    pages = torch.randperm(POOL, generator=g)[: B * 4].view(B, 4)
    ctx = [int(x) for x in torch.randint(1, 4 * BS - 1, (B,), generator=g)] if prompt_len is None \
        else [prompt_len] * B
    q = torch.randn(LAYERS, B, 1, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(LAYERS, B, 1, KVH, D, generator=g).to(torch.bfloat16)
    v = torch.randn(LAYERS, B, 1, KVH, D, generator=g).to(torch.bfloat16)
    return q, k, v, [row.tolist() for row in pages], ctx


def run(graphed, batch, device, use_graph):
    q, k, v, tables, ctx = batch
    return graphed.decode(q.to(device), k.to(device), v.to(device), tables, ctx,
                          use_graph=use_graph)


def test_bucket_parity(graphed, device):
    """tests/test_cuda_graph.py:39-45: graph equals eager (here bit-exactly)."""
    for B in (1, 2):
        note(f"bucket parity B={B}")
        batch = make_batch(B, seed=B)
        eager = run(graphed, batch, device, False)
        graph = run(graphed, batch, device, True)
        assert torch.equal(eager, graph), f"bucket {B}"


def test_double_buffer_alternation(graphed, device):
    """tests/test_cuda_graph.py:48-55."""
    batch = make_batch(2, seed=7)
    start = len(graphed.replay_log)
    for _ in range(4):
        run(graphed, batch, device, True)
    assert [i for _, i in graphed.replay_log[start:]] == [0, 1, 0, 1]


@pytest.mark.parametrize("B", [3, 5, 7, 12, 20, 24])
def test_interpolation_matches_eager(graphed, device, B):
    """tests/test_cuda_graph.py:58-65: off-bucket batches replay the next bucket."""
    note(f"interpolation B={B}")
    batch = make_batch(B, seed=B * 3)
    eager = run(graphed, batch, device, False)
    graph = run(graphed, batch, device, True)
    assert graph.shape == (LAYERS, B, 1, H, D)
    assert torch.equal(eager, graph)


def test_ragged_real_pad_mix_bucket16(graphed, device):
    """tests/test_cuda_graph.py:68-80: 5 real rows + 11 pad rows (table -1, ctx 0) at
    bucket 16 match eager on the padded batch and eager on the 5 rows; pad rows touch
    no cache page and return zeros."""
    q, k, v, tables, ctx = make_batch(5, seed=42)
    pad = 11
    zq = torch.zeros(LAYERS, pad, 1, H, D, dtype=torch.bfloat16)
    zk = torch.zeros(LAYERS, pad, 1, KVH, D, dtype=torch.bfloat16)
    padded = (torch.cat([q, zq], 1), torch.cat([k, zk], 1), torch.cat([v, zk], 1),
              tables + [[-1]] * pad, ctx + [0] * pad)
    # pad rows: every table entry is a hole, so their write and their key are skipped
    before = [layer.k_cache.clone() for layer in graphed.layers]
    graph = run(graphed, padded, device, True)
    eager_padded = run(graphed, padded, device, False)
    eager_small = run(graphed, (q, k, v, tables, ctx), device, False)
    assert torch.equal(graph, eager_padded)
    assert torch.equal(graph[:, :5], eager_small)
    assert not graph[:, 5:].any()
    real_pages = {p for row in tables for p in row}
    for layer, old in zip(graphed.layers, before):
        changed = (layer.k_cache != old).flatten(1).any(1).nonzero().flatten().tolist()
        assert set(changed) <= real_pages


def test_graph_pool_persistence_memory(graphed):
    """tests/test_cuda_graph.py:83-86: statics are shared by all buckets' graphs."""
    report = graphed.memory_report()
    assert report["total_static_bytes"] > 0 and report["shared_pool"]
    assert len(report["buckets_captured"]) >= 3
    assert report["total_over_max"] < 2.0


def test_decode_steps_match_oracle(device):
    """Several decode steps through the graph (write_kv inside the graph each step):
    the caches hold exactly what the oracle's write_kv puts there, and every step's
    output matches the float64 oracle over the updated caches."""
    g = torch.Generator().manual_seed(11)
    pool, width, B = 64, 8, 3
    pa = PagedAttention(H, KVH, D, num_blocks=pool, block_size=BS, dtype=torch.bfloat16,
                        kv_dtype=torch.bfloat16, device=device)
    kc = torch.randn(pool, BS, KVH, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(pool, BS, KVH, D, generator=g).to(torch.bfloat16)
    runner = GraphedDecodeRunner([DecodeLayer(pa, kc.to(device), vc.to(device))],
                                 table_width=width, buckets=(1, 2, 4))
    tables = torch.randperm(pool, generator=g)[: B * width].view(B, width)
    ctx = [5, 30, 100]
    kc_ref, vc_ref = kc.clone(), vc.clone()
    for step in range(6):
        note(f"decode step {step}")
        q = torch.randn(1, B, 1, H, D, generator=g).to(torch.bfloat16)
        k = torch.randn(1, B, 1, KVH, D, generator=g).to(torch.bfloat16)
        v = torch.randn(1, B, 1, KVH, D, generator=g).to(torch.bfloat16)
        out = runner.decode(q.to(device), k.to(device), v.to(device),
                            [r.tolist() for r in tables], ctx)
        paged_sdpa.write_kv(kc_ref, vc_ref, k[0], v[0], tables, start=ctx)
        lens = [c + 1 for c in ctx]
        ref = dense.paged_attention_f64(q[0], kc_ref, vc_ref, tables, lens)
        err = np.abs(out[0].double().cpu().numpy() - ref).max() / np.abs(ref).max()
        assert err < 2e-2
        assert torch.equal(runner.layers[0].k_cache.cpu(), kc_ref)
        assert torch.equal(runner.layers[0].v_cache.cpu(), vc_ref)
        ctx = [c + 1 for c in ctx]


def test_capture_of_new_bucket_leaves_freed_pages_alone(device):
    """Capturing a bucket warms the step up on its input sets. After a decode, a set still
    holds that step's rows; if one of their pages has since been freed and reused by
    another sequence, the warm-up must not write the old k/v into it."""
    g = torch.Generator().manual_seed(5)
    pool, width = 64, 4
    pa = PagedAttention(H, KVH, D, num_blocks=pool, block_size=BS, dtype=torch.bfloat16,
                        kv_dtype=torch.bfloat16, device=device)
    kc = torch.randn(pool, BS, KVH, D, generator=g).to(torch.bfloat16).to(device)
    vc = torch.randn(pool, BS, KVH, D, generator=g).to(torch.bfloat16).to(device)
    runner = GraphedDecodeRunner([DecodeLayer(pa, kc, vc)], table_width=width, buckets=(1, 2, 4))
    tables = torch.randperm(pool, generator=g)[: 2 * width].view(2, width)
    ctx = [10, 20]
    for _ in range(2):  # both input sets now hold these rows (bucket 2 captured)
        q = torch.randn(1, 2, 1, H, D, generator=g).to(torch.bfloat16).to(device)
        k = torch.randn(1, 2, 1, KVH, D, generator=g).to(torch.bfloat16).to(device)
        v = torch.randn(1, 2, 1, KVH, D, generator=g).to(torch.bfloat16).to(device)
        runner.decode(q, k, v, [r.tolist() for r in tables], ctx)
    # The pages the last step wrote into are freed and handed to another sequence,
    # which fills them with its own keys and values.
    freed = [int(tables[b, ctx[b] // BS]) for b in range(2)]
    for p in freed:
        kc[p] = 7.0
        vc[p] = -7.0
    k_before, v_before = kc.clone(), vc.clone()
    note("capture bucket 4 after the pages were reused")
    other = torch.randperm(pool, generator=g)[: 3 * width].view(3, width)
    other = [[p for p in row.tolist() if p not in freed][:width] for row in other]
    q = torch.zeros(1, 3, 1, H, D, dtype=torch.bfloat16, device=device)
    k = torch.zeros(1, 3, 1, KVH, D, dtype=torch.bfloat16, device=device)
    runner.decode(q, k, k, other, [0, 0, 0])  # bucket 4: a new capture
    torch.cuda.synchronize()
    for p in freed:
        assert torch.equal(kc[p], k_before[p]) and torch.equal(vc[p], v_before[p]), \
            f"page {p} was overwritten by the capture's warm-up"
