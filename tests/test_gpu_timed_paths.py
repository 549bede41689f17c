"""GPU parity on exactly the paths bench.py times, at the benchmark configurations' full
sizes (BASELINE.json configs C2-C4; inputs from miniserve_amd.workloads):

  * C4 decodes through the cascade entry point (shared prefix read once per KV head):
    every row against the float64 oracle, and the one-pass decode of the same batch too;
  * C2 captures all 24 layers in one hipGraph: every layer's output against the oracle;
  * the bucketed graph runner at bucket 64 with C3's geometry and contexts.

Bars as in test_gpu_parity.py: bf16 max|out - ref| / max|ref| <= 2e-2.
"""
import numpy as np
import pytest
import torch

from miniserve_amd import PagedAttention, paged_attention
from miniserve_amd.graphs import DecodeLayer, GraphedDecodeRunner
from miniserve_amd.workloads import make_workload
from oracle import dense, paged_sdpa

pytestmark = pytest.mark.gpu

BF16_REL = 2e-2


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)


def rel_err(out: torch.Tensor, ref: np.ndarray) -> float:
    o = out.double().cpu().numpy()
    return float(np.abs(o - ref).max() / max(np.abs(ref).max(), 1e-30))


def test_c4_cascade_and_one_pass_every_row(device):
    """C4 (8 rows, 32k-131k tokens, the first 512 pages shared): the cascade decode the
    bench times and the one-pass decode, all 8 rows, against the float64 oracle; the two
    agree with each other within the same bar."""
    w = make_workload(4, device=device, values_device=device)
    B, bs = w.batch, w.block_size
    cap = w.table.shape[1] * bs
    kc, vc = w.k_caches[0], w.v_caches[0]
    q = w.query
    note(f"C4: B={B} ctx {min(w.lens)}..{max(w.lens)} prefix={w.shared_prefix_pages} pages")
    cascade = paged_attention(q, kc, vc, w.table, w.lens, max_context=cap,
                              prefix_pages=w.shared_prefix_pages)
    one_pass = paged_attention(q, kc, vc, w.table, w.lens, max_context=cap)
    torch.cuda.synchronize()
    kcpu, vcpu, qcpu = kc.cpu(), vc.cpu(), q.cpu()
    for b in range(B):
        ref = dense.paged_attention_f64(qcpu[b:b + 1], kcpu, vcpu, w.table[b:b + 1],
                                        [w.lens[b]])
        e_c = rel_err(cascade[b:b + 1], ref)
        e_o = rel_err(one_pass[b:b + 1], ref)
        note(f"C4 row {b} (ctx {w.lens[b]}): cascade {e_c:.3e}, one-pass {e_o:.3e}")
        assert e_c < BF16_REL and e_o < BF16_REL
    assert rel_err(cascade, one_pass.double().cpu().numpy()) < BF16_REL


def test_c2_all_layers_in_one_graph(device):
    """C2 as bench.py runs it: 24 layers' decodes (each over its own caches, one shared
    table) captured in one hipGraph with static table, lengths, workspace and outputs;
    after replays every layer's output matches the float64 oracle."""
    w = make_workload(2, device=device, values_device=device)
    dev = device
    B, H, KVH, D, bs = w.batch, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size
    table = w.table.to(device=dev, dtype=torch.int32).contiguous()
    lens = torch.tensor(w.lens, dtype=torch.int32, device=dev)
    cap = table.shape[1] * bs
    q = w.query.contiguous()
    from miniserve_amd import _native as nat
    ws = torch.zeros(nat.lib().msattn_workspace_bytes(B, 1, H, KVH, D, cap), dtype=torch.uint8,
                     device=dev)
    outs = [torch.empty_like(q) for _ in range(w.layers)]

    def step():
        for layer in range(w.layers):
            paged_attention(q, w.k_caches[layer], w.v_caches[layer], table, lens,
                            max_context=cap, workspace=ws, out=outs[layer])

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(dev).wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for o in outs:
        o.zero_()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    note(f"C2: {w.layers} layers replayed, B={B} ctx {min(w.lens)}..{max(w.lens)}")
    qcpu = q.cpu()
    worst = 0.0
    for layer in range(w.layers):
        ref = dense.paged_attention_f64(qcpu, w.k_caches[layer].cpu(), w.v_caches[layer].cpu(),
                                        w.table, w.lens)
        err = rel_err(outs[layer], ref)
        worst = max(worst, err)
        assert err < BF16_REL, f"layer {layer}: {err}"
    note(f"C2 worst layer max-rel {worst:.3e}")


def test_graphed_runner_bucket64_c3_geometry(device):
    """The bucketed runner at bucket 64 with C3's geometry (H32/KVH8/D128), tables and
    contexts: one decode step writes each row's new K/V at position ctx - 1 and attends
    over ctx tokens. Graph replay equals eager bit for bit; the caches equal the oracle's
    write_kv; the output is within the bar of the float64 oracle."""
    w = make_workload(3, device=device, values_device=device)
    B, H, KVH, D, bs = w.batch, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size
    assert B == 64
    width = w.table.shape[1]
    pa = PagedAttention(H, KVH, D, num_blocks=w.num_blocks, block_size=bs,
                        dtype=torch.bfloat16, kv_dtype=torch.bfloat16, device=device)
    kc, vc = w.k_caches[0], w.v_caches[0]
    kc_ref, vc_ref = kc.cpu(), vc.cpu()
    runner = GraphedDecodeRunner([DecodeLayer(pa, kc, vc)], table_width=width)
    g = torch.Generator().manual_seed(64)
    tables = [w.table[b, : (w.lens[b] + bs - 1) // bs].tolist() for b in range(B)]
    ctx = [L - 1 for L in w.lens]  # tokens already cached; the step adds one each
    q = torch.randn(1, B, 1, H, D, generator=g).to(torch.bfloat16)
    k = torch.randn(1, B, 1, KVH, D, generator=g).to(torch.bfloat16)
    v = torch.randn(1, B, 1, KVH, D, generator=g).to(torch.bfloat16)
    note(f"runner bucket 64, C3 geometry: ctx {min(w.lens)}..{max(w.lens)}")
    out_graph = runner.decode(q.to(device), k.to(device), v.to(device), tables, ctx)
    assert runner.memory_report()["buckets_captured"] == [64]
    out_eager = runner.decode(q.to(device), k.to(device), v.to(device), tables, ctx,
                              use_graph=False)
    assert torch.equal(out_graph, out_eager)
    paged_sdpa.write_kv(kc_ref, vc_ref, k[0], v[0], w.table, start=ctx)
    assert torch.equal(kc.cpu(), kc_ref) and torch.equal(vc.cpu(), vc_ref)
    ref = dense.paged_attention_f64(q[0], kc_ref, vc_ref, w.table, w.lens)
    err = rel_err(out_graph[0], ref)
    note(f"runner bucket 64 max-rel {err:.3e}")
    assert err < BF16_REL
