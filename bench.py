"""Paged-decode benchmark on one MI355X (gfx950).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--no-cpu-baseline]
                    [--kv-fp8] [--no-cascade] [--prefill] [--graph-steps G]

A step is one layer's paged-attention decode over the whole batch (split-K
partials kernel + merge kernel; one launch where the partition kernel merges
in-kernel), replayed from a captured hipGraph with the
block tables, context lengths, workspace and output in static device buffers.
The default workload is BASELINE.json's headline config C3 (Llama-3-8B
attention geometry, bf16, batch 64, context log-uniform in [1024, 8192]); C2
captures all 24 layers in one graph and reports per-layer figures. One graph
holds G consecutive steps (G the largest divisor of K up to 10, or --graph-steps),
so the host's per-replay launch cost is spread as a model's decode graph spreads
it over its layers; K / G replays time exactly K steps. The line also reports the
step time with one step per replay.

Printed: one JSON line with the throughput (algorithmic KV-read GB/s), the
per-layer latency, the roofline of the dominant kernel (HIP events around the
partials kernel on the stream it runs on) and the reference's CPU path timed
on this host's cores (the oracle's restatement of attention.py, bounded
sample).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = ("paged-decode µs/layer; KV-read HBM GB/s as % of peak (bs64, ctx<=8k, 1 GPU)")
HBM_PEAK_GBS = 8000.0
PROFILES = ROOT / "profiles"
MIN_WARMUP_REPLAYS = 5


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", type=int, default=3, choices=[1, 2, 3, 4, 5])
    ap.add_argument("--graph-steps", type=int, default=0,
                    help="steps captured per graph (0: largest divisor of --steps up to 10)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--kv-dtype", choices=["same", "fp8", "fp32"], default="same",
                    help="store the caches as fp8 e4m3 (half the KV bytes) or fp32 (twice; the "
                         "reference runner's cache type, model_runner.py:122-123) instead of the "
                         "config dtype; the query stays in the config dtype and the cache is "
                         "cast to it as it is read. Bytes follow the cache's element size.")
    ap.add_argument("--kv-fp8", action="store_true", help="same as --kv-dtype fp8")
    ap.add_argument("--q-dtype", choices=["same", "fp32"], default="same",
                    help="the query (and output) in fp32 instead of the config dtype; with "
                         "--kv-dtype fp32 this is the reference runner's default pair "
                         "(model_runner.py:122-123), on the fp32 MFMA decode kernels")
    ap.add_argument("--no-cascade", action="store_true",
                    help="decode a shared-prefix workload (config 4) in one pass per sequence "
                         "instead of the cascade entry point")
    ap.add_argument("--prefill", action="store_true",
                    help="C5's chunked-prefill part (2 x 512 query tokens onto 4096 cached): "
                         "MFMA-bound, reported in TFLOP/s; with --q-dtype fp32 --kv-dtype fp32 "
                         "the reference runner's types, priced against the fp32 matrix peak")
    ap.add_argument("--runner", action="store_true",
                    help="time GraphedDecodeRunner.decode (one bucketed hipGraph decode step "
                         "per call, write_kv included, host-side input staging included) on "
                         "the config's decode shape (C2: bucket 32, 24 layers; C3: bucket 64)")
    ap.add_argument("--eager", action="store_true",
                    help="time PagedAttention.write_kv + forward called per layer as the "
                         "reference runner calls them (model_runner.py:72-76: transposed q/k/v "
                         "views, an int64 device table, Python-list starts and lengths), "
                         "against the kernel's own time")
    ap.add_argument("--decode-sweep", action="store_true",
                    help="time decodes of the shapes around the stream-K threshold (table "
                         "capacities of 49k-261k tiles), one line per shape with the route "
                         "the library took; compare builds made with --define overrides of "
                         "MSATTN_STREAMK_MIN_TILES*")
    ap.add_argument("--prefill-sweep", action="store_true",
                    help="time chunked prefills of 16-224 tasks (sequence x KV head x 128-row "
                         "block) on the prefill kernel, one line per shape; compare builds "
                         "made with --define MSATTN_PF_STREAMK=0 / 1")
    ap.add_argument("--warm-ms", type=float, default=200.0,
                    help="untimed graph replays before each timed loop last at least this "
                         "long (and at least --warmup steps), so timing starts at steady "
                         "clocks")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="target CPU time of the cpu_baseline sample")
    ap.add_argument("--stream-probe", action="store_true",
                    help="instead of the decode bench, time torch's out = in * 1 over 1 GiB "
                         "fp32 (the reference dispatch for scaling rocprofv3 "
                         "FETCH_SIZE/WRITE_SIZE) and the plain streaming-read kernel")
    args = ap.parse_args()
    if args.kv_fp8:
        args.kv_dtype = "fp8"
    return args


def stream_probe(steps: int):
    """1 GiB fp32 read + 1 GiB written per dispatch by torch's elementwise multiply."""
    import torch

    dev = torch.device("cuda:0")
    n = (1 << 30) // 4
    src = torch.ones(n, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        torch.mul(src, 1.0, out=dst)
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / steps
    gbs = 2 * (1 << 30) / (ms * 1e-3) / 1e9
    print(json.dumps({"metric": "streaming kernel HBM bandwidth (read + write)",
                      "value": round(gbs, 1), "unit": "GB/s", "ms_per_dispatch": round(ms, 4),
                      "bytes_read_per_dispatch": 1 << 30, "bytes_written_per_dispatch": 1 << 30,
                      "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}), flush=True)
    rd = stream_read_gbs(dev, max(steps, 5))
    print(json.dumps({"metric": "streaming read kernel HBM bandwidth (msattn_probe_stream_read)",
                      "value": round(rd, 1), "unit": "GB/s", "bytes_read_per_dispatch": 2 << 30,
                      "frac_of_hbm_peak": round(rd / HBM_PEAK_GBS, 4)}), flush=True)


def stream_read_gbs(dev, launches: int = 20) -> float:
    """GB/s of msattn_probe_stream_read (a plain 16-byte-load read kernel) over 2 GiB,
    timed with HIP events on the stream it is launched on: the read rate a plain kernel
    reaches on this device, reported beside the decode kernel's."""
    import torch

    from miniserve_amd import _native as nat

    nbytes = 2 << 30
    buf = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    sink = torch.empty((nbytes + 65535) // 65536, dtype=torch.int32, device=dev)
    lib, stream = nat.lib(), nat.stream_handle(dev)

    def launch():
        nat.check("msattn_probe_stream_read",
                  lib.msattn_probe_stream_read(buf.data_ptr(), nbytes, sink.data_ptr(), stream))

    for _ in range(3):
        launch()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(launches):
        launch()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / launches
    del buf, sink
    torch.cuda.empty_cache()
    return nbytes / (ms * 1e-3) / 1e9


def warm(replay, warm_ms: float, min_replays: int) -> None:
    """Replay a captured graph at least `min_replays` times and for at least `warm_ms` of
    wall time, then synchronise. Under sustained load the MFMA-bound prefill kernel runs
    ~10 % faster after the first ~20 ms (its time falls from ~91 to ~81 us per launch over
    the first ~150 launches of a run, while a decode kernel's stays flat): timing starts
    in that steady state."""
    import torch

    t0 = time.perf_counter()
    done = 0
    while done < min_replays or (time.perf_counter() - t0) * 1e3 < warm_ms:
        for _ in range(8):
            replay()
        done += 8
        torch.cuda.synchronize()


def warmup_replays(warmup: int, steps_per_graph: int) -> int:
    """Untimed replays of a captured graph before the timed ones: the --warmup steps'
    worth, and never fewer than MIN_WARMUP_REPLAYS (the first replays of a new graph run
    slower than the steady state: a 20-step run after 5 warm-up steps, one replay, came
    out 3.5 % above a 200-step run)."""
    return max(MIN_WARMUP_REPLAYS, -(-warmup // steps_per_graph))


def graph_steps(args) -> int:
    """Steps captured per graph: --graph-steps, else the largest divisor of K up to 10."""
    if args.graph_steps > 0:
        if args.steps % args.graph_steps:
            raise SystemExit("--steps must be a multiple of --graph-steps")
        return args.graph_steps
    return max(g for g in range(1, 11) if args.steps % g == 0)


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build is a one-GPU kernel library: bench.py runs on "
                                   "exactly one GPU (--gpus 1); multi-GPU figures are not "
                                   "produced", "n_gpus": args.gpus}))
        sys.exit(2)
    if args.stream_probe:
        stream_probe(args.steps)
        return
    if args.prefill:
        prefill_bench(args)
        return
    if args.runner:
        runner_bench(args)
        return
    if args.decode_sweep:
        decode_sweep()
        return
    if args.prefill_sweep:
        prefill_sweep(args)
        return
    if args.eager:
        eager_bench(args)
        return

    import torch

    from miniserve_amd import _native as nat
    from miniserve_amd.attention import kernel_route, paged_attention
    from miniserve_amd.workloads import make_workload

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a ROCm GPU")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = nat.lib()

    t0 = time.time()
    w = make_workload(args.config, device=dev, values_device=dev, part="decode")
    print(f"[bench] built {w.name}: B={w.batch} H={w.num_heads} KVH={w.num_kv_heads} "
          f"D={w.head_dim} layers={w.layers} pool={w.num_blocks} pages, "
          f"ctx {min(w.lens)}..{max(w.lens)} (sum {sum(w.lens)}) in {time.time() - t0:.1f}s",
          file=sys.stderr, flush=True)
    kv_torch = {"fp8": torch.float8_e4m3fn, "fp32": torch.float32}.get(args.kv_dtype)
    if kv_torch is not None:  # the same values stored as kv_torch; bytes follow the dtype
        w.k_caches = [c.to(kv_torch) for c in w.k_caches]
        w.v_caches = [c.to(kv_torch) for c in w.v_caches]
    if args.q_dtype == "fp32":  # the query's values in fp32; q/out bytes follow
        w.query = w.query.float()
        w.dtype = torch.float32

    B, H, KVH, D, bs = w.batch, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size
    table = w.table.to(device=dev, dtype=torch.int32).contiguous()
    lens = torch.tensor(w.lens, dtype=torch.int32, device=dev)
    W = table.shape[1]
    max_ctx = W * bs  # capture-safe bound: the table capacity
    q = w.query.to(dev).contiguous()
    ws_bytes = lib.msattn_workspace_bytes(B, 1, H, KVH, D, max_ctx)
    # Shared-prefix workloads decode through the cascade entry point (shared pages read
    # once per KV head for the batch) unless --no-cascade.
    cascade = w.shared_prefix_pages if not args.no_cascade else 0
    if cascade:
        ws_bytes = lib.msattn_prefix_workspace_bytes(B, H, KVH, D, bs, max_ctx, cascade)
    part_tokens = lib.msattn_partition_tokens(B, 1, H, KVH, D, max_ctx)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)  # merge tickets start at zero
    outs = [torch.empty_like(q) for _ in range(w.layers)]
    qcode, kvcode = nat.dtype_code(w.dtype), nat.dtype_code(w.k_caches[0].dtype)

    def step():
        for layer in range(w.layers):
            paged_attention(q, w.k_caches[layer], w.v_caches[layer], table, lens,
                            max_context=max_ctx, workspace=ws, out=outs[layer],
                            prefix_pages=cascade or None)

    # eager warm-up on a side stream, then capture the step into a hipGraph
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    gsteps = graph_steps(args)

    def timed(n_in_graph):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(n_in_graph):
                step()
        torch.cuda.synchronize()
        warm(graph.replay, args.warm_ms, warmup_replays(args.warmup, n_in_graph))
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps // n_in_graph):
            graph.replay()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / args.steps

    ms_single = timed(1)  # one step per replay: each replay pays the graph launch
    ms_per_step = timed(gsteps) if gsteps > 1 else ms_single
    print(f"[bench] graph replay: {ms_per_step * 1e3:.2f} us/step over {args.steps} steps "
          f"({gsteps} per graph; {ms_single * 1e3:.2f} us with one per graph)",
          file=sys.stderr, flush=True)

    # Dominant kernel: the partials kernel, bracketed by HIP events on the stream it
    # is launched on (torch's current stream), over its own timed loop. A decode that
    # merges in-kernel (workspace kind 2 after the step) is one launch: the whole
    # msattn_paged_attention call is timed instead, and the merge column is 0.
    stream = nat.stream_handle(dev)
    kc, vc = w.k_caches[0], w.v_caches[0]
    fused = not cascade and int(ws[:4].view(torch.int32).item()) == 2
    n_k = max(10, min(args.steps, 200))
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
            torch.cuda.Event(enable_timing=True)) for _ in range(n_k)]
    for i in range(n_k + 5):
        e = evs[i - 5] if i >= 5 else None
        if e:
            e[0].record()
        if fused:
            st = lib.msattn_paged_attention(
                q.data_ptr(), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
                kc.stride(2), table.data_ptr(), lens.data_ptr(), outs[0].data_ptr(),
                ws.data_ptr(), ws_bytes, B, 1, H, KVH, D, bs, w.num_blocks, W, max_ctx, 1, 0,
                w.scale, qcode, kvcode, stream)
            nat.check("fused decode", st)
            if e:
                e[1].record()
                e[2].record()
            continue
        st = lib.msattn_paged_attention_partials(
            q.data_ptr(), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2),
            table.data_ptr(), lens.data_ptr(), ws.data_ptr(), ws_bytes, B, 1, H, KVH, D, bs,
            w.num_blocks, W, max_ctx, 1, 0, w.scale, qcode, kvcode, stream)
        nat.check("partials", st)
        if e:
            e[1].record()
        st = lib.msattn_merge_partials(ws.data_ptr(), ws_bytes, lens.data_ptr(),
                                       outs[0].data_ptr(), B, 1, H, KVH, D, max_ctx, qcode, stream)
        nat.check("merge", st)
        if e:
            e[2].record()
    torch.cuda.synchronize()
    # Which partials kernel ran: the workspace header's first word is the layout kind
    # (1 = stream-K); otherwise the partition kernel, on MFMA with head_dim 64 or 128 for a
    # bf16/fp16 query over its own type, fp8 or fp32 and for an fp32 query over any cache,
    # else the generic kernel.
    hdr = ws[:64].view(torch.int32).cpu()
    kind = int(hdr[0])
    # The partition kernels record their launch's partition length and waves per
    # workgroup in header words 8 and 9 (the wide shape takes longer partitions than
    # msattn_partition_tokens reports), and in word 14 the workgroups per CU the MFMA
    # kernel was built to keep resident (0: the compiler's own occupancy).
    if kind in (0, 2) and int(hdr[8]) > 0:
        part_tokens, part_waves = int(hdr[8]), int(hdr[9])
        part_residency = int(hdr[14])
    else:
        part_waves = part_residency = None
    # The kernel the library routes this call to (msattn_paged_attention_route); the
    # header's kind after the call must agree with it.
    route = kernel_route(q, w.k_caches[0], table, max_context=max_ctx, out=outs[0])
    kernel_name = {
        "partition-fused": "msattn::decode_mfma_kernel (partition split-K, merged in-kernel)",
        "stream-K": "msattn::decode_streamk_kernel (stream-K split-K partials)",
        "partition": "msattn::decode_mfma_kernel (partition split-K partials)",
        "generic": "msattn::split_kernel (generic partition split-K partials)",
    }[route]
    if cascade:  # the suffix pass: stream-K or the partition kernel, then the merge
        kernel_name = ("msattn::decode_streamk_kernel (stream-K split-K partials)" if kind == 1
                       else "msattn::decode_mfma_kernel (partition split-K partials)")
    elif {"partition-fused": 2, "stream-K": 1}.get(route, 0) != kind:
        raise SystemExit(f"route {route} but workspace kind {kind}")
    split_ms = sorted(a.elapsed_time(b) for a, b, _ in evs)
    merge_ms = sorted(b.elapsed_time(c) for _, b, c in evs)
    split_avg = sum(split_ms) / len(split_ms)
    merge_avg = 0.0 if fused else sum(merge_ms) / len(merge_ms)

    per_layer_bytes = w.algorithmic_bytes(unique=True)
    layer_us = ms_per_step * 1e3 / w.layers
    value_gbs = per_layer_bytes * w.layers / (ms_per_step * 1e-3) / 1e9
    achieved = per_layer_bytes / (split_avg * 1e-3) / 1e9

    read_ceiling = stream_read_gbs(dev)

    traffic, traffic_note = traffic_record(w.name, args)
    lib_sha = library_sha256()

    result = {
        "metric": METRIC,
        "value": round(value_gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_layer": round(layer_us, 2),
        "frac_of_hbm_peak": round(value_gbs / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {torch.bfloat16: "bf16", torch.float32: "f32"}[w.dtype],
        "data": "synthetic: seeded N(0,1) q/K/V, seeded scattered block tables (16-token pages)",
        "config": {
            "workload": f"{w.name}: paged decode, H{H}/KVH{KVH}/D{D}, batch {B}, "
                        f"ctx {min(w.lens)}..{max(w.lens)}, {w.layers} layer(s), hipGraph replay",
            "batch": B, "q_len": 1, "num_heads": H, "num_kv_heads": KVH, "head_dim": D,
            "block_size": bs, "layers": w.layers, "context_tokens": sum(w.lens),
            "pool_pages": w.num_blocks, "partition_tokens": part_tokens,
            "partition_waves": part_waves, "partition_wg_per_cu": part_residency,
            "algorithmic_bytes_per_layer": per_layer_bytes,
            "shared_prefix_pages": w.shared_prefix_pages, "cascade": bool(cascade),
            "kv_dtype": str(w.k_caches[0].dtype).replace("torch.", ""),
            "steps_per_graph": gsteps, "us_per_step_one_per_graph": round(ms_single * 1e3, 2),
        },
        "roofline": {
            "kernel": kernel_name,
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": traffic_note,
            "library_sha256": lib_sha,
            "kernel_avg_us": round(split_avg * 1e3, 2),
            "kernel_median_us": round(split_ms[len(split_ms) // 2] * 1e3, 2),
            "merge_avg_us": round(merge_avg * 1e3, 2),
            "stream_read_gbs": round(read_ceiling, 1),
            "frac_of_stream_read": round(achieved / read_ceiling, 4),
        },
        "cpu_baseline": None,
        "reference_gpu": None,
    }
    ref = reference_forward_us(w, table, lens, 1)
    ref["speedup"] = round(ref["us"] / layer_us, 1)
    result["reference_gpu"] = ref
    if not args.no_cpu_baseline and args.kv_dtype == "same" and args.q_dtype == "same":
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds)
    print(json.dumps(result), flush=True)


def prefill_bench(args):
    """C5 prefill: one forward over 2 x 512 query rows, captured in a hipGraph; the kernel
    itself timed per launch with HIP events on its stream; the reference's CPU path on a
    bounded sample of the same call."""
    import torch

    from miniserve_amd import _native as nat
    from miniserve_amd.attention import kernel_route, paged_attention
    from miniserve_amd.workloads import make_workload

    dev = torch.device("cuda:0")
    w = make_workload(5, device=dev, values_device=dev, part="prefill")
    if args.q_dtype == "fp32":
        w.query = w.query.float()
    kv_torch = {"fp8": torch.float8_e4m3fn, "fp32": torch.float32}.get(args.kv_dtype)
    if kv_torch is not None:
        w.k_caches = [c.to(kv_torch) for c in w.k_caches]
        w.v_caches = [c.to(kv_torch) for c in w.v_caches]
    B, T, H, D = w.query.shape
    KVH = w.num_kv_heads
    table = w.table.to(device=dev, dtype=torch.int32).contiguous()
    lens = torch.tensor(w.lens, dtype=torch.int32, device=dev)
    cap = table.shape[1] * w.block_size
    out = torch.empty_like(w.query)
    lib = nat.lib()
    ws_bytes = lib.msattn_workspace_bytes(B, T, H, KVH, D, cap)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    kc, vc = w.k_caches[0], w.v_caches[0]
    route = kernel_route(w.query, kc, table, max_context=cap, out=out)

    def step():
        paged_attention(w.query, kc, vc, table, lens, max_context=cap, workspace=ws, out=out)

    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream(dev).wait_stream(side)
    gsteps = graph_steps(args)

    def timed(n_in_graph):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(n_in_graph):
                step()
        warm(graph.replay, args.warm_ms, warmup_replays(args.warmup, n_in_graph))
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(args.steps // n_in_graph):
            graph.replay()
        stop.record()
        torch.cuda.synchronize()
        return start.elapsed_time(stop) / args.steps

    ms_single = timed(1)
    ms = timed(gsteps) if gsteps > 1 else ms_single

    # The kernel per launch: msattn_paged_attention is one launch on this route (the
    # prefill kernel, or the partition kernel merging in-kernel), bracketed by HIP events
    # on the stream it is launched on, back to back as in the graph.
    stream = nat.stream_handle(dev)
    qcode, kvcode = nat.dtype_code(w.query.dtype), nat.dtype_code(kc.dtype)
    n_k = max(10, min(args.steps, 200))
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(n_k)]
    for i in range(n_k + 5):
        e = evs[i - 5] if i >= 5 else None
        if e:
            e[0].record()
        st = lib.msattn_paged_attention(
            w.query.data_ptr(), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
            kc.stride(2), table.data_ptr(), lens.data_ptr(), out.data_ptr(), ws.data_ptr(),
            ws_bytes, B, T, H, KVH, D, w.block_size, w.num_blocks, table.shape[1], cap, 1, 0,
            w.scale, qcode, kvcode, stream)
        nat.check("prefill", st)
        if e:
            e[1].record()
    torch.cuda.synchronize()
    k_ms = sorted(a.elapsed_time(b) for a, b in evs)
    k_avg = sum(k_ms) / len(k_ms)

    # causal: row i of a sequence with context L sees L - T + i + 1 keys
    flops = sum(4 * D * H * (L - T + i + 1) for L in w.lens for i in range(T) if L - T + i + 1 > 0)
    tflops = flops / (ms * 1e-3) / 1e12
    k_tflops = flops / (k_avg * 1e-3) / 1e12
    fp32 = w.query.dtype == torch.float32
    # MI355X dense matrix peaks: bf16 2.5 PFLOP/s, fp32 157.3 TFLOP/s.
    peak = 157.3 if fp32 else 2500.0
    traffic, traffic_note = traffic_record(w.name, args)
    kernel = {"prefill": "msattn::prefill_mfma_kernel",
              "prefill stream-K": "msattn::prefill_mfma_kernel (stream-K schedule)",
              "partition-fused": "msattn::decode_mfma_kernel (16-row tiles, merged in-kernel)"
              }.get(route, route)
    result = {
        "metric": "C5 chunked-prefill attention (2 x 512 tokens onto 4096 cached)",
        "value": round(tflops, 1), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None,
        "dtype": "f32" if fp32 else "bf16",
        "data": "synthetic: seeded N(0,1) q/K/V, scattered block tables",
        "config": {"workload": "C5-prefill: causal chunked prefill, H28/KVH4/D128, 2 sequences "
                               "x 512 new tokens onto 4096 cached, hipGraph replay",
                   "batch": B, "q_len": T, "num_heads": H,
                   "num_kv_heads": KVH, "head_dim": D, "flops": flops,
                   "kv_dtype": str(kc.dtype).replace("torch.", ""), "route": route,
                   "steps_per_graph": gsteps,
                   "us_per_step_one_per_graph": round(ms_single * 1e3, 2)},
        "roofline": {"kernel": kernel, "bound": "mfma",
                     "achieved": round(k_tflops, 1), "peak": peak, "unit": "TFLOP/s",
                     "frac": round(k_tflops / peak, 4), "traffic": traffic,
                     "traffic_source": traffic_note,
                     "kernel_avg_us": round(k_avg * 1e3, 2),
                     "kernel_median_us": round(k_ms[len(k_ms) // 2] * 1e3, 2),
                     "kernel_min_us": round(k_ms[0] * 1e3, 2),
                     "library_sha256": library_sha256()},
        "cpu_baseline": None,
        "reference_gpu": reference_forward_us(w, table, lens, T),
    }
    if not args.no_cpu_baseline and args.kv_dtype == "same" and args.q_dtype == "same":
        result["cpu_baseline"] = cpu_baseline_prefill(w, args.cpu_seconds)
    print(json.dumps(result), flush=True)


def reference_forward_us(w, table, lens, T) -> dict:
    """The reference's own forward for this call, restated in torch on the same GPU and
    timed with events: gather every row's K/V up to the longest context through the block
    table, expand the KV heads to the query heads, causal mask over the context, and
    scaled_dot_product_attention in the query dtype (miniserve/attention.py:155-171,
    :235-250), over the first layer's caches. Eager, as the reference runs it."""
    import torch
    import torch.nn.functional as F

    dev = w.query.device
    B, _, H, D = w.query.shape
    KVH = w.num_kv_heads
    max_l = max(w.lens)
    tl = table.long()
    pos = torch.arange(max_l, device=dev)
    L = lens.long()
    q_pos = L[:, None] - T + torch.arange(T, device=dev)[None, :]
    mask = ((pos[None, None, :] <= q_pos[:, :, None]) & (pos[None, None, :] < L[:, None, None]))[:, None]
    kc, vc = w.k_caches[0], w.v_caches[0]

    def forward():
        pages = tl[:, pos // w.block_size]
        slots = (pos % w.block_size)[None, :]
        k = kc[pages, slots].to(w.query.dtype).repeat_interleave(H // KVH, dim=2).transpose(1, 2)
        v = vc[pages, slots].to(w.query.dtype).repeat_interleave(H // KVH, dim=2).transpose(1, 2)
        return F.scaled_dot_product_attention(w.query.transpose(1, 2), k, v, attn_mask=mask)

    for _ in range(3):
        forward()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    n = 10
    for _ in range(n):
        forward()
    stop.record()
    torch.cuda.synchronize()
    return {"us": round(start.elapsed_time(stop) / n * 1e3, 1),
            "what": "the reference's forward (block-table gather, GQA expand, masked SDPA) "
                    "restated in torch, eager, on this GPU"}


def traffic_record(workload: str, args):
    """HBM bytes per launch of the dominant kernel from rocprofv3 counter runs (FETCH_SIZE,
    WRITE_SIZE) recorded in profiles/traffic_<workload>[-<kv dtype>][-q<q dtype>].json,
    reported only when the record was taken on the library this run loaded (same sha256);
    else None, with the reason."""
    tname = (f"traffic_{workload}{'' if args.kv_dtype == 'same' else '-' + args.kv_dtype}"
             f"{'' if args.q_dtype == 'same' else '-q' + args.q_dtype}.json")
    tfile = PROFILES / tname
    lib_sha = library_sha256()
    if not tfile.exists():
        return None, f"no profiles/{tname} for this workload"
    try:
        rec = json.loads(tfile.read_text())
    except (ValueError, OSError):
        rec = {}
    if rec.get("library_sha256") == lib_sha:
        return (rec.get("hbm_bytes_per_launch"),
                f"profiles/{tname}: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE on this library")
    return None, (f"profiles/{tname} was measured on library {rec.get('library_sha256')}, "
                  f"not on this one ({lib_sha})")


def library_sha256() -> str:
    """First 16 hex digits of the sha256 of the libmsattn.so this run loads."""
    import hashlib

    from miniserve_amd import _native as nat

    return hashlib.sha256(nat.LIB_PATH.read_bytes()).hexdigest()[:16]


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo, what lscpu reports as 'Model name')."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def cpu_baseline(w, target_s: float):
    """The reference's CPU path (oracle restatement of attention.py:205-250, torch SDPA)
    on a bounded sample of the same batch: the first rows whose contexts sum to a share
    that runs about `target_s` seconds in total. Reported as KV-read GB/s."""
    import torch

    from oracle import paged_sdpa

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    kc = w.k_caches[0].cpu()
    vc = w.v_caches[0].cpu()
    q = w.query.cpu()
    n_rows = 1
    probe = None
    while True:
        rows = list(range(n_rows))
        args = (q[rows], kc, vc, w.table[rows], [w.lens[i] for i in rows])
        t = time.perf_counter()
        paged_sdpa.paged_attention_sdpa(*args)
        probe = time.perf_counter() - t
        if probe * 5 >= target_s or n_rows >= w.batch:
            break
        n_rows = min(w.batch, max(n_rows * 2, int(n_rows * target_s / max(5 * probe, 1e-3))))
    times = []
    for _ in range(5):
        t = time.perf_counter()
        paged_sdpa.paged_attention_sdpa(*args)
        times.append(time.perf_counter() - t)
    med = sorted(times)[len(times) // 2]
    tokens = sum(w.lens[i] for i in rows)
    kv_bytes = tokens * w.kv_bytes_per_token()
    full_tokens = sum(w.lens)
    gbs = kv_bytes / med / 1e9
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": f"rows 0..{n_rows - 1} of {w.name} ({tokens} of {full_tokens} context tokens), "
                  f"median of 5 runs of the oracle's SDPA restatement in {str(w.dtype)[6:]}",
        "us_per_layer_extrapolated": round(med * 1e6 * full_tokens / tokens, 1),
        "cpu_model": cpu_model(),
        "torch": torch.__version__,
    }


# (batch, H, KVH, D, lo, hi, log-uniform, max_context or None for hi, cache, query)
SWEEP_SHAPES = [
    (64, 32, 8, 128, 1024, 8192, True, 8158, "bf16", "bf16"),
    (64, 32, 8, 128, 1024, 8192, True, 6144, "bf16", "bf16"),
    (48, 32, 8, 128, 1024, 8192, True, None, "bf16", "bf16"),
    (40, 32, 8, 128, 2048, 8192, False, None, "bf16", "bf16"),
    (32, 32, 8, 128, 1024, 8192, False, None, "bf16", "bf16"),
    (64, 32, 8, 128, 512, 4096, False, None, "bf16", "bf16"),
    (24, 32, 8, 128, 4096, 16384, False, None, "bf16", "bf16"),
    (12, 32, 8, 128, 8192, 32768, False, None, "bf16", "bf16"),
    (192, 14, 2, 64, 2048, 8192, False, None, "bf16", "bf16"),
    (240, 14, 2, 64, 1024, 8192, False, None, "bf16", "bf16"),
    (128, 14, 2, 64, 1024, 8192, False, None, "bf16", "bf16"),
    (96, 28, 4, 128, 1024, 8192, False, None, "bf16", "bf16"),
    (120, 28, 4, 128, 1024, 8192, False, None, "bf16", "bf16"),
    (64, 28, 4, 128, 2048, 8192, False, None, "bf16", "bf16"),
    (64, 32, 8, 128, 1024, 8192, True, 8158, "fp8", "bf16"),
    (48, 32, 8, 128, 1024, 8192, True, None, "fp8", "bf16"),
    (40, 32, 8, 128, 2048, 8192, False, None, "fp8", "bf16"),
    (64, 32, 8, 128, 1024, 8192, True, 8158, "fp32", "fp32"),
    (48, 32, 8, 128, 1024, 8192, True, None, "fp32", "fp32"),
    (16, 32, 8, 128, 1024, 8192, False, None, "bf16", "bf16"),
    (16, 32, 8, 128, 1024, 8192, True, None, "bf16", "bf16"),
    (8, 32, 8, 128, 8192, 16384, False, None, "bf16", "bf16"),
    (4, 32, 8, 128, 16384, 32768, False, None, "bf16", "bf16"),
    (24, 32, 8, 128, 1024, 8192, False, None, "bf16", "bf16"),
    (24, 32, 8, 128, 1024, 8192, True, None, "bf16", "bf16"),
    (12, 32, 8, 128, 4096, 16384, False, None, "bf16", "bf16"),
    (48, 32, 8, 128, 512, 4096, False, None, "bf16", "bf16"),
    (28, 32, 8, 128, 1024, 8192, True, None, "bf16", "bf16"),
    (12, 32, 8, 128, 1024, 8192, False, None, "bf16", "bf16"),
    (128, 14, 2, 64, 1024, 4096, False, None, "bf16", "bf16"),
    (64, 14, 2, 64, 2048, 8192, False, None, "bf16", "bf16"),
    (96, 14, 2, 64, 1024, 8192, False, None, "bf16", "bf16"),
    (96, 14, 2, 64, 1024, 8192, True, None, "bf16", "bf16"),
    (32, 28, 4, 128, 1024, 8192, False, None, "bf16", "bf16"),
    (48, 28, 4, 128, 1024, 8192, False, None, "bf16", "bf16"),
    (48, 28, 4, 128, 1024, 8192, True, None, "bf16", "bf16"),
    (16, 32, 8, 128, 1024, 8192, False, None, "fp8", "bf16"),
    (24, 32, 8, 128, 1024, 8192, False, None, "fp8", "bf16"),
    (16, 32, 8, 128, 1024, 8192, False, None, "fp32", "fp32"),
    (24, 32, 8, 128, 1024, 8192, False, None, "fp32", "fp32"),
    (24, 32, 8, 128, 1024, 8192, False, None, "fp32", "bf16"),
]


def decode_sweep():
    """Per-call time of each SWEEP_SHAPES decode (ten calls per hipGraph, 20 replays after
    5), with the route the library took."""
    import torch

    from miniserve_amd.attention import kernel_route, paged_attention

    dev = torch.device("cuda:0")
    types = {"bf16": torch.bfloat16, "fp8": torch.float8_e4m3fn, "fp32": torch.float32}
    for i, (B, H, KVH, D, lo, hi, logu, cap, kvn, qn) in enumerate(SWEEP_SHAPES):
        g = torch.Generator().manual_seed(i)
        if logu:
            lens = torch.exp(torch.empty(B).uniform_(math.log(lo), math.log(hi), generator=g))
            lens = lens.floor().long()
        else:
            lens = torch.randint(lo, hi + 1, (B,), generator=g)
        cap = cap or hi
        lens = lens.clamp(max=cap)
        W = -(-cap // 16)
        pool = int(sum(-(-int(L) // 16) for L in lens)) + 8
        kc = torch.randn(pool, 16, KVH, D, device=dev).to(types[kvn])
        vc = torch.randn(pool, 16, KVH, D, device=dev).to(types[kvn])
        perm = torch.randperm(pool, generator=g).int().to(dev)
        table = torch.zeros(B, W, dtype=torch.int32, device=dev)
        cur = 0
        for b in range(B):
            n = -(-int(lens[b]) // 16)
            table[b, :n] = perm[cur:cur + n]
            cur += n
        q = torch.randn(B, 1, H, D, device=dev).to(types[qn])
        ln = lens.int().to(dev)
        out = torch.empty_like(q)
        ws = torch.zeros(256 << 20, dtype=torch.uint8, device=dev)
        step = lambda: paged_attention(q, kc, vc, table, ln, max_context=cap, workspace=ws,
                                       out=out)
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream(dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(10):
                step()
        for _ in range(MIN_WARMUP_REPLAYS):
            graph.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(20):
            graph.replay()
        stop.record()
        torch.cuda.synchronize()
        print(json.dumps({"batch": B, "geometry": f"H{H}/KVH{KVH}/D{D}",
                          "contexts": f"{lo}..{hi} {'log-U' if logu else 'U'}",
                          "max_context": cap, "table_tiles": B * KVH * W,
                          "query": qn, "cache": kvn,
                          "route": kernel_route(q, kc, table, max_context=cap, out=out),
                          "us_per_call": round(start.elapsed_time(stop) * 1e3 / 200, 2)}),
              flush=True)
        del kc, vc, ws
        torch.cuda.empty_cache()


# (batch, H, KVH, q_len, context): causal bf16 chunks at the end of the context, D = 128
PREFILL_SWEEP_SHAPES = [
    (1, 32, 8, 64, 16384),     # 16 tasks
    (1, 32, 8, 128, 8192),     # 32
    (1, 8, 8, 512, 32768),     # 32
    (1, 32, 8, 256, 8192),     # 64
    (2, 32, 8, 192, 6144),     # 96
    (1, 28, 4, 512, 4608),     # 112
    (1, 32, 8, 512, 8192),     # 128
    (4, 32, 8, 128, 2048),     # 128
    (2, 32, 8, 384, 4096),     # 192
    (2, 28, 4, 512, 4608),     # 224 (C5)
]


def prefill_sweep(args):
    """Graph-step time of each PREFILL_SWEEP_SHAPES call (ten per graph, 20 replays after
    the warm-up) with its task count and TFLOP/s."""
    import torch

    from miniserve_amd.attention import kernel_route, paged_attention

    dev = torch.device("cuda:0")
    for i, (B, H, KVH, T, L) in enumerate(PREFILL_SWEEP_SHAPES):
        g = torch.Generator(device=dev).manual_seed(i)
        D, bs = 128, 16
        pages = -(-L // bs)
        pool = B * pages + 4
        kc = torch.randn(pool, bs, KVH, D, generator=g, device=dev).to(torch.bfloat16)
        vc = torch.randn(pool, bs, KVH, D, generator=g, device=dev).to(torch.bfloat16)
        table = torch.randperm(pool, device=dev)[: B * pages].view(B, pages).int()
        q = torch.randn(B, T, H, D, generator=g, device=dev).to(torch.bfloat16)
        lens = torch.full((B,), L, dtype=torch.int32, device=dev)
        out = torch.empty_like(q)
        ws = torch.zeros(256 << 20, dtype=torch.uint8, device=dev)
        step = lambda: paged_attention(q, kc, vc, table, lens, max_context=L, workspace=ws,
                                       out=out)
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream(dev).wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(10):
                step()
        warm(graph.replay, args.warm_ms, MIN_WARMUP_REPLAYS)
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(20):
            graph.replay()
        stop.record()
        torch.cuda.synchronize()
        us = start.elapsed_time(stop) * 1e3 / 200
        rows = T * (H // KVH)
        tasks = -(-rows // 128) * KVH * B
        flops = B * sum(4 * D * H * (L - T + j + 1) for j in range(T))
        print(json.dumps({"batch": B, "geometry": f"H{H}/KVH{KVH}/D{D}", "q_len": T,
                          "context": L, "tasks": tasks,
                          "route": kernel_route(q, kc, table, max_context=L, out=out),
                          "us_per_call": round(us, 2),
                          "tflops": round(flops / (us * 1e-6) / 1e12, 1)}), flush=True)
        del kc, vc, ws
        torch.cuda.empty_cache()


def _decode_inputs(w, dev):
    """Per-layer new-token q/k/v of a decode step ([layers, batch, 1, heads, D]), seeded."""
    import torch

    g = torch.Generator(device=dev).manual_seed(7)
    shape_q = (w.layers, w.batch, 1, w.num_heads, w.head_dim)
    shape_kv = (w.layers, w.batch, 1, w.num_kv_heads, w.head_dim)
    q = torch.randn(shape_q, generator=g, device=dev).to(w.dtype)
    k = torch.randn(shape_kv, generator=g, device=dev).to(w.dtype)
    v = torch.randn(shape_kv, generator=g, device=dev).to(w.dtype)
    return q, k, v


def runner_bench(args):
    """GraphedDecodeRunner.decode on the config's decode batch: each call stages the
    inputs (q/k/v copies, block tables and lengths from host lists), replays the bucket's
    captured graph (write_kv + attention per layer) and copies the output out. Timed on
    the host clock over whole calls (synchronised at the end), and the device time of the
    replays alone with events."""
    import torch

    from miniserve_amd import PagedAttention
    from miniserve_amd.graphs import DecodeLayer, GraphedDecodeRunner
    from miniserve_amd.workloads import make_workload

    dev = torch.device("cuda:0")
    w = make_workload(args.config, device=dev, values_device=dev, part="decode")
    B, H, KVH, D, bs = w.batch, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size
    layers = [DecodeLayer(PagedAttention(H, KVH, D, num_blocks=w.num_blocks, block_size=bs,
                                         dtype=w.dtype, kv_dtype=w.k_caches[i].dtype,
                                         device=dev), w.k_caches[i], w.v_caches[i])
              for i in range(w.layers)]
    width = w.table.shape[1]
    runner = GraphedDecodeRunner(layers, table_width=width, buckets=(1, 2, 4, 8, 16, 32, 64))
    # every row's last cached token is rewritten with its new k/v each step, so the
    # context stays the workload's
    ctx = [max(L - 1, 0) for L in w.lens]
    tables = [w.table[b, : -(-w.lens[b] // bs)].tolist() for b in range(B)]
    q, k, v = _decode_inputs(w, dev)
    bucket = next(b for b in runner.buckets if b >= B)
    for _ in range(max(MIN_WARMUP_REPLAYS, args.warmup)):  # captures both input sets
        runner.decode(q, k, v, tables, ctx)
    torch.cuda.synchronize()
    n = args.steps
    t0 = time.perf_counter()
    for _ in range(n):
        runner.decode(q, k, v, tables, ctx)
    torch.cuda.synchronize()
    wall_us = (time.perf_counter() - t0) / n * 1e6
    # device time of the replays alone
    graphs = runner._graphs[bucket]
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(n):
        graphs[i % 2]()
    stop.record()
    torch.cuda.synchronize()
    replay_us = start.elapsed_time(stop) / n * 1e3
    bytes_step = w.algorithmic_bytes(unique=True) * w.layers
    print(json.dumps({
        "metric": "GraphedDecodeRunner.decode step (bucketed hipGraph: write_kv + attention "
                  "per layer)",
        "value": round(wall_us, 2), "unit": "us/step (host clock, whole call)",
        "n_gpus": 1, "steps": n, "higher_is_better": False,
        "replay_us_per_step": round(replay_us, 2),
        "replay_us_per_layer": round(replay_us / w.layers, 2),
        "host_us_per_step": round(wall_us - replay_us, 2),
        "replay_gbs": round(bytes_step / (replay_us * 1e-6) / 1e9, 1),
        "config": {"workload": f"{w.name} decode through GraphedDecodeRunner", "batch": B,
                   "bucket": bucket, "layers": w.layers, "num_heads": H, "num_kv_heads": KVH,
                   "head_dim": D, "table_width": width,
                   "dtype": str(w.dtype).replace("torch.", "")},
    }), flush=True)


def eager_bench(args):
    """The reference runner's eager per-layer calls (model_runner.py:72-76) on the
    config's decode batch: write_kv with transposed k/v views and a Python-list start,
    then forward with a transposed q view, the int64 device block table and a
    Python-list context_lens. Host clock over N layers (synchronised at the end), against
    the attention kernel alone (HIP events, the same call through the C ABI)."""
    import torch

    from miniserve_amd import PagedAttention
    from miniserve_amd import _native as nat
    from miniserve_amd.workloads import make_workload

    dev = torch.device("cuda:0")
    w = make_workload(args.config, device=dev, values_device=dev, part="decode")
    B, H, KVH, D, bs = w.batch, w.num_heads, w.num_kv_heads, w.head_dim, w.block_size
    kc, vc = w.k_caches[0], w.v_caches[0]
    pa = PagedAttention(H, KVH, D, num_blocks=w.num_blocks, block_size=bs, dtype=w.dtype,
                        kv_dtype=kc.dtype, device=dev)
    table64 = w.table.to(dev)  # int64, as the reference runner keeps it
    starts = [max(L - 1, 0) for L in w.lens]
    lens_list = [s + 1 for s in starts]
    q5, k5, v5 = _decode_inputs(w, dev)
    # the runner's views: [B, H, 1, D] projections transposed to [B, 1, H, D]
    q = q5[0].transpose(1, 2).contiguous().transpose(1, 2)
    k = k5[0].transpose(1, 2).contiguous().transpose(1, 2)
    v = v5[0].transpose(1, 2).contiguous().transpose(1, 2)

    def layer_call(write=True):
        if write:
            pa.write_kv(kc, vc, k, v, table64, start=starts)
        return pa.forward(q, kc, vc, table64, lens_list)

    for _ in range(max(MIN_WARMUP_REPLAYS, args.warmup)):
        layer_call()
    torch.cuda.synchronize()
    n = args.steps

    def host_clock(write):
        t0 = time.perf_counter()
        for _ in range(n):
            layer_call(write)
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e6

    both_us = host_clock(True)
    fwd_us = host_clock(False)
    # the attention kernel alone, through the C ABI on prepared device inputs
    lib = nat.lib()
    qc = q.contiguous()
    table = table64.to(torch.int32)
    lens = torch.tensor(lens_list, dtype=torch.int32, device=dev)
    max_ctx = max(lens_list)
    ws_bytes = lib.msattn_workspace_bytes(B, 1, H, KVH, D, max_ctx)
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=dev)
    out = torch.empty_like(qc)
    stream = nat.stream_handle(dev)

    def raw():
        nat.check("attention", lib.msattn_paged_attention(
            qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1),
            kc.stride(2), table.data_ptr(), lens.data_ptr(), out.data_ptr(), ws.data_ptr(),
            ws_bytes, B, 1, H, KVH, D, bs, w.num_blocks, table.shape[1], max_ctx, 1, 0, w.scale,
            nat.dtype_code(w.dtype), nat.dtype_code(kc.dtype), stream))

    for _ in range(5):
        raw()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(n):
        raw()
    stop.record()
    torch.cuda.synchronize()
    kernel_us = start.elapsed_time(stop) / n * 1e3
    t0 = time.perf_counter()
    for _ in range(n):
        raw()
    torch.cuda.synchronize()
    raw_host_us = (time.perf_counter() - t0) / n * 1e6
    print(json.dumps({
        "metric": "eager PagedAttention per layer as the reference runner calls it "
                  "(write_kv + forward)",
        "value": round(both_us, 2), "unit": "us/layer (host clock)", "n_gpus": 1, "steps": n,
        "higher_is_better": False,
        "forward_us": round(fwd_us, 2),
        "write_kv_us": round(both_us - fwd_us, 2),
        "kernel_us": round(kernel_us, 2),
        "c_abi_call_host_us": round(raw_host_us, 2),
        "forward_overhead_us": round(fwd_us - max(kernel_us, raw_host_us), 2),
        "config": {"workload": f"{w.name} decode, one layer, eager", "batch": B,
                   "num_heads": H, "num_kv_heads": KVH, "head_dim": D,
                   "dtype": str(w.dtype).replace("torch.", ""),
                   "kv_dtype": str(kc.dtype).replace("torch.", "")},
    }), flush=True)


def cpu_baseline_prefill(w, target_s: float):
    """The reference's CPU path for the C5 prefill call (the oracle's restatement of
    attention.py:205-250: gather to the longest context, GQA expand, causal mask, torch
    SDPA in the config dtype) on a bounded sample: the whole call when it runs in about
    `target_s` seconds or less, else its first sequence (same chunk, same context).
    Reported as TFLOP/s of the sample's causal attention."""
    import torch

    from oracle import paged_sdpa

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    kc, vc, q = w.k_caches[0].cpu(), w.v_caches[0].cpu(), w.query.cpu()
    T, H, D = q.shape[1], q.shape[2], q.shape[3]
    rows = list(range(w.batch))
    args = (q, kc, vc, w.table, list(w.lens))
    t = time.perf_counter()
    paged_sdpa.paged_attention_sdpa(*args)
    first = time.perf_counter() - t
    if first * 3 > target_s and w.batch > 1:
        rows = [0]
        args = (q[rows], kc, vc, w.table[rows], [w.lens[0]])
    runs = 3
    times = []
    for _ in range(runs):
        t = time.perf_counter()
        paged_sdpa.paged_attention_sdpa(*args)
        times.append(time.perf_counter() - t)
    med = sorted(times)[len(times) // 2]
    flops = sum(4 * D * H * (w.lens[b] - T + i + 1) for b in rows for i in range(T)
                if w.lens[b] - T + i + 1 > 0)
    return {
        "value": round(flops / med / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": f"sequence(s) {rows} of C5-prefill ({len(rows) * T} query rows onto "
                  f"{w.lens[0]}-token contexts), median of {runs} runs of the oracle's SDPA "
                  f"restatement in {str(q.dtype)[6:]}",
        "us_per_call_extrapolated": round(med * 1e6 * w.batch / len(rows), 1),
        "cpu_model": cpu_model(),
        "torch": torch.__version__,
    }


if __name__ == "__main__":
    main()
