"""MoE-layer decode benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config NAME]

A step is one MoE-layer decode step (router GEMV, softmax, top-k,
renormalisation, routed SwiGLU experts, sigmoid-gated shared expert,
weighted combine) for one batch of synthetic tokens, on weights resident in
HBM.  The K timed steps cycle through `--replicas` distinct seeded layers
(each with all E experts) and distinct inputs, so the bytes a step touches
come from HBM, not from the 256 MB last-level cache.  The steps are
captured in one HIP graph and replayed.  A batch-1 step is one kernel (the
single-launch path), so the graph's average step is that kernel's average
launch; for batches (three launches) the per-kernel durations come from graph
replays of each stage on its own, timed with HIP events.  Prints one JSON
line.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published

# HBM bytes per launch from two rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE),
# each scaled by what the counter reads for a 256 MiB device copy (FETCH x 2.0, WRITE x 1.0);
# the runs' commands and raw counts are kept with the kernel-trace summaries.  Keyed (workload, kernel).
MEASURED_TRAFFIC = {
    ("qwen3.6-35b-a3b-q4-b1", "moe_fused"): 18_163_424,
    ("qwen3.6-35b-a3b-q4-b1", "moe_stage1"): 2_692_148,
    ("qwen3.6-35b-a3b-q4-b1", "moe_stage2"): 14_590_849,
    ("qwen3.6-35b-a3b-q4-b1", "moe_stage3"): 5_743_112,
}

CONFIGS = {
    # name: (shape key, batch)
    "qwen3.6-35b-a3b-q4-b1": ("qwen3.6-35b-a3b-q4", 1),
    "qwen3-next-80b-a3b-q4-b1": ("qwen3-next-80b-a3b-q4", 1),
    "qwen3.6-35b-a3b-q8-b1": ("qwen3.6-35b-a3b-q8", 1),
    "qwen3.6-35b-a3b-q8-b4": ("qwen3.6-35b-a3b-q8", 4),
}


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=960)
    ap.add_argument("--warmup", type=int, default=96)
    ap.add_argument("--config", default="qwen3.6-35b-a3b-q4-b1", choices=sorted(CONFIGS))
    ap.add_argument("--replicas", type=int, default=48, help="distinct layers cycled through (MALL defeat)")
    ap.add_argument("--seed", type=int, default=20261201)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bound on the CPU baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--path", default="auto", choices=("auto", "fused", "staged"),
                    help="auto: the single launch for batch 1, the three launches otherwise")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="first run three plain device-to-device copies of MIB MiB, a kernel of known "
                         "traffic that scales the FETCH_SIZE / WRITE_SIZE counters")
    return ap.parse_args()


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}). "
              "The MoE decode step would shard by experts across GPUs with one all-reduce of the "
              "[batch, hidden] output.", file=sys.stderr)
        sys.exit(2)

    import torch
    from swiftlet_amd import _lib, moe, synth
    from swiftlet_amd._lib import check

    if not _lib.LIB_PATH.exists():
        from swiftlet_amd import build
        build.build()
    lib = _lib.load()

    shape_key, batch = CONFIGS[args.config]
    path = args.path if args.path != "auto" else ("fused" if batch == 1 else "staged")
    MASK = _lib.SWQ_STAGES_FUSED if path == "fused" else 7
    shape = synth.SHAPES[shape_key]
    R = args.replicas
    dev = "cuda"
    torch.cuda.init()
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- resident weights: R distinct layers, all experts --------------
    layers = [moe.synth_layer(shape, args.seed, r, dev) for r in range(R)]
    xs_bits = synth.activations_bf16(args.seed + 7, R * batch, shape.hidden).reshape(R, batch, shape.hidden)
    xs = torch.from_numpy(xs_bits.view(np.int16)).view(torch.bfloat16).to(dev)
    wss = [l.new_workspace(batch) for l in layers]
    outs = torch.empty((R, batch, shape.hidden), dtype=torch.bfloat16, device=dev)
    ids = torch.empty((R, batch, shape.top_k), dtype=torch.int32, device=dev)
    wts = torch.empty((R, batch, shape.top_k), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()

    # prebuilt ctypes argument tuples, one per replica
    calls = []
    for r, l in enumerate(layers):
        calls.append((ctypes.byref(l._c), ctypes.c_void_p(xs[r].data_ptr()), _lib.SWQ_BF16, batch,
                      ctypes.c_void_p(outs[r].data_ptr()), _lib.SWQ_BF16, ctypes.c_void_p(ids[r].data_ptr()),
                      ctypes.c_void_p(wts[r].data_ptr()), ctypes.c_void_p(wss[r].data_ptr()), wss[r].numel(), 0))

    def step(i, mask=MASK):
        c = calls[i % R]
        check(lib.swq_moe_decode_stages(*c, mask, sh), "moe_decode")

    # ---- graph of K steps -----------------------------------------------
    K, W = args.steps, args.warmup
    for i in range(min(W, R)):
        step(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for i in range(K):
            c = calls[i % R]
            check(lib.swq_moe_decode_stages(*c, MASK, cap), "moe_decode (capture)")
    torch.cuda.synchronize()
    for _ in range(max(1, (W + K - 1) // K)):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    graph_ms = e0.elapsed_time(e1)
    us_per_step = graph_ms * 1000.0 / K

    # ---- per-kernel durations ------------------------------------------------
    # fused: one kernel per step, so the graph's average step is its average
    # launch.  staged: graphs of single-stage steps (each replica's workspace
    # already holds its routing from the replays above, so a stage on its own
    # reads valid inputs); HIP events around one replay give the average launch.
    n_st = min(K, 4 * R)
    if path == "fused":
        stage_us = [us_per_step]
    else:
        stage_us = []
        for mask in (1, 2, 4):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                for i in range(n_st):
                    c = calls[i % R]
                    check(lib.swq_moe_decode_stages(*c, mask, cap), "moe_decode stage (capture)")
            g.replay()
            torch.cuda.synchronize()
            a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a0.record()
            g.replay()
            a1.record()
            torch.cuda.synchronize()
            stage_us.append(a0.elapsed_time(a1) * 1000.0 / n_st)
            del g
    # eager (no graph) launches of whole steps, for reference
    check(lib.swq_bench_stall(20000, sh), "stall")
    t_eager0 = torch.cuda.Event(enable_timing=True)
    t_eager1 = torch.cuda.Event(enable_timing=True)
    t_eager0.record()
    for i in range(n_st):
        step(i)
    t_eager1.record()
    torch.cuda.synchronize()
    eager_us_per_step = t_eager0.elapsed_time(t_eager1) * 1000.0 / n_st
    # unique experts per step (batch > 1 reads each distinct expert once)
    ids_h = ids.cpu().numpy()
    uniq = [len(np.unique(ids_h[r])) for r in range(R)]
    mean_uniq = float(np.mean(uniq))

    H, I, Is, E = shape.hidden, shape.inter, shape.shared_inter, shape.experts
    mb = shape.matrix_bytes
    eb, rb = shape.expert_bits, shape.router_bits
    xb = batch * H * 2
    step_bytes = shape.decode_bytes(mean_uniq, batch)
    if path == "fused":
        stage_bytes = [step_bytes]
        kernels = ["moe_fused"]
    else:
        stage_bytes = [
            mb(E, H, rb) + mb(1, H, rb) + 2 * mb(Is, H, eb) + xb,    # router + shared gate + shared gate/up
            mean_uniq * 2 * mb(I, H, eb) + xb,                       # routed gate/up
            mean_uniq * mb(H, I, eb) + mb(H, Is, eb) + xb,           # routed + shared down, bf16 out
        ]
        kernels = ["moe_stage1", "moe_stage2", "moe_stage3"]
    dom = int(np.argmax(stage_us))
    achieved = stage_bytes[dom] / (stage_us[dom] * 1e-6) / 1e9
    dom_kernel = kernels[dom]

    result = {
        "metric": "us per MoE-layer decode step; achieved HBM GB/s as fraction of peak (1 GPU)",
        "value": round(us_per_step, 3),
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(us_per_step / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4-affine x bf16, fp32 accumulate" if eb == 4 else "q8-affine x bf16, fp32 accumulate",
        "data": f"synthetic seeded weights (seed {args.seed}), {R} distinct resident layers cycled, bf16 x ~N(0,1)",
        "config": {"workload": args.config, "hidden": H, "experts": E, "top_k": shape.top_k,
                   "moe_intermediate": I, "shared_intermediate": Is, "expert_bits": eb,
                   "router_bits": rb, "group": shape.group, "batch": batch, "replicas": R,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "kernel": dom_kernel,
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": MEASURED_TRAFFIC.get((args.config, dom_kernel)),
                     "algorithmic_bytes_per_launch": int(stage_bytes[dom]),
                     "avg_launch_us": round(stage_us[dom], 3)},
        "path": path,
        "kernel_us": dict(zip(kernels, [round(v, 3) for v in stage_us])),
        "kernel_bytes": dict(zip(kernels, [int(v) for v in stage_bytes])),
        "step_bytes": int(step_bytes),
        "step_gbs_wall": round(step_bytes / (us_per_step * 1e-6) / 1e9, 1),
        "step_gbs_kernels": round(step_bytes / (sum(stage_us) * 1e-6) / 1e9, 1),
        "eager_us_per_step": round(eager_us_per_step, 3),
        "unique_experts_per_step": mean_uniq,
    }

    # ---- CPU baseline: the C restatement of the reference CPU path -------
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args, shape, batch, layers[0], xs_bits[0])

    print(json.dumps(result), flush=True)


def cpu_baseline(args, shape, batch, layer0, x0_bits):
    """oracle/liboracle.so (QwenCPUModel.moeForward restated in C) on layer 0
    of the same workload, fresh x per step, bounded by --cpu-seconds."""
    from oracle import cref
    from swiftlet_amd import moe, synth

    if not cref.LIB.exists():
        import subprocess
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True, capture_output=True)
    arrays = moe.host_layer_arrays(shape, args.seed, 0)
    c = cref.CMoE(arrays, shape.hidden, shape.experts, shape.top_k, shape.inter, shape.shared_inter,
                  shape.group, shape.norm_topk_prob)
    xs = synth.bf16_to_f32(synth.activations_bf16(args.seed + 99, 64 * batch, shape.hidden))
    res = {}
    for threads in (1, cref.max_threads()):
        n, t0 = 0, time.perf_counter()
        times = []
        while n < 64 and time.perf_counter() - t0 < args.cpu_seconds / 2:
            t = time.perf_counter()
            c.forward(xs[n * batch:(n + 1) * batch], threads)
            times.append(time.perf_counter() - t)
            n += 1
        res[threads] = (float(np.median(times)) * 1e6, n)
    one_us, one_n = res[1]
    mt = max(res)
    return {"value": round(one_us, 1), "unit": "us/layer-step", "cores": 1, "kind": "port",
            "sample": f"{one_n} decode steps of layer 0 (batch {batch}), median; C restatement of "
                      f"QwenCPUModel.moeForward, experts dequantised per call",
            "multithread": {"value": round(res[mt][0], 1), "cores": mt, "steps": res[mt][1]},
            "cpu": cpu_model(), "nproc": os.cpu_count()}


if __name__ == "__main__":
    main()
