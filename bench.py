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

The prefill workload (--config qwen3.6-35b-a3b-q4-prefill512) times one
512-token chunk through swq_moe_prefill: router GEMM, top-k and grouping of
the 4096 (token, expert) pairs, grouped gate/up and down on the bf16 matrix
cores, combine.  A per-expert logit bias skews the expert load towards
Zipf(1.1).  The decode line carries a summary of the same measurement under
"prefill" (skip it with --no-prefill).
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
# each scaled by what the counter reads for a 256 MiB device copy (FETCH x 2.0, WRITE x 1.0),
# 48 distinct layers cycled;
# the runs' commands and raw counts are kept with the kernel-trace summaries.  Keyed (workload, kernel).
MEASURED_TRAFFIC = {
    ("qwen3.6-35b-a3b-q4-b1", "moe_fused"): 17_652_196,
    ("qwen3.6-35b-a3b-q4-b1", "moe_stage1"): 2_757_384,
    ("qwen3.6-35b-a3b-q4-b1", "moe_stage2"): 9_698_457,
    ("qwen3.6-35b-a3b-q4-b1", "moe_stage3"): 5_713_406,
    ("qwen3.6-35b-a3b-q8-b4", "moe_fused"): 115_208_204,
    ("qwen3.6-35b-a3b-q8-b4", "moe_stage1"): 5_580_301,
    ("qwen3.6-35b-a3b-q8-b4", "moe_stage2"): 69_525_396,
    ("qwen3.6-35b-a3b-q8-b4", "moe_stage3"): 36_430_644,
    ("qwen3.6-35b-a3b-q4-prefill512", "gate_up"): 344_679_983,
    ("qwen3.6-35b-a3b-q4-prefill512", "down"): 209_619_859,
}

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16, published

# prefill workloads: name -> (shape key, tokens, Zipf seed of the logit bias)
PREFILL_CONFIGS = {
    "qwen3.6-35b-a3b-q4-prefill512": ("qwen3.6-35b-a3b-q4", 512, 2024),
}
PREFILL_STAGES = [("router", 2), ("route", 4), ("gate_up", 8), ("down", 16), ("combine", 32)]

CONFIGS = {
    # name: (shape key, batch)
    "single-expert-q4-b1": ("single-expert-q4", 1),
    "qwen3.6-35b-a3b-q4-b1": ("qwen3.6-35b-a3b-q4", 1),
    "qwen3-next-80b-a3b-q4-b1": ("qwen3-next-80b-a3b-q4", 1),
    "qwen3.6-35b-a3b-q8-b1": ("qwen3.6-35b-a3b-q8", 1),
    "qwen3.6-35b-a3b-q8-b4": ("qwen3.6-35b-a3b-q8", 4),
}


# the other decode workloads the default line summarises, and the resident
# layers each cycles (enough distinct bytes to exceed the 256 MB MALL: one
# 1.77 MB expert per layer for the single expert; 48 layers for the 80B stack)
OTHER_DECODE_CONFIGS = ["single-expert-q4-b1", "qwen3-next-80b-a3b-q4-b1", "qwen3.6-35b-a3b-q8-b1",
                        "qwen3.6-35b-a3b-q8-b4"]
DEFAULT_REPLICAS = {"single-expert-q4-b1": 256, "qwen3-next-80b-a3b-q4-b1": 48, "qwen3.6-35b-a3b-q8-b1": 48,
                    "qwen3.6-35b-a3b-q8-b4": 48, "qwen3.6-35b-a3b-q4-b1": 48}


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=960)
    ap.add_argument("--warmup", type=int, default=96)
    ap.add_argument("--config", default="qwen3.6-35b-a3b-q4-b1", choices=sorted(CONFIGS) + sorted(PREFILL_CONFIGS))
    ap.add_argument("--no-prefill", action="store_true", help="decode line without the prefill summary")
    ap.add_argument("--no-configs", action="store_true",
                    help="decode line without the single-expert, 80B, q8 batch-1 and batch-4 summaries")
    ap.add_argument("--no-lmhead", action="store_true", help="decode line without the lm_head + sampling summary")
    ap.add_argument("--no-load", action="store_true", help="decode line without the qpack layer-load rate")
    ap.add_argument("--no-deltanet", action="store_true", help="decode line without the DeltaNet layer summary")
    ap.add_argument("--no-attention", action="store_true", help="decode line without the attention layer summary")
    ap.add_argument("--no-model", action="store_true", help="decode line without the whole-model token summary")
    ap.add_argument("--attention-context", type=int, default=4096, help="cached positions of the attention summary")
    ap.add_argument("--prefill-steps", type=int, default=40, help="prefill chunks timed")
    ap.add_argument("--prefill-replicas", type=int, default=3, help="distinct layers the prefill chunks cycle")
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

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    if args.config in PREFILL_CONFIGS:
        res = prefill_measure(args, torch, lib, args.config)
        line = prefill_line(args, res)
        if not args.no_cpu_baseline:
            line["cpu_baseline"] = prefill_cpu_baseline(args, res)
        print(json.dumps(line), flush=True)
        return

    shape_key, batch = CONFIGS[args.config]
    path = args.path if args.path != "auto" else auto_path(batch)
    shape = synth.SHAPES[shape_key]
    torch.cuda.init()
    K, W = args.steps, args.warmup
    m = decode_measure(args, torch, lib, args.config, args.replicas, K, W, path, keep=True)
    layers, wss, calls, ids, wts, xs_bits = m.pop("_keep")
    R = len(layers)
    dev = "cuda"
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    MASK = _lib.SWQ_STAGES_FUSED if path == "fused" else 7

    def step(i, mask=MASK):
        check(lib.swq_moe_decode_stages(*calls[i % R], mask, sh), "moe_decode")

    # ---- per-kernel durations ------------------------------------------------
    # fused: one kernel per step, so the graph's average step is its average
    # launch.  staged: graphs of single-stage steps (each replica's workspace
    # already holds its routing from the replays above, so a stage on its own
    # reads valid inputs); HIP events around one replay give the average launch.
    n_st = max(R, min(K, 4 * R))
    if path == "fused":
        stage_us = [m["us_per_step"]]
    else:
        stage_us = []
        for mask in (1, 2, 4):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                for i in range(n_st):
                    check(lib.swq_moe_decode_stages(*calls[i % R], mask, cap), "moe_decode stage (capture)")
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
    # ---- the layer tail: attention residual add + post-attention RMSNorm
    # (swq_rmsnorm), then the MoE step adding into the f32 residual stream,
    # as a graph over the same resident layers
    hs = torch.randn((R, batch, shape.hidden), dtype=torch.float32, device=dev)
    rs = torch.randn((R, batch, shape.hidden), dtype=torch.float32, device=dev)
    wnorm = (1.0 + 0.1 * torch.randn(shape.hidden, device=dev)).to(torch.bfloat16)
    xn = torch.empty((R, batch, shape.hidden), dtype=torch.bfloat16, device=dev)
    tail_calls = []
    for r, l in enumerate(layers):
        tail_calls.append((
            (ctypes.c_void_p(hs[r].data_ptr()), ctypes.c_void_p(rs[r].data_ptr()), ctypes.c_void_p(wnorm.data_ptr()),
             _lib.SWQ_BF16, ctypes.c_float(1e-6), batch, shape.hidden, ctypes.c_void_p(xn[r].data_ptr()), _lib.SWQ_BF16),
            (ctypes.byref(l._c), ctypes.c_void_p(xn[r].data_ptr()), _lib.SWQ_BF16, batch,
             ctypes.c_void_p(hs[r].data_ptr()), _lib.SWQ_F32, ctypes.c_void_p(ids[r].data_ptr()),
             ctypes.c_void_p(wts[r].data_ptr()), ctypes.c_void_p(wss[r].data_ptr()), wss[r].numel(),
             _lib.SWQ_MOE_ACCUMULATE)))
    n_tail = max(R, K)
    gt = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gt):
        cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for i in range(n_tail):
            nrm, dec = tail_calls[i % R]
            check(lib.swq_rmsnorm(*nrm, cap), "rmsnorm (capture)")
            check(lib.swq_moe_decode_stages(*dec, MASK, cap), "moe_decode (capture)")
    gt.replay()
    torch.cuda.synchronize()
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    b0.record()
    gt.replay()
    b1.record()
    torch.cuda.synchronize()
    tail_sep_us = b0.elapsed_time(b1) * 1000.0 / n_tail
    del gt
    # the same tail with the residual add and the norm folded into the MoE
    # step's launch (swq_moe_decode_norm; batch 1, the single-launch path)
    tail_us = tail_sep_us
    tail_folded = False
    if batch == 1:
        hs_out = torch.empty_like(hs)
        fold_calls = [(ctypes.byref(l._c), ctypes.c_void_p(hs[r].data_ptr()), ctypes.c_void_p(rs[r].data_ptr()),
                       ctypes.c_void_p(wnorm.data_ptr()), _lib.SWQ_BF16, ctypes.c_float(1e-6),
                       ctypes.c_void_p(hs_out[r].data_ptr()), ctypes.c_void_p(ids[r].data_ptr()),
                       ctypes.c_void_p(wts[r].data_ptr()), ctypes.c_void_p(wss[r].data_ptr()), wss[r].numel())
                      for r, l in enumerate(layers)]
        if lib.swq_moe_decode_norm(*fold_calls[0], sh) == _lib.SWQ_OK:
            gf = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gf):
                cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
                for i in range(n_tail):
                    check(lib.swq_moe_decode_norm(*fold_calls[i % R], cap), "moe_decode_norm (capture)")
            gf.replay()
            torch.cuda.synchronize()
            b0.record()
            gf.replay()
            b1.record()
            torch.cuda.synchronize()
            tail_us = b0.elapsed_time(b1) * 1000.0 / n_tail
            tail_folded = True
            del gf
    for r in range(R):
        check(layers[r].workspace_status(wss[r]), "workspace status after the timed replays")

    H, I, Is, E = shape.hidden, shape.inter, shape.shared_inter, shape.experts
    mb = shape.matrix_bytes
    eb, rb = shape.expert_bits, shape.router_bits
    xb = batch * H * 2
    mean_uniq = m["unique_experts_per_step"]
    step_bytes = m["step_bytes"]
    if path == "fused":
        stage_bytes = [step_bytes]
        kernels = ["moe_fused"]
    else:
        sh_b = (2 * mb(Is, H, eb) + mb(1, H, rb)) if Is else 0
        stage_bytes = [
            mb(E, H, rb) + sh_b + xb,                                # router + shared gate + shared gate/up
            mean_uniq * 2 * mb(I, H, eb) + xb,                       # routed gate/up
            mean_uniq * mb(H, I, eb) + (mb(H, Is, eb) if Is else 0) + xb,  # routed + shared down, bf16 out
        ]
        kernels = ["moe_stage1", "moe_stage2", "moe_stage3"]
    dom = int(np.argmax(stage_us))
    achieved = stage_bytes[dom] / (stage_us[dom] * 1e-6) / 1e9
    dom_kernel = kernels[dom]

    result = {
        "metric": "us per MoE-layer decode step; achieved HBM GB/s as fraction of peak (1 GPU)",
        "value": m["value"],
        "unit": "us/layer-step",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(m["value"] / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4-affine x bf16, fp32 accumulate" if eb == 4 else "q8-affine x bf16, fp32 accumulate",
        "data": m["data"],
        "config": m["config"],
        "roofline": {"bound": "hbm", "kernel": dom_kernel,
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": MEASURED_TRAFFIC.get((args.config, dom_kernel)),
                     "algorithmic_bytes_per_launch": int(stage_bytes[dom]),
                     "avg_launch_us": round(stage_us[dom], 3)},
        "step_us_distribution": m["distribution"],
        "path": path,
        "kernel_us": dict(zip(kernels, [round(v, 3) for v in stage_us])),
        "kernel_bytes": dict(zip(kernels, [int(v) for v in stage_bytes])),
        "step_bytes": int(step_bytes),
        "step_gbs_wall": m["step_gbs"],
        "step_gbs_kernels": round(step_bytes / (sum(stage_us) * 1e-6) / 1e9, 1),
        "eager_us_per_step": round(eager_us_per_step, 3),
        "layer_tail_us": round(tail_us, 3),
        "layer_tail_separate_us": round(tail_sep_us, 3),
        "layer_tail_note": ("residual add + post-attention RMSNorm + MoE step: one launch (swq_moe_decode_norm); "
                            "layer_tail_separate_us: swq_rmsnorm then the MoE step" if tail_folded else
                            "swq_rmsnorm then the MoE step"),
        "unique_experts_per_step": mean_uniq,
    }

    # ---- CPU baseline: the C restatement of the reference CPU path -------
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args, shape, batch, layers[0], xs_bits[0])

    # ---- the token tail: final norm, lm_head GEMV, sampling -----------------
    if not args.no_lmhead and shape_key.startswith("qwen3.6-35b"):
        result["lm_head"] = lmhead_measure(args, torch, lib, shape.hidden)

    # ---- one token through the whole model ---------------------------------
    if not args.no_model and shape_key == "qwen3.6-35b-a3b-q4" and batch == 1:
        result["model_decode"] = model_measure(args, torch, lib, shape, layers, wss)

    # ---- the DeltaNet layer (the layer type of 30 of the 40 layers) ---------
    if not args.no_deltanet and shape_key.startswith("qwen3.6-35b"):
        result["deltanet"] = deltanet_measure(args, torch, lib, shape.hidden)

    # ---- the full-attention layer (every 4th layer) -------------------------
    if not args.no_attention and shape_key.startswith("qwen3.6-35b"):
        result["attention"] = attention_measure(args, torch, lib, shape.hidden)

    # ---- loading: one .qpack layer file into HBM ----------------------------
    if not args.no_load and shape_key.startswith("qwen3.6-35b"):
        result["qpack_load"] = qpack_load_measure(torch, lib, shape)

    del layers, wss, calls
    torch.cuda.synchronize()
    torch.cuda.empty_cache()

    # ---- the other decode workloads, each on its own resident stack ---------
    if not args.no_configs and args.config == "qwen3.6-35b-a3b-q4-b1":
        result["configs"] = {}
        for name in OTHER_DECODE_CONFIGS:
            sm = decode_measure(args, torch, lib, name, None, None, None, "auto")
            result["configs"][name] = {k: sm[k] for k in (
                "value", "unit", "distribution", "roofline", "step_bytes", "unique_experts_per_step", "config",
                "data")}
            torch.cuda.synchronize()
            torch.cuda.empty_cache()

    # ---- the prefill chunk, summarised --------------------------------------
    if not args.no_prefill:
        res = prefill_measure(args, torch, lib, "qwen3.6-35b-a3b-q4-prefill512")
        line = prefill_line(args, res)
        result["prefill"] = {k: line[k] for k in ("config", "value", "unit", "roofline", "kernel_us", "mfma")}

    print(json.dumps(result), flush=True)


def auto_path(batch):
    """The single launch takes 1, 2 or 4 tokens; other batches run as three launches."""
    return "fused" if batch in (1, 2, 4) else "staged"


def decode_measure(args, torch, lib, name, R=None, K=None, W=None, path="auto", keep=False):
    """µs per MoE-layer decode step of workload `name` on R resident seeded
    layers (all experts each), cycled with a distinct input per layer.

    K steps are captured in one HIP graph (step i runs layer i mod R; by
    default 480: a replay carries a fixed start-up cost, ~60-100 us on the
    first timed replay, which 96-step graphs spread into ~1 us per step).
    The first timed replay, bracketed by a synchronize on both sides, gives
    `value` (K steps exactly); further replays of the same graph, at least
    100 steps in all and at least 11 replays, give the distribution of the
    per-step time over replays (median, p10, p90).  Algorithmic bytes count
    each distinct expert of a step once, from the ids the timed steps wrote
    (only the layers the graph ran)."""
    from swiftlet_amd import _lib, moe, synth
    from swiftlet_amd._lib import check
    shape_key, batch = CONFIGS[name]
    shape = synth.SHAPES[shape_key]
    R = R or DEFAULT_REPLICAS.get(name, 48)
    K = K or max(R, 480)
    W = W if W is not None else R
    path = path if path != "auto" else auto_path(batch)
    mask = _lib.SWQ_STAGES_FUSED if path == "fused" else 7
    dev = "cuda"
    layers = [moe.synth_layer(shape, args.seed, r, dev) for r in range(R)]
    xs_bits = synth.activations_bf16(args.seed + 7, R * batch, shape.hidden).reshape(R, batch, shape.hidden)
    xs = torch.from_numpy(xs_bits.view(np.int16)).view(torch.bfloat16).to(dev)
    wss = [l.new_workspace(batch) for l in layers]
    outs = torch.empty((R, batch, shape.hidden), dtype=torch.bfloat16, device=dev)
    ids = torch.full((R, batch, shape.top_k), -1, dtype=torch.int32, device=dev)
    wts = torch.empty((R, batch, shape.top_k), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    calls = [(ctypes.byref(l._c), ctypes.c_void_p(xs[r].data_ptr()), _lib.SWQ_BF16, batch,
              ctypes.c_void_p(outs[r].data_ptr()), _lib.SWQ_BF16, ctypes.c_void_p(ids[r].data_ptr()),
              ctypes.c_void_p(wts[r].data_ptr()), ctypes.c_void_p(wss[r].data_ptr()), wss[r].numel(), 0)
             for r, l in enumerate(layers)]
    sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for i in range(W):
        check(lib.swq_moe_decode_stages(*calls[i % R], mask, sh), "moe_decode")
    torch.cuda.synchronize()
    ids.fill_(-1)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for i in range(K):
            check(lib.swq_moe_decode_stages(*calls[i % R], mask, cap), "moe_decode (capture)")
    torch.cuda.synchronize()
    graph.replay()  # warm: the graph's own first replay
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    samples = []
    n_rep = max(11, -(-100 // K))
    for _ in range(n_rep):
        torch.cuda.synchronize()
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        samples.append(e0.elapsed_time(e1) * 1000.0 / K)
    for r in range(min(K, R)):
        check(layers[r].workspace_status(wss[r]), f"{name}: workspace status after the timed replays")
    ran = min(K, R)
    ids_h = ids.cpu().numpy()[:ran]
    assert (ids_h >= 0).all(), "a timed step did not write its routing"
    uniq = float(np.mean([len(np.unique(ids_h[r])) for r in range(ran)]))
    step_bytes = shape.decode_bytes(uniq, batch)
    value = samples[0]
    med = float(np.median(samples))
    achieved = step_bytes / (med * 1e-6) / 1e9
    out = {
        "value": round(value, 3),
        "unit": "us/layer-step",
        "us_per_step": med,
        "distribution": {"median": round(med, 3), "p10": round(float(np.percentile(samples, 10)), 3),
                         "p90": round(float(np.percentile(samples, 90)), 3), "replays": n_rep,
                         "steps_per_replay": K, "timed_steps": n_rep * K,
                         "note": "per-step time of each graph replay (K steps, event-timed)"},
        "roofline": {"bound": "hbm", "kernel": "moe_fused" if path == "fused" else "three launches",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "algorithmic_bytes_per_launch": int(step_bytes),
                     "avg_launch_us": round(med, 3)},
        "step_bytes": int(step_bytes),
        "step_gbs": round(step_bytes / (value * 1e-6) / 1e9, 1),
        "unique_experts_per_step": uniq,
        "data": f"synthetic seeded weights (seed {args.seed}), {ran} distinct resident layers cycled by the "
                f"{K} timed steps ({R} resident), bf16 x ~N(0,1), a distinct x per layer",
        "config": {"workload": name, "hidden": shape.hidden, "experts": shape.experts, "top_k": shape.top_k,
                   "moe_intermediate": shape.inter, "shared_intermediate": shape.shared_inter,
                   "expert_bits": shape.expert_bits, "router_bits": shape.router_bits, "group": shape.group,
                   "batch": batch, "replicas": R, "layers_cycled": ran, "path": path,
                   "parallelism": "single GPU"},
    }
    if keep:
        out["_keep"] = (layers, wss, calls, ids, wts, xs_bits)
    else:
        del graph, layers, wss, calls
    return out


MODEL_LAYERS = 40  # qwen3.6-35b: 30 DeltaNet layers, every 4th one full attention


def model_measure(args, torch, lib, shape, moe_layers, moe_ws, tokens=4):
    """One decode token through the whole 35B-shape model, every kernel on
    the device, as one graph: per layer the input RMSNorm + projections (one
    launch), the DeltaNet step or the attention step (cache of
    --attention-context positions), out_proj / o_proj, then the residual add,
    post-attention RMSNorm and MoE step in one launch (the 40 resident MoE
    layers of the decode measurement); then the final RMSNorm, the q4
    lm_head (248,320 rows) and Qwen's default sampling.  Synthetic weights
    of the real shapes; the hidden state alternates between two buffers."""
    from swiftlet_amd import _lib, moe
    from swiftlet_amd._lib import check
    from swiftlet_amd.attention import AttentionGPU
    from swiftlet_amd.deltanet import DeltaNetGPU
    dev = "cuda"
    H = shape.hidden
    nk, nv, dk, dv, K = 16, 32, 128, 128, 4
    convD, valD = 2 * nk * dk + nv * dv, nv * dv
    AH, AKV, ahd = 16, 2, 256
    pos = args.attention_context - 1
    g = torch.Generator(device="cpu").manual_seed(args.seed + 2)

    def bf16_ones():
        return (1.0 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)

    blocks = []
    for i in range(MODEL_LAYERS):
        seed_base = 5000 + 16 * i
        if (i + 1) % 4 != 0:
            projs = [moe.synth_linear(args.seed, seed_base + j, "router", None, rows, H, 4, 64, dev)
                     for j, rows in enumerate((convD, valD, nv, nv))]
            out = moe.synth_linear(args.seed, seed_base + 4, "router", None, H, valD, 4, 64, dev)
            blk = DeltaNetGPU(nk, nv, dk, dv, K, _lib.SWQ_DELTA_SPLIT, 1e-6,
                              torch.randn(convD * K, generator=g) * 0.3, torch.randn(nv, generator=g) * 0.5,
                              torch.randn(nv, generator=g) * 0.5, 1.0 + 0.1 * torch.randn(dv, generator=g),
                              projections=projs, out_proj=out, device=dev)
            blocks.append(("delta", blk, blk.new_state()))
        else:
            projs = [moe.synth_linear(args.seed, seed_base + j, "router", None, rows, H, 4, 64, dev)
                     for j, rows in enumerate((AH * 2 * ahd, AKV * ahd, AKV * ahd))]
            o = moe.synth_linear(args.seed, seed_base + 3, "router", None, H, AH * ahd, 4, 64, dev)
            blk = AttentionGPU(AH, AKV, ahd, 64, 1e7, 1e-6, pos + 1, 1.0 + 0.1 * torch.randn(ahd, generator=g),
                               1.0 + 0.1 * torch.randn(ahd, generator=g), projections=projs, o_proj=o, device=dev)
            cache = blk.new_cache()
            ck, cv = blk.cache_views(cache)
            ck[:pos].normal_(0.0, 0.5)
            cv[:pos].normal_()
            blocks.append(("attn", blk, (cache, blk.new_workspace())))
    w_in = [bf16_ones() for _ in range(MODEL_LAYERS)]
    w_post = [bf16_ones() for _ in range(MODEL_LAYERS)]
    w_final = bf16_ones()
    head = moe.synth_linear(args.seed, 990, "router", None, LMHEAD_VOCAB, H, 4, 64, dev)
    hbuf = [torch.randn(H, generator=g).to(dev), torch.empty(H, dtype=torch.float32, device=dev)]
    proj_out = torch.empty(convD + valD, dtype=torch.float32, device=dev)
    ba = torch.empty(2 * nv, dtype=torch.float32, device=dev)
    q = torch.empty(AH * 2 * ahd, dtype=torch.float32, device=dev)
    kk = torch.empty(AKV * ahd, dtype=torch.float32, device=dev)
    vv = torch.empty(AKV * ahd, dtype=torch.float32, device=dev)
    y = torch.empty(max(valD, AH * ahd), dtype=torch.float32, device=dev)
    r = torch.empty(H, dtype=torch.float32, device=dev)
    logits = torch.empty(LMHEAD_VOCAB, dtype=torch.float32, device=dev)
    n_ws = lib.swq_sample_workspace_bytes(LMHEAD_VOCAB)
    sws = torch.zeros(n_ws, dtype=torch.uint8, device=dev)
    seen = torch.arange(0, 64 * 997, 997, dtype=torch.int32, device=dev) % LMHEAD_VOCAB
    counts = torch.ones(64, dtype=torch.int32, device=dev)
    banned = torch.tensor([LMHEAD_VOCAB - 1], dtype=torch.int32, device=dev)
    tok = torch.empty(1, dtype=torch.int32, device=dev)
    ids = torch.empty((1, shape.top_k), dtype=torch.int32, device=dev)
    wts = torch.empty((1, shape.top_k), dtype=torch.float32, device=dev)
    opt = _lib.SampleOptions(0.7, 20, 0.8, 1.5, 0.5)
    eps = ctypes.c_float(1e-6)
    multi = []
    for kind, blk, _ in blocks:
        if kind == "delta":
            ptrs = (proj_out.data_ptr(), proj_out.data_ptr() + 4 * convD, ba.data_ptr(), ba.data_ptr() + 4 * nv)
        else:
            ptrs = (q.data_ptr(), kk.data_ptr(), vv.data_ptr())
        multi.append(((_lib.QLinear * len(ptrs))(*[l.c() for l in blk.projections]), (ctypes.c_void_p * len(ptrs))(*ptrs)))
    outs_c = [blk.out_proj.c() if kind == "delta" else blk.o_proj.c() for kind, blk, _ in blocks]
    head_c = head.c()
    head_lins = (_lib.QLinear * 1)(head_c)
    head_ys = (ctypes.c_void_p * 1)(logits.data_ptr())
    launches = 0

    def token(cap, t):
        nonlocal launches
        for i, (kind, blk, st) in enumerate(blocks):
            hc, hn = hbuf[i % 2], hbuf[(i + 1) % 2]
            lins, ys = multi[i]
            check(lib.swq_encode_gemv_multi(lins, len(ys), ys, hc.data_ptr(), w_in[i].data_ptr(), _lib.SWQ_BF16, eps,
                                            cap), "norm + projections")
            if kind == "delta":
                check(lib.swq_deltanet_step(ctypes.byref(blk._c), proj_out.data_ptr(), ba.data_ptr(), st.data_ptr(),
                                            st.numel(), pos + t, y.data_ptr(), cap), "deltanet")
                launches += 1
            else:
                cache, ws = st
                check(lib.swq_attention_step(ctypes.byref(blk._c), q.data_ptr(), kk.data_ptr(), vv.data_ptr(),
                                             cache.data_ptr(), cache.numel(), pos, y.data_ptr(), ws.data_ptr(),
                                             ws.numel(), cap), "attention")
                launches += 2
            check(lib.swq_encode_gemv(ctypes.byref(outs_c[i]), 0, 0, 0, 0, y.data_ptr(), 0, r.data_ptr(), 0, cap),
                  "out_proj")
            ml = moe_layers[i]
            check(lib.swq_moe_decode_norm(ctypes.byref(ml._c), hc.data_ptr(), r.data_ptr(), w_post[i].data_ptr(),
                                          _lib.SWQ_BF16, eps, hn.data_ptr(), ids.data_ptr(), wts.data_ptr(),
                                          moe_ws[i].data_ptr(), moe_ws[i].numel(), cap), "moe")
            launches += 3
        hc = hbuf[MODEL_LAYERS % 2]
        # the final norm inside the lm_head's launch
        check(lib.swq_encode_gemv_multi(head_lins, 1, head_ys, hc.data_ptr(), w_final.data_ptr(), _lib.SWQ_BF16, eps,
                                        cap), "final norm + lm_head")
        check(lib.swq_sample(logits.data_ptr(), LMHEAD_VOCAB, ctypes.byref(opt), seen.data_ptr(), counts.data_ptr(),
                             64, banned.data_ptr(), 1, ctypes.c_float(0.5), tok.data_ptr(), sws.data_ptr(), n_ws, cap),
              "sample")
        launches += 2

    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for t in range(tokens):
            token(cap, t)
    gr.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    gr.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1000.0 / tokens
    # every MoE step of the replays completed normally (a stalled single
    # launch leaves its record in the workspace; its outputs would be invalid)
    for i, ws in enumerate(moe_ws):
        check(lib.swq_moe_workspace_status(ws.data_ptr(), ws.numel(), 1, None), f"model: MoE layer {i} workspace status")
    del gr, blocks, head
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return {"us_per_token": round(us, 1), "tokens_per_s": round(1e6 / us, 1), "layers": MODEL_LAYERS,
            "attention_context": pos + 1, "launches_per_token": launches // tokens,
            "note": "one decode token of the 35B-A3B-shape 4-bit model (30 DeltaNet + 10 attention layers, 40 MoE "
                    "steps, final norm inside the 248,320-row lm_head's launch, sampling), all on the device, graph of 4 "
                    "tokens; "
                    "synthetic weights; context only: the reference publishes 7-11 tok/s for this model on an "
                    "M5 Mac (README.md:21), whole decode including its SSD expert streaming"}


DN_LAYERS = 30  # qwen3.6-35b: 40 layers, every 4th one full attention


def deltanet_measure(args, torch, lib, hidden, tokens=8):
    """The 35B DeltaNet layer per token (split projections, nk 16, nv 32,
    dk = dv = 128, conv 4; q4 group-64 projections with fp16 scales): input
    RMSNorm, in_proj_qkv / z / b / a GEMVs, swq_deltanet_step, out_proj GEMV,
    residual add + post-attention RMSNorm — a graph over 30 resident layers
    (537 MB of projections, more than the 256 MB MALL) and 8 tokens; and the
    step kernel alone from a graph of the same steps."""
    from swiftlet_amd import _lib, moe
    from swiftlet_amd._lib import check
    from swiftlet_amd.deltanet import DeltaNetGPU
    dev = "cuda"
    nk, nv, dk, dv, K = 16, 32, 128, 128, 4
    convD, valD = 2 * nk * dk + nv * dv, nv * dv
    g = torch.Generator(device="cpu").manual_seed(args.seed)
    layers = []
    for r in range(DN_LAYERS):
        projs = [moe.synth_linear(args.seed, 3000 + 8 * r + j, "router", None, rows, hidden, 4, 64, dev)
                 for j, rows in enumerate((convD, valD, nv, nv))]
        out = moe.synth_linear(args.seed, 3000 + 8 * r + 4, "router", None, hidden, valD, 4, 64, dev)
        blk = DeltaNetGPU(nk, nv, dk, dv, K, _lib.SWQ_DELTA_SPLIT, 1e-6,
                          torch.randn(convD * K, generator=g) * 0.3, torch.randn(nv, generator=g) * 0.5,
                          torch.randn(nv, generator=g) * 0.5, 1.0 + 0.1 * torch.randn(dv, generator=g),
                          projections=projs, out_proj=out, device=dev)
        layers.append((blk, blk.new_state(), (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(dev),
                       (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(dev)))
    h = torch.randn((DN_LAYERS, hidden), generator=g).to(dev)
    x = torch.empty((DN_LAYERS, hidden), dtype=torch.float32, device=dev)
    qkvz = torch.empty((DN_LAYERS, convD + valD), dtype=torch.float32, device=dev)
    ba = torch.empty((DN_LAYERS, 2 * nv), dtype=torch.float32, device=dev)
    y = torch.empty((DN_LAYERS, valD), dtype=torch.float32, device=dev)
    rr = torch.empty((DN_LAYERS, hidden), dtype=torch.float32, device=dev)
    x2 = torch.empty((DN_LAYERS, hidden), dtype=torch.float32, device=dev)
    eps = ctypes.c_float(1e-6)
    multi = []
    for r, (blk, _, _, _) in enumerate(layers):
        lins = (_lib.QLinear * 4)(*[lin.c() for lin in blk.projections])
        ys = (ctypes.c_void_p * 4)(qkvz[r].data_ptr(), qkvz[r].data_ptr() + 4 * convD, ba[r].data_ptr(),
                                   ba[r].data_ptr() + 4 * nv)
        multi.append((lins, ys))

    def graph_of(step_only):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for t in range(tokens):
                for r, (blk, st, w_in, w_post) in enumerate(layers):
                    if not step_only:  # input RMSNorm + the four projections: one launch
                        lins, ys = multi[r]
                        check(lib.swq_encode_gemv_multi(lins, 4, ys, h[r].data_ptr(), w_in.data_ptr(), _lib.SWQ_BF16,
                                                        eps, cap), "norm + projections")
                    check(lib.swq_deltanet_step(ctypes.byref(blk._c), qkvz[r].data_ptr(), ba[r].data_ptr(),
                                                st.data_ptr(), st.numel(), t, y[r].data_ptr(), cap), "deltanet")
                    if not step_only:
                        c = blk.out_proj.c()
                        check(lib.swq_encode_gemv(ctypes.byref(c), 0, 0, 0, 0, y[r].data_ptr(), 0,
                                                  rr[r].data_ptr(), 0, cap), "out_proj")
                        check(lib.swq_rmsnorm(h[r].data_ptr(), rr[r].data_ptr(), w_post.data_ptr(), _lib.SWQ_BF16,
                                              eps, 1, hidden, x2[r].data_ptr(), _lib.SWQ_F32, cap), "post norm")
        return gr

    def timed(gr):
        gr.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        gr.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / (tokens * DN_LAYERS)

    qkvz.normal_()
    ba.normal_()
    step_us = timed(graph_of(True))
    layer_us = timed(graph_of(False))
    step_bytes = (2 * nv * dv * dk + (K - 1) * convD + convD + convD * K + convD + valD + 2 * nv + valD) * 4
    proj_bytes = sum(lin.matrix_bytes for lin in layers[0][0].projections) + layers[0][0].out_proj.matrix_bytes
    layer_bytes = proj_bytes + step_bytes + 2 * hidden * 4 * 4
    gbs = step_bytes / (step_us * 1e-6) / 1e9
    del layers
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return {"step_us": round(step_us, 3), "step_bytes": int(step_bytes), "step_gbs": round(gbs, 1),
            "step_frac": round(gbs / HBM_PEAK_GBS, 4), "layer_us": round(layer_us, 3),
            "layer_bytes": int(layer_bytes),
            "layer_gbs": round(layer_bytes / (layer_us * 1e-6) / 1e9, 1),
            "note": "35B DeltaNet layer per token (split layout, q4 projections), graph over 30 resident layers "
                    "x 8 tokens: input norm + 4 projections (one launch) + swq_deltanet_step + out_proj + "
                    "residual/post-norm; "
                    "step_us from a graph of the step alone (state 2 MB read + written per layer)"}


ATTN_LAYERS = 10  # qwen3.6-35b: every 4th of 40 layers


def attention_measure(args, torch, lib, hidden, reps=8):
    """The 35B full-attention layer per token at a cache of
    --attention-context positions (16 query heads over 2 kv heads, hd 256,
    64 rotary dims; q4 group-64 projections): input RMSNorm, q/k/v_proj
    GEMVs, swq_attention_step, o_proj GEMV, residual add + post-attention
    RMSNorm — a graph over 10 resident layers x 8 repetitions of the same
    position; and the step alone (two launches) from a graph of the steps."""
    from swiftlet_amd import _lib, moe
    from swiftlet_amd._lib import check
    from swiftlet_amd.attention import AttentionGPU
    dev = "cuda"
    H, KVH, hd, rot = 16, 2, 256, 64
    pos = args.attention_context - 1
    g = torch.Generator(device="cpu").manual_seed(args.seed + 1)
    layers = []
    for r in range(ATTN_LAYERS):
        projs = [moe.synth_linear(args.seed, 4000 + 8 * r + j, "router", None, rows, hidden, 4, 64, dev)
                 for j, rows in enumerate((H * 2 * hd, KVH * hd, KVH * hd))]
        o = moe.synth_linear(args.seed, 4000 + 8 * r + 3, "router", None, hidden, H * hd, 4, 64, dev)
        blk = AttentionGPU(H, KVH, hd, rot, 1e7, 1e-6, pos + 1, 1.0 + 0.1 * torch.randn(hd, generator=g),
                           1.0 + 0.1 * torch.randn(hd, generator=g), projections=projs, o_proj=o, device=dev)
        cache = blk.new_cache()
        ck, cv = blk.cache_views(cache)
        ck[:pos].normal_(0.0, 0.5)
        cv[:pos].normal_()
        layers.append((blk, cache, blk.new_workspace(),
                       (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(dev),
                       (1.0 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(dev)))
    n = ATTN_LAYERS
    h = torch.randn((n, hidden), generator=g).to(dev)
    x = torch.empty((n, hidden), dtype=torch.float32, device=dev)
    q = torch.randn((n, H * 2 * hd), generator=g).to(dev)
    kk = torch.randn((n, KVH * hd), generator=g).to(dev)
    vv = torch.randn((n, KVH * hd), generator=g).to(dev)
    att = torch.empty((n, H * hd), dtype=torch.float32, device=dev)
    rr = torch.empty((n, hidden), dtype=torch.float32, device=dev)
    x2 = torch.empty((n, hidden), dtype=torch.float32, device=dev)
    eps = ctypes.c_float(1e-6)
    multi = []
    for r, (blk, _, _, _, _) in enumerate(layers):
        multi.append(((_lib.QLinear * 3)(*[lin.c() for lin in blk.projections]),
                      (ctypes.c_void_p * 3)(q[r].data_ptr(), kk[r].data_ptr(), vv[r].data_ptr())))

    def graph_of(step_only):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for _ in range(reps):
                for r, (blk, cache, ws, w_in, w_post) in enumerate(layers):
                    if not step_only:  # input RMSNorm + q/k/v_proj: one launch
                        lins, ys = multi[r]
                        check(lib.swq_encode_gemv_multi(lins, 3, ys, h[r].data_ptr(), w_in.data_ptr(), _lib.SWQ_BF16,
                                                        eps, cap), "norm + projections")
                    check(lib.swq_attention_step(ctypes.byref(blk._c), q[r].data_ptr(), kk[r].data_ptr(),
                                                 vv[r].data_ptr(), cache.data_ptr(), cache.numel(), pos,
                                                 att[r].data_ptr(), ws.data_ptr(), ws.numel(), cap), "attention")
                    if not step_only:
                        c = blk.o_proj.c()
                        check(lib.swq_encode_gemv(ctypes.byref(c), 0, 0, 0, 0, att[r].data_ptr(), 0,
                                                  rr[r].data_ptr(), 0, cap), "o_proj")
                        check(lib.swq_rmsnorm(h[r].data_ptr(), rr[r].data_ptr(), w_post.data_ptr(), _lib.SWQ_BF16,
                                              eps, 1, hidden, x2[r].data_ptr(), _lib.SWQ_F32, cap), "post norm")
        return gr

    def timed(gr):
        gr.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        gr.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / (reps * n)

    step_us = timed(graph_of(True))
    layer_us = timed(graph_of(False))
    # k and v rows of every cached position + the new token's projections and the output
    step_bytes = 2 * (pos + 1) * KVH * hd * 4 + (H * 2 * hd + 2 * KVH * hd + H * hd) * 4
    proj_bytes = sum(lin.matrix_bytes for lin in layers[0][0].projections) + layers[0][0].o_proj.matrix_bytes
    gbs = step_bytes / (step_us * 1e-6) / 1e9
    del layers
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return {"context": pos + 1, "step_us": round(step_us, 3), "step_bytes": int(step_bytes),
            "step_gbs": round(gbs, 1), "step_frac": round(gbs / HBM_PEAK_GBS, 4), "layer_us": round(layer_us, 3),
            "layer_bytes": int(proj_bytes + step_bytes + 4 * hidden * 4),
            "note": "35B attention layer per token with an f32 KV cache of `context` positions, graph over 10 "
                    "resident layers x 8: input norm + q/k/v_proj (one launch) + swq_attention_step + o_proj + "
                    "residual/post-norm; "
                    "step_us from a graph of the step alone"}


PCIE_PEAK_GBS = 64.0  # PCIe 5.0 x16, one direction


def qpack_load_measure(torch, lib, shape, reps=3):
    """One layer file of a .qpack container (E blobs of the layer's gate, up
    and down codes, scales and biases, 16 KiB-aligned) read from the page
    cache and copied into HBM by swq_qpack_load_experts: pread into two
    pinned 16 MiB staging buffers, host-to-device copies overlapped with the
    next read.  The file is written to a temporary directory first (synthetic
    bytes) and read once untimed."""
    import shutil
    import tempfile

    from swiftlet_amd._lib import check
    H, I, E, bits = shape.hidden, shape.inter, shape.experts, shape.expert_bits
    g = shape.group
    sections, off = [], 0
    for proj, rows, cols in (("gate_proj", I, H), ("up_proj", I, H), ("down_proj", H, I)):
        for part, dt, per_shape, size in (("weight", "U32", [rows, cols * bits // 32], rows * cols * bits // 8),
                                          ("scales", "F16", [rows, cols // g], rows * cols // g * 2),
                                          ("biases", "F16", [rows, cols // g], rows * cols // g * 2)):
            sections.append({"name": f"{proj}.{part}", "dtype": dt, "shape": per_shape, "offset": off, "size": size})
            off += size
    stride = (off + 16383) // 16384 * 16384
    d = tempfile.mkdtemp(prefix="swq-qpack-", dir="/tmp")
    try:
        os.makedirs(os.path.join(d, "packed_experts"))
        with open(os.path.join(d, "packed_experts", "layout.json"), "w") as f:
            json.dump({"expertCount": E, "layerCount": 1, "expertStride": stride, "sections": sections,
                       "linearLayers": [True]}, f)
        with open(os.path.join(d, "manifest.json"), "w") as f:
            json.dump({"magic": "QPACK", "version": 1, "modelName": "synthetic", "sourceCheckpoint": "synthetic",
                       "quantBits": bits, "quantGroupSize": g, "files": {}}, f)
        blob = np.arange(stride // 4, dtype=np.uint32).tobytes()
        with open(os.path.join(d, "packed_experts", "layer_00.bin"), "wb") as f:
            for _ in range(E):
                f.write(blob)
        n = E * stride
        h = ctypes.c_void_p()
        check(lib.swq_qpack_open(d.encode(), ctypes.byref(h)), "qpack open")
        dst = torch.empty(n, dtype=torch.uint8, device="cuda")
        times = []
        for i in range(reps + 1):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            check(lib.swq_qpack_load_experts(h, 0, 0, E, ctypes.c_void_p(dst.data_ptr()), n, None), "load")
            torch.cuda.synchronize()
            if i:
                times.append(time.perf_counter() - t0)
        lib.swq_qpack_close(h)
        ok = bytes(dst[:stride].cpu().numpy()) == blob
        del dst
        best = min(times)
        return {"layer_file_bytes": n, "expert_stride": stride, "ms": round(best * 1e3, 2),
                "gbs": round(n / best / 1e9, 2), "pcie_peak_gbs": PCIE_PEAK_GBS,
                "frac": round(n / best / 1e9 / PCIE_PEAK_GBS, 3), "first_blob_intact": ok,
                "note": "one 35B-shape layer file (E blobs), page-cache warm, best of "
                        f"{reps}: pread into pinned staging + host-to-device copies"}
    finally:
        shutil.rmtree(d, ignore_errors=True)


LMHEAD_VOCAB = 248320  # qwen3.6-35b vocab_size (model config)


def lmhead_measure(args, torch, lib, hidden):
    """Final RMSNorm and the q4 lm_head GEMV in one launch
    (swq_encode_gemv_multi with the norm weight), then Qwen's default sampling
    (swq_sample: T 0.7, top-k 20, top-p 0.8, presence 1.5, frequency 0.5, 64
    seen tokens) per token, as a graph over two resident lm_heads (2 x 286 MB,
    more than the 256 MB MALL).  gemv_us: the GEMV alone (swq_encode_gemv)."""
    from swiftlet_amd import _lib, moe
    from swiftlet_amd._lib import check
    dev = "cuda"
    V, R, K = LMHEAD_VOCAB, 2, 64
    heads = [moe.synth_linear(args.seed, 900 + r, "router", None, V, hidden, 4, 64, dev) for r in range(R)]
    h = torch.randn((R, hidden), dtype=torch.float32, device=dev)
    wn = (1.0 + 0.1 * torch.randn(hidden, device=dev)).to(torch.bfloat16)
    # the GEMV-alone graph's input: the normalised rows the fused launch computes
    x = ((h * torch.rsqrt((h * h).mean(dim=1, keepdim=True) + 1e-6)) * wn.float()).contiguous()
    logits = torch.empty((R, V), dtype=torch.float32, device=dev)
    n_ws = lib.swq_sample_workspace_bytes(V)
    wss = [torch.zeros(n_ws, dtype=torch.uint8, device=dev) for _ in range(R)]
    seen = torch.arange(0, 64 * 997, 997, dtype=torch.int32, device=dev) % V
    counts = torch.ones(64, dtype=torch.int32, device=dev)
    banned = torch.tensor([V - 1], dtype=torch.int32, device=dev)
    toks = torch.empty(R, dtype=torch.int32, device=dev)
    opt = _lib.SampleOptions(0.7, 20, 0.8, 1.5, 0.5)
    cs = [c.c() for c in heads]
    lins1 = [(_lib.QLinear * 1)(c) for c in cs]
    ys1 = [(ctypes.c_void_p * 1)(logits[r].data_ptr()) for r in range(R)]

    def graph_of(parts):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for i in range(K):
                r = i % R
                if "norm+gemv" in parts:
                    check(lib.swq_encode_gemv_multi(lins1[r], 1, ys1[r], h[r].data_ptr(), wn.data_ptr(), _lib.SWQ_BF16,
                                                    ctypes.c_float(1e-6), cap), "final norm + lm_head")
                if "gemv" in parts:
                    check(lib.swq_encode_gemv(ctypes.byref(cs[r]), 0, 0, 0, 0, x[r].data_ptr(), 0,
                                              logits[r].data_ptr(), 0, cap), "lm_head gemv")
                if "sample" in parts:
                    check(lib.swq_sample(logits[r].data_ptr(), V, ctypes.byref(opt), seen.data_ptr(),
                                         counts.data_ptr(), 64, banned.data_ptr(), 1, ctypes.c_float(0.5),
                                         toks[r:].data_ptr(), wss[r].data_ptr(), n_ws, cap), "sample")
        return g

    def timed(g):
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / K

    us_step = timed(graph_of(("norm+gemv", "sample")))
    us_gemv = timed(graph_of(("gemv",)))
    us_sample = timed(graph_of(("sample",)))
    gemv_bytes = heads[0].matrix_bytes + hidden * 4 + V * 4
    gbs = gemv_bytes / (us_gemv * 1e-6) / 1e9
    del heads
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return {"vocab": V, "us_per_token": round(us_step, 3), "gemv_us": round(us_gemv, 3),
            "sample_us": round(us_sample, 3), "gemv_bytes": int(gemv_bytes), "gemv_gbs": round(gbs, 1),
            "gemv_frac": round(gbs / 8000.0, 4),
            "note": "final norm + q4 lm_head GEMV (one launch) + top-k/top-p sampling per token, graph of 64 "
                    "tokens over 2 resident lm_heads; gemv_us from a graph of the GEMV alone"}


def prefill_measure(args, torch, lib, name):
    """Time the prefill chunk: a graph of --prefill-steps full chunks cycling
    --prefill-replicas layers, then each launch alone (graph replays of that
    stage over the replicas, whose workspaces hold the earlier stages'
    outputs)."""
    from swiftlet_amd import _lib, moe, synth
    from swiftlet_amd._lib import check

    shape_key, T, zipf_seed = PREFILL_CONFIGS[name]
    shape = synth.SHAPES[shape_key]
    H, E, K = shape.hidden, shape.experts, shape.top_k
    R = args.prefill_replicas
    dev = "cuda"
    layers = [moe.synth_layer(shape, args.seed, 100 + r, dev) for r in range(R)]
    bias = torch.from_numpy(synth.zipf_logit_bias(zipf_seed, E)).to(dev)
    xs_bits = synth.activations_bf16(args.seed + 11, R * T, H).reshape(R, T, H)
    xs = torch.from_numpy(xs_bits.view(np.int16)).view(torch.bfloat16).to(dev)
    wss = [l.new_prefill_workspace(T) for l in layers]
    outs = torch.empty((R, T, H), dtype=torch.bfloat16, device=dev)
    ids = torch.empty((R, T, K), dtype=torch.int32, device=dev)
    wts = torch.empty((R, T, K), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    calls = [(ctypes.byref(l._c), ctypes.c_void_p(xs[r].data_ptr()), _lib.SWQ_BF16, T,
              ctypes.c_void_p(outs[r].data_ptr()), _lib.SWQ_BF16, ctypes.c_void_p(ids[r].data_ptr()),
              ctypes.c_void_p(wts[r].data_ptr()), ctypes.c_void_p(bias.data_ptr()),
              ctypes.c_void_p(wss[r].data_ptr()), wss[r].numel(), 0) for r, l in enumerate(layers)]

    def graph_of(n, mask):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
            for i in range(n):
                check(lib.swq_moe_prefill_stages(*calls[i % R], mask, cap), "moe_prefill (capture)")
        return g

    def timed(g, n):
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1000.0 / n

    sh = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for r in range(R):
        check(lib.swq_moe_prefill_stages(*calls[r], _lib.SWQ_PREFILL_ALL, sh), "moe_prefill")
    torch.cuda.synchronize()
    Kp = args.prefill_steps
    us_chunk = timed(graph_of(Kp, _lib.SWQ_PREFILL_ALL), Kp)
    n_st = 4 * R
    stage_us = {nm: timed(graph_of(n_st, bit), n_st) for nm, bit in PREFILL_STAGES}

    ids_h = ids.cpu().numpy()
    counts = [np.bincount(ids_h[r].ravel(), minlength=E) for r in range(R)]
    touched = float(np.mean([(c > 0).sum() for c in counts]))
    tiles = float(np.mean([((c + 63) // 64).sum() for c in counts])) + (T + 63) // 64
    I, Is = shape.inter, shape.shared_inter
    mb, eb, rb = shape.matrix_bytes, shape.expert_bits, shape.router_bits
    xb = T * H * 2
    P = T * K
    kbytes = {
        "router": mb(E, H, rb) + xb,
        "route": mb(1, H, rb) + xb,
        "gate_up": touched * 2 * mb(I, H, eb) + 2 * mb(Is, H, eb) + xb,
        "down": touched * mb(H, I, eb) + mb(H, Is, eb),
        "combine": xb,
    }
    kflops = {
        "router": 2.0 * T * E * H,
        "gate_up": 2.0 * 2 * (P * I + T * Is) * H,
        "down": 2.0 * (P * I + T * Is) * H,
    }
    chunk_bytes = touched * shape.expert_bytes() + shape.shared_bytes() + shape.router_bytes() \
        + shape.seg_bytes() + 2 * xb
    return {"name": name, "shape": shape, "T": T, "R": R, "zipf_seed": zipf_seed, "us_chunk": us_chunk,
            "stage_us": stage_us, "kbytes": kbytes, "kflops": kflops, "chunk_bytes": chunk_bytes,
            "touched": touched, "tiles": tiles, "max_count": int(np.max([c.max() for c in counts])),
            "counts_sorted": sorted((int(v) for v in counts[0]), reverse=True)}


def prefill_line(args, res):
    shape, T = res["shape"], res["T"]
    st, kb, kf = res["stage_us"], res["kbytes"], res["kflops"]
    dom = max(st, key=st.get)
    gbs = kb[dom] / (st[dom] * 1e-6) / 1e9
    mfma = {k: {"tflops": round(kf[k] / (st[k] * 1e-6) / 1e12, 1),
                "frac": round(kf[k] / (st[k] * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)} for k in kf}
    return {
        "metric": "us per 512-token MoE-layer prefill chunk; achieved HBM GB/s and MFMA TFLOP/s as fractions of peak (1 GPU)",
        "value": round(res["us_chunk"], 2),
        "unit": "us/chunk",
        "n_gpus": 1,
        "steps": args.prefill_steps,
        "warmup": res["R"],
        "ms_per_step": round(res["us_chunk"] / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4-affine x bf16 on bf16 MFMA, fp32 accumulate",
        "data": f"synthetic seeded weights (seed {args.seed}), {res['R']} distinct resident layers cycled, "
                f"bf16 x ~N(0,1), Zipf(1.1) per-expert logit bias (seed {res['zipf_seed']})",
        "config": {"workload": res["name"], "tokens": T, "hidden": shape.hidden, "experts": shape.experts,
                   "top_k": shape.top_k, "moe_intermediate": shape.inter,
                   "shared_intermediate": shape.shared_inter, "expert_bits": shape.expert_bits,
                   "router_bits": shape.router_bits, "group": shape.group, "parallelism": "single GPU",
                   "experts_touched": res["touched"], "tiles": res["tiles"], "max_expert_pairs": res["max_count"]},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": MEASURED_TRAFFIC.get((res["name"], dom)),
                     "algorithmic_bytes_per_launch": int(kb[dom]), "avg_launch_us": round(st[dom], 3)},
        "mfma": mfma,
        "kernel_us": {k: round(v, 3) for k, v in st.items()},
        "chunk_bytes": int(res["chunk_bytes"]),
        "chunk_gbs": round(res["chunk_bytes"] / (res["us_chunk"] * 1e-6) / 1e9, 1),
        "expert_pairs_sorted": res["counts_sorted"][:32],
    }


def prefill_cpu_baseline(args, res):
    """The C restatement of the reference's per-token path (each pick's expert
    dequantised per token, QwenCPUModel.moeForward at S = 1, as the reference
    runs a prompt token by token) on a 16-token sample of layer 0's shape,
    scaled to the chunk."""
    from oracle import cref
    from swiftlet_amd import moe, synth

    if not cref.LIB.exists():
        import subprocess
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle")], check=True, capture_output=True)
    shape = res["shape"]
    arrays = moe.host_layer_arrays(shape, args.seed, 0)
    c = cref.CMoE(arrays, shape.hidden, shape.experts, shape.top_k, shape.inter, shape.shared_inter,
                  shape.group, shape.norm_topk_prob)
    xs = synth.bf16_to_f32(synth.activations_bf16(args.seed + 98, 16, shape.hidden))
    times = []
    t0 = time.perf_counter()
    for i in range(16):
        if time.perf_counter() - t0 > args.cpu_seconds:
            break
        t = time.perf_counter()
        c.forward(xs[i:i + 1], 1)
        times.append(time.perf_counter() - t)
    per_tok = float(np.median(times)) * 1e6
    return {"value": round(per_tok * res["T"], 1), "unit": "us/chunk", "cores": 1, "kind": "port",
            "sample": f"{len(times)} single-token steps (median {per_tok:.1f} us) x {res['T']} tokens; "
                      f"C restatement of QwenCPUModel.moeForward, experts dequantised per token",
            "cpu": cpu_model(), "nproc": os.cpu_count()}


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
