"""Benchmark of the block-FP8 MoE layer (fwd+bwd) on one MI355X.

Default workload: BASELINE config 3, the Qwen3-30B-A3B-shaped MoE layer
(T=16384 tokens, hidden 2048, expert width 768, 128 experts, top-8),
bf16 inputs and bf16 master weights quantized per call to 128x128 block-FP8,
block-FP8 GEMMs for forward, input gradients and weight gradients. One step =
``mlops_amd.moe`` forward + backward (with the aux-loss cotangent) on
synthetic N(0,1) activations, router weights N(0,1/H) (logits ~ N(0,1)) and
expert weights N(0,0.02).

Prints ONE JSON line with tokens/s, the grouped-GEMM roofline (fp8 MFMA peak)
measured live with device events around every GEMM launch on its stream, and
the CPU baseline: the reference's native PyTorch path (restated in
``oracle.native_moe``) on a bounded sample (128 tokens) of the same layer
shape, timed on the host cores.
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

FP8_PEAK_TFLOPS = 5000.0   # MI355X dense fp8 MFMA
HBM_PEAK_GBS = 8000.0      # MI355X HBM3E

CONFIGS = {
    "qwen3_30b_a3b": dict(tokens=16384, hidden=2048, inter=768, experts=128, top_k=8),
    # One EP rank's share of DeepSeek-V3: 32 local experts and 32768 routed
    # token-slots, each slot's expert drawn i.i.d. Zipf(s=1.2) (forced through
    # the routing override, so group sizes are as ragged as the draw makes
    # them), bf16 master weights N(0, 0.006).
    "deepseek_v3_shard": dict(tokens=32768, hidden=7168, inter=2048, experts=32, top_k=1,
                              zipf=1.2, weight_std=0.006),
    "mixtral_8x7b": dict(tokens=8192, hidden=4096, inter=14336, experts=8, top_k=2),
    # Expert LoRA on a frozen block-FP8 base: rank-16 bf16 factors, logits
    # N(0,1) + 2 on expert 0; gradients reach the factors, the router and the
    # hidden rows only.
    "mixtral_8x7b_lora": dict(tokens=8192, hidden=4096, inter=14336, experts=8, top_k=2,
                              lora_rank=16),
    # C3's layer at compute_precision="fp8_current" (per-row e4m3 scaling, the
    # reference's other FP8 format): the same per-call bf16 masters.
    "qwen3_30b_a3b_fp8_current": dict(tokens=16384, hidden=2048, inter=768, experts=128,
                                      top_k=8, precision="fp8_current"),
    "config1": dict(tokens=256, hidden=512, inter=1024, experts=8, top_k=2),
    # The single grouped GEMM (E=8, K=4096, N=2048, M_e ~ U{256..4096} step
    # 128, seeded): one step is one launch on resident e4m3 operands.
    "grouped_gemm_c2": dict(gemm_only=True, experts=8, k=4096, n=2048, seed=2),
}


def make_gemm_inputs(cfg, device):
    """C2's operands, quantized once (1x128 activation and 128x128 weight
    scales): ``(xq, xs, wq, ws, offsets, rows)``."""
    import numpy as np
    from mlops_amd import kernels as K

    rng = np.random.default_rng(cfg["seed"])
    counts = (rng.integers(2, 33, size=cfg["experts"]) * 128).tolist()
    offsets = torch.tensor([0] + list(np.cumsum(counts)), dtype=torch.int32, device=device)
    rows = int(sum(counts))
    g = torch.Generator(device=device).manual_seed(cfg["seed"])
    x = torch.randn(rows, cfg["k"], generator=g, device=device).to(torch.bfloat16)
    w = torch.randn(cfg["experts"], cfg["n"], cfg["k"], generator=g, device=device) * 0.02
    xq, xs = K.quantize_rows(x)
    wq, ws = K.quantize_weight_blocks(w.to(torch.bfloat16))
    return xq, xs, wq, ws, offsets, rows


def gemm_main(args, cfg):
    """One grouped GEMM per step; prints the JSON line for C2."""
    from mlops_amd import kernels as K

    device = torch.device("cuda", 0)
    xq, xs, wq, ws, offsets, rows = make_gemm_inputs(cfg, device)
    step = lambda: K.gemm(xq, xs, wq, ws, offsets)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # the kernel's own duration: a second pass with events around each launch
    timer = K.LaunchTimer()
    K.set_launch_timer(timer)
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    K.set_launch_timer(None)
    gemm = timer.summary()["gemm_fp8_block"]
    flops = 2 * rows * cfg["n"] * cfg["k"]
    achieved = gemm["flops"] / (gemm["ms_total"] * 1e-3) / 1e12
    print(json.dumps({
        "metric": "block-FP8 grouped GEMM TFLOP/s (% MFMA peak), 1 GPU",
        "value": flops * args.steps / elapsed / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "fp8_e4m3 (block-scaled), fp32 accumulate, bf16 out",
        "data": "synthetic (N(0,1) activations, N(0,0.02) weights)",
        "config": {"workload": "grouped_gemm_c2 single grouped GEMM", "experts": cfg["experts"],
                   "k": cfg["k"], "n": cfg["n"], "rows": rows},
        "roofline": {"kernel": "mi355x_gemm_fp8_block", "bound": "mfma", "achieved": achieved,
                     "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": achieved / FP8_PEAK_TFLOPS, "traffic": None},
    }))


def vendor_gemm_main(args, cfg):
    """Calibration, not the benchmark line: the four GEMM shapes of one layer
    step as ONE dense problem each (rows = tokens*top_k, one group), timed
    through hipBLASLt (``torch._scaled_mm``, per-tensor and per-row scales)
    and through this package's row-scaled and 128x128 block-scaled kernels
    with the same operands. Prints one JSON line per shape."""
    from mlops_amd import kernels as K

    device = torch.device("cuda", 0)
    rows = cfg["tokens"] * cfg["top_k"]
    h, i = cfg["hidden"], cfg["inter"]
    shapes = {"up": (2 * i, h), "down": (h, i), "dgrad_down": (i, h), "dgrad_up": (h, 2 * i)}
    g = torch.Generator(device=device).manual_seed(0)

    def timed(fn, reps=20):
        for _ in range(3):
            fn()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / reps

    offsets = torch.tensor([0, rows], dtype=torch.int32, device=device)
    for name, (n, k) in shapes.items():
        x = torch.randn(rows, k, generator=g, device=device).to(torch.bfloat16)
        w = (torch.randn(1, n, k, generator=g, device=device) * 0.02).to(torch.bfloat16)
        xq_r, xs_r = K.quantize_rows_current(x)
        wq_r, _, ws_r, _ = K.quantize_weights_current(w)
        xq_b, xs_b = K.quantize_rows(x)
        wq_b, ws_b = K.quantize_weight_blocks(w)
        one = torch.ones((), device=device)
        runs = {
            "hipblaslt_tensorwise": lambda: torch._scaled_mm(
                xq_r, wq_r[0].t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16),
            "hipblaslt_rowwise": lambda: torch._scaled_mm(
                xq_r, wq_r[0].t(), scale_a=xs_r[:, None], scale_b=ws_r[0][None, :],
                out_dtype=torch.bfloat16),
            "mi355x_gemm_fp8_rowwise": lambda: K.gemm_rowwise(xq_r, xs_r, wq_r, ws_r, offsets),
            "mi355x_gemm_fp8_block": lambda: K.gemm(xq_b, xs_b, wq_b, ws_b, offsets),
        }
        flops = 2 * rows * n * k
        line = {"shape": name, "rows": rows, "n": n, "k": k}
        for label, fn in runs.items():
            ms = timed(fn)
            line[label] = {"us": round(ms * 1e3, 1), "tflops": round(flops / ms / 1e9, 1)}
        print(json.dumps(line), flush=True)
        del x, w, xq_r, xs_r, wq_r, ws_r, xq_b, xs_b, wq_b, ws_b


def make_inputs(cfg, device, seed=0):
    g = torch.Generator(device=device).manual_seed(seed)
    t, h, i, e = cfg["tokens"], cfg["hidden"], cfg["inter"], cfg["experts"]
    x = torch.randn(t, h, generator=g, device=device).to(torch.bfloat16)
    res = torch.randn(t, h, generator=g, device=device).to(torch.bfloat16)
    wr = torch.randn(e, h, generator=g, device=device) / math.sqrt(h)
    std = cfg.get("weight_std", 0.02)
    w13 = (torch.randn(e, 2 * i, h, generator=g, device=device) * std).to(torch.bfloat16)
    w2 = (torch.randn(e, h, i, generator=g, device=device) * std).to(torch.bfloat16)
    dy = torch.randn(t, h, generator=g, device=device).to(torch.bfloat16)
    return x, res, wr, w13, w2, dy


def make_lora_inputs(cfg, device, seed=0):
    """The LoRA workload: the layer's inputs with a frozen block-FP8 base, a
    +2 logit on expert 0 (a constant hidden feature the router reads) and
    factors A ~ N(0, 0.01), B = 0.1 N(0, 1) in bf16."""
    from mlops_amd import BlockFP8Weight

    x, res, wr, w13, w2, dy = make_inputs(cfg, device, seed)
    x[:, 0] = 1.0
    wr[:, 0] = 0.0
    wr[0, 0] = 2.0
    g = torch.Generator(device=device).manual_seed(seed + 1)
    e, r, h, i = cfg["experts"], cfg["lora_rank"], cfg["hidden"], cfg["inter"]

    def factor(*shape, std):
        return (torch.randn(*shape, generator=g, device=device) * std).to(torch.bfloat16)

    factors = [factor(e, r, h, std=0.01), factor(e, 2 * i, r, std=0.1),
               factor(e, r, i, std=0.01), factor(e, h, r, std=0.1)]
    for t in factors:
        t.requires_grad_(True)
    w13c, w2c = BlockFP8Weight.quantize(w13), BlockFP8Weight.quantize(w2)
    return x, res, wr, w13c, w2c, factors, dy


def lora_step(args, cfg):
    from mlops_amd.lora import expert_lora

    x, res, wr, w13c, w2c, factors, dy = args
    for t in (x, wr, *factors):
        t.grad = None
    out, aux, counts, psum = expert_lora(x, res, wr, w13c, w2c, *factors, top_k=cfg["top_k"],
                                         routing_mode="topk_then_softmax", scale=2.0)
    torch.autograd.backward([out, aux], [dy, torch.full_like(aux, 0.01)])


def zipf_ids(cfg, device, seed=0):
    """``[tokens, top_k]`` expert ids with every slot's expert drawn i.i.d. from
    Zipf(s) over the experts (p_e proportional to (e + 1)^-s); needs top_k = 1
    (i.i.d. slots could repeat an expert within a token otherwise)."""
    import numpy as np

    if cfg["top_k"] != 1:
        raise ValueError("i.i.d. Zipf slots are drawn with top_k = 1")
    p = np.arange(1, cfg["experts"] + 1, dtype=np.float64) ** -cfg["zipf"]
    rng = np.random.default_rng(seed)
    ids = rng.choice(cfg["experts"], size=(cfg["tokens"], 1), p=p / p.sum())
    return torch.from_numpy(ids.astype(np.int32)).to(device)


def gpu_step(moe, args, cfg, forced=None):
    x, res, wr, w13, w2, dy = args
    # A training step starts from cleared gradients (optimizer.zero_grad(set_to_none=True));
    # without this, autograd would add each step's weight gradients into the last ones.
    for t in (wr, w13, w2):
        t.grad = None
    kwargs = dict(top_k=cfg["top_k"], routing_mode="topk_then_softmax",
                  compute_precision=cfg.get("precision", "fp8_block"))
    if forced is None:
        out, aux, counts, psum = moe(x, res, wr, w13, w2, **kwargs)
    else:
        from mlops_amd.routing import routing_override

        with routing_override([forced]):
            out, aux, counts, psum = moe(x, res, wr, w13, w2, **kwargs)
    torch.autograd.backward([out, aux], [dy, torch.full_like(aux, 0.01)])


def host_cores():
    """The cores this process may run on (its affinity set; os.cpu_count() can
    count cores of the machine that are not ours)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(cfg_name, sample_tokens=128, budget_s=20.0, max_iters=10, warmups=2,
                 threads=None):
    """The reference's native path (``oracle.native_moe``, the restatement of
    moe_reference.py:20-109: every expert on every token, masked, torch
    autograd, fp32 as the reference computes off the GPU) on a bounded sample of the benchmark's own workload: the
    same layer shape with ``sample_tokens`` tokens, on the host CPU. Median of
    up to ``max_iters`` fwd+bwd runs after 2 warmups, bounded by ``budget_s``;
    reported as tokens/s of that sample."""
    from oracle import moe_oracle as O

    threads = max(1, min(host_cores(), 16)) if threads is None else int(threads)
    torch.set_num_threads(threads)
    cfg = dict(CONFIGS[cfg_name], tokens=int(sample_tokens))
    x, res, wr, w13, w2, dy = make_inputs(cfg, torch.device("cpu"))
    x.requires_grad_(True)
    wr.requires_grad_(True)
    lora = None
    if "lora_rank" in cfg:
        # Frozen base, trainable factors (the LoRA workload's gradients).
        e, r, h, i = cfg["experts"], cfg["lora_rank"], cfg["hidden"], cfg["inter"]
        g = torch.Generator().manual_seed(1)
        lora = (*[(torch.randn(*shape, generator=g) * std).requires_grad_(True)
                  for shape, std in (((e, r, h), 0.01), ((e, 2 * i, r), 0.1),
                                     ((e, r, i), 0.01), ((e, h, r), 0.1))], 2.0)
        w13, w2 = list(w13), list(w2)
    else:
        # Per-expert leaf weights (same values): the gradients are the same, without
        # autograd materializing a full [E, ...] gradient for every expert's slice.
        w13 = [w.clone().requires_grad_(True) for w in w13]
        w2 = [w.clone().requires_grad_(True) for w in w2]

    def step():
        out, aux, counts, psum = O.native_moe(x, res, wr, w13, w2, top_k=cfg["top_k"],
                                              routing_mode="topk_then_softmax",
                                              compute_dtype=torch.float32, lora=lora)
        torch.autograd.backward([out, aux], [dy, torch.full_like(aux, 0.01)])

    for _ in range(warmups):
        step()
    times = []
    start = time.perf_counter()
    while len(times) < max_iters and time.perf_counter() - start < budget_s:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    median = statistics.median(times)
    return {
        "value": cfg["tokens"] / median,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"{cfg_name} layer shape (H={cfg['hidden']}, I={cfg['inter']}, E={cfg['experts']}, "
                   f"k={cfg['top_k']}{', LoRA r=' + str(cfg['lora_rank']) + ' on a frozen base' if lora else ''}) "
                   f"with {cfg['tokens']} tokens: reference native path (dense "
                   f"per-expert loop, masked, per-expert weight leaves) fwd+bwd in fp32 via torch autograd, median of "
                   f"{len(times)} runs after {warmups} warmups, {threads} threads"),
        "ms_per_step": median * 1e3,
    }


# Sources whose code decides the GEMMs' memory traffic: the traffic
# figures in profiles/traffic.json hold the digest of these files as they were
# when the counters were read, and are reported only while it still matches.
TRAFFIC_SOURCES = ("mlops_amd/csrc/gemm_v2.hip", "mlops_amd/csrc/gemm_pipe.h",
                   "mlops_amd/csrc/gemm_wgrad.hip")


def source_digest():
    import hashlib

    h = hashlib.sha256()
    for rel in TRAFFIC_SOURCES:
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def load_traffic(kernel):
    """HBM bytes per launch of ``kernel`` from the committed counter summary,
    or None when the summary is missing or was taken on other sources."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        data = json.load(f)
    if data.get("_sources") != source_digest():
        return None
    return data.get(kernel)


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--config", default="qwen3_30b_a3b", choices=sorted(CONFIGS))
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--cpu-sample-tokens", type=int, default=128)
    parser.add_argument("--implementation", default=None,
                        help="force a registered moe implementation (default: the registry's "
                             "choice, mi355x.moe.block_fp8), e.g. mi355x.moe.composed")
    parser.add_argument("--calibration-copy-mib", type=int, default=0,
                        help="after the timed steps, run one device copy of this many MiB "
                             "(the known-size kernel that calibrates rocprofv3 byte counters)")
    parser.add_argument("--calibration-read-mib", type=int, default=0,
                        help="after the timed steps, run one read-only reduction over this many "
                             "MiB (calibrates rocprofv3 FETCH_SIZE)")
    parser.add_argument("--vendor-gemm", action="store_true",
                        help="instead of the benchmark line, time the layer's four GEMM shapes "
                             "as dense problems through hipBLASLt and this package's kernels")
    args = parser.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; --gpus must be 1 "
                          "(multi-GPU sharding is a design note only)"}))
        sys.exit(2)

    import mlops_amd
    from mlops_amd import kernels

    cfg = CONFIGS[args.config]
    if args.vendor_gemm:
        vendor_gemm_main(args, cfg)
        return
    if cfg.get("gemm_only"):
        gemm_main(args, cfg)
        return
    device = torch.device("cuda", 0)
    lora = "lora_rank" in cfg
    if lora:
        inputs = make_lora_inputs(cfg, device)
        inputs[0].requires_grad_(True)
        inputs[2].requires_grad_(True)
        step = lambda: lora_step(inputs, cfg)
    else:
        inputs = make_inputs(cfg, device)
        _, _, wr, w13, w2, _ = inputs
        for t in (wr, w13, w2):
            t.requires_grad_(True)
        forced = zipf_ids(cfg, device) if "zipf" in cfg else None
        step = lambda: gpu_step(mlops_amd.moe, inputs, cfg, forced)
    if args.implementation is not None:
        from mlops_amd.dispatch import set_implementations

        set_implementations({"moe": args.implementation})

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # The ~270K Python objects alive by now (torch, the model inputs) move to
    # the collector's permanent generation: a full collection would otherwise
    # rescan them all, ~50 ms with the host thread (and so the GPU queue)
    # stalled, once every few dozen steps. Nothing of a step is skipped.
    gc.collect()
    gc.freeze()

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    # Per-kernel durations come from a second pass of the same K steps with a
    # pair of HIP events around every launch, on the launch's stream, so that
    # no marker sits inside the pass that gives `value`.
    timer = kernels.LaunchTimer()
    kernels.set_launch_timer(timer)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    instrumented = time.perf_counter() - t1
    kernels.set_launch_timer(None)
    summary = timer.summary()

    ms_per_step = elapsed / args.steps * 1e3
    tokens_per_s = cfg["tokens"] * args.steps / elapsed
    a = cfg["tokens"] * cfg["top_k"]
    # fwd + input gradients + weight gradients; a frozen base has no weight
    # gradients (the rank-r LoRA products add under 1%, not counted).
    layer_flops = (12 if lora else 18) * a * cfg["hidden"] * cfg["inter"]

    gemm_kernel = "gemm_fp8_rowwise" if cfg.get("precision") == "fp8_current" else "gemm_fp8_block"
    gemm = summary.get(gemm_kernel, {})
    achieved = gemm["flops"] / (gemm["ms_total"] * 1e-3) / 1e12 if gemm else None
    per_kernel = {}
    for name, entry in summary.items():
        secs = entry["ms_total"] * 1e-3
        item = {"launches_per_step": entry["launches"] / args.steps, "ms_avg": entry["ms_avg"]}
        if entry["flops"]:
            item["tflops"] = entry["flops"] / secs / 1e12
            item["frac_fp8_peak"] = item["tflops"] / FP8_PEAK_TFLOPS
        if entry["bytes"] and not entry["flops"]:
            item["gbs"] = entry["bytes"] / secs / 1e9
            item["frac_hbm_peak"] = item["gbs"] / HBM_PEAK_GBS
        per_kernel[name] = item
    all_gemm_ms = sum(summary[n]["ms_total"] for n in summary if n.startswith("gemm"))
    all_gemm_flops = sum(summary[n]["flops"] for n in summary if n.startswith("gemm"))

    result = {
        "metric": "MoE layer fwd+bwd tokens/s and grouped-GEMM fp8 TFLOP/s (% MFMA peak), 1 GPU",
        "value": tokens_per_s,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "ms_per_step_with_kernel_events": instrumented / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (block-scaled) GEMMs, fp32 accumulate, bf16 activations",
        "data": (f"synthetic (N(0,1) activations, N(0,{cfg.get('weight_std', 0.02)}) bf16 master "
                 "weights, random init"
                 + (f", expert of each slot drawn Zipf({cfg['zipf']}))" if "zipf" in cfg else ")")),
        "config": {
            "workload": f"{args.config} MoE layer fwd+bwd, block-FP8",
            **cfg,
            **({"implementation": args.implementation} if args.implementation else {}),
            "routing_mode": "topk_then_softmax",
            "weights": ("frozen block-FP8 base (128x128 blocks), rank-16 bf16 LoRA factors, "
                        "logits +2 on expert 0" if lora else
                        "bf16 masters quantized per call (one descale per row, both "
                        "orientations)" if cfg.get("precision") == "fp8_current" else
                        "bf16 masters quantized per call (128x128 blocks)"),
        },
        "layer_tflops": layer_flops * args.steps / elapsed / 1e12,
        "gemm_tflops_all": all_gemm_flops / (all_gemm_ms * 1e-3) / 1e12 if all_gemm_ms else None,
        "roofline": {
            "kernel": f"mi355x_{gemm_kernel} (grouped fwd/dgrad GEMM)",
            "bound": "mfma",
            "achieved": achieved,
            "peak": FP8_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / FP8_PEAK_TFLOPS if achieved else None,
            "traffic": load_traffic(gemm_kernel),
        },
        "kernels": per_kernel,
    }
    if args.calibration_read_mib > 0:
        # A read-only kernel of known size: torch's sum of n bytes (the output
        # is 4 bytes), for the FETCH_SIZE calibration of rocprofv3 runs.
        n = args.calibration_read_mib << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=device)
        torch.cuda.synchronize()
        total = src.sum()
        torch.cuda.synchronize()
        result["calibration_read_bytes"] = n
        del src, total
    if args.calibration_copy_mib > 0:
        n = args.calibration_copy_mib << 20
        src = torch.empty(n, dtype=torch.uint8, device=device).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = n
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args.config, args.cpu_sample_tokens)
        # BASELINE's own CPU case: config 1 (T=256, H=512, I=1024, E=8, k=2) on
        # every core this process has, 3 warmups, median of 20.
        result["cpu_baseline_config1"] = cpu_baseline(
            "config1", CONFIGS["config1"]["tokens"], budget_s=120.0, max_iters=20, warmups=3,
            threads=host_cores())
    print(json.dumps(result))


if __name__ == "__main__":
    main()
