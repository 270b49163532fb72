"""Benchmark: one MuonAdamW.step() on MI355X (gfx950).

Headline workload: a full step over the
Llama-3-8B-shaped parameter set (fp32 params/grads; 224 Muon matrices,
67 AdamW tensors; ns_steps = 5) with synthetic N(0, 0.02) weights and
N(0, 1e-3) gradients already resident in HBM.  `value` is milliseconds per
step (lower is better).  Extras on the same JSON line:

* gpt2   : full step, GPT-2-124M-shaped set (config 4), ms per step
* adamw  : AdamW-only step on config 2 (256 tensors, 2**26 elements), HBM GB/s with the
           memory-side cache flushed before each step
* ns     : Muon-only step on the config 3 matrices, NS TFLOP/s and % of peak over the step's device time

`roofline` describes the dominant kernel of the headline step (the one with
the largest total device time), from per-dispatch HIP events recorded by the
library over the timed steps.  `cpu_baseline` times this build's
PyTorchMuonAdamW (the reference's torch.optim wrapper, restated) on the host
CPU over a bounded sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extras]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT / "triton-muonadamw_amd"), str(ROOT), str(ROOT / "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MuonAdamW step ms (GPT-2-124M, Llama-8B shapes); AdamW HBM GB/s; NS MFMA %"
PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 flop/clk)
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
MODE_NUM = {"gram": 0, "poly": 1, "update": 2, "apply": 3}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def kernel_label(name: str, variant: int) -> str:
    """Demangled template name of a GEMM launch as rocprofv3 reports it."""
    if name.startswith("ns_gemm_kernel:"):
        mode = name.split(":")[1]
        return f"ns_gemm_kernel<{variant // 2}, {MODE_NUM[mode]}, {'true' if variant % 2 else 'false'}>"
    return name


def traffic_bytes(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (profiles/hbm_traffic_llama8b.txt, scaled by a copy kernel of known size); None if absent."""
    path = ROOT / "profiles" / "hbm_traffic_llama8b.txt"
    try:
        text = path.read_text()
    except OSError:
        return None
    for line in text.splitlines():
        if line.startswith("kernel="):
            fields = dict(kv.split("=", 1) for kv in line.split("; "))
            if fields.get("kernel") == kernel:
                return float(fields["bytes_per_launch"])
    return None


def make_params(layout, dev, seed: int):
    """Parameters (N(0,0.02)) with gradients (N(0,1e-3)), generated on the device from a seeded generator."""
    import torch

    gen = torch.Generator(device=dev).manual_seed(seed)
    named = []
    for name, shape, branch in layout:
        p = torch.nn.Parameter(torch.empty(shape, device=dev).normal_(0.0, 0.02, generator=gen))
        p.grad = torch.empty(shape, device=dev).normal_(0.0, 1e-3, generator=gen)
        named.append((name, p, branch))
    return named


def split(named):
    return {"adam": [p for _, p, b in named if b == "adam"], "muon": [p for _, p, b in named if b == "muon"]}


def configs():
    from triton_muon_adamw import AdamConfig, MuonConfig

    mc = MuonConfig(lr=1e-3, beta=0.95, eps=1e-7, weight_decay=0.1, coeffs=(3.4445, -4.7750, 2.0315),
                    nesterov=True, ns_steps=5, adjust_lr_fn="original")
    ac = AdamConfig(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    return mc, ac


def time_steps(opt, steps: int, warmup: int, profile: bool, between=None):
    """Warm up, then time exactly `steps` steps between device synchronisations.

    `between` (optional) runs before every step, inside the timed region: the
    per-kernel records (HIP events per dispatch) exclude it, the step time
    does not.
    """
    import torch

    from triton_muon_adamw import _lib

    for _ in range(warmup):
        if between is not None:
            between()
        opt.step()
    torch.cuda.synchronize()
    if profile:
        _lib.prof_start()
    t0 = time.perf_counter()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        if between is not None:
            between()
        opt.step()
    ev1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    recs = []
    if profile:
        _lib.prof_stop()
        recs = _lib.prof_collect()
    return ev0.elapsed_time(ev1) / steps, wall, recs


def summarize_kernels(recs):
    agg = {}
    for r in recs:
        key = kernel_label(r["kernel"], r["variant"])
        a = agg.setdefault(key, {"launches": 0, "ms": 0.0, "flops": 0.0, "bytes": 0.0})
        a["launches"] += 1
        a["ms"] += r["ms"]
        a["flops"] += r["flops"]
        a["bytes"] += r["bytes"]
    return agg


def bench_full_step(layout, dev, steps, warmup, seed, label):
    import torch

    from triton_muon_adamw import MuonAdamW

    mc, ac = configs()
    named = make_params(layout, dev, seed)
    opt = MuonAdamW(split(named), muon_config=mc, adam_config=ac, parameter_split="explicit")
    log(f"[{label}] {sum(p.numel() for _, p, _ in named):,} params; warmup {warmup}, timed {steps}")
    ms, wall, recs = time_steps(opt, steps, warmup, profile=True)
    agg = summarize_kernels(recs)
    note = " (shape classes concurrent: kernel times below overlap)" if opt.muon._concurrent else ""
    log(f"[{label}] {ms:.3f} ms/step (device events), {wall:.3f} ms/step (host wall){note}")
    for k, a in sorted(agg.items(), key=lambda kv: -kv[1]["ms"]):
        tf = a["flops"] / (a["ms"] * 1e-3) / 1e12 if a["flops"] else 0.0
        log(f"    {k:42s} {a['launches']:4d} launches {a['ms'] / steps:9.3f} ms/step  {tf:8.1f} TFLOP/s")
    del opt, named
    torch.cuda.empty_cache()
    return ms, agg


def bench_adamw_c2(dev, steps, warmup):
    import torch

    from helpers import c2_sizes
    from triton_muon_adamw.adamw import HipAdamW

    sizes = c2_sizes()
    gen = torch.Generator(device=dev).manual_seed(0)
    params = []
    for s in sizes:
        p = torch.nn.Parameter(torch.empty(s, device=dev).normal_(0.0, 0.02, generator=gen))
        p.grad = torch.empty(s, device=dev).normal_(0.0, 1e-3, generator=gen)
        params.append(p)
    opt = HipAdamW(params, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8)
    for p in params:
        opt.m[p].normal_(0.0, 1e-4, generator=gen)
        opt.v[p].normal_(0.0, 1e-6, generator=gen).abs_()
    opt.step_num = 9
    # A 512 MB write before every step evicts the 256 MB memory-side cache, so
    # the kernel's bandwidth is the HBM's (without it: about +1 point).
    flush = torch.empty(1 << 27, device=dev)
    ms, wall, recs = time_steps(opt, steps, warmup, profile=True, between=lambda: flush.fill_(0.0))
    kern = [r for r in recs if r["kernel"] == "adamw_mt_kernel"]
    kms = sum(r["ms"] for r in kern) / len(kern)
    nbytes = 28.0 * sum(sizes)
    gbs = nbytes / (kms * 1e-3) / 1e9
    log(f"[adamw c2] {len(sizes)} tensors, {sum(sizes):,} elements (cache flushed before each step): "
        f"step incl. flush {ms:.4f} ms, kernel {kms:.4f} ms "
        f"-> {gbs:.0f} GB/s ({100 * gbs / PEAK_HBM_GBS:.1f}% of 8 TB/s)")
    del opt, params, flush
    torch.cuda.empty_cache()
    return {"kernel_ms": round(kms, 4), "GB/s": round(gbs, 1),
            "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes_per_step": nbytes}


def bench_ns_c3(dev, steps, warmup):
    import torch

    from helpers import C3_SHAPES, ns_flops
    from triton_muon_adamw.muon import HipMuon

    mc, _ = configs()
    gen = torch.Generator(device=dev).manual_seed(1)
    params = []
    for s in C3_SHAPES:
        p = torch.nn.Parameter(torch.empty(s, device=dev).normal_(0.0, 0.02, generator=gen))
        p.grad = torch.empty(s, device=dev).normal_(0.0, 1.0, generator=gen)
        params.append(p)
    opt = HipMuon(params, lr=mc.lr, weight_decay=mc.weight_decay, coeffs=mc.coeffs, nesterov=True, beta=0.95,
                  ns_steps=5, eps=mc.eps)
    for p in params:
        opt.momentum[p].normal_(0.0, 1e-3, generator=gen)
    ms, wall, recs = time_steps(opt, steps, warmup, profile=False)
    # The four shape classes of this small step run concurrently on side
    # streams, so kernel durations overlap: the rate is taken over the whole
    # step's device time (prep, norm and scale included), a lower bound on the
    # GEMMs' own rate.
    flops = sum(ns_flops(s) for s in C3_SHAPES)
    tf = flops / (ms * 1e-3) / 1e12
    log(f"[ns c3] step {ms:.3f} ms ({'concurrent' if opt._concurrent else 'in order'} shape classes) -> "
        f"{tf:.1f} TFLOP/s of NS work over the whole step ({100 * tf / PEAK_BF16_TFLOPS:.1f}% of bf16 peak)")
    del opt, params
    torch.cuda.empty_cache()
    return {"step_ms": round(ms, 4), "TFLOP/s_over_step": round(tf, 1),
            "mfma_frac_over_step": round(tf / PEAK_BF16_TFLOPS, 4), "ns_flops": flops}


def cpu_baseline(layout, seed: int = 0, budget_s: float = 30.0):
    """PyTorchMuonAdamW on host CPU tensors over a bounded sample of the Llama-8B step.

    Sample: one decoder layer's seven Muon matrices plus 1/32 of the AdamW
    elements (the embedding and LM head cut to 1/32 of their rows, and two
    norm vectors); the step time is scaled by 32 (the layer count), labelled
    extrapolated.
    """
    import torch

    from triton_muon_adamw import PyTorchMuonAdamW

    mc, ac = configs()
    layer = [(n, s, b) for n, s, b in layout if n.startswith("l0.")]
    adam = [(n, (s[0] // 32, s[1]), b) for n, s, b in layout if n in ("embed", "lm_head")]
    sample = layer + adam
    gen = torch.Generator().manual_seed(seed)
    params = {"adam": [], "muon": []}
    for _, shape, b in sample:
        p = torch.nn.Parameter(torch.randn(shape, generator=gen) * 0.02)
        p.grad = torch.randn(shape, generator=gen) * 1e-3
        params[b].append(p)
    opt = PyTorchMuonAdamW(params, muon_config=mc, adam_config=ac, parameter_split="explicit")
    t0 = time.perf_counter()
    opt.step()  # warm-up
    first = time.perf_counter() - t0
    log(f"[cpu baseline] warm-up step {first:.1f} s on {torch.get_num_threads()} threads")
    times = []
    n_timed = max(1, min(3, int(budget_s / max(first, 1e-3)) - 1))
    for i in range(n_timed):
        t0 = time.perf_counter()
        opt.step()
        times.append(time.perf_counter() - t0)
        log(f"[cpu baseline] step {i + 1}/{n_timed}: {times[-1]:.2f} s")
    sample_ms = statistics.median(times) * 1e3
    n_adam = sum(math.prod(s) for _, s, b in sample if b == "adam")
    return {
        "value": round(sample_ms * 32, 1),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"PyTorchMuonAdamW (fused torch AdamW + torch Muon) on CPU: Llama-8B layer 0 "
                   f"(7 Muon matrices) + {n_adam:,} AdamW elements (1/32 of the set); median of {n_timed} "
                   f"step(s) = {sample_ms:.0f} ms, x32 layers = extrapolated full step"),
        "os_cpu_count": os.cpu_count(),
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extras", action="store_true", help="only the headline Llama-8B step")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--calib-copy", action="store_true",
                    help="only copy 1 GiB three times (torch copy_): the known-size kernel that scales the "
                         "FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc run")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        log("bench.py measures one GPU: this build has no multi-GPU path (collectives, sharding). "
            "Run it with --gpus 1.")
        sys.exit(2)

    import torch

    from helpers import gpt2_layout, llama8b_layout

    dev = torch.device("cuda:0")
    log(f"device: {torch.cuda.get_device_name(dev)}; torch {torch.__version__}")
    if args.calib_copy:
        x = torch.empty(1 << 28, device=dev).normal_()
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        torch.cuda.synchronize()
        print(json.dumps({"calib_copy_bytes_each_way": x.numel() * 4, "copies": 3}), flush=True)
        return
    layout = llama8b_layout()
    ms, agg = bench_full_step(layout, dev, args.steps, args.warmup, args.seed, "llama8b")
    dom_name, dom = max(agg.items(), key=lambda kv: kv[1]["ms"])
    achieved = dom["flops"] / (dom["ms"] * 1e-3) / 1e12
    roofline = {
        "bound": "mfma",
        "achieved": round(achieved, 1),
        "peak": PEAK_BF16_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
        "traffic": traffic_bytes(dom_name),
        "kernel": dom_name,
        "avg_launch_ms": round(dom["ms"] / dom["launches"], 4),
        "launches": dom["launches"],
        "share_of_step": round(dom["ms"] / args.steps / ms, 3),
    }
    ns_all = [a for k, a in agg.items() if k.startswith("ns_gemm_kernel")]
    ns_ms = sum(a["ms"] for a in ns_all) / args.steps
    ns_flops = sum(a["flops"] for a in ns_all) / args.steps
    extras = {"llama8b": {"ns_gemm_ms_per_step": round(ns_ms, 3),
                          "ns_TFLOP/s": round(ns_flops / (ns_ms * 1e-3) / 1e12, 1),
                          "ns_mfma_frac": round(ns_flops / (ns_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}}
    if not args.no_extras:
        g_ms, _ = bench_full_step(gpt2_layout(), dev, max(args.steps, 20), max(args.warmup, 5), args.seed, "gpt2")
        extras["gpt2_step_ms"] = round(g_ms, 4)
        extras["adamw_c2"] = bench_adamw_c2(dev, max(args.steps, 20), max(args.warmup, 3))
        extras["ns_c3"] = bench_ns_c3(dev, args.steps, args.warmup)
    cpu = None
    if not args.no_cpu:
        log("[cpu baseline] PyTorchMuonAdamW on host CPU (bounded sample) ...")
        cpu = cpu_baseline(layout)
        log(f"[cpu baseline] {cpu['value']} ms extrapolated; {cpu['sample']}")
    line = {
        "metric": METRIC,
        "value": round(ms, 3),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) params, N(0,1e-3) grads, generated on the device)",
        "config": {"workload": "MuonAdamW.step, Llama-3-8B-shaped fp32 parameter set (config 5)",
                   "params": 8030261248, "muon_matrices": 224, "adamw_tensors": 67, "ns_steps": 5,
                   "arithmetic": "AdamW fp32; Newton-Schulz bf16 MFMA with fp32 accumulate"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
