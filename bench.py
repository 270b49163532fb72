"""Benchmark: one MuonAdamW.step() on MI355X (gfx950).

Headline workload: a full step over the
Llama-3-8B-shaped parameter set (fp32 params/grads; 224 Muon matrices,
67 AdamW tensors; ns_steps = 5) with synthetic N(0, 0.02) weights and
N(0, 1e-3) gradients already resident in HBM.  `value` is milliseconds per
step (lower is better), timed with the library's per-dispatch profiler off.
A second pass over the same steps with the profiler on (an event pair bound
to every dispatch) gives the per-kernel table and `roofline`.  Extras on the
same JSON line:

* gpt2   : full step, GPT-2-124M-shaped set (config 4), ms per step; a
           profiled pass with the shape classes in order gives per-kernel rates
* adamw  : AdamW-only step on config 2 (256 tensors, 2**26 elements), HBM GB/s with the
           memory-side cache flushed before each step
* ns     : Muon-only step on the config 3 matrices, NS TFLOP/s and % of peak over the step's device time
* vs_torch_gpu : the reference's own comparison on this GPU (event-timed step
           loops as in its benchmark scripts): this build against
           PyTorchMuonAdamW (eager and torch.compile'd) / fused torch AdamW on
           the same parameters
* peak_mem : device memory each optimizer (this build, PyTorchMuonAdamW) adds
           to the resident GPT-2 and Llama-8B parameter sets
* c1_step_ms : config 1 (toy MLP) step on the GPU

`cpu_baseline.configs` times configs 1-4 in full on the same host cores.

`roofline` describes the dominant kernel of the headline step (the one with
the largest total device time).  `cpu_baseline` times this build's
PyTorchMuonAdamW (the reference's torch.optim wrapper, restated) on the host
CPU over a bounded sample of the same workload: the GPU run's own layer-0
values, copied to the host before the first step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extras]
       (single-workload modes for profiling: --calib-copy, --adamw-set c2|llama8b, --muon-group BxRxC,
       --gpt2-in-order)
"""

from __future__ import annotations

import argparse
import json
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
        flags = ["true" if (variant >> b) & 1 else "false" for b in range(3)]  # k-blocked, k-major, lower A
        tile = variant // 8  # 128, 256, or 192 for the 128 x 192 update tile
        bm, bn = (128, 192) if tile == 192 else (tile, tile)
        return f"ns_gemm_kernel<{bm}, {MODE_NUM[mode]}, {', '.join(flags)}, {bn}>"
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


def time_steps(opt, steps: int, warmup: int, profile: bool = False, between=None):
    """Warm up, then time exactly `steps` steps between device synchronisations.

    With `profile`, the library's per-dispatch profiler records an event pair
    around every kernel launch of the timed steps (returned as records); the
    step time of such a pass includes that instrumentation and is not used as
    `value`.  `between` (optional) runs before every step, inside the timed
    region: the per-kernel records exclude it, the step time does not.
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


def event_loop_ms(step_fn, warmup: int, iterations: int, repeats: int = 1) -> float:
    """The reference's timing loop (muon_adamw_benchmark.py:99-114,
    adam_benchmark.py:75-95): warm-up calls, a synchronisation, then CUDA/HIP
    events around `iterations` calls; the mean over `repeats` such loops."""
    import torch

    total = 0.0
    for _ in range(repeats):
        for _ in range(warmup):
            step_fn()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(iterations):
            step_fn()
        end.record()
        torch.cuda.synchronize()
        total += start.elapsed_time(end) / iterations
    return total / repeats


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


def log_kernels(label, agg, steps):
    for k, a in sorted(agg.items(), key=lambda kv: -kv[1]["ms"]):
        tf = a["flops"] / (a["ms"] * 1e-3) / 1e12 if a["flops"] else 0.0
        log(f"    {k:42s} {a['launches']:4d} launches {a['ms'] / steps:9.3f} ms/step  {tf:8.1f} TFLOP/s")


def optimizer_memory(make_opt, dev, label):
    """Device memory an optimizer adds to a resident parameter set (the
    reference benchmarks print torch.cuda.max_memory_allocated,
    muon_adamw_benchmark.py:149-151): `held_gb`, what it keeps between steps
    (state, workspace), measured after its first step; `peak_gb`, the most
    allocated at once during a later step, both above the parameters and
    gradients."""
    import torch

    torch.cuda.synchronize(dev)
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated(dev)
    opt = make_opt()
    opt.step()  # the first step allocates lazily created state and workspace
    torch.cuda.synchronize(dev)
    held = torch.cuda.memory_allocated(dev) - base
    torch.cuda.reset_peak_memory_stats(dev)
    opt.step()
    torch.cuda.synchronize(dev)
    peak = torch.cuda.max_memory_allocated(dev) - base
    out = {"held_gb": round(held / 1e9, 3), "peak_gb": round(peak / 1e9, 3)}
    ws = getattr(getattr(opt, "muon", None), "_ws", None)
    if isinstance(ws, dict):
        out["muon_workspace_gb"] = round(sum(w.numel() for w in ws.values()) / 1e9, 3)
    log(f"[{label}] memory: {out}")
    del opt
    torch.cuda.synchronize(dev)
    torch.cuda.empty_cache()
    return out


def bench_full_step(layout, dev, steps, warmup, seed, label, keep_host=None, profile_in_order=False,
                    memory=False):
    """Clean timed pass (`value`), then a profiled pass of the same length.

    `keep_host(named)` (optional) copies what the CPU baseline needs to host
    memory before the first step.  `profile_in_order`: the profiled pass runs
    the Muon shape classes in order (the clean pass keeps the library's
    choice), so that per-kernel durations do not overlap.  `memory`: after
    the passes, the device memory this build's optimizer and PyTorchMuonAdamW
    each add to the same resident parameters (optimizer_memory).
    """
    import torch

    from triton_muon_adamw import MuonAdamW, PyTorchMuonAdamW

    mc, ac = configs()
    named = make_params(layout, dev, seed)
    host = keep_host(named) if keep_host is not None else None
    opt = MuonAdamW(split(named), muon_config=mc, adam_config=ac, parameter_split="explicit")
    log(f"[{label}] {sum(p.numel() for _, p, _ in named):,} params; warmup {warmup}, timed {steps}")
    ms, wall, _ = time_steps(opt, steps, warmup)
    conc = opt.muon._concurrent
    log(f"[{label}] {ms:.3f} ms/step (device events, profiler off), {wall:.3f} ms/step (host wall)"
        f"{' (shape classes concurrent)' if conc else ''}")
    if profile_in_order and conc:
        opt.muon.concurrent_flops_limit = 0.0
        opt.muon._plan_key = None  # rebuild the launch plan with the classes in order
    pms, _, recs = time_steps(opt, steps, 1, profile=True)
    agg = summarize_kernels(recs)
    log(f"[{label}] profiled pass: {pms:.3f} ms/step with an event pair per dispatch"
        f"{' (shape classes in order)' if profile_in_order and conc else ''}")
    log_kernels(label, agg, steps)
    del opt
    mem = None
    if memory:
        mem = {"this_build": optimizer_memory(lambda: MuonAdamW(split(named), muon_config=mc, adam_config=ac,
                                                                 parameter_split="explicit"), dev, label),
               "torch_wrapper": optimizer_memory(lambda: PyTorchMuonAdamW(split(named), muon_config=mc,
                                                                          adam_config=ac,
                                                                          parameter_split="explicit"),
                                                 dev, label + " PyTorchMuonAdamW"),
               "params_and_grads_gb": round(sum(2 * p.numel() * p.element_size() for _, p, _ in named) / 1e9, 3)}
    del named
    torch.cuda.empty_cache()
    return ms, pms, agg, host, mem


def c1_layout():
    """Config 1: Linear(512, 2048) -> LayerNorm(2048) -> Linear(2048, 512), torch Linear layout."""
    return [("fc1.w", (2048, 512), "muon"), ("fc1.b", (2048,), "adam"), ("ln.w", (2048,), "adam"),
            ("ln.b", (2048,), "adam"), ("fc2.w", (512, 2048), "muon"), ("fc2.b", (512,), "adam")]


def bench_c1(dev, seed: int):
    """Config 1 (the toy MLP of BASELINE.json config 1) on the GPU: one MuonAdamW step, ms (event loop of
    20 steps after 5 warm-up)."""
    import torch

    from triton_muon_adamw import MuonAdamW

    mc, _ = configs()
    _, ac = configs()
    named = make_params(c1_layout(), dev, seed)
    opt = MuonAdamW(split(named), muon_config=mc, adam_config=ac, parameter_split="explicit")
    ms = event_loop_ms(opt.step, 5, 20)
    log(f"[c1] toy MLP step {ms:.4f} ms")
    del opt, named
    torch.cuda.empty_cache()
    return round(ms, 4)


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


def bench_kv_class(dev, steps, warmup):
    """The Llama-8B step's k/v shape class alone: 64 matrices of 1024 x 4096
    (32 layers x k_proj, v_proj) through HipMuon, as the full step groups
    them.  Reports the class's step time (prep, norm and scale included), the
    Newton-Schulz GEMM time from a profiled pass, and both rates over the
    symmetric-minimal NS work."""
    import torch

    from helpers import ns_flops
    from triton_muon_adamw.muon import HipMuon

    mc, _ = configs()
    gen = torch.Generator(device=dev).manual_seed(2)
    params = []
    for _ in range(64):
        p = torch.nn.Parameter(torch.empty((1024, 4096), device=dev).normal_(0.0, 0.02, generator=gen))
        p.grad = torch.empty((1024, 4096), device=dev).normal_(0.0, 1e-3, generator=gen)
        params.append(p)
    opt = HipMuon(params, lr=mc.lr, weight_decay=mc.weight_decay, coeffs=mc.coeffs, nesterov=True, beta=0.95,
                  ns_steps=5, eps=mc.eps)
    ms, _, _ = time_steps(opt, steps, warmup)
    _, _, recs = time_steps(opt, steps, 1, profile=True)
    ns_ms = sum(r["ms"] for r in recs if r["kernel"].startswith("ns_gemm")) / steps
    flops = 64 * ns_flops((1024, 4096))
    groups = [c.n for c in opt._calls]
    log(f"[kv class] 64 x 1024x4096 in groups {groups}: step {ms:.3f} ms, NS GEMMs {ns_ms:.3f} ms -> "
        f"{flops / (ns_ms * 1e-3) / 1e12:.1f} TFLOP/s over the GEMMs")
    del opt, params
    torch.cuda.empty_cache()
    return {"groups": groups, "step_ms": round(ms, 4), "ns_gemm_ms": round(ns_ms, 4), "ns_flops": flops,
            "TFLOP/s_over_step": round(flops / (ms * 1e-3) / 1e12, 1),
            "mfma_frac_over_step": round(flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "TFLOP/s_over_gemms": round(flops / (ns_ms * 1e-3) / 1e12, 1),
            "mfma_frac_over_gemms": round(flops / (ns_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)}


def llama_cpu_sample(named):
    """Host copies of the CPU baseline's sample, taken from the GPU run's own
    tensors before its first step: layer 0's seven Muon matrices and two
    norms, and 1/32 of the rows of the embedding and the LM head, each with its
    gradient.  Returns [(name, param, grad, branch)]."""
    out = []
    for name, p, b in named:
        if name.startswith("l0."):
            out.append((name, p.detach().cpu(), p.grad.cpu(), b))
        elif name in ("embed", "lm_head"):
            rows = p.shape[0] // 32
            out.append((name, p.detach()[:rows].cpu(), p.grad[:rows].cpu(), b))
    return out


def host_cpu_info():
    """lscpu model and core counts of the host the process runs on."""
    info = {"os_cpu_count": os.cpu_count()}
    try:
        info["cpus_available"] = len(os.sched_getaffinity(0))
    except AttributeError:
        info["cpus_available"] = os.cpu_count()
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        kv = {}
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                kv[k.strip()] = v.strip()
        info["model"] = kv.get("Model name")
        cores, sockets = kv.get("Core(s) per socket"), kv.get("Socket(s)")
        if cores and sockets and cores.isdigit() and sockets.isdigit():
            info["physical_cores"] = int(cores) * int(sockets)
        tpc = kv.get("Thread(s) per core")
        if tpc and tpc.isdigit():
            info["threads_per_core"] = int(tpc)
    except (OSError, ValueError):
        pass
    return info


def cpu_baseline(sample, budget_s: float = 30.0):
    """PyTorchMuonAdamW on host CPU tensors over a bounded sample of the Llama-8B step.

    Sample: one decoder layer's seven Muon matrices and two norms plus 1/32
    of the embedding and LM-head rows (the GPU run's own initial values and
    gradients); the step time is scaled by 32 (the layer count), labelled
    extrapolated.  Threads: the host's physical cores, capped by the CPUs this
    process may run on.
    """
    import torch

    from triton_muon_adamw import PyTorchMuonAdamW

    info = host_cpu_info()
    threads = min(info.get("physical_cores") or info["cpus_available"], info["cpus_available"])
    torch.set_num_threads(max(1, threads))
    mc, ac = configs()
    params = {"adam": [], "muon": []}
    for _, p0, g0, b in sample:
        p = torch.nn.Parameter(p0.clone())
        p.grad = g0.clone()
        params[b].append(p)
    opt = PyTorchMuonAdamW(params, muon_config=mc, adam_config=ac, parameter_split="explicit")
    t0 = time.perf_counter()
    opt.step()  # warm-up
    first = time.perf_counter() - t0
    log(f"[cpu baseline] warm-up step {first:.1f} s on {torch.get_num_threads()} threads ({info.get('model')})")
    times = []
    n_timed = max(1, min(3, int(budget_s / max(first, 1e-3)) - 1))
    for i in range(n_timed):
        t0 = time.perf_counter()
        opt.step()
        times.append(time.perf_counter() - t0)
        log(f"[cpu baseline] step {i + 1}/{n_timed}: {times[-1]:.2f} s")
    sample_ms = statistics.median(times) * 1e3
    n_adam = sum(p0.numel() for _, p0, _, b in sample if b == "adam")
    return {
        "value": round(sample_ms * 32, 1),
        "unit": "ms",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"PyTorchMuonAdamW (fused torch AdamW + torch Muon) on CPU over the GPU run's own initial "
                   f"layer-0 values: 7 Muon matrices + {n_adam:,} AdamW elements (layer 0's two norms and 1/32 of "
                   f"the embedding and LM-head rows); median of {n_timed} step(s) = {sample_ms:.0f} ms, "
                   f"x32 layers = extrapolated full step"),
        "cpu_model": info.get("model"),
        "physical_cores": info.get("physical_cores"),
        "threads_per_core": info.get("threads_per_core"),
        "cpus_available": info["cpus_available"],
        "os_cpu_count": info["os_cpu_count"],
    }


def cpu_baseline_configs(threads: int):
    """Configs 1-4 on the host CPU with the reference's torch.optim path, median of 3 timed steps after
    one warm-up step (config 3: of 2): config 1 (toy MLP) and config 4 (GPT-2 set) through
    PyTorchMuonAdamW, config 2 through fused torch.optim.AdamW (the reference's AdamW comparison,
    adam_benchmark.py:35-42), config 3 through torch.optim.Muon (muon_benchmark.py:33-34).  Values:
    seeded N(0, 0.02) parameters and N(0, 1e-3) gradients (config 3: N(0, 1)), drawn on the CPU."""
    import torch

    from helpers import C3_SHAPES, c2_sizes, gpt2_layout
    from triton_muon_adamw import PyTorchMuonAdamW

    torch.set_num_threads(max(1, threads))
    mc, ac = configs()
    gen = torch.Generator().manual_seed(0)

    def params(shapes, gstd=1e-3):
        out = []
        for s in shapes:
            p = torch.nn.Parameter(torch.randn(s, generator=gen) * 0.02)
            p.grad = torch.randn(s, generator=gen) * gstd
            out.append(p)
        return out

    def wrapper(layout):
        ps = params([s for _, s, _ in layout])
        d = {"adam": [p for p, (_, _, b) in zip(ps, layout) if b == "adam"],
             "muon": [p for p, (_, _, b) in zip(ps, layout) if b == "muon"]}
        return PyTorchMuonAdamW(d, muon_config=mc, adam_config=ac, parameter_split="explicit")

    cases = {
        "c1_toy_mlp": (lambda: wrapper(c1_layout()), 3),
        "c2_adamw": (lambda: torch.optim.AdamW(params([(n,) for n in c2_sizes()]), lr=ac.lr, betas=ac.betas,
                                               eps=ac.eps, weight_decay=ac.weight_decay, fused=True), 3),
        "c3_ns": (lambda: torch.optim.Muon(params(C3_SHAPES, gstd=1.0), lr=mc.lr, momentum=mc.beta,
                                           weight_decay=mc.weight_decay, nesterov=mc.nesterov,
                                           ns_coefficients=tuple(mc.coeffs), eps=mc.eps, ns_steps=mc.ns_steps), 2),
        "c4_gpt2": (lambda: wrapper(gpt2_layout()), 3),
    }
    out = {}
    for name, (make, n) in cases.items():
        opt = make()
        opt.step()  # warm-up (allocates the state)
        times = []
        for _ in range(n):
            t0 = time.perf_counter()
            opt.step()
            times.append(time.perf_counter() - t0)
        out[name] = {"ms": round(statistics.median(times) * 1e3, 2), "timed_steps": n}
        log(f"[cpu baseline] {name}: median {out[name]['ms']} ms of {n} steps")
        del opt
    return out


def bench_vs_torch_gpu(dev, seed: int = 0):
    """The reference's own comparison, on this GPU, with its event-timed loop.

    Each case builds two identical parameter sets with N(0, 1e-3) gradients
    (a backward pass does not change the optimizer's work) and times this
    build's optimizer and the torch.optim one it is compared with:

    * ref_hybrid_mlp: the reference's hybrid benchmark model
      (muon_adamw_benchmark.py:9-20,28-39,41-52; 2-D weights to Muon), this
      build's MuonAdamW against PyTorchMuonAdamW, eager and, as the reference
      times it, compiled by torch.compile (inductor); warm-up 50, 100 timed
      steps, mean of 5 loops (:99-126).  Published: 1.24-1.26x against the
      compiled step (the reference's README.md:48).
    * ref_muon_mlp: the reference's Muon benchmark model (five bias-free
      linear layers, muon_benchmark.py:14-24, all to Muon), HipMuon against
      torch.optim.Muon with the reference's settings (:33-35), eager and
      compiled; warm-up 50, 100 timed steps, mean of 5 loops (:66-92).
      Published: 1.33-1.35x eager, 1.27-1.30x compiled (the reference's README.md:46-47).
    * ref_adamw_mlp: the reference's AdamW benchmark model
      (adam_benchmark.py:14-25,33-42), HipAdamW against fused torch AdamW
      and against torch's default (foreach) AdamW; warm-up 100, 500 timed
      steps, mean of 10 loops (:75-108).  Published: 0.97-0.99x against the
      fused and 2.65-2.70x against the foreach step (the reference's README.md:44-45).
    * gpt2, llama_layer (layer 0 plus 1/32 of the embedding and LM head),
      c2_adamw: configurations 4, 5 and 2, shorter loops.
    """
    import torch
    import torch.nn as nn

    from helpers import c2_sizes, gpt2_layout, llama8b_layout
    from triton_muon_adamw import AdamConfig, MuonAdamW, MuonConfig, PyTorchMuonAdamW
    from triton_muon_adamw.adamw import HipAdamW

    gen = torch.Generator(device=dev).manual_seed(seed)

    def twin(shapes_branches):
        a, b = {"adam": [], "muon": []}, {"adam": [], "muon": []}
        for shape, br, init in shapes_branches:
            w = init(shape)
            g = torch.empty(shape, device=dev).normal_(0.0, 1e-3, generator=gen)
            for d in (a, b):
                p = nn.Parameter(w.clone())
                p.grad = g.clone()
                d[br].append(p)
        return a, b

    def normal(std):
        return lambda shape: torch.empty(shape, device=dev).normal_(0.0, std, generator=gen)

    def mlp_shapes(dims):
        out = []
        for i, (fi, fo) in enumerate(zip(dims[:-1], dims[1:])):
            out += [((fo, fi), "muon", normal(fi ** -0.5)), ((fo,), "adam", normal(fi ** -0.5))]
            if i < len(dims) - 2:
                out += [((fo,), "adam", lambda s: torch.ones(s, device=dev)),
                        ((fo,), "adam", lambda s: torch.zeros(s, device=dev))]
        return out

    def ratio(mine, theirs):
        return {"this_build_ms": round(mine, 4), "torch_ms": round(theirs, 4),
                "speedup": round(theirs / mine, 3)}

    out = {}
    # reference hybrid benchmark (its configs, muon_adamw_benchmark.py:28-39)
    mc_ref = MuonConfig(lr=1e-3, beta=0.95, eps=1e-7, weight_decay=0.1, coeffs=(3.445, -4.775, 2.0315),
                        nesterov=True, ns_steps=5, adjust_lr_fn="original")
    ac_ref = AdamConfig(lr=1e-3, betas=(0.9, 0.999), eps=1e-7, weight_decay=0.01)
    a, b = twin(mlp_shapes([1024, 2048, 4096, 4096, 1024]))
    mine = MuonAdamW(a, muon_config=mc_ref, adam_config=ac_ref, parameter_split="explicit")
    ref = PyTorchMuonAdamW(b, muon_config=mc_ref, adam_config=ac_ref, parameter_split="explicit")
    mine_ms = event_loop_ms(mine.step, 50, 100, 5)
    r = ratio(mine_ms, event_loop_ms(ref.step, 50, 100, 5))
    r["published_speedup"] = "1.24-1.26 (vs the torch.compile'd wrapper step)"
    # The reference's own comparison point: torch.compile(pytorch_optimizer.step)
    # (muon_adamw_benchmark.py:66,123), compiled here by inductor for this GPU.
    try:
        t0 = time.perf_counter()
        compiled = torch.compile(ref.step)
        compiled()
        torch.cuda.synchronize(dev)
        r["compile_s"] = round(time.perf_counter() - t0, 1)
        c_ms = event_loop_ms(compiled, 50, 100, 5)
        r["compiled_torch_ms"] = round(c_ms, 4)
        r["speedup_vs_compiled"] = round(c_ms / mine_ms, 3)
    except Exception as e:  # inductor is optional: record why the compiled point is missing
        r["compiled_torch_error"] = f"{type(e).__name__}: {str(e)[:200]}"
    out["ref_hybrid_mlp"] = r
    log(f"[vs torch gpu] reference hybrid MLP: {r}")
    del mine, ref, a, b
    # reference Muon benchmark (muon_benchmark.py:14-24,33-35)
    from triton_muon_adamw.muon import HipMuon

    dims = [1024, 2048, 4096, 4096, 4096, 1024]
    a, b = twin([((fo, fi), "muon", normal(fi ** -0.5)) for fi, fo in zip(dims[:-1], dims[1:])])
    mine = HipMuon(a["muon"], coeffs=(3.4445, -4.775, 2.0315), beta=0.95, lr=1e-3, weight_decay=0.1, ns_steps=5)
    ref = torch.optim.Muon(b["muon"], lr=1e-3, momentum=0.95, nesterov=True, ns_steps=5)
    mine_ms = event_loop_ms(mine.step, 50, 100, 5)
    r = ratio(mine_ms, event_loop_ms(ref.step, 50, 100, 5))
    r["published_speedup"] = "1.33-1.35 (vs torch.optim.Muon), 1.27-1.30 (vs its torch.compile'd step)"
    try:
        compiled = torch.compile(ref.step)
        compiled()
        torch.cuda.synchronize(dev)
        c_ms = event_loop_ms(compiled, 50, 100, 5)
        r["compiled_torch_ms"] = round(c_ms, 4)
        r["speedup_vs_compiled"] = round(c_ms / mine_ms, 3)
    except Exception as e:  # inductor is optional: record why the compiled point is missing
        r["compiled_torch_error"] = f"{type(e).__name__}: {str(e)[:200]}"
    out["ref_muon_mlp"] = r
    log(f"[vs torch gpu] reference Muon MLP: {r}")
    del mine, ref, a, b
    # reference AdamW benchmark (adam_benchmark.py:33-42)
    a, b = twin(mlp_shapes([1024, 4096, 4096, 4096, 1024]))
    pa, pb = a["adam"] + a["muon"], b["adam"] + b["muon"]
    mine = HipAdamW(pa, lr=1e-3, betas=(0.9, 0.999), weight_decay=1e-4, eps=1e-8)
    ref = torch.optim.AdamW(pb, lr=1e-3, betas=(0.9, 0.999), weight_decay=1e-4, eps=1e-8, fused=True)
    mine_ms = event_loop_ms(mine.step, 100, 500, 10)
    r = ratio(mine_ms, event_loop_ms(ref.step, 100, 500, 10))
    r["published_speedup"] = "0.97-0.99 (vs fused torch AdamW), 2.65-2.70 (vs foreach AdamW)"
    ref_fe = torch.optim.AdamW(pb, lr=1e-3, betas=(0.9, 0.999), weight_decay=1e-4, eps=1e-8, foreach=True)
    fe_ms = event_loop_ms(ref_fe.step, 100, 500, 10)
    r["foreach_torch_ms"] = round(fe_ms, 4)
    r["speedup_vs_foreach"] = round(fe_ms / mine_ms, 3)
    out["ref_adamw_mlp"] = r
    log(f"[vs torch gpu] reference AdamW MLP: {r}")
    del mine, ref, ref_fe, a, b, pa, pb
    # BASELINE.json configurations
    mc, ac = configs()
    for name, layout in (("gpt2", gpt2_layout()),
                         ("llama_layer", [(n, s, br) for n, s, br in llama8b_layout() if n.startswith("l0.")]
                          + [(n, (s[0] // 32, s[1]), br) for n, s, br in llama8b_layout()
                             if n in ("embed", "lm_head")])):
        a, b = twin([(s, br, normal(0.02)) for _, s, br in layout])
        mine = MuonAdamW(a, muon_config=mc, adam_config=ac, parameter_split="explicit")
        ref = PyTorchMuonAdamW(b, muon_config=mc, adam_config=ac, parameter_split="explicit")
        r = ratio(event_loop_ms(mine.step, 5, 20), event_loop_ms(ref.step, 5, 20))
        out[name] = r
        log(f"[vs torch gpu] {name}: {r}")
        del mine, ref, a, b
        torch.cuda.empty_cache()
    sizes = c2_sizes()
    a, b = twin([((s,), "adam", normal(0.02)) for s in sizes])
    mine = HipAdamW(a["adam"], lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8)
    ref = torch.optim.AdamW(b["adam"], lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8, fused=True)
    r = ratio(event_loop_ms(mine.step, 10, 50), event_loop_ms(ref.step, 10, 50))
    out["c2_adamw"] = r
    log(f"[vs torch gpu] c2 AdamW: {r}")
    del mine, ref, a, b
    torch.cuda.empty_cache()
    return out


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
    ap.add_argument("--adamw-set", choices=["c2", "llama8b"],
                    help="only the AdamW step on one tensor set (config 2, or the Llama-8B AdamW tensors: embedding, "
                         "LM head, 65 norms), 6 steps with the memory-side cache flushed before each: the workload of "
                         "the rocprofv3 memory-path counter runs")
    ap.add_argument("--muon-group", metavar="BxRxC",
                    help="only the Muon step of one launch group of B matrices R x C (N(0,0.02) parameters, "
                         "N(0,1e-3) gradients), --steps timed after --warmup: the workload of the per-kernel "
                         "counter runs on single shape classes")
    ap.add_argument("--gpt2-in-order", action="store_true",
                    help="only the GPT-2 (config 4) step with its Muon shape classes run in order (no side "
                         "streams), for a kernel trace whose per-kernel durations do not overlap")
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
    if args.adamw_set:
        from helpers import c2_sizes
        from triton_muon_adamw.adamw import HipAdamW

        sizes = c2_sizes() if args.adamw_set == "c2" else [
            int(torch.Size(s).numel()) for _, s, b in llama8b_layout() if b == "adam"]
        gen = torch.Generator(device=dev).manual_seed(args.seed)
        params = []
        for n in sizes:
            p = torch.nn.Parameter(torch.empty(n, device=dev).normal_(0.0, 0.02, generator=gen))
            p.grad = torch.empty(n, device=dev).normal_(0.0, 1e-3, generator=gen)
            params.append(p)
        opt = HipAdamW(params, lr=3e-4, betas=(0.9, 0.95), weight_decay=0.1, eps=1e-8)
        flush = torch.empty(1 << 27, device=dev)
        ms = []
        for _ in range(6):
            flush.fill_(0.0)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            opt.step()
            e1.record()
            torch.cuda.synchronize()
            ms.append(e0.elapsed_time(e1))
        gbs = 28.0 * sum(sizes) / (statistics.median(ms[1:]) * 1e-3) / 1e9
        print(json.dumps({"workload": f"AdamW step alone, {args.adamw_set} set", "elements": sum(sizes),
                          "tensors": len(sizes), "step_ms_median": round(statistics.median(ms[1:]), 4),
                          "GB/s": round(gbs, 1)}), flush=True)
        return
    if args.muon_group:
        from triton_muon_adamw.muon import HipMuon

        count, rows, cols = (int(v) for v in args.muon_group.split("x"))
        gen = torch.Generator(device=dev).manual_seed(args.seed)
        params = []
        for _ in range(count):
            p = torch.nn.Parameter(torch.empty((rows, cols), device=dev).normal_(0.0, 0.02, generator=gen))
            p.grad = torch.empty((rows, cols), device=dev).normal_(0.0, 1e-3, generator=gen)
            params.append(p)
        mc, _ = configs()
        opt = HipMuon(params, lr=mc.lr, weight_decay=mc.weight_decay, coeffs=mc.coeffs, nesterov=True, beta=0.95,
                      ns_steps=5, eps=mc.eps)
        ms, wall, _ = time_steps(opt, args.steps, args.warmup)
        print(json.dumps({"workload": f"Muon step of {count} x {rows}x{cols}", "groups": [c.n for c in opt._calls],
                          "ms_per_step": round(ms, 4), "steps": args.steps, "warmup": args.warmup}), flush=True)
        return
    if args.gpt2_in_order:
        from triton_muon_adamw import MuonAdamW

        mc, ac = configs()
        named = make_params(gpt2_layout(), dev, args.seed)
        opt = MuonAdamW(split(named), muon_config=mc, adam_config=ac, parameter_split="explicit")
        opt.muon.concurrent_flops_limit = 0.0
        ms, wall, _ = time_steps(opt, args.steps, args.warmup)
        print(json.dumps({"workload": "GPT-2 (config 4) MuonAdamW.step, Muon shape classes in order",
                          "ms_per_step": round(ms, 4), "steps": args.steps, "warmup": args.warmup,
                          "concurrent": opt.muon._concurrent}), flush=True)
        return
    layout = llama8b_layout()
    keep = None if args.no_cpu else llama_cpu_sample
    ms, pms, agg, sample, l_mem = bench_full_step(layout, dev, args.steps, args.warmup, args.seed, "llama8b",
                                                  keep_host=keep, memory=not args.no_extras)
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
        "share_of_step": round(dom["ms"] / args.steps / pms, 3),
        "source": "profiled pass (an event pair bound to each dispatch) over the same steps as `value`",
        "traffic_note": "FETCH_SIZE + WRITE_SIZE per launch averaged over the launch groups of one step "
                        "(unequal group sizes), from profiles/hbm_traffic_llama8b.txt",
    }
    ns_all = [a for k, a in agg.items() if k.startswith("ns_gemm_kernel")]
    ns_ms = sum(a["ms"] for a in ns_all) / args.steps
    ns_flops = sum(a["flops"] for a in ns_all) / args.steps
    per_kernel = {k: {"ms_per_step": round(a["ms"] / args.steps, 3), "launches_per_step": a["launches"] // args.steps,
                      **({"TFLOP/s": round(a["flops"] / (a["ms"] * 1e-3) / 1e12, 1)} if a["flops"] else {})}
                  for k, a in sorted(agg.items(), key=lambda kv: -kv[1]["ms"])}
    extras = {"llama8b": {"profiled_pass_ms": round(pms, 3),
                          "ns_gemm_ms_per_step": round(ns_ms, 3),
                          "ns_TFLOP/s": round(ns_flops / (ns_ms * 1e-3) / 1e12, 1),
                          "ns_mfma_frac": round(ns_flops / (ns_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                          "kernels": per_kernel}}
    if not args.no_extras:
        g_steps, g_warm = max(args.steps, 20), max(args.warmup, 5)
        g_ms, g_pms, g_agg, _, g_mem = bench_full_step(gpt2_layout(), dev, g_steps, g_warm, args.seed, "gpt2",
                                                       profile_in_order=True, memory=True)
        g_ns = [a for k, a in g_agg.items() if k.startswith("ns_gemm_kernel")]
        g_ns_ms = sum(a["ms"] for a in g_ns) / g_steps
        g_ns_fl = sum(a["flops"] for a in g_ns) / g_steps
        extras["gpt2_step_ms"] = round(g_ms, 4)
        extras["gpt2"] = {"step_ms": round(g_ms, 4),
                          "ns_TFLOP/s_over_step": round(g_ns_fl / (g_ms * 1e-3) / 1e12, 1),
                          "ns_mfma_frac_over_step": round(g_ns_fl / (g_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                          "in_order_profiled_ms": round(g_pms, 4),
                          "in_order_ns_gemm_ms": round(g_ns_ms, 4),
                          "kernels_in_order": {k: {"ms_per_step": round(a["ms"] / g_steps, 4),
                                                   **({"TFLOP/s": round(a["flops"] / (a["ms"] * 1e-3) / 1e12, 1)}
                                                      if a["flops"] else {})}
                                               for k, a in sorted(g_agg.items(), key=lambda kv: -kv[1]["ms"])}}
        extras["peak_mem"] = {
            "note": "device memory each optimizer adds to the resident fp32 parameters and gradients: held_gb "
                    "between steps (state, workspace), peak_gb at most during a step, both above the "
                    "parameters and gradients",
            "llama8b": l_mem, "gpt2": g_mem}
        extras["c1_step_ms"] = bench_c1(dev, args.seed)
        extras["adamw_c2"] = bench_adamw_c2(dev, max(args.steps, 20), max(args.warmup, 3))
        extras["ns_c3"] = bench_ns_c3(dev, args.steps, args.warmup)
        extras["llama_kv_class"] = bench_kv_class(dev, args.steps, args.warmup)
        extras["vs_torch_gpu"] = bench_vs_torch_gpu(dev, args.seed)
    cpu = None
    if not args.no_cpu:
        log("[cpu baseline] PyTorchMuonAdamW on host CPU (bounded sample) ...")
        cpu = cpu_baseline(sample)
        log(f"[cpu baseline] {cpu['value']} ms extrapolated; {cpu['sample']}")
        cpu["configs"] = cpu_baseline_configs(cpu["cores"])
        cpu["configs_note"] = ("configs 1-4 in full on the same host cores: median ms per step (the reference's "
                               "torch.optim path; config 2 fused AdamW, config 3 torch Muon)")
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
        "data": "synthetic (seeded N(0,0.02) params, N(0,1e-3) grads, generated on the device; the CPU "
                "baseline copies layer 0 of these to the host)",
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
