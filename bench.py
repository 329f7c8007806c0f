#!/usr/bin/env python3
"""Benchmark: batched soft-raster forward + MSE + backward on one MI355X.

One step = one drh_fused_loss_backward call (setup_records, then
fused_tile_kernel, whose last workgroups also sum the scenes' losses) over the
headline workload: B=16 scenes at 256x256,
T=128 triangles each, sigma=0.0015, synthetic seeded scenes (diffrast.synth)
and targets rendered from independently seeded scenes. Inputs and outputs
stay in HBM; the timed region is K steps between two synchronizations.

Printed (one JSON line on stdout): throughput in dense pixel-triangle
evaluations per second, ms per batch, the dominant kernel's roofline position
(fused_tile_kernel: its algorithmic FLOP per launch over its event-timed average
duration, against the FP32 vector peak; under "two_kernel_path" the same step
with forward_kernel and backward_kernel, DRH_UNFUSED=1, and their rooflines;
configurations that take the two kernels report them directly), the CPU
baseline (the C oracle, one thread per scene, on this host's cores), and under
"configs" the same measurements for every benchmark workload: c0 (B=1 64x64 T=32), c1 (B=16 128x128 T=128), c2 (the
headline), c3 (B=8 256x256 T=512 small triangles) and c4 (the 800-iteration
fit at 176x176, T=150, against the oracle's fit on one core).

The headline is measured first in the process, then every other GPU leg, then
the CPU legs. The GPU's clocks ramp up over ~18 ms of sustained load (the c2
step from ~111 to ~100 us), so with a few warm-up steps the headline runs in
that ramp; "sustained" reports the same step after 200 untimed steps beside it.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
    python bench.py --copy-calibration     # plain device copy, for PMC scaling
    python bench.py --crossover            # GPU vs this host's CPU over the reference's crossover cells
    python bench.py --config c3 --no-cpu-baseline --steps 20 --warmup 5   # one workload alone
    python bench.py --config c3 --after-headline ...   # the same, after 150 untimed headline steps
"""

from __future__ import annotations

import argparse
import contextlib
import gc
import json
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PKG = ROOT / "differentiable-rasterizer_amd"
for _p in (ROOT, PKG):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

import numpy as np  # noqa: E402

METRIC = "fwd+bwd ms/batch & pixel·tri/s, B=16 256² T=128; % FP32 VALU peak"
UNIT = "pixel·tri/s"
PEAK_FP32_TFLOPS = 157.3      # MI355X FP32 vector (AMD published); plain v_fma_f32 on VGPR
                              # operands issues at this rate too (~2 cycles per wave64 per SIMD)
SIGMA = 0.0015                # python/diffrast/torch_layer.py:73
# Algorithmic FLOP convention for this path (each + - * / sqrt exp min max
# compare counts 1; per-triangle invariants hoisted):
#   coverage evaluation 74 per box pair, once forward and once backward
#   forward composite 10 per contributing pair, backward chain 51
#   loss + dL/dpixel 15 per pixel
# forward_kernel: 74 box + 10 contrib + 15 pixel; backward_kernel: 74 box + 51 contrib
FLOP_FWD = (74, 10, 15)
FLOP_BWD = (74, 51, 0)
# parameter groups of the per-group gradient parity figures
GROUPS = {"vertices": slice(0, 6), "colours": slice(6, 9), "alpha": slice(9, 10)}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


@contextlib.contextmanager
def quiet_gc():
    """A timed region without the cyclic garbage collector, as timeit runs its
    loops: a full collection of this process (torch loaded) takes 30-45 ms and
    would otherwise land inside whichever loop crosses its allocation count.
    Nothing is collected on entry either: that would leave the GPU idle for as
    long right before loops whose clocks have just ramped up."""
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def box_cpu_share() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def make_inputs(torch, ctx, cfg, seed, dev):
    from diffrast import synth

    B, H, W, T = cfg["B"], cfg["H"], cfg["W"], cfg["T"]
    params = synth.batch(cfg["kind"], B, T, seed)
    tparams = synth.batch(cfg["kind"], B, T, seed, target_offset=1000)
    p = torch.from_numpy(params).to(dev)
    tp = torch.from_numpy(tparams).to(dev)
    bg = torch.zeros((B, 3), device=dev)
    targets = torch.empty((B, H, W, 3), device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    ctx.render_ptr(tp.data_ptr(), bg.data_ptr(), B, T, H, W, SIGMA, targets.data_ptr(), stream)
    torch.cuda.synchronize()
    return params, p, bg, targets


def time_fused(torch, ctx, cfg, p, bg, targets, steps, warmup, dev):
    """Wall ms per step over `steps` calls, synchronized on both sides."""
    B, H, W, T = cfg["B"], cfg["H"], cfg["W"], cfg["T"]
    losses = torch.empty((B,), device=dev)
    grads = torch.empty((B, T, 10), device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def step():
        ctx.fused_ptr(p.data_ptr(), bg.data_ptr(), targets.data_ptr(), B, T, H, W, SIGMA,
                      losses.data_ptr(), grads.data_ptr(), None, stream)

    with quiet_gc():
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / steps
    return ms, losses, grads


def fused_kernel_name(B, H, W, T, deterministic=False):
    """The kernel the library's fused gradient path takes for this shape: the
    segmented kernel for grids of at most 2048 8x8 tiles with 16 to 160
    triangles (runtime.h: use_segments), else the one-wave tile kernel (the
    four-wave block kernel with fixed-order sums)."""
    tiles = B * ((W + 15) // 16) * ((H + 15) // 16) * 4
    if 16 <= T <= 160 and tiles <= 2048:
        return "fused_seg_kernel" + (" (fixed order)" if deterministic else "")
    return "fused_kernel (fixed order)" if deterministic else "fused_tile_kernel"


def kernel_times(torch, ctx, cfg, p, bg, targets, steps, dev, two_kernels=False):
    """Event-timed average duration of each kernel of the step: setup_records, then
    either the fused kernel (and sum_losses where it runs: fused kernels that
    sum the losses themselves launch none), or (two_kernels: DRH_UNFUSED=1, and
    the paths that always take them) forward_kernel and backward_kernel."""
    if two_kernels:
        os.environ["DRH_UNFUSED"] = "1"
    ctx.timing(True)
    try:
        time_fused(torch, ctx, cfg, p, bg, targets, steps, 0, dev)
        t = ctx.read_timings()
    finally:
        ctx.timing(False)
        os.environ.pop("DRH_UNFUSED", None)
    ms = {f: t[f"{f}_ms"] / max(t[f"{f}_n"], 1) for f in ("setup", "raster", "backward", "reduce")}
    if t["backward_n"] == 0 and t["raster_n"] > 0:
        out = {"setup": ms["setup"], "fused": ms["raster"]}
        if t["reduce_n"] > 0:
            out["sum_losses"] = ms["reduce"]
        return out
    return {"setup": ms["setup"], "forward": ms["raster"], "backward": ms["backward"], "reduce": ms["reduce"]}


def pmc_profile(config):
    return ROOT / "profiles" / f"raster_kernels_{config}_pmc.md"


def traffic_from_profiles(kernel, config="c2"):
    """HBM bytes per launch of `kernel` at `config`, read from the committed PMC
    summary of that workload (a counter run of an earlier invocation, not this
    run's measurement), or None."""
    f = pmc_profile(config)
    if not f.exists():
        return None
    m = re.search(re.escape(kernel) + r" traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def timed_reps(fn, warmup=3, budget_s=0.4, min_reps=3, max_reps=50):
    """benches/raster.rs:22-40 protocol: `warmup` untimed runs, then timed runs until
    `budget_s` seconds and `min_reps` runs have passed; returns the per-run seconds."""
    for _ in range(warmup):
        fn()
    times = []
    with quiet_gc():
        while (sum(times) < budget_s or len(times) < min_reps) and len(times) < max_reps:
            t0 = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t0)
    return times


def cpu_baseline(cfg, params, targets_np, budget_s):
    """The oracle's backward_batch analogue on this host (grad.rs:192-207): one thread
    per scene as rayon's par_iter, capped by the cores this process may use (16 per
    GPU on a shared box, whatever the machine's total); and one item on one thread."""
    from oracle import oracle

    B = cfg["B"]
    threads = max(1, min(B, box_cpu_share(), 16))
    counts = oracle.Counts()
    losses, grads = oracle.loss_backward_batch(params, targets_np, SIGMA, nthreads=threads, counts=counts)
    times = timed_reps(lambda: oracle.loss_backward_batch(params, targets_np, SIGMA, nthreads=threads),
                       warmup=2, budget_s=budget_s)  # the counted run above is the first warm-up
    single = timed_reps(lambda: oracle.loss_backward_batch(params[:1], targets_np[:1], SIGMA, nthreads=1),
                        warmup=1, budget_s=min(budget_s, 0.4), min_reps=2)
    return dict(per_batch_s=float(np.mean(times)), median_s=float(np.median(times)), reps=len(times),
                threads=threads, single_item_ms=float(np.median(single)) * 1e3, losses=losses, grads=grads,
                n_box=int(counts.n_box), n_contrib=int(counts.n_contrib))


def fit_gpu(ctx):
    """Config c4 on the GPU: the device fit loop, 800 iterations at 176x176, T=150
    (fit.rs:243-288), three timed fits after a short warm-up, then one with the
    kernels event-timed. Throughput is dense pixel x triangle evaluations per
    second over the whole fit (800 H W T / seconds)."""
    from diffrast import synth

    cfg = synth.CONFIGS["c4"]
    H, W, T, iters = cfg["H"], cfg["W"], cfg["T"], cfg["iters"]
    target = synth.blob_target(4, H, W)
    init, bg = synth.seed_scene(target, T, 4)
    ctx.fit(target, init, bg, iters=20, patience=None)  # warm-up
    runs = []
    with quiet_gc():
        for _ in range(3):
            t0 = time.perf_counter()
            r = ctx.fit(target, init, bg, iters=iters, patience=None)
            runs.append(time.perf_counter() - t0)
    dt = float(np.median(runs))
    ctx.timing(True)
    try:
        ctx.fit(target, init, bg, iters=iters, patience=None)
        t = ctx.read_timings()
    finally:
        ctx.timing(False)
    kt = {"setup": t["setup_ms"] / max(t["setup_n"], 1), "fused": t["raster_ms"] / max(t["raster_n"], 1),
          "fit_step": t["adam_ms"] / max(t["adam_n"], 1)}
    out = dict(workload=f"device fit loop, B=1 {H}x{W} T={T}, {iters} iterations (patience off), "
                        "sigma 0.02 -> 0.0015, Adam lr 0.004/0.02/0.01",
               iterations=len(r["losses"]), seconds=round(dt, 4), ms_per_iteration=dt * 1e3 / iters,
               pixel_tri_per_s=iters * H * W * T / dt, kernel_ms={k: round(v, 5) for k, v in kt.items()},
               launches={"fused": t["raster_n"]},
               first_loss=float(r["losses"][0]), best_loss=r["best_loss"], best_iter=r["best_iter"],
               improvement=float(r["losses"][0] / r["best_loss"]))
    log(f"c4: {dt * 1e3 / iters:.4f} ms/iteration; kernel avg ms {kt}")
    return out, dict(target=target, init=init, bg=bg, dt=dt, kt=kt)


def fit_cpu(out, keep):
    """Config c4 on the CPU, after fit_gpu: the oracle's fit of the same start on
    one core, timed; its pair counts give the fit's algorithmic FLOP (148 N_box +
    61 N_contrib + 15 H W summed over the iterations), and the roofline is the
    fixed-order fused kernel's: that FLOP per launch over its event-timed
    average duration."""
    from diffrast import synth
    from oracle import oracle

    cfg = synth.CONFIGS["c4"]
    H, W, T, iters = cfg["H"], cfg["W"], cfg["T"], cfg["iters"]
    dt, kt = keep["dt"], keep["kt"]
    dense = iters * H * W * T
    counts = oracle.Counts()
    t0 = time.perf_counter()
    c = oracle.fit(keep["target"], keep["init"], keep["bg"], iters=iters, patience=None, counts=counts)
    cpu_s = time.perf_counter() - t0
    out["cpu_baseline"] = {"value": dense / cpu_s, "unit": UNIT, "cores": 1, "kind": "port",
                           "sample": f"the whole {iters}-iteration fit once, one thread",
                           "seconds": round(cpu_s, 3), "ms_per_iteration": cpu_s * 1e3 / iters,
                           "iterations_per_s": iters / cpu_s,
                           "best_loss": c["best_loss"], "best_iter": c["best_iter"]}
    out["speedup_gpu_over_cpu"] = cpu_s / dt
    flop = (FLOP_FWD[0] + FLOP_BWD[0]) * counts.n_box + (FLOP_FWD[1] + FLOP_BWD[1]) * counts.n_contrib \
        + FLOP_FWD[2] * iters * H * W
    kname = fused_kernel_name(1, H, W, T, deterministic=True)
    out["roofline"] = roof(kname, flop / iters, kt["fused"], traffic_from_profiles(kname.split(" ")[0], "c4"))
    out["roofline"]["n_box_pairs_all_iterations"] = int(counts.n_box)
    out["roofline"]["n_contrib_pairs_all_iterations"] = int(counts.n_contrib)
    out["roofline_step"] = roof("whole iteration (wall)", flop / iters, dt * 1e3 / iters)
    return out


def fit_config(ctx, with_cpu=True):
    """fit_gpu, then (with_cpu) fit_cpu."""
    out, keep = fit_gpu(ctx)
    return fit_cpu(out, keep) if with_cpu else out


def torch_op_ms(torch, cfg, p, targets, dev, steps=50):
    """End to end through the drop-in autograd op: fused_mse forward + backward."""
    from diffrast import torch_layer

    tgt = targets.permute(0, 3, 1, 2).contiguous()
    q = p.clone().requires_grad_(True)
    for _ in range(10):
        torch_layer.fused_mse(q, tgt, sigma=SIGMA).backward()
    torch.cuda.synchronize()
    with quiet_gc():
        t0 = time.perf_counter()
        for _ in range(steps):
            q.grad = None
            torch_layer.fused_mse(q, tgt, sigma=SIGMA).backward()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps


def torch_rasterize_ms(torch, cfg, p, targets, dev, keep_record=True, steps=50):
    """End to end through the drop-in autograd op: rasterize, an MSE in torch, backward.
    keep_record=False times the backward that renders again, as the reference's does."""
    from diffrast import torch_layer

    tgt = targets.permute(0, 3, 1, 2).contiguous()
    q = p.clone().requires_grad_(True)

    def step():
        img = torch_layer._Rasterize.apply(q, cfg["H"], cfg["W"], SIGMA, (0.0, 0.0, 0.0), "gpu", True,
                                           keep_record)
        ((img - tgt) ** 2).mean().backward()

    for _ in range(10):
        step()
    torch.cuda.synchronize()
    with quiet_gc():
        t0 = time.perf_counter()
        for _ in range(steps):
            q.grad = None
            step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / steps


def forward_side(torch, ctx, dev, cpu=True):
    """Forward-only renders (drh_render): the reference's GPU forward benchmark cells, one
    Scene::random-shaped scene each at sigma 0.0015 (gpu_bench.rs:18-69), the fit binary's
    1024-pixel export (fit.rs:95-99), and the c2 batch rendered without gradients. Device
    time with params and image in HBM; `host_ms` adds the copies in and out (the
    reference's `render` returns a host canvas)."""
    from diffrast import synth

    cells = [("fwd_128_T64", 1, 128, 128, 64, 0.0015, "random", 11),
             ("fwd_256_T128", 1, 256, 256, 128, 0.0015, "random", 11),
             ("fwd_512_T256", 1, 512, 512, 256, 0.0015, "random", 11),
             ("fwd_512_T1024", 1, 512, 512, 1024, 0.0015, "random", 11),
             ("export_1024_T150", 1, 1024, 1024, 150, 0.0015 * 176 / 1024, "export", 12),
             ("fwd_c2_B16_256_T128", 16, 256, 256, 128, 0.0015, "uniform", 1)]
    stream = torch.cuda.current_stream(dev).cuda_stream
    res = {}
    for name, B, H, W, T, sig, kind, seed in cells:
        if kind == "export":
            params = synth.random_scene(seed, T, 0.18)[None]
        elif kind == "random":
            params = synth.random_scene(seed, T)[None]
        else:
            params = synth.batch(kind, B, T, seed)
        bg = np.tile(np.array([[0.1, 0.11, 0.14]], np.float32), (B, 1))
        p = torch.from_numpy(params).to(dev)
        b = torch.from_numpy(bg).to(dev)
        out = torch.empty((B, H, W, 3), device=dev)

        def run():
            ctx.render_ptr(p.data_ptr(), b.data_ptr(), B, T, H, W, sig, out.data_ptr(), stream)

        for _ in range(3):
            run()
        torch.cuda.synchronize()
        n = 20
        with quiet_gc():
            t0 = time.perf_counter()
            for _ in range(n):
                run()
            torch.cuda.synchronize()
            dev_ms = (time.perf_counter() - t0) * 1e3 / n
        for _ in range(2):
            ctx.render(params, H, W, sig, bg)
        with quiet_gc():
            t0 = time.perf_counter()
            for _ in range(5):
                ctx.render(params, H, W, sig, bg)
            host_ms = (time.perf_counter() - t0) * 1e3 / 5
        res[name] = {"B": B, "H": H, "W": W, "T": T, "sigma": sig, "ms": round(dev_ms, 4),
                     "host_ms": round(host_ms, 4), "pixel_tri_per_s": B * H * W * T / (dev_ms / 1e3)}
        if name == "fwd_512_T1024":
            res[name]["_inputs"] = (params, bg)
    if cpu:
        forward_cpu(res)
    return res


def forward_cpu(res):
    """The oracle's single-thread render of the 512x512 T=1024 cell, beside forward_side's GPU time."""
    from oracle import oracle

    r = res.get("fwd_512_T1024")
    if not r or "_inputs" not in r:
        return
    params, bg = r.pop("_inputs")
    t0 = time.perf_counter()
    oracle.render_batch(params, r["H"], r["W"], r["sigma"], bg, nthreads=1)
    cpu_ms = (time.perf_counter() - t0) * 1e3
    r["cpu_oracle_1thread_ms"] = round(cpu_ms, 2)
    r["speedup_vs_cpu_1thread"] = round(cpu_ms / r["ms"], 1)


def copy_calibration(torch):
    """A plain device copy of known size: the scale for FETCH_SIZE/WRITE_SIZE."""
    n = 64 << 20  # floats (256 MiB)
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_each_way": n * 4}), flush=True)


def roof(kernel, flop, ms_k, traffic=None):
    achieved = flop / (ms_k / 1e3) / 1e12
    return {
        "bound": "valu",
        "achieved": achieved,
        "peak": PEAK_FP32_TFLOPS,
        "unit": "TFLOP/s",
        "frac": achieved / PEAK_FP32_TFLOPS,
        "traffic": traffic,
        "traffic_source": "committed PMC summary under profiles/ (FETCH_SIZE, WRITE_SIZE), not this run"
                          if traffic is not None else None,
        "kernel": kernel,
        "flop_per_launch": flop,
        "ms_per_launch": ms_k,
    }


def gpu_leg(torch, ctx, name, dev, steps, warmup, two_kernels=True):
    """The GPU side of one batched workload: wall ms per fused step over `steps`
    calls after `warmup`, per-kernel event times, and (two_kernels) the same step
    on the two-kernel path. Returns the config's line and what cpu_leg needs."""
    from diffrast import synth

    cfg = synth.CONFIGS[name]
    B, H, W, T = cfg["B"], cfg["H"], cfg["W"], cfg["T"]
    params, p, bg, targets = make_inputs(torch, ctx, cfg, 1, dev)
    with quiet_gc():  # also between the timed steps and the event-timed ones
        ms, losses, grads = time_fused(torch, ctx, cfg, p, bg, targets, steps, warmup, dev)
        kt = kernel_times(torch, ctx, cfg, p, bg, targets, max(10, min(steps, 50)), dev)
    log(f"{name}: {ms:.4f} ms/batch over {steps} steps; kernel avg ms {kt}")
    # the same step on the two-kernel path, for its per-kernel figures
    two = None
    if "fused" in kt and two_kernels:
        os.environ["DRH_UNFUSED"] = "1"
        try:
            ms2 = time_fused(torch, ctx, cfg, p, bg, targets, steps, warmup, dev)[0]
        finally:
            os.environ.pop("DRH_UNFUSED", None)
        two = {"ms_per_batch": ms2,
               "kernel_ms": kernel_times(torch, ctx, cfg, p, bg, targets, max(10, min(steps, 50)), dev, True)}
        log(f"{name}: two-kernel path {ms2:.4f} ms/batch; kernel avg ms {two['kernel_ms']}")
    dense = B * H * W * T
    out = {
        "workload": f"batched soft-raster forward+MSE+backward, B={B} {H}x{W} T={T} sigma={SIGMA}"
                    + (" (small triangles)" if cfg["kind"] == "small" else ""),
        "B": B, "H": H, "W": W, "T": T,
        "steps": steps, "warmup": warmup,
        "ms_per_batch": ms,
        "pixel_tri_per_s": dense / (ms / 1e3),
        "kernel_ms": {k: round(v, 5) for k, v in kt.items()},
    }
    keep = dict(name=name, cfg=cfg, params=params, targets_np=targets.cpu().numpy(),
                losses=losses.cpu().numpy(), grads=grads.cpu().numpy(), kt=kt, two=two)
    return out, keep


def cpu_leg(out, keep, cpu_budget, traffic=True):
    """The CPU side of one batched workload, after its gpu_leg: the oracle on the
    same batch (parity figures, N_box and N_contrib), the rooflines of the GPU
    leg's kernels and the same-run CPU baseline."""
    name, cfg, kt, two = keep["name"], keep["cfg"], keep["kt"], keep["two"]
    B, H, W, T = cfg["B"], cfg["H"], cfg["W"], cfg["T"]
    ms = out["ms_per_batch"]
    dense = B * H * W * T
    c = cpu_baseline(cfg, keep["params"], keep["targets_np"], cpu_budget)
    log(f"{name}: cpu baseline {c['per_batch_s'] * 1e3:.1f} ms/batch on {c['threads']} threads")
    g = keep["grads"].reshape(B, -1, 10).astype(np.float64)
    cg = c["grads"].reshape(B, -1, 10).astype(np.float64)
    par = {"grad_max_abs_over_norm": max(float(np.abs(g[b] - cg[b]).max() / np.linalg.norm(cg[b]))
                                         for b in range(B))}
    for gname, sl in GROUPS.items():
        par[f"grad_{gname}"] = max(float(np.abs(g[b][:, sl] - cg[b][:, sl]).max() /
                                         max(np.linalg.norm(cg[b][:, sl]), 1e-30)) for b in range(B))
    l = keep["losses"].astype(np.float64)
    par["loss_rel"] = float(np.max(np.abs(l - c["losses"]) / np.abs(c["losses"])))
    out["parity_vs_oracle"] = par
    counts = (c["n_box"], c["n_contrib"], B * H * W)
    flop_f = sum(a * b for a, b in zip(FLOP_FWD, counts))
    flop_b = sum(a * b for a, b in zip(FLOP_BWD, counts))

    def two_kernel_roofs(k):
        return {"roofline_backward": roof("backward_kernel", flop_b, k["backward"],
                                          traffic_from_profiles("backward_kernel", name) if traffic else None),
                "roofline_forward": roof("forward_kernel", flop_f, k["forward"],
                                         traffic_from_profiles("forward_kernel", name) if traffic else None),
                "roofline_pair": roof("forward_kernel+backward_kernel", flop_f + flop_b,
                                      k["forward"] + k["backward"])}

    if "fused" in kt:
        kname = fused_kernel_name(B, H, W, T)
        out["roofline"] = roof(kname, flop_f + flop_b, kt["fused"],
                               traffic_from_profiles(kname, name) if traffic else None)
        if two is not None:
            two.update(two_kernel_roofs(two["kernel_ms"]))
            two["kernel_ms"] = {k: round(v, 5) for k, v in two["kernel_ms"].items()}
            out["two_kernel_path"] = two
    else:
        r = two_kernel_roofs(kt)
        out["roofline"] = r.pop("roofline_backward")
        out.update(r)
    out["roofline"]["n_box_pairs"] = c["n_box"]
    out["roofline"]["n_contrib_pairs"] = c["n_contrib"]
    out["roofline_step"] = roof("whole step (wall)", flop_f + flop_b, ms)
    out["cpu_baseline"] = {
        "value": dense / c["per_batch_s"],
        "unit": UNIT,
        "cores": c["threads"],
        "kind": "port",
        "sample": f"the full B={B} {H}x{W} T={T} batch: 3 warm-ups, then {c['reps']} timed runs "
                  f"(>= 0.4 s), one thread per scene",
        "ms_per_batch": c["per_batch_s"] * 1e3,
        "median_ms_per_batch": c["median_s"] * 1e3,
        "single_thread_ms_per_item": c["single_item_ms"],
        "cpu_model": cpu_model(),
        "nproc": os.cpu_count(),
        "threads": c["threads"],
        "speedup_gpu_over_cpu": c["per_batch_s"] * 1e3 / ms,
    }
    return out


def measure_batch(torch, ctx, name, dev, steps, warmup, cpu, cpu_budget, traffic=True):
    """gpu_leg, then (with `cpu`) cpu_leg."""
    out, keep = gpu_leg(torch, ctx, name, dev, steps, warmup)
    return cpu_leg(out, keep, cpu_budget, traffic) if cpu else out


def crossover(torch, ctx, dev):
    """GPU against this host's CPU over the reference's crossover cells (batch of 16,
    64/128/256 pixels, 32/128/512 triangles, sigma 0.01, Scene::random-shaped scenes,
    flat targets; crates/diffrast-gpu/src/bin/gpu_bench.rs:157-182) and small cells
    near the reference's dispatch floor (crates/diffrast-py/src/lib.rs:138-147). The
    GPU is timed with host arrays in and out, as the reference's backward_many takes
    them, and with device-resident arrays."""
    from diffrast import synth
    from oracle import oracle

    cells = [(16, n, t) for n in (64, 128, 256) for t in (32, 128, 512)]
    cells += [(1, 16, 2), (1, 32, 8), (2, 32, 16), (1, 64, 32), (2, 64, 32), (4, 64, 64), (1, 128, 64)]
    rows = []
    stream = torch.cuda.current_stream(dev).cuda_stream
    for B, n, T in cells:
        params = np.stack([synth.random_scene(11 + b, T) for b in range(B)])
        targets = np.empty((B, n, n, 3), np.float32)
        targets[:] = (0.4, 0.5, 0.6)
        threads = max(1, min(B, box_cpu_share(), 16))
        cpu = np.median(timed_reps(lambda: oracle.loss_backward_batch(params, targets, 0.01, nthreads=threads),
                                   warmup=1, budget_s=0.2))
        host = np.median(timed_reps(lambda: ctx.fused_loss_backward(params, targets, 0.01), warmup=2,
                                    budget_s=0.1, min_reps=5))
        p, tg = torch.from_numpy(params).to(dev), torch.from_numpy(targets).to(dev)
        bg = torch.zeros((B, 3), device=dev)
        l, g = torch.empty(B, device=dev), torch.empty((B, T, 10), device=dev)

        def dev_step():
            ctx.fused_ptr(p.data_ptr(), bg.data_ptr(), tg.data_ptr(), B, T, n, n, 0.01, l.data_ptr(), g.data_ptr(),
                          None, stream)
            torch.cuda.synchronize()

        devt = np.median(timed_reps(dev_step, warmup=2, budget_s=0.1, min_reps=5))
        rows.append(dict(batch=B, size=n, tris=T, work=B * T * n * n, cpu_ms=cpu * 1e3, cpu_threads=threads,
                         gpu_host_ms=host * 1e3, gpu_device_ms=devt * 1e3, gpu_host_over_cpu=cpu / host,
                         reference_rule_prefers_gpu=bool(B >= 2 and B * T * n * n >= 250_000)))
        log(json.dumps(rows[-1]))
    print(json.dumps({"crossover": rows, "cpu_model": cpu_model(), "nproc": os.cpu_count(),
                      "device": ctx.device_info()}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-budget", type=float, default=0.4, help="seconds of timed CPU baseline runs per config")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-side", action="store_true", help="skip the other workloads")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--crossover", action="store_true")
    ap.add_argument("--config", choices=["c0", "c1", "c2", "c3", "c4"],
                    help="measure this one workload alone and print its line (for profiling)")
    ap.add_argument("--after-headline", action="store_true",
                    help="with --config: first run the headline's fused steps untimed (150 of them), as the "
                         "full run's headline leg precedes every other workload, so that the workload runs at "
                         "the clocks it has there (the GPU's clocks ramp over ~18 ms of load)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: there is no multi-GPU path "
              "(scenes are independent: each GPU would take a slice of the batch)", file=sys.stderr)
        sys.exit(2)

    import torch

    if args.copy_calibration:
        copy_calibration(torch)
        return

    from diffrast import _lib, synth

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    ctx = _lib.Context()
    log("device:", ctx.device_info())
    if args.crossover:
        crossover(torch, ctx, dev)
        return
    if args.config:
        cpu = not args.no_cpu_baseline
        if args.after_headline and args.config != "c2":
            hcfg = synth.CONFIGS["c2"]
            _, hp, hbg, htg = make_inputs(torch, ctx, hcfg, 1, dev)
            time_fused(torch, ctx, hcfg, hp, hbg, htg, 150, 0, dev)
        if args.config == "c4":
            one = fit_config(ctx, with_cpu=cpu)
        else:
            one = measure_batch(torch, ctx, args.config, dev, args.steps, args.warmup, cpu, args.cpu_budget)
        print(json.dumps({"config": args.config, "steps": args.steps, "warmup": args.warmup, **one}), flush=True)
        return
    cfg = synth.CONFIGS["c2"]
    B, H, W, T = cfg["B"], cfg["H"], cfg["W"], cfg["T"]
    cpu = not args.no_cpu_baseline
    # Order of the run: every GPU leg first, then the CPU legs (the oracle),
    # during which the GPU idles:
    # - the headline: c2 with `warmup` untimed and `steps` timed steps, first
    #   thing in the process;
    # - the other configurations' GPU legs (c0, c1, c3, the c4 fit);
    # - "sustained": the same c2 step again after 200 more untimed steps (the
    #   GPU's clocks ramp up over ~18 ms of sustained load), reported beside
    #   the headline, not as it;
    # - the torch-op and forward-only side measurements.
    head, head_keep = gpu_leg(torch, ctx, "c2", dev, args.steps, args.warmup)
    legs, fit = {}, None
    if not args.no_side:
        for name in ("c0", "c1", "c3"):
            legs[name] = gpu_leg(torch, ctx, name, dev, 20, 5)
        fit = fit_gpu(ctx)
    sustained, _ = gpu_leg(torch, ctx, "c2", dev, 100, 200, two_kernels=False)
    side = {}
    if not args.no_side:
        p = torch.from_numpy(synth.batch("uniform", B, T, 1)).to(dev)
        _, _, _, targets = make_inputs(torch, ctx, cfg, 1, dev)
        side["c2_torch_fused_mse_fwd_bwd_ms"] = round(torch_op_ms(torch, cfg, p, targets, dev), 4)
        side["c2_torch_rasterize_mse_fwd_bwd_ms"] = round(torch_rasterize_ms(torch, cfg, p, targets, dev), 4)
        side["c2_torch_rasterize_mse_fwd_bwd_rerender_ms"] = round(
            torch_rasterize_ms(torch, cfg, p, targets, dev, keep_record=False), 4)
        side["forward_only"] = forward_side(torch, ctx, dev, cpu=False)
    # the CPU legs
    if cpu:
        head = cpu_leg(head, head_keep, args.cpu_budget)
        for name, (o, k) in legs.items():
            legs[name] = (cpu_leg(o, k, args.cpu_budget), k)
        if fit is not None:
            fit = (fit_cpu(*fit), None)
        if not args.no_side:
            forward_cpu(side["forward_only"])
    for r in side.get("forward_only", {}).values():
        r.pop("_inputs", None)
    ms = head["ms_per_batch"]
    dense = B * H * W * T
    out = {
        "metric": METRIC,
        "value": dense / (ms / 1e3),
        "unit": UNIT,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64 scenes; targets rendered from independently seeded scenes)",
        "config": {"workload": head["workload"], "B": B, "H": H, "W": W, "T": T, "sigma": SIGMA,
                   "scenes": "uniform vertices"},
        "kernel_ms": head["kernel_ms"],
        "parity_vs_oracle": head.get("parity_vs_oracle"),
        "roofline": head.get("roofline"),
        "roofline_step": head.get("roofline_step"),
        "two_kernel_path": head.get("two_kernel_path"),
        "cpu_baseline": head.get("cpu_baseline"),
        "sustained": {"ms_per_step": sustained["ms_per_batch"], "kernel_ms": sustained["kernel_ms"],
                      "steps": 100, "warmup": 200,
                      "note": "the same step measured again later in the run, after 200 untimed steps: the GPU's "
                              "clocks ramp up over ~18 ms of sustained load, so a training loop runs at this "
                              "rate; the headline above keeps the requested warm-up"},
    }
    if "roofline" in head and cpu:
        flop = head["roofline"]["flop_per_launch"]
        out["sustained"]["roofline_frac"] = flop / (sustained["kernel_ms"]["fused"] / 1e3) / 1e12 / PEAK_FP32_TFLOPS
        out["sustained"]["roofline_step_frac"] = flop / (sustained["ms_per_batch"] / 1e3) / 1e12 / PEAK_FP32_TFLOPS
    if not args.no_side:
        configs = {name: legs[name][0] for name in ("c0", "c1")}
        configs["c2"] = head
        configs["c3"] = legs["c3"][0]
        configs["c4"] = fit[0]
        out["configs"] = configs
        out["side"] = side
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
