#!/usr/bin/env python3
"""Benchmark: batched soft-raster forward + MSE + backward on one MI355X.

One step = one drh_fused_loss_backward call (setup_records, forward_kernel,
backward_kernel) over the headline workload: B=16 scenes at 256x256,
T=128 triangles each, sigma=0.0015, synthetic seeded scenes (diffrast.synth)
and targets rendered from independently seeded scenes. Inputs and outputs
stay in HBM; the timed region is K steps between two synchronizations.

Printed (one JSON line on stdout): throughput in dense pixel-triangle
evaluations per second, ms per batch, the dominant kernel's roofline position
(backward_kernel: its algorithmic FLOP per launch over its event-timed average
duration, against the FP32 vector peak; the forward kernel and the pair are
reported beside it), the CPU baseline (the C oracle, one thread per scene, on
this host's cores), and side measurements of the other workloads.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
    python bench.py --copy-calibration     # plain device copy, for PMC scaling
"""

from __future__ import annotations

import argparse
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


def log(*a):
    print(*a, file=sys.stderr, flush=True)


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

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    return ms, losses, grads


def kernel_times(torch, ctx, cfg, p, bg, targets, steps, dev):
    """Event-timed average duration of each kernel of the step."""
    ctx.timing(True)
    try:
        time_fused(torch, ctx, cfg, p, bg, targets, steps, 0, dev)
        t = ctx.read_timings()
    finally:
        ctx.timing(False)
    names = {"setup": "setup", "forward": "raster", "backward": "backward", "reduce": "reduce"}
    return {k: t[f"{f}_ms"] / max(t[f"{f}_n"], 1) for k, f in names.items()}


def traffic_from_profiles(kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summary, if any."""
    f = ROOT / "profiles" / "raster_kernels_c2_pmc.md"
    if not f.exists():
        return None
    m = re.search(kernel + r" traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


def cpu_baseline(cfg, params, targets_np, budget_s):
    """The oracle's backward_batch analogue on this host (grad.rs:192-207)."""
    from oracle import oracle

    B, H, W, T = cfg["B"], cfg["H"], cfg["W"], cfg["T"]
    # one thread per scene, capped by the cores this process may use (16 per
    # GPU on a shared box, whatever the machine's total)
    threads = max(1, min(B, box_cpu_share(), 16))
    counts = oracle.Counts()
    t0 = time.perf_counter()
    losses, grads = oracle.loss_backward_batch(params, targets_np, SIGMA, nthreads=threads,
                                               counts=counts)
    first = time.perf_counter() - t0
    reps, t_total = 0, 0.0
    while t_total < budget_s and reps < 50:
        t0 = time.perf_counter()
        oracle.loss_backward_batch(params, targets_np, SIGMA, nthreads=threads)
        t_total += time.perf_counter() - t0
        reps += 1
    per_batch = t_total / reps if reps else first
    return dict(per_batch_s=per_batch, reps=reps, threads=threads, losses=losses, grads=grads,
                n_box=int(counts.n_box), n_contrib=int(counts.n_contrib))


def fit_side(ctx):
    """Config c4: the device fit loop, 800 iterations at 176x176, T=150."""
    from diffrast import synth

    target = synth.blob_target(4, 176, 176)
    init, bg = synth.seed_scene(target, 150, 4)
    ctx.fit(target, init, bg, iters=20, patience=None)  # warm-up
    t0 = time.perf_counter()
    r = ctx.fit(target, init, bg, iters=800, patience=None)
    dt = time.perf_counter() - t0
    return dict(seconds=round(dt, 4), iterations=len(r["losses"]), first_loss=float(r["losses"][0]),
                best_loss=r["best_loss"], improvement=float(r["losses"][0] / r["best_loss"]))


def torch_op_ms(torch, cfg, p, targets, dev, steps=10):
    """End to end through the drop-in autograd op: fused_mse forward + backward."""
    from diffrast import torch_layer

    tgt = targets.permute(0, 3, 1, 2).contiguous()
    q = p.clone().requires_grad_(True)
    for _ in range(3):
        torch_layer.fused_mse(q, tgt, sigma=SIGMA).backward()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        q.grad = None
        torch_layer.fused_mse(q, tgt, sigma=SIGMA).backward()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3 / steps


def torch_rasterize_ms(torch, cfg, p, targets, dev, keep_record=True, steps=10):
    """End to end through the drop-in autograd op: rasterize, an MSE in torch, backward.
    keep_record=False times the backward that renders again, as the reference's does."""
    from diffrast import torch_layer

    tgt = targets.permute(0, 3, 1, 2).contiguous()
    q = p.clone().requires_grad_(True)

    def step():
        img = torch_layer._Rasterize.apply(q, cfg["H"], cfg["W"], SIGMA, (0.0, 0.0, 0.0), "gpu", True,
                                           keep_record)
        ((img - tgt) ** 2).mean().backward()

    for _ in range(3):
        step()
    torch.cuda.synchronize()
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
        t0 = time.perf_counter()
        for _ in range(n):
            run()
        torch.cuda.synchronize()
        dev_ms = (time.perf_counter() - t0) * 1e3 / n
        for _ in range(2):
            ctx.render(params, H, W, sig, bg)
        t0 = time.perf_counter()
        for _ in range(5):
            ctx.render(params, H, W, sig, bg)
        host_ms = (time.perf_counter() - t0) * 1e3 / 5
        res[name] = {"B": B, "H": H, "W": W, "T": T, "sigma": sig, "ms": round(dev_ms, 4),
                     "host_ms": round(host_ms, 4), "pixel_tri_per_s": B * H * W * T / (dev_ms / 1e3)}
        if cpu and name == "fwd_512_T1024":
            from oracle import oracle

            t0 = time.perf_counter()
            oracle.render_batch(params, H, W, sig, bg, nthreads=1)
            cpu_ms = (time.perf_counter() - t0) * 1e3
            res[name]["cpu_oracle_1thread_ms"] = round(cpu_ms, 2)
            res[name]["speedup_vs_cpu_1thread"] = round(cpu_ms / dev_ms, 1)
    return res


def copy_calibration(torch):
    """A plain device copy of known size: the scale for FETCH_SIZE/WRITE_SIZE."""
    n = 64 << 20  # floats (256 MiB)
    a = torch.ones(n, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_each_way": n * 4}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--cpu-budget", type=float, default=8.0, help="seconds of CPU baseline timing")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-side", action="store_true", help="skip the other workloads")
    ap.add_argument("--copy-calibration", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(scenes are independent; see DESIGN.md for how batches would shard)", file=sys.stderr)
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
    cfg = synth.CONFIGS["c2"]
    B, H, W, T = cfg["B"], cfg["H"], cfg["W"], cfg["T"]

    params, p, bg, targets = make_inputs(torch, ctx, cfg, 1, dev)
    ms, losses, grads = time_fused(torch, ctx, cfg, p, bg, targets, args.steps, args.warmup, dev)
    log(f"c2: {ms:.4f} ms/batch over {args.steps} steps")
    kt = kernel_times(torch, ctx, cfg, p, bg, targets, max(10, min(args.steps, 50)), dev)
    log("kernel avg ms:", kt)

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
        "config": {"workload": "batched soft-raster forward+MSE+backward, B=16 256x256 T=128 sigma=0.0015",
                   "B": B, "H": H, "W": W, "T": T, "sigma": SIGMA, "scenes": "uniform vertices"},
        "kernel_ms": {k: round(v, 5) for k, v in kt.items()},
    }

    cpu = None
    if not args.no_cpu_baseline:
        targets_np = targets.cpu().numpy()
        cpu = cpu_baseline(cfg, params, targets_np, args.cpu_budget)
        log(f"cpu baseline: {cpu['per_batch_s'] * 1e3:.1f} ms/batch on {cpu['threads']} threads")
        g = grads.cpu().numpy().reshape(B, -1).astype(np.float64)
        cg = cpu["grads"].reshape(B, -1).astype(np.float64)
        grad_rel = max(float(np.abs(g[b] - cg[b]).max() / np.linalg.norm(cg[b])) for b in range(B))
        l = losses.cpu().numpy().astype(np.float64)
        loss_rel = float(np.max(np.abs(l - cpu["losses"]) / np.abs(cpu["losses"])))
        out["parity_vs_oracle"] = {"grad_max_abs_over_norm": grad_rel, "loss_rel": loss_rel}
        counts = (cpu["n_box"], cpu["n_contrib"], B * H * W)
        flop_f = sum(a * b for a, b in zip(FLOP_FWD, counts))
        flop_b = sum(a * b for a, b in zip(FLOP_BWD, counts))

        def roof(kernel, flop, ms_k):
            achieved = flop / (ms_k / 1e3) / 1e12
            return {
                "bound": "valu",
                "achieved": achieved,
                "peak": PEAK_FP32_TFLOPS,
                "unit": "TFLOP/s",
                "frac": achieved / PEAK_FP32_TFLOPS,
                "traffic": traffic_from_profiles(kernel),
                "kernel": kernel,
                "flop_per_launch": flop,
                "ms_per_launch": ms_k,
            }

        out["roofline"] = roof("backward_kernel", flop_b, kt["backward"])
        out["roofline"]["n_box_pairs"] = cpu["n_box"]
        out["roofline"]["n_contrib_pairs"] = cpu["n_contrib"]
        out["roofline_forward"] = roof("forward_kernel", flop_f, kt["forward"])
        both = roof("forward_kernel+backward_kernel", flop_f + flop_b, kt["forward"] + kt["backward"])
        both["traffic"] = None
        out["roofline_pair"] = both
        out["cpu_baseline"] = {
            "value": dense / cpu["per_batch_s"],
            "unit": UNIT,
            "cores": cpu["threads"],
            "kind": "port",
            "sample": f"the full B=16 256x256 T=128 batch, {cpu['reps']} timed repetitions "
                      f"({cpu['per_batch_s'] * 1e3:.1f} ms each) after one untimed run, "
                      "one thread per scene",
            "ms_per_batch": cpu["per_batch_s"] * 1e3,
            "speedup_gpu_over_cpu": cpu["per_batch_s"] * 1e3 / ms,
        }
    else:
        out["roofline"] = None
        out["cpu_baseline"] = None

    if not args.no_side:
        side = {}
        for name in ("c0", "c1", "c3"):
            c = synth.CONFIGS[name]
            _, pp, bb, tt = make_inputs(torch, ctx, c, 1, dev)
            m, _, _ = time_fused(torch, ctx, c, pp, bb, tt, 20, 5, dev)
            side[name] = {"ms_per_batch": round(m, 4), "B": c["B"], "H": c["H"], "W": c["W"], "T": c["T"],
                          "pixel_tri_per_s": c["B"] * c["H"] * c["W"] * c["T"] / (m / 1e3)}
        side["c4_fit_800_iters"] = fit_side(ctx)
        side["c2_torch_fused_mse_fwd_bwd_ms"] = round(torch_op_ms(torch, cfg, p, targets, dev), 4)
        side["c2_torch_rasterize_mse_fwd_bwd_ms"] = round(torch_rasterize_ms(torch, cfg, p, targets, dev), 4)
        side["c2_torch_rasterize_mse_fwd_bwd_rerender_ms"] = round(
            torch_rasterize_ms(torch, cfg, p, targets, dev, keep_record=False), 4)
        side["forward_only"] = forward_side(torch, ctx, dev, cpu=not args.no_cpu_baseline)
        out["side"] = side

    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
