"""The five benchmark workloads, each against the CPU oracle at its full size.

Inputs are the documented ones (diffrast.synth, seed 1, background (0, 0, 0),
sigma 0.0015, the drop-in default of python/diffrast/torch_layer.py:73):
  c0  B=1 64x64 T=32, uniform scene of seed 1; target = render of the seed-2 scene
  c1  B=16 128x128 T=128, scene b of seed 1+b, target b rendered from seed 1001+b
  c2  B=16 256x256 T=128 (the headline batch), seeds as c1
  c3  B=8 256x256 T=512 small triangles (centre + offsets within 0.05), seeds as c1
  c4  the fit of the `fit` binary: B=1 176x176 blob target, T=150, 800 iterations
Bars are tests/bars.py's: images 1e-5, losses 1e-4 relative, gradients 1e-4 of the
norm per scene and per parameter group (vertices, colours, alpha).
"""

import numpy as np
import pytest

from bars import assert_grads, check_image, check_losses
from diffrast import synth

pytestmark = pytest.mark.gpu

SIGMA = 0.0015


@pytest.fixture(scope="module")
def ctx():
    from diffrast import _lib

    c = _lib.Context()
    yield c
    c.close()


def batch_inputs(orc, name, seed=1):
    cfg = synth.CONFIGS[name]
    B, H, W, T = cfg["B"], cfg["H"], cfg["W"], cfg["T"]
    params = synth.batch(cfg["kind"], B, T, seed)
    targets = orc.render_batch(synth.batch(cfg["kind"], B, T, seed, target_offset=1000), H, W, SIGMA)
    return params, targets, H, W


def check_batch(ctx, orc, name, params, targets, deterministic=False):
    H, W = targets.shape[1], targets.shape[2]
    print(f"{name}: B={params.shape[0]} {H}x{W} T={params.shape[1]} det={deterministic}", flush=True)
    gl, gg, gimg = ctx.fused_loss_backward(params, targets, SIGMA, want_images=True,
                                           deterministic=deterministic)
    counts = orc.Counts()
    cl, cg = orc.loss_backward_batch(params, targets, SIGMA, counts=counts)
    print(f"{name}: box pairs {counts.n_box}, contributing pairs {counts.n_contrib}", flush=True)
    check_image(gimg, orc.render_batch(params, H, W, SIGMA), label=name)
    check_losses(gl, cl, label=name)
    assert_grads(gg, cg, label=name)
    # the render-only entry point draws the same image
    check_image(ctx.render(params, H, W, SIGMA), gimg, label=f"{name} render")
    return gg, cg


def test_c0_single_image_fit_step(ctx, orc):
    # B=1, 64x64, T=32: one forward + MSE + backward against the render of the next seed
    params = synth.batch("uniform", 1, 32, 1)
    targets = orc.render_batch(synth.batch("uniform", 1, 32, 2), 64, 64, SIGMA)
    check_batch(ctx, orc, "c0", params, targets)
    for exact in (False, True):
        gl, gg = ctx.fused_loss_backward(params, targets, SIGMA, exact=exact)
        cl, cg = orc.loss_backward_batch(params, targets, SIGMA)
        check_losses(gl, cl)
        assert_grads(gg, cg, label=f"c0 exact={exact}")


def test_c1_batch_128(ctx, orc):
    params, targets, H, W = batch_inputs(orc, "c1")
    check_batch(ctx, orc, "c1", params, targets)


def test_c2_headline_batch(ctx, orc):
    params, targets, H, W = batch_inputs(orc, "c2")
    check_batch(ctx, orc, "c2", params, targets)
    # upstream-gradient mode on the same batch
    gin = ((synth.uniforms(5, params.shape[0] * H * W * 3) - 0.5) * 1e-4).reshape(-1, H, W, 3).astype(np.float32)
    assert_grads(ctx.backward_from_grad(params, gin, SIGMA), orc.backward_from_grad_batch(params, gin, SIGMA),
                 label="c2 from_grad")


def test_c3_high_contention(ctx, orc):
    # T=512 small triangles: four triangle chunks per tile, the most gradient
    # adds per triangle; both the atomic and the fixed-order reductions
    params, targets, H, W = batch_inputs(orc, "c3")
    g_atomic, cg = check_batch(ctx, orc, "c3", params, targets)
    g_det, _ = check_batch(ctx, orc, "c3", params, targets, deterministic=True)
    assert_grads(g_atomic, g_det, tol=1e-6, label="c3 atomic vs fixed order")


def patience_stop(losses, patience=250, min_delta=1e-7):
    """Iteration count at which fit.rs:267-281's patience would have stopped, or None."""
    best, since = np.inf, 0
    for i, L in enumerate(losses):
        if L + np.float32(min_delta) < best:
            best, since = L, 0
        else:
            since += 1
        if since >= patience:
            return i + 1
    return None


def test_c4_fit_800_iterations(ctx, orc):
    cfg = synth.CONFIGS["c4"]
    H, W, T, iters = cfg["H"], cfg["W"], cfg["T"], cfg["iters"]
    target = synth.blob_target(4, H, W)
    init, bg = synth.seed_scene(target, T, 4)
    print(f"c4: {H}x{W} T={T} {iters} iterations", flush=True)
    g = ctx.fit(target, init, bg, iters=iters, patience=None)
    c = orc.fit(target, init, bg, iters=iters, patience=None)
    assert g["stop_reason"] == c["stop_reason"] == "Completed"
    assert len(g["losses"]) == len(c["losses"]) == iters
    rel = np.abs(g["losses"] - c["losses"]) / c["losses"]
    print(f"c4: loss rel err first 20 {rel[:20].max():.2e}, first 100 {rel[:100].max():.2e}, "
          f"all {rel.max():.2e}; best gpu {g['best_loss']:.6e} @{g['best_iter']} "
          f"oracle {c['best_loss']:.6e} @{c['best_iter']}", flush=True)
    assert rel[:20].max() <= 1e-4
    # the trajectories stay together: the first 100 losses, and the best
    # snapshot (iteration and loss) as the reference's loop picks it
    assert rel[:100].max() <= 1e-3
    assert g["best_iter"] == c["best_iter"]
    assert abs(g["best_loss"] - c["best_loss"]) <= 1e-3 * c["best_loss"]
    # the best snapshot is the scene its loss was measured on, at that iteration's sigma
    sig = orc.sigma_at(0.02, 0.0015, iters, g["best_iter"])
    again = orc.mse(orc.render(g["best_params"], H, W, sig, bg), target)
    print(f"c4: best params re-rendered {again:.6e} vs recorded {g['best_loss']:.6e}", flush=True)
    assert abs(again - g["best_loss"]) <= 1e-4 * g["best_loss"]
    assert g["best_loss"] == g["losses"][g["best_iter"]]
    # the fit improves as the reference's does (integration.rs:23-45: > 10x)
    assert g["losses"][0] / g["best_loss"] > 10
    # whether the default patience (Some(250)) would have stopped this fit early
    print(f"c4: patience 250 would stop the GPU fit at {patience_stop(g['losses'])}, "
          f"the oracle's at {patience_stop(c['losses'])}", flush=True)
    r = ctx.fit(target, init, bg, iters=iters, patience=250)
    assert len(r["losses"]) == (patience_stop(g["losses"]) or iters)
