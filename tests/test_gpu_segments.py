"""fused_seg_kernel: the gradient calls on grids of few tiles (a single scene of
a few hundred 8x8 tiles, the fit), where each tile's triangles are split over
eight waves that evaluate their weights and sweep their gradients in parallel,
while the composite between them runs in scene order.

Against the oracle at the usual bars (tests/bars.py); against the other fused
kernels (DRH_NO_SEGMENTS=1): the same image and losses bit for bit (the
composite is theirs), the gradients to float-atomic order; its fixed-order
mode bit-reproducible, with the default mode's losses bit for bit (both sum the
per-tile loss partials four per 16x16 block, as sum_losses does).
"""

import numpy as np
import pytest

from bars import assert_grads, check_image, check_losses, grad_err
from diffrast import synth

pytestmark = pytest.mark.gpu

# (name, B, H, W, T, sigma, kind): every one within the segmented kernel's
# share (at most 2048 tiles, 16 to 160 triangles)
CASES = [
    ("64x64-T32", 1, 64, 64, 32, 0.0015, "uniform"),
    ("fit-176-T150", 1, 176, 176, 150, 0.02, "uniform"),
    ("odd-T19", 3, 37, 45, 19, 0.01, "uniform"),
    ("small-T144", 2, 64, 96, 144, 0.004, "small"),
    ("tiny-sigma", 2, 32, 32, 24, 1e-4, "uniform"),
    ("T160", 1, 40, 56, 160, 0.006, "small"),
]


@pytest.fixture(scope="module")
def ctx():
    from diffrast import _lib

    c = _lib.Context()
    yield c
    c.close()


def make_case(B, H, W, T, kind, seed=500, opaque_every=0):
    params = synth.batch(kind, B, T, seed)
    if opaque_every:
        # alpha 1: wherever such a triangle covers a pixel fully its weight is
        # exactly 1, a zero factor of the transmittance (counted, not multiplied)
        params[:, ::opaque_every, 9] = 1.0
    bgs = synth.uniforms(seed + 7, B * 3).reshape(B, 3).astype(np.float32)
    return params, bgs


def targets_for(orc, B, H, W, T, sigma, kind, bgs, seed=500):
    return orc.render_batch(synth.batch(kind, B, T, seed, target_offset=1000), H, W, sigma, bgs[::-1].copy())


@pytest.mark.parametrize("exact", [False, True], ids=["fast", "exact"])
@pytest.mark.parametrize("name,B,H,W,T,sigma,kind", CASES, ids=[c[0] for c in CASES])
def test_segments_match_oracle(ctx, orc, name, B, H, W, T, sigma, kind, exact):
    params, bgs = make_case(B, H, W, T, kind)
    targets = targets_for(orc, B, H, W, T, sigma, kind, bgs)
    print(f"segments {name} exact={exact}", flush=True)
    gl, gg, gimg = ctx.fused_loss_backward(params, targets, sigma, bgs, exact=exact, want_images=True)
    check_image(gimg, orc.render_batch(params, H, W, sigma, bgs), label=name)
    cl, cg = orc.loss_backward_batch(params, targets, sigma, bgs)
    check_losses(gl, cl, label=name)
    assert_grads(gg, cg, label=name)
    gin = ((synth.uniforms(9, B * H * W * 3) - 0.5) * 1e-3).reshape(B, H, W, 3).astype(np.float32)
    assert_grads(ctx.backward_from_grad(params, gin, sigma, bgs, exact=exact),
                 orc.backward_from_grad_batch(params, gin, sigma, bgs), label=f"{name} from_grad")


@pytest.mark.parametrize("name,B,H,W,T,sigma,kind", CASES, ids=[c[0] for c in CASES])
def test_segments_fixed_order_and_other_kernels(ctx, orc, name, B, H, W, T, sigma, kind, monkeypatch):
    params, bgs = make_case(B, H, W, T, kind, seed=600)
    targets = targets_for(orc, B, H, W, T, sigma, kind, bgs, seed=600)
    print(f"segments fixed order {name}", flush=True)
    gl, gg, gimg = ctx.fused_loss_backward(params, targets, sigma, bgs, want_images=True)
    d1 = ctx.fused_loss_backward(params, targets, sigma, bgs, deterministic=True)
    d2 = ctx.fused_loss_backward(params, targets, sigma, bgs, deterministic=True)
    assert np.array_equal(d1[0], d2[0]) and np.array_equal(d1[1], d2[1])
    assert np.array_equal(d1[0], gl)
    assert grad_err(gg, d1[1]) <= 1e-6
    cl, cg = orc.loss_backward_batch(params, targets, sigma, bgs)
    assert_grads(d1[1], cg, label=f"{name} fixed order")
    # the other fused kernels: the same composite, so the same image and
    # losses; gradients summed in another order
    monkeypatch.setenv("DRH_NO_SEGMENTS", "1")
    nl, ng, nimg = ctx.fused_loss_backward(params, targets, sigma, bgs, want_images=True)
    assert np.array_equal(gimg, nimg) and np.array_equal(gl, nl)
    assert grad_err(gg, ng) <= 1e-6
    nd = ctx.fused_loss_backward(params, targets, sigma, bgs, deterministic=True)
    assert np.array_equal(nd[0], d1[0])
    assert grad_err(nd[1], d1[1]) <= 1e-6


def test_segments_with_zero_factors_and_deep_stacks(ctx, orc):
    # Every 5th triangle opaque (alpha 1: exact zero factors where it covers a
    # pixel fully) and 160 large triangles per scene (transmittance products
    # below 2^-64, rescaled): every segment's backward starts from a prefix
    # with zero and rescaling counts.
    B, H, W, T, sigma = 2, 48, 40, 160, 0.003
    params, bgs = make_case(B, H, W, T, "uniform", seed=700, opaque_every=5)
    targets = targets_for(orc, B, H, W, T, sigma, "uniform", bgs, seed=700)
    print("segments with zero factors", flush=True)
    gl, gg, gimg = ctx.fused_loss_backward(params, targets, sigma, bgs, want_images=True)
    check_image(gimg, orc.render_batch(params, H, W, sigma, bgs), label="zero factors")
    cl, cg = orc.loss_backward_batch(params, targets, sigma, bgs)
    check_losses(gl, cl, label="zero factors")
    assert_grads(gg, cg, label="zero factors")
    dl, dg = ctx.fused_loss_backward(params, targets, sigma, bgs, deterministic=True)
    assert np.array_equal(dl, gl)
    assert_grads(dg, cg, label="zero factors, fixed order")
    # the zero loss of a scene against its own render (grad.rs:462-469): the
    # composite is the render's, bit for bit
    zl, zg = ctx.fused_loss_backward(params, gimg, sigma, bgs)
    assert np.all(zl == 0.0) and np.all(zg == 0.0)
