"""The raster kernels' heaviest-first block order, through every path that makes it.

setup_records orders the blocks of a batch (B > 1) whose grid has more blocks than
the device has CUs (256 on MI355X): the backward kernel always follows the order, the
forward kernel when T <= 256, and the one-wave fused kernel an order of 8x8 tiles where
the scene's tile grid fits the order's cells (else the block order, four tiles per
block). The order only changes which tile a launch slot works on, so every result must
equal the oracle's at this path's bars (images 1e-5, gradients 1e-4 of the scene's
gradient norm), and, with DRH_DETERMINISTIC, be bit-identical from call to call. The
cases are sized to take the ordered paths: 4 scenes of 160 x 200 px are 4 x 10 x 13 =
520 blocks; 2 scenes of 720 x 768 px have 90 x 96 tiles each, past the tile order's
8192 cells, so their one-wave fused kernel takes the block order; 2 scenes of 1100
small triangles take the order workgroup's triangles in three batches of up to 512
and the records in nine workgroups of 128. From 256 triangles on, the one-wave
fused kernel's lists scan only the triangles of their tile row, which setup_records
lists (the small-triangle cases, and 300 large triangles at 256 x 256).
"""

import numpy as np
import pytest

from diffrast import _lib, synth

pytestmark = pytest.mark.gpu

IMG_TOL = 1e-5
GRAD_RTOL = 1e-4


@pytest.fixture(scope="module")
def ctx():
    c = _lib.Context()
    yield c
    c.close()


def grad_err(gpu, cpu):
    worst = 0.0
    for a, b in zip(np.asarray(gpu, np.float64).reshape(len(gpu), -1),
                    np.asarray(cpu, np.float64).reshape(len(cpu), -1)):
        worst = max(worst, float(np.abs(a - b).max()) / max(np.linalg.norm(b), 1e-12) if a.size else 0.0)
    return worst


def scenes(kind, B, T, seed):
    params = synth.batch(kind, B, T, seed)
    bgs = synth.uniforms(seed + 7, B * 3).reshape(B, 3).astype(np.float32)
    return params, bgs


# (kind, B, H, W, T, sigma): forward and backward ordered; backward only (T > 256)
CASES = [("uniform", 4, 160, 200, 100, 0.002), ("small", 3, 200, 208, 300, 0.003),
         ("uniform", 2, 720, 768, 40, 0.002), ("small", 2, 256, 256, 1100, 0.002),
         ("uniform", 2, 256, 256, 300, 0.002)]


@pytest.mark.parametrize("kind,B,H,W,T,sigma", CASES,
                         ids=["ordered", "backward-ordered", "large-block-order", "many-triangles", "row-lists-large"])
def test_ordered_render_fused_and_from_grad_match_oracle(ctx, orc, kind, B, H, W, T, sigma):
    assert B * -(-H // 16) * -(-W // 16) > 256  # more blocks than CUs: the order is made
    params, bgs = scenes(kind, B, T, 50)
    print(f"order {kind} B={B} {H}x{W} T={T}", flush=True)
    img = ctx.render(params, H, W, sigma, bgs)
    want_img = orc.render_batch(params, H, W, sigma, bgs)
    assert np.abs(img - want_img).max() <= IMG_TOL
    targets = orc.render_batch(synth.batch(kind, B, T, 51), H, W, sigma, bgs)
    for det in (False, True):
        losses, grads = ctx.fused_loss_backward(params, targets, sigma, bgs, deterministic=det)
        cl, cg = orc.loss_backward_batch(params, targets, sigma, bgs)
        assert np.all(np.abs(losses - cl) <= 1e-4 * np.abs(cl) + 1e-7)
        assert grad_err(grads, cg) <= GRAD_RTOL
    gi = np.random.default_rng(3).standard_normal((B, H, W, 3)).astype(np.float32) * 1e-3
    g = ctx.backward_from_grad(params, gi, sigma, bgs)
    assert grad_err(g, orc.backward_from_grad_batch(params, gi, sigma, bgs)) <= GRAD_RTOL


def test_ordered_results_repeat_bit_for_bit(ctx):
    # the order comes from the scenes alone, and a deterministic sum does not
    # depend on it: two calls agree exactly
    params, bgs = scenes("uniform", 4, 100, 60)
    targets = synth.batch("uniform", 4, 100, 61)
    targets = ctx.render(targets, 160, 200, 0.002, bgs)
    a = ctx.fused_loss_backward(params, targets, 0.002, bgs, deterministic=True)
    b = ctx.fused_loss_backward(params, targets, 0.002, bgs, deterministic=True)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    assert np.array_equal(ctx.render(params, 160, 200, 0.002, bgs), ctx.render(params, 160, 200, 0.002, bgs))


def test_ordered_record_path(ctx, orc):
    # the order kept in a forward record serves its backward
    import torch

    B, H, W, T, sigma = 4, 160, 200, 100, 0.002
    params, bgs = scenes("uniform", B, T, 70)
    gi = np.random.default_rng(4).standard_normal((B, H, W, 3)).astype(np.float32) * 1e-3
    dev = torch.device("cuda:0")
    p, bg, g = (torch.from_numpy(x).to(dev) for x in (params, bgs, gi))
    s = torch.cuda.current_stream(dev).cuda_stream
    n = _lib.record_bytes(B, T, H, W)
    rec = torch.empty((n,), dtype=torch.uint8, device=dev)
    img = torch.empty((B, H, W, 3), device=dev)
    out = torch.empty((B, T, 10), device=dev)
    ctx.render_record_ptr(p.data_ptr(), bg.data_ptr(), B, T, H, W, sigma, img.data_ptr(), rec.data_ptr(), n, s)
    ctx.backward_recorded_ptr(rec.data_ptr(), n, g.data_ptr(), B, T, H, W, sigma, out.data_ptr(), s,
                              _lib.DETERMINISTIC)
    ref = torch.empty_like(out)
    ctx.from_grad_ptr(p.data_ptr(), bg.data_ptr(), g.data_ptr(), B, T, H, W, sigma, ref.data_ptr(), s,
                      _lib.DETERMINISTIC)
    torch.cuda.synchronize()
    assert np.abs(img.cpu().numpy() - orc.render_batch(params, H, W, sigma, bgs)).max() <= IMG_TOL
    assert torch.equal(out, ref)
    assert grad_err(out.cpu().numpy(), orc.backward_from_grad_batch(params, gi, sigma, bgs)) <= GRAD_RTOL
