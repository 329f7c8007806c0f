"""A render kept for its backward pass (drh_render_record / drh_backward_recorded).

The reference has no such pair: its PyTorch op renders in forward and renders the batch
again in backward (python/diffrast/torch_layer.py:40-66, via backward_batch,
crates/diffrast-py/src/lib.rs:245-324). The pair must therefore give what that
render + re-render path gives: the image of drh_render bit for bit, and, under
DRH_DETERMINISTIC (a fixed summation order), the gradients of drh_backward_from_grad bit
for bit; both are also checked against the oracle at this path's bars (images 1e-5,
gradients 1e-4 of the scene's gradient norm).
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
    """Per-scene max |d| / ||g_cpu||_2, worst over the batch."""
    worst = 0.0
    for a, b in zip(np.asarray(gpu, np.float64).reshape(len(gpu), -1),
                    np.asarray(cpu, np.float64).reshape(len(cpu), -1)):
        worst = max(worst, float(np.abs(a - b).max()) / max(np.linalg.norm(b), 1e-12) if a.size else 0.0)
    return worst


def both_paths(ctx, params, bgs, grad_images, H, W, sigma, flags=0, backwards=1):
    """(record image, [record grads per backward call], render image, from_grad grads), numpy."""
    import torch

    dev = torch.device("cuda:0")
    B, T = params.shape[0], params.shape[1]
    p = torch.from_numpy(np.ascontiguousarray(params, np.float32)).to(dev)
    bg = torch.from_numpy(np.ascontiguousarray(bgs, np.float32)).to(dev)
    gi = torch.from_numpy(np.ascontiguousarray(grad_images, np.float32)).to(dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    n = _lib.record_bytes(B, T, H, W)
    rec = torch.empty((n,), dtype=torch.uint8, device=dev)
    shape = (B, 3, H, W) if flags & _lib.CHANNELS_FIRST else (B, H, W, 3)
    img_r, img_a = torch.empty(shape, device=dev), torch.empty(shape, device=dev)
    print(f"record B={B} T={T} {H}x{W} sigma={sigma} flags={flags:#x} bytes={n}", flush=True)
    ctx.render_record_ptr(p.data_ptr(), bg.data_ptr(), B, T, H, W, sigma, img_r.data_ptr(), rec.data_ptr(), n,
                          s, flags)
    grads_r = []
    for _ in range(backwards):
        g = torch.full((B, T, 10), 7.0, device=dev)  # the call must overwrite every value
        ctx.backward_recorded_ptr(rec.data_ptr(), n, gi.data_ptr(), B, T, H, W, sigma, g.data_ptr(), s, flags)
        grads_r.append(g)
    ctx.render_ptr(p.data_ptr(), bg.data_ptr(), B, T, H, W, sigma, img_a.data_ptr(), s, flags)
    grads_a = torch.empty((B, T, 10), device=dev)
    ctx.from_grad_ptr(p.data_ptr(), bg.data_ptr(), gi.data_ptr(), B, T, H, W, sigma, grads_a.data_ptr(), s, flags)
    torch.cuda.synchronize()
    return (img_r.cpu().numpy(), [g.cpu().numpy() for g in grads_r], img_a.cpu().numpy(),
            grads_a.cpu().numpy())


@pytest.fixture(autouse=True)
def _sequential_rows(monkeypatch):
    # The recorded backward sums its fixed-order rows per 16x16 block, as the
    # fused kernels other than fused_seg_kernel do (which small grids take by
    # default, with rows per 8x8 tile): those are the path these tests compare
    # it with bit for bit.
    monkeypatch.setenv("DRH_NO_SEGMENTS", "1")


def case(B, H, W, T, kind, seed):
    params = synth.batch(kind, B, T, seed)
    bgs = synth.uniforms(seed + 7, B * 3).reshape(B, 3).astype(np.float32)
    gi = np.random.default_rng(seed).standard_normal((B, H, W, 3)).astype(np.float32) * 1e-3
    return params, bgs, gi


@pytest.mark.parametrize("exact", [False, True], ids=["fast", "exact"])
@pytest.mark.parametrize("B,H,W,T,sigma,kind", [
    (4, 128, 128, 64, 0.0015, "uniform"),
    (2, 37, 53, 200, 0.004, "small"),
    (1, 64, 64, 32, 0.02, "uniform"),
])
def test_record_path_equals_the_render_and_rerender_path(ctx, orc, B, H, W, T, sigma, kind, exact, monkeypatch):
    params, bgs, gi = case(B, H, W, T, kind, 40 + T)
    flags = _lib.DETERMINISTIC | (_lib.EXACT_MATH if exact else 0)
    # bit-equal to the other fused kernels (the fixture), and to
    # fused_seg_kernel up to the association of its per-tile rows
    monkeypatch.delenv("DRH_NO_SEGMENTS")
    img_s, _, _, g_s = both_paths(ctx, params, bgs, gi, H, W, sigma, flags)
    monkeypatch.setenv("DRH_NO_SEGMENTS", "1")
    img_r, (g_r,), img_a, g_a = both_paths(ctx, params, bgs, gi, H, W, sigma, flags)
    assert np.array_equal(img_r, img_a) and np.array_equal(img_s, img_r)
    assert np.array_equal(g_r, g_a)
    assert grad_err(g_s, g_r) <= 1e-6
    assert np.abs(img_r - orc.render_batch(params, H, W, sigma, bgs)).max() <= IMG_TOL
    assert grad_err(g_r, orc.backward_from_grad_batch(params, gi, sigma, bgs)) <= GRAD_RTOL


def test_record_path_with_atomics(ctx, orc):
    # the default summation (float atomics): equal to the other path up to the order of the adds
    params, bgs, gi = case(3, 96, 80, 128, "uniform", 5)
    img_r, (g_r,), img_a, g_a = both_paths(ctx, params, bgs, gi, 96, 80, 0.002)
    assert np.array_equal(img_r, img_a)
    assert grad_err(g_r, g_a) <= 1e-6
    assert grad_err(g_r, orc.backward_from_grad_batch(params, gi, 0.002, bgs)) <= GRAD_RTOL


def test_one_record_serves_repeated_backward_calls(ctx):
    params, bgs, gi = case(2, 48, 48, 40, "uniform", 9)
    _, grads, _, g_a = both_paths(ctx, params, bgs, gi, 48, 48, 0.004, _lib.DETERMINISTIC, backwards=3)
    for g in grads:
        assert np.array_equal(g, g_a)


def test_channels_first_record(ctx):
    params, bgs, gi = case(2, 33, 41, 50, "uniform", 3)
    gi_chw = np.ascontiguousarray(gi.transpose(0, 3, 1, 2))
    flags = _lib.DETERMINISTIC | _lib.CHANNELS_FIRST
    img_r, (g_r,), img_a, g_a = both_paths(ctx, params, bgs, gi_chw, 33, 41, 0.004, flags)
    assert img_r.shape == (2, 3, 33, 41)
    assert np.array_equal(img_r, img_a) and np.array_equal(g_r, g_a)
    img_h, (g_h,), _, _ = both_paths(ctx, params, bgs, gi, 33, 41, 0.004, _lib.DETERMINISTIC)
    assert np.array_equal(img_r, img_h.transpose(0, 3, 1, 2)) and np.array_equal(g_r, g_h)


def test_nan_alpha_is_drawn_but_not_differentiated(ctx, orc):
    # render composites a NaN alpha (raster.rs:48-51); the taped forward culls it
    # (grad.rs:61-62): the record's image and gradients each follow their path
    params, bgs, gi = case(1, 24, 24, 6, "uniform", 12)
    params[0, 2, 9] = float("nan")
    img_r, (g_r,), img_a, g_a = both_paths(ctx, params, bgs, gi, 24, 24, 0.01, _lib.DETERMINISTIC)
    assert np.array_equal(np.isnan(img_r), np.isnan(img_a)) and np.isnan(img_r).any()
    ok = ~np.isnan(img_a)
    assert np.array_equal(img_r[ok], img_a[ok])
    assert np.isfinite(g_r).all() and np.array_equal(g_r, g_a) and np.all(g_r[0, 2] == 0)
    assert grad_err(g_r, orc.backward_from_grad_batch(params, gi, 0.01, bgs)) <= GRAD_RTOL


def test_record_past_the_recorded_entries(ctx, orc, monkeypatch):
    # a record sized below T entries per tile: the backward kernel rebuilds the rest
    params, bgs, gi = case(2, 40, 48, 300, "small", 21)
    want = orc.backward_from_grad_batch(params, gi, 0.004, bgs)
    full = _lib.record_bytes(2, 300, 40, 48)
    for cap in ("3", "40"):
        monkeypatch.setenv("DRH_MAX_TILE_ENTRIES", cap)
        assert _lib.record_bytes(2, 300, 40, 48) < full
        img_r, (g_r,), img_a, g_a = both_paths(ctx, params, bgs, gi, 40, 48, 0.004, _lib.DETERMINISTIC)
        assert np.array_equal(img_r, img_a) and np.array_equal(g_r, g_a)
        assert grad_err(g_r, want) <= GRAD_RTOL


def test_record_arguments_are_checked(ctx):
    import torch

    dev = torch.device("cuda:0")
    B, T, H, W = 2, 8, 16, 16
    n = _lib.record_bytes(B, T, H, W)
    rec = torch.empty((n + 512,), dtype=torch.uint8, device=dev)
    p = torch.zeros((B, T, 10), device=dev)
    bg = torch.zeros((B, 3), device=dev)
    img = torch.empty((B, H, W, 3), device=dev)
    g = torch.empty((B, T, 10), device=dev)
    with pytest.raises(_lib.DiffrastError) as e:  # wrong size
        ctx.render_record_ptr(p.data_ptr(), bg.data_ptr(), B, T, H, W, 0.01, img.data_ptr(), rec.data_ptr(),
                              n + 256, None, _lib.SYNC)
    assert e.value.code == 6
    with pytest.raises(_lib.DiffrastError) as e:  # misaligned
        ctx.render_record_ptr(p.data_ptr(), bg.data_ptr(), B, T, H, W, 0.01, img.data_ptr(),
                              rec.data_ptr() + 4, n, None, _lib.SYNC)
    assert e.value.code == 6
    with pytest.raises(_lib.DiffrastError) as e:  # sizes that do not match the record
        ctx.backward_recorded_ptr(rec.data_ptr(), n, img.data_ptr(), B, T, H + 8, W, 0.01, g.data_ptr(), None,
                                  _lib.SYNC)
    assert e.value.code == 6
    with pytest.raises(_lib.DiffrastError) as e:
        ctx.backward_recorded_ptr(None, n, img.data_ptr(), B, T, H, W, 0.01, g.data_ptr(), None, _lib.SYNC)
    assert e.value.code == 6


def test_torch_op_keeps_the_record_only_when_autograd_needs_it(orc):
    import torch

    from diffrast import torch_layer as tl

    dev = torch.device("cuda:0")
    params, bgs, gi = case(2, 40, 56, 48, "uniform", 31)
    bg = tuple(float(v) for v in bgs[0])
    p = torch.from_numpy(params).to(dev).requires_grad_(True)
    upstream = torch.from_numpy(gi.transpose(0, 3, 1, 2).copy()).to(dev)
    img = tl.rasterize(p, 40, 56, sigma=0.004, background=bg)
    assert len(img.grad_fn.saved_tensors) == 2  # params and the record
    (img * upstream).sum().backward()
    want = orc.backward_from_grad_batch(params, gi, 0.004, np.broadcast_to(bgs[0], (2, 3)))
    assert grad_err(p.grad.cpu().numpy(), want) <= GRAD_RTOL
    with torch.no_grad():
        img2 = tl.rasterize(p, 40, 56, sigma=0.004, background=bg)
    assert img2.grad_fn is None and torch.equal(img2, img.detach())
    # without the record (the re-rendering backward) the gradients agree
    q = p.detach().clone().requires_grad_(True)
    img3 = tl._Rasterize.apply(q, 40, 56, 0.004, bg, "gpu", True, False)
    assert len(img3.grad_fn.saved_tensors) == 1
    (img3 * upstream).sum().backward()
    assert grad_err(q.grad.cpu().numpy(), p.grad.cpu().numpy()) <= 1e-6
