"""Pins for the CPU oracle beyond the reference's own tests.

Closed forms computed independently in float64, exact symmetries of the
reference's arithmetic, and finite differences. Each is chosen so that a
plausible restatement mistake (a swapped axis, a wrong compositing order, a
dropped chain-rule factor, a wrong bias correction) fails it.
"""

import math

import numpy as np
import pytest

from diffrast import synth


def tri(verts, color, alpha):
    return np.array([*np.ravel(verts), *color, alpha], np.float32)


def sig64(x):
    return 1.0 / (1.0 + math.exp(-x)) if x >= 0 else math.exp(x) / (1.0 + math.exp(x))


# ---- pixel_bounds (raster.rs:144-168) ----

def test_bounds_closed_form(orc):
    t = tri([[0.25, 0.25], [0.5, 0.25], [0.25, 0.5]], [1, 1, 1], 1)
    # pad = 0.06: floor((0.25-0.06)*64) = 12, ceil((0.5+0.06)*64)+1 = 37
    assert orc.pixel_bounds(t, 64, 64, 0.01) == (12, 12, 37, 37)
    # clipped at both sides, and x uses W while y uses H
    t2 = tri([[-0.5, 0.25], [1.5, 0.25], [0.5, 0.5]], [1, 1, 1], 1)
    assert orc.pixel_bounds(t2, 32, 64, 0.01) == (0, 12, 32, 37)


def test_bounds_cull_rules(orc):
    nan, inf = float("nan"), float("inf")
    assert orc.pixel_bounds(tri([[nan, 0.2], [0.5, 0.5], [0.6, 0.1]], [1] * 3, 1), 16, 16, 0.01) is None
    assert orc.pixel_bounds(tri([[inf, 0.2], [0.5, 0.5], [0.6, 0.1]], [1] * 3, 1), 16, 16, 0.01) is None
    assert orc.pixel_bounds(tri([[2.0, 2.0], [3.0, 2.0], [2.5, 3.0]], [1] * 3, 1), 16, 16, 0.01) is None
    # ceil((hi+pad)*W) >= 2**64 saturates, and the `+ 1` of a release build wraps to 0
    assert orc.pixel_bounds(tri([[0.1, 0.1], [1e20, 0.1], [0.2, 0.3]], [1] * 3, 1), 256, 256, 0.01) is None
    assert orc.pixel_bounds(tri([[0.1, 0.1], [1e15, 0.1], [0.2, 0.3]], [1] * 3, 1), 256, 256, 0.01)[2] == 256


# ---- coverage (raster.rs:74-134) ----

@pytest.mark.parametrize("py,sigma", [(0.25, 0.01), (0.21, 0.01), (0.3, 0.02), (0.203, 0.002)])
def test_coverage_inside_closed_form(orc, py, sigma):
    # the bottom edge y = 0.2 is the nearest edge for these points on x = 0.5
    t = tri([[0.2, 0.2], [0.8, 0.2], [0.5, 0.8]], [1, 0, 0], 1)
    d = py - 0.2
    assert abs(orc.coverage(t, 0.5, py, sigma) - sig64(d / sigma)) < 2e-6


@pytest.mark.parametrize("px,py", [(0.15, 0.15), (0.85, 0.1), (0.5, 0.85)])
def test_coverage_outside_near_vertex_closed_form(orc, px, py):
    v = np.array([[0.2, 0.2], [0.8, 0.2], [0.5, 0.8]])
    t = tri(v, [1, 0, 0], 1)
    d = min(np.hypot(px - v[:, 0], py - v[:, 1]))
    assert orc.signed_distance(t, px, py) < 0
    assert abs(orc.coverage(t, px, py, 0.05) - sig64(-d / 0.05)) < 2e-6


def test_point_triangle_counts_as_inside(orc):
    # All three crosses are 0 for coincident vertices, so is_inside() (raster.rs:111-116)
    # says inside and the coverage is sigmoid(+d/sigma) around the point.
    t = tri([[0.5, 0.5]] * 3, [1, 1, 1], 1)
    assert orc.signed_distance(t, 0.52, 0.5) > 0
    assert abs(orc.coverage(t, 0.52, 0.5, 0.01) - sig64(0.02 / 0.01)) < 2e-6


@pytest.mark.parametrize("px,py", [(0.45, 0.35), (0.3, 0.22), (0.1, 0.1), (0.62, 0.6), (0.5, 0.19)])
def test_coverage_gradient_matches_finite_differences(orc, px, py):
    t = tri([[0.2, 0.2], [0.8, 0.25], [0.45, 0.8]], [1, 0, 0], 1)
    sigma = 0.05
    _, d = orc.coverage_with_grad(t, px, py, sigma)
    eps = 1e-3
    for i in range(6):
        hi, lo = t.copy(), t.copy()
        hi[i] += eps
        lo[i] -= eps
        fd = (orc.coverage(hi, px, py, sigma) - orc.coverage(lo, px, py, sigma)) / (2 * eps)
        assert abs(d.ravel()[i] - fd) < 2e-3 + 2e-2 * abs(fd), (i, d.ravel()[i], fd)


# ---- exact symmetries of the arithmetic ----

def test_transpose_symmetry_is_exact(orc):
    p = synth.uniform_scene(5, 12)
    q = p.copy()
    q[:, [0, 2, 4]], q[:, [1, 3, 5]] = p[:, [1, 3, 5]], p[:, [0, 2, 4]]
    a = orc.render(p, 48, 48, 0.01)
    b = orc.render(q, 48, 48, 0.01)
    assert np.array_equal(a, b.transpose(1, 0, 2))


def test_vertex_rotation_is_exact(orc):
    p = synth.uniform_scene(6, 12)
    q = p.copy()
    q[:, 0:6] = np.roll(p[:, 0:6], -2, axis=1)
    assert np.array_equal(orc.render(p, 40, 40, 0.01), orc.render(q, 40, 40, 0.01))


def test_whole_pixel_translation_is_exact(orc):
    # Coordinates on a 2**-12 grid make the shift exact, so only the pixel
    # indexing can break equality.
    p = synth.uniform_scene(7, 8)
    p[:, :6] = np.round(p[:, :6] * 0.5 * 4096) / 4096 + 0.125
    q = p.copy()
    q[:, [0, 2, 4]] += np.float32(8 / 64)
    q[:, [1, 3, 5]] += np.float32(4 / 64)
    a = orc.render(p, 64, 64, 0.004)
    b = orc.render(q, 64, 64, 0.004)
    assert np.array_equal(a[10:50, 10:50], b[14:54, 18:58])


# ---- compositing order (raster.rs:37-68): index 0 is the back ----

def test_two_layer_over_closed_form(orc):
    back = tri([[0.0, 0.0], [1.0, 0.0], [0.0, 1.0]], [0.9, 0.1, 0.2], 0.6)
    front = tri([[1.0, 1.0], [0.0, 1.0], [1.0, 0.0]], [0.1, 0.7, 0.4], 0.3)
    big = tri([[-1, -1], [3, -1], [-1, 3]], [0.2, 0.3, 0.9], 0.5)
    bg = np.array([0.05, 0.1, 0.15])
    img = orc.render(np.stack([back, big, front]), 32, 32, 0.002, bg)
    # pixel (4, 4) is deep inside `back` and `big`, far outside `front`
    expect = bg * (1 - 0.6) + np.array([0.9, 0.1, 0.2]) * 0.6
    expect = expect * (1 - 0.5) + np.array([0.2, 0.3, 0.9]) * 0.5
    assert np.allclose(img[4, 4], expect, atol=1e-6)
    # pixel (28, 28): front + big only
    expect = bg * 0.5 + np.array([0.2, 0.3, 0.9]) * 0.5
    expect = expect * (1 - 0.3) + np.array([0.1, 0.7, 0.4]) * 0.3
    assert np.allclose(img[28, 28], expect, atol=1e-6)


def test_per_item_backgrounds(orc):
    p = synth.batch("uniform", 3, 6, 11)
    bgs = np.array([[0.1, 0.2, 0.3], [0.9, 0.5, 0.0], [0.3, 0.3, 0.3]], np.float32)
    out = orc.render_batch(p, 20, 24, 0.01, bgs)
    for b in range(3):
        assert np.array_equal(out[b], orc.render(p[b], 20, 24, 0.01, bgs[b]))


# ---- gradients (grad.rs:98-182) ----

def single_tri_case(orc, alpha):
    t = tri([[0.15, 0.2], [0.85, 0.3], [0.4, 0.85]], [0.8, 0.3, 0.1], alpha)
    bg = np.array([0.1, 0.2, 0.6], np.float32)
    target = synth.uniforms(3, 32 * 32 * 3).reshape(32, 32, 3).astype(np.float32)
    loss, g, img = orc.loss_backward(t[None], target, 0.02, bg, want_image=True)
    return t, bg, target, loss, g, img


def test_single_triangle_color_and_alpha_gradients_closed_form(orc):
    t, bg, target, loss, g, img = single_tri_case(orc, 0.7)
    r = img.astype(np.float64)
    # r = c w + bg (1 - w)  =>  w = (r - bg) / (c - bg), per channel (here channel 0)
    w = (r[..., 0] - bg[0]) / (t[6] - bg[0])
    scale = 2.0 / r.size
    resid = scale * (r - target)
    for ch in range(3):
        expect = float(np.sum(resid[..., ch] * w))
        assert abs(g[0, 6 + ch] - expect) <= 1e-5 * max(abs(expect), 1e-3)
    cov = w / 0.7
    expect_a = float(np.sum(resid * (t[6:9] - bg)[None, None, :] * cov[..., None]))
    assert abs(g[0, 9] - expect_a) <= 1e-5 * max(abs(expect_a), 1e-3)
    assert abs(loss - np.mean((r - target) ** 2)) < 1e-7


def box_is_locally_constant(orc, p, i, eps, H, W, sigma):
    """The integer cull box (raster.rs:144-168) jumps when a vertex crosses a
    pixel boundary, and the pixels it adds still carry ~2.5e-3 coverage, so the
    loss is discontinuous there and a central difference straddling the jump
    measures the step, not the slope. Such parameters are left out of FD checks."""
    k, j = divmod(i, 10)
    base = orc.pixel_bounds(p[k], W, H, sigma)
    for s in (eps, -eps):
        q = p[k].copy()
        q[j] += s
        if orc.pixel_bounds(q, W, H, sigma) != base:
            return False
    return True


def test_multi_layer_gradient_matches_finite_differences(orc):
    p = synth.uniform_scene(21, 6)
    p[:, :6] = p[:, :6] * 0.6 + 0.2
    target = synth.uniforms(22, 28 * 28 * 3).reshape(28, 28, 3).astype(np.float32)
    _, a = orc.loss_backward(p, target, 0.025, (0.3, 0.3, 0.3))
    _, n = orc.finite_difference(p, target, 0.025, 1e-4, (0.3, 0.3, 0.3))
    keep = [i for i in range(p.size) if box_is_locally_constant(orc, p, i, 1e-4, 28, 28, 0.025)]
    assert len(keep) > 0.8 * p.size
    a, n = a.ravel()[keep].astype(np.float64), n.ravel()[keep].astype(np.float64)
    assert np.linalg.norm(a - n) / np.linalg.norm(n) < 0.02
    assert a @ n / (np.linalg.norm(a) * np.linalg.norm(n)) > 0.999


def test_backward_from_grad_agrees_with_the_loss_path(orc):
    p = synth.uniform_scene(31, 10)
    target = synth.uniforms(32, 24 * 30 * 3).reshape(24, 30, 3).astype(np.float32)
    _, g_loss, img = orc.loss_backward(p, target, 0.01, want_image=True)
    gin = (np.float32(2.0 / img.size) * (img - target)).astype(np.float32)
    direct = orc.backward_from_grad(p, gin, 0.01)
    inverted = orc.backward_from_grad(p, gin, 0.01, inverted=True)
    norm = np.linalg.norm(g_loss)
    assert np.abs(direct - g_loss).max() / norm < 1e-6
    assert np.abs(inverted - g_loss).max() / norm < 1e-4


def test_backward_is_linear_in_the_upstream_gradient(orc):
    p = synth.uniform_scene(41, 10)
    g1 = (synth.uniforms(42, 20 * 20 * 3).reshape(20, 20, 3) - 0.5).astype(np.float32)
    g2 = (synth.uniforms(43, 20 * 20 * 3).reshape(20, 20, 3) - 0.5).astype(np.float32)
    a = orc.backward_from_grad(p, g1, 0.01).astype(np.float64)
    b = orc.backward_from_grad(p, g2, 0.01).astype(np.float64)
    c = orc.backward_from_grad(p, (2 * g1 - 3 * g2).astype(np.float32), 0.01)
    assert np.abs(c - (2 * a - 3 * b)).max() / np.linalg.norm(c) < 1e-5


def test_nan_alpha_paints_in_render_and_is_culled_by_the_tape(orc):
    t = tri([[0.2, 0.2], [0.8, 0.2], [0.5, 0.8]], [1, 0, 0], float("nan"))
    img = orc.render(t[None], 16, 16, 0.01)
    assert np.isnan(img[8, 8]).all()  # raster.rs:48-51: `alpha <= 0` is false for NaN
    target = np.zeros((16, 16, 3), np.float32)
    loss, g, taped = orc.loss_backward(t[None], target, 0.01, want_image=True)
    assert np.all(taped == 0) and loss == 0 and np.all(g == 0)  # grad.rs:61-62


# ---- optimizer and schedule (optim.rs, fit.rs) ----

def test_adam_constant_gradient_closed_form(orc):
    # With a constant gradient the bias-corrected moments equal g and g^2, so
    # each step moves lr * g / (|g| + eps): a wrong bias correction fails this.
    adam = orc.Adam(3)
    p = np.zeros(3, np.float32)
    g = np.array([0.5, -2.0, 1e-3], np.float32)
    lr = np.array([0.1, 0.01, 0.05], np.float32)
    for _ in range(10):
        adam.step(p, g, lr)
    expect = -10 * lr * g / (np.abs(g) + 1e-8)
    assert np.allclose(p, expect, rtol=2e-5, atol=0)


def test_sigma_schedule_matches_the_geometric_form(orc):
    for i in range(0, 800, 37):
        expect = 0.02 * (0.0015 / 0.02) ** (i / 799)
        assert abs(orc.sigma_at(0.02, 0.0015, 800, i) - expect) < 1e-6 * expect


def test_mse_matches_float64(orc):
    a = synth.uniforms(51, 3000).astype(np.float32)
    b = synth.uniforms(52, 3000).astype(np.float32)
    expect = np.mean((a - b).astype(np.float64) ** 2)
    assert abs(orc.mse(a, b) - expect) <= 1e-7 * expect


def test_mean_color_and_sample(orc):
    img = synth.blob_target(3, 20, 30)
    assert np.allclose(orc.mean_color(img), img.reshape(-1, 3).astype(np.float64).mean(0), atol=1e-7)
    assert np.array_equal(synth.mean_color(img), orc.mean_color(img))
    for x, y in [(0.0, 0.0), (0.999, 0.5), (1.5, -0.3), (0.51, 0.49)]:
        assert np.array_equal(orc.sample(img, x, y), synth.sample(img, x, y))


def test_sample_truncates_toward_zero_and_clamps(orc):
    # fit.rs:381-385: `(x * W as f32) as isize`, clamped to [0, W - 1]; Rust's
    # float-to-int cast truncates toward zero, saturates, and sends NaN to 0.
    # The image stores each pixel's own column and row, so the sample names
    # the pixel it read.
    H, W = 7, 11
    img = np.zeros((H, W, 3), np.float32)
    img[..., 0] = np.arange(W, dtype=np.float32)[None, :]
    img[..., 1] = np.arange(H, dtype=np.float32)[:, None]
    img[..., 2] = 5.0
    nan, inf = float("nan"), float("inf")
    cases = [  # (x, y, column, row)
        (0.0, 0.0, 0, 0),
        (0.5, 0.5, 5, 3),              # 5.5 and 3.5 truncate; x scales by W, y by H
        (2.99 / W, 4.999 / H, 2, 4),   # truncation, not rounding
        (-0.05, -0.1, 0, 0),           # -0.55 and -0.7 truncate to 0
        (-0.5, -3.0, 0, 0),            # negative: clamped to 0
        (1.0, 1.0, W - 1, H - 1),      # exactly 1: W and H, clamped to the last pixel
        (1.5, 2.0, W - 1, H - 1),      # above 1: clamped
        (nan, nan, 0, 0),              # NaN casts to 0
        (inf, -inf, W - 1, 0),         # saturating casts
        (0.95, 0.0, 10, 0),            # 10.45 -> 10
    ]
    for x, y, cx, cy in cases:
        got = orc.sample(img, x, y)
        assert got.tolist() == [float(cx), float(cy), 5.0], (x, y, got)
        assert np.array_equal(synth.sample(img, x, y), got), (x, y)
