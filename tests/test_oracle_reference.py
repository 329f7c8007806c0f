"""The reference's own tests, restated against the CPU oracle.

Each test names the reference test it ports (file:line). These literal scenes
are the reference's only fixtures (it ships no golden files), so they are what
pins the oracle to the reference's behaviour. Scenes the reference draws from
rand::StdRng use this repository's seeded generator instead; the properties
asserted are the reference's.
"""

import numpy as np
import pytest

from diffrast import synth


def tri(verts, color, alpha):
    return np.array([*np.ravel(verts), *color, alpha], np.float32)


UNIT_TRI = tri([[0.2, 0.2], [0.8, 0.2], [0.5, 0.8]], [1.0, 0.0, 0.0], 1.0)  # raster.rs:174-176


# ---------------- raster.rs:170-241 ----------------

def test_centroid_is_inside_and_far_corner_is_outside(orc):  # raster.rs:178-183
    assert orc.signed_distance(UNIT_TRI, 0.5, 0.4) > 0
    assert orc.signed_distance(UNIT_TRI, 0.0, 0.0) < 0


def test_coverage_is_half_on_the_edge(orc):  # raster.rs:185-191
    c = orc.coverage(UNIT_TRI, 0.5, 0.2, 0.01)
    assert abs(c - 0.5) < 1e-4


def test_coverage_saturates_away_from_the_edge(orc):  # raster.rs:193-198
    assert orc.coverage(UNIT_TRI, 0.5, 0.4, 0.002) > 0.999
    assert orc.coverage(UNIT_TRI, 0.02, 0.98, 0.002) < 1e-3


def test_winding_order_does_not_matter(orc):  # raster.rs:200-210
    flipped = UNIT_TRI.copy()
    flipped[[0, 1, 2, 3]] = UNIT_TRI[[2, 3, 0, 1]]
    a = orc.signed_distance(UNIT_TRI, 0.5, 0.4)
    b = orc.signed_distance(flipped, 0.5, 0.4)
    assert (a > 0) == (b > 0)


def test_opaque_triangle_paints_over_background(orc):  # raster.rs:212-220
    img = orc.render(UNIT_TRI[None], 64, 64, 0.002)
    inside = img[25, 32]
    assert inside[0] > 0.99 and inside[1] < 0.01
    assert list(img[63, 0]) == [0.0, 0.0, 0.0]


def test_offscreen_triangle_is_culled(orc):  # raster.rs:233-240
    t = tri([[5.0, 5.0], [6.0, 5.0], [5.5, 6.0]], [1.0] * 3, 1.0)
    img = orc.render(t[None], 32, 32, 0.01, background=(0.1, 0.1, 0.1))
    assert np.all(np.abs(img - 0.1) < 1e-6)


# ---------------- grad.rs:325-495 ----------------

def scene_pair(orc, sigma):  # grad.rs:329-346
    W = H = 48
    bg = (0.1, 0.12, 0.15)
    target_scene = np.stack([
        tri([[0.25, 0.30], [0.80, 0.22], [0.55, 0.78]], [0.9, 0.3, 0.2], 0.8),
        tri([[0.15, 0.60], [0.70, 0.65], [0.40, 0.20]], [0.2, 0.6, 0.9], 0.6),
    ])
    target = orc.render(target_scene, H, W, sigma, bg)
    scene = np.stack([
        tri([[0.21, 0.34], [0.77, 0.26], [0.58, 0.72]], [0.7, 0.4, 0.3], 0.7),
        tri([[0.18, 0.55], [0.66, 0.69], [0.44, 0.24]], [0.3, 0.5, 0.8], 0.5),
    ])
    return scene, target, bg


def test_tape_render_matches_plain_render(orc):  # grad.rs:348-354
    scene, target, bg = scene_pair(orc, 0.02)
    plain = orc.render(scene, 48, 48, 0.02, bg)
    _, _, taped = orc.loss_backward(scene, target, 0.02, bg, want_image=True)
    assert np.array_equal(plain, taped)


def test_analytic_gradient_matches_finite_differences(orc):  # grad.rs:356-374
    scene, target, bg = scene_pair(orc, 0.03)
    loss, analytic = orc.loss_backward(scene, target, 0.03, bg)
    fd_loss, numeric = orc.finite_difference(scene, target, 0.03, 1e-3, bg)
    assert abs(loss - fd_loss) < 1e-6
    norm = max(float(np.sqrt(np.sum(numeric.astype(np.float32) ** 2))), 1e-8)
    err = np.abs(analytic - numeric) / norm
    assert err.max() < 0.02, err


def test_color_gradient_is_exact_for_a_single_triangle(orc):  # grad.rs:376-399
    t = tri([[0.2, 0.25], [0.85, 0.35], [0.5, 0.8]], [0.6, 0.4, 0.2], 1.0)
    tt = t.copy()
    tt[6:9] = [0.1, 0.9, 0.5]
    target = orc.render(tt[None], 32, 32, 0.02)
    _, analytic = orc.loss_backward(t[None], target, 0.02)
    _, numeric = orc.finite_difference(t[None], target, 0.02, 1e-3)
    for ch in range(3):
        a, n = analytic[0, 6 + ch], numeric[0, 6 + ch]
        assert abs(a - n) / max(abs(n), 1e-6) < 0.01


def test_batch_gradients_match_sequential_ones(orc):  # grad.rs:401-420
    scene, target, bg = scene_pair(orc, 0.02)
    losses, grads = orc.loss_backward_batch(np.stack([scene] * 4), np.stack([target] * 4), 0.02, bg)
    loss, g = orc.loss_backward(scene, target, 0.02, bg)
    for i in range(4):
        assert losses[i] == np.float32(loss)
        assert np.array_equal(grads[i], g)


def test_batch_render_matches_sequential_render(orc):  # grad.rs:422-430
    scene, _, bg = scene_pair(orc, 0.01)
    batched = orc.render_batch(np.stack([scene] * 3), 48, 48, 0.01, bg)
    single = orc.render(scene, 48, 48, 0.01, bg)
    for img in batched:
        assert np.array_equal(img, single)


def test_batch_preserves_input_order(orc):  # grad.rs:432-453
    scenes, targets, bgs = [], [], []
    for i in range(6):
        shade = i / 6.0
        scenes.append(tri([[0.2, 0.2], [0.8, 0.3], [0.5, 0.8]], [1.0, 0.0, 0.0], 0.5)[None])
        bgs.append([shade] * 3)
        targets.append(np.full((16, 16, 3), [1.0 - shade, 0.5, 0.5], np.float32))
    losses, _ = orc.loss_backward_batch(np.stack(scenes), np.stack(targets), 0.02, np.array(bgs))
    for i in range(6):
        expected, _ = orc.loss_backward(scenes[i], targets[i], 0.02, bgs[i])
        assert losses[i] == np.float32(expected), f"item {i} out of order"


def test_zero_loss_gives_zero_gradient(orc):  # grad.rs:462-469
    scene, _, bg = scene_pair(orc, 0.02)
    rendered = orc.render(scene, 48, 48, 0.02, bg)
    loss, grads = orc.loss_backward(scene, rendered, 0.02, bg)
    assert loss == 0.0
    assert np.all(grads == 0.0)


def test_clamped_alpha_receives_no_gradient(orc):  # grad.rs:471-481
    t = tri([[0.2, 0.2], [0.8, 0.3], [0.5, 0.8]], [1.0, 0.0, 0.0], 1.0)
    target = np.full((32, 32, 3), [0.0, 0.0, 1.0], np.float32)
    _, grads = orc.loss_backward(t[None], target, 0.02)
    assert grads[0, 9] == 0.0


def test_culled_triangle_contributes_no_gradient(orc):  # grad.rs:483-494
    t = tri([[5.0, 5.0], [6.0, 5.0], [5.5, 6.0]], [1.0] * 3, 1.0)
    target = np.full((32, 32, 3), 0.9, np.float32)
    c = orc.Counts()
    _, grads = orc.loss_backward(t[None], target, 0.02, (0.2, 0.2, 0.2), counts=c)
    assert np.all(grads == 0.0)
    assert c.n_box == 0  # the tape is empty (memory_bytes() == 0)


# ---------------- optim.rs:63-98 ----------------

def test_adam_descends_a_quadratic(orc):  # optim.rs:67-79
    adam = orc.Adam(1)
    p = np.zeros(1, np.float32)
    for _ in range(500):
        adam.step(p, 2.0 * (p - 3.0), [0.1])
    assert abs(p[0] - 3.0) < 1e-2
    assert adam.steps_taken == 500


def test_adam_zero_gradient_leaves_params_untouched(orc):  # optim.rs:81-88
    adam = orc.Adam(3)
    p = np.array([1.0, -2.0, 0.5], np.float32)
    before = p.copy()
    adam.step(p, np.zeros(3, np.float32), [0.1] * 3)
    assert np.array_equal(p, before)


def test_adam_per_parameter_rates_are_respected(orc):  # optim.rs:90-97
    adam = orc.Adam(2)
    p = np.zeros(2, np.float32)
    adam.step(p, [1.0, 1.0], [0.5, 0.01])
    assert abs(p[0]) > abs(p[1]) * 10.0


# ---------------- fit.rs:426-636 ----------------

def target_scene():  # fit.rs:431-440
    return np.stack([
        tri([[0.20, 0.25], [0.80, 0.30], [0.50, 0.80]], [0.90, 0.30, 0.20], 0.9),
        tri([[0.30, 0.55], [0.85, 0.60], [0.60, 0.15]], [0.20, 0.60, 0.90], 0.7),
    ])


def target_at(orc, size):  # fit.rs:468-470
    return orc.render(target_scene(), size, size, 0.002, (0.08, 0.09, 0.12))


def run_fit(orc, target, triangles, seed, **cfg):
    init, bg = synth.seed_scene(target, triangles, seed)
    return orc.fit(target, init, bg, **cfg)


def test_sigma_anneals_from_start_to_end(orc):  # fit.rs:442-451
    s0, s1 = 0.02, 0.0015
    assert abs(orc.sigma_at(s0, s1, 100, 0) - s0) < 1e-9
    assert abs(orc.sigma_at(s0, s1, 100, 99) - s1) < 1e-9
    for i in range(1, 100):
        assert orc.sigma_at(s0, s1, 100, i) < orc.sigma_at(s0, s1, 100, i - 1)


def test_single_iteration_config_uses_final_sigma(orc):  # fit.rs:453-457
    assert orc.sigma_at(0.02, 0.0015, 1, 0) == np.float32(0.0015)


def test_projection_keeps_parameters_in_range(orc):  # fit.rs:459-466
    p = orc.project([-5.0, 5.0, 0.5, 0.5, 0.5, 0.5, -1.0, 2.0, 0.5, 1.7])
    assert list(p[0:2]) == [-0.25, 1.25]
    assert list(p[6:9]) == [0.0, 1.0, 0.5]
    assert p[9] == np.float32(0.999)


def test_loss_decreases_on_a_synthetic_target(orc):  # fit.rs:472-485
    r = run_fit(orc, target_at(orc, 48), 16, 7, iters=200)
    first = r["losses"][0]
    assert r["best_loss"] < first * 0.5
    assert np.isfinite(r["best_loss"])
    assert first / r["best_loss"] > 2.0


def test_fitting_is_deterministic_for_a_fixed_seed(orc):  # fit.rs:487-496
    target = target_at(orc, 32)
    a = run_fit(orc, target, 8, 42, iters=30)
    b = run_fit(orc, target, 8, 42, iters=30)
    assert np.array_equal(a["losses"], b["losses"])
    assert np.array_equal(a["best_params"], b["best_params"])


def test_progress_reports_every_iteration(orc):  # fit.rs:498-506
    target = np.full((32, 32, 3), [0.5, 0.2, 0.7], np.float32)
    r = run_fit(orc, target, 4, 0, iters=10, patience=None)
    assert len(r["losses"]) == 10


def test_non_square_targets_are_fitted_without_cropping(orc):  # fit.rs:508-518
    target = np.full((24, 64, 3), [0.3, 0.6, 0.2], np.float32)
    r = run_fit(orc, target, 8, 0, iters=20)
    out = orc.render(r["best_params"], 24, 64, 0.002)
    assert out.shape == (24, 64, 3)
    assert np.isfinite(r["best_loss"])


def test_best_scene_is_returned_not_the_last(orc):  # fit.rs:520-528
    r = run_fit(orc, target_at(orc, 40), 12, 3, iters=150)
    assert r["best_loss"] <= r["losses"][-1]
    assert r["best_loss"] == r["losses"][r["best_iter"]]


def test_patience_stops_a_stalled_fit_early(orc):  # fit.rs:530-540
    target = np.full((24, 24, 3), [0.4, 0.4, 0.4], np.float32)
    r = run_fit(orc, target, 4, 0, iters=1000, patience=5)
    assert r["stop_reason"] == "Converged"
    assert len(r["losses"]) < 1000


def test_projection_replaces_non_finite_parameters(orc):  # fit.rs:566-571
    nan, inf = float("nan"), float("inf")
    p = orc.project([nan, inf, 0.5, 0.5, 0.5, 0.5, nan, 0.2, 0.3, nan])
    assert np.all(np.isfinite(p))


def test_zero_iterations_is_not_an_error(orc):  # fit.rs:628-635
    r = run_fit(orc, np.full((16, 16, 3), 0.5, np.float32), 4, 0, iters=0)
    assert len(r["losses"]) == 0
    assert r["stop_reason"] == "Completed"


# ---------------- integration.rs:23-145 ----------------

def reference_scene():  # integration.rs:12-17
    return np.stack([
        tri([[0.20, 0.25], [0.80, 0.30], [0.50, 0.80]], [0.90, 0.30, 0.20], 0.9),
        tri([[0.30, 0.55], [0.85, 0.60], [0.60, 0.15]], [0.20, 0.60, 0.90], 0.7),
    ])


REF_BG = (0.10, 0.11, 0.14)


def reference_target(orc, w, h):
    return orc.render(reference_scene(), h, w, 0.002, REF_BG)


def test_fit_reduces_loss_substantially(orc):  # integration.rs:23-30
    r = run_fit(orc, reference_target(orc, 64, 64), 24, 1, iters=400)
    assert r["losses"][0] / r["best_loss"] > 10.0
    assert r["stop_reason"] != "Diverged"


def test_fitted_scene_upscales_without_refitting(orc):  # integration.rs:32-45
    r = run_fit(orc, reference_target(orc, 64, 64), 24, 2, iters=300)
    init, bg = synth.seed_scene(reference_target(orc, 64, 64), 24, 2)
    big = orc.render(r["best_params"], 256, 256, 0.0015 / 4.0, bg)
    big_target = reference_target(orc, 256, 256)
    loss_big = orc.mse(big, big_target)
    baseline = orc.mse(np.full((256, 256, 3), 0.5, np.float32), big_target)
    assert loss_big < baseline


def test_render_is_deterministic(orc):  # integration.rs:60-65
    a = orc.render(reference_scene(), 96, 96, 0.004, REF_BG)
    b = orc.render(reference_scene(), 96, 96, 0.004, REF_BG)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("w,h", [(32, 32), (64, 48), (17, 41)])
def test_taped_render_matches_plain_render_at_several_sizes(orc, w, h):  # integration.rs:67-75
    plain = orc.render(reference_scene(), h, w, 0.01, REF_BG)
    _, _, taped = orc.loss_backward(reference_scene(), plain, 0.01, REF_BG, want_image=True)
    assert np.array_equal(plain, taped)


def test_gradient_points_downhill(orc):  # integration.rs:77-101
    target = reference_target(orc, 48, 48)
    scene = reference_scene()
    scene[0, 0] += 0.08
    scene[0, 6:9] = 0.3
    loss, grads = orc.loss_backward(scene, target, 0.02, REF_BG)
    step = 1e-3 / max(float(np.sqrt(np.sum(grads * grads))), 1e-12)
    stepped = (scene - np.float32(step) * grads).astype(np.float32)
    new_loss = orc.mse(orc.render(stepped, 48, 48, 0.02, REF_BG), target)
    assert new_loss < loss


@pytest.mark.parametrize("w,h", [(1, 1), (1, 64), (64, 1), (37, 11)])
def test_non_square_and_tiny_canvases_are_handled(orc, w, h):  # integration.rs:103-111
    target = np.full((h, w, 3), [0.4, 0.5, 0.6], np.float32)
    r = run_fit(orc, target, 4, 0, iters=10, patience=None)
    assert np.isfinite(r["best_loss"])


def test_empty_scene_renders_the_background(orc):  # integration.rs:113-118
    img = orc.render(np.zeros((0, 10), np.float32), 16, 16, 0.01, (0.2, 0.4, 0.6))
    assert np.all(img == np.array([0.2, 0.4, 0.6], np.float32))


# ---------------- python/test_torch_layer.py:56-90 ----------------

def test_gradient_matches_numerical_differentiation(orc):  # test_torch_layer.py:56-90
    p = synth.uniform_scene(0, 5)
    p[:, :6] = p[:, :6] * 0.3 + 0.35  # small triangles scattered near the centre
    target = synth.uniforms(1, 24 * 24 * 3).reshape(24, 24, 3).astype(np.float32)
    _, analytic = orc.loss_backward(p, target, 0.03)
    _, numeric = orc.finite_difference(p, target, 0.03, 5e-4)
    a, n = analytic.ravel().astype(np.float64), numeric.ravel().astype(np.float64)
    rel = np.linalg.norm(a - n) / np.linalg.norm(n)
    cos = a @ n / (np.linalg.norm(a) * np.linalg.norm(n))
    assert rel < 0.02 and cos > 0.999, (rel, cos)
