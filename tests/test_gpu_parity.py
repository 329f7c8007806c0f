"""HIP path vs the CPU oracle, through the C ABI, on edge cases and odd shapes.

The bars (images 1e-5, losses 1e-4 relative, gradients 1e-4 of the norm per scene
and per parameter group) are in tests/bars.py; the benchmark configurations have
their own tests in test_gpu_configs.py.
"""

import numpy as np
import pytest

from bars import GRAD_RTOL, IMG_TOL, assert_grads, check_image, check_losses, grad_err
from diffrast import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from diffrast import _lib

    c = _lib.Context()
    print("device:", c.device_info(), flush=True)
    yield c
    c.close()


CASES = [
    # (name, B, H, W, T, sigma, kind)
    ("64x64-T32", 1, 64, 64, 32, 0.0015, "uniform"),
    ("odd-sizes", 2, 19, 37, 33, 0.02, "uniform"),
    ("tall", 1, 41, 17, 65, 0.02, "uniform"),
    ("wide-sigma", 3, 48, 40, 12, 0.05, "uniform"),
    ("chunks", 2, 40, 48, 300, 0.004, "small"),
    ("tiny-sigma", 2, 32, 32, 24, 1e-4, "uniform"),
    ("pixel-1x1", 1, 1, 1, 4, 0.02, "uniform"),
    ("row", 1, 1, 64, 8, 0.01, "uniform"),
    ("column", 1, 64, 1, 8, 0.01, "uniform"),
    ("37x11", 1, 11, 37, 8, 0.01, "uniform"),
]


def make_case(B, H, W, T, kind, seed=100):
    params = synth.batch(kind, B, T, seed)
    bgs = synth.uniforms(seed + 7, B * 3).reshape(B, 3).astype(np.float32)
    return params, bgs


@pytest.mark.parametrize("exact", [False, True], ids=["fast", "exact"])
@pytest.mark.parametrize("name,B,H,W,T,sigma,kind", CASES, ids=[c[0] for c in CASES])
def test_render_matches_oracle(ctx, orc, name, B, H, W, T, sigma, kind, exact):
    params, bgs = make_case(B, H, W, T, kind)
    print(f"render {name} exact={exact}", flush=True)
    gpu = ctx.render(params, H, W, sigma, bgs, exact=exact)
    cpu = orc.render_batch(params, H, W, sigma, bgs)
    check_image(gpu, cpu)


@pytest.mark.parametrize("exact", [False, True], ids=["fast", "exact"])
@pytest.mark.parametrize("name,B,H,W,T,sigma,kind", CASES, ids=[c[0] for c in CASES])
def test_fused_loss_backward_matches_oracle(ctx, orc, name, B, H, W, T, sigma, kind, exact):
    params, bgs = make_case(B, H, W, T, kind)
    targets = orc.render_batch(synth.batch(kind, B, T, 100, target_offset=1000), H, W, sigma,
                               bgs[::-1].copy())
    print(f"fused {name} exact={exact}", flush=True)
    gl, gg, gimg = ctx.fused_loss_backward(params, targets, sigma, bgs, exact=exact, want_images=True)
    cl, cg = orc.loss_backward_batch(params, targets, sigma, bgs)
    assert np.abs(gimg - orc.render_batch(params, H, W, sigma, bgs)).max() <= IMG_TOL
    check_losses(gl, cl)
    assert_grads(gg, cg)


@pytest.mark.parametrize("name,B,H,W,T,sigma,kind", CASES[:6], ids=[c[0] for c in CASES[:6]])
def test_backward_from_grad_matches_oracle(ctx, orc, name, B, H, W, T, sigma, kind):
    params, bgs = make_case(B, H, W, T, kind)
    gin = ((synth.uniforms(5, B * H * W * 3) - 0.5) * 1e-3).reshape(B, H, W, 3).astype(np.float32)
    print(f"from_grad {name}", flush=True)
    gpu = ctx.backward_from_grad(params, gin, sigma, bgs)
    cpu = orc.backward_from_grad_batch(params, gin, sigma, bgs)
    assert_grads(gpu, cpu, label=name)
    # the reference CPU binding's target-inversion route agrees to the same bar
    inv = np.stack([orc.backward_from_grad(params[b], gin[b], sigma, bgs[b], inverted=True)
                    for b in range(B)])
    assert_grads(gpu, inv, label=f"{name} inverted")


@pytest.mark.parametrize("name,B,H,W,T,sigma,kind", [CASES[0], CASES[1], CASES[4]],
                         ids=[CASES[0][0], CASES[1][0], CASES[4][0]])
def test_fused_and_two_kernel_paths_agree(ctx, orc, name, B, H, W, T, sigma, kind, monkeypatch):
    # The gradient paths run as one fused kernel; DRH_UNFUSED=1 keeps
    # forward_kernel and backward_kernel, the path that fixed-order sums, the
    # split backward and the rebuild past the recorded entries take. The loss
    # and image come from the same per-block sums (bit-equal); the gradients
    # differ only in the order of their float atomics, and not at all with
    # fixed-order sums. On grids this small the default would take
    # fused_seg_kernel (tests/test_gpu_segments.py), which composites in
    # segments and rounds differently: DRH_NO_SEGMENTS=1 keeps the others.
    monkeypatch.setenv("DRH_NO_SEGMENTS", "1")
    params, bgs = make_case(B, H, W, T, kind)
    targets = orc.render_batch(synth.batch(kind, B, T, 100, target_offset=1000), H, W, sigma, bgs[::-1].copy())
    gin = ((synth.uniforms(8, B * H * W * 3) - 0.5) * 1e-3).reshape(B, H, W, 3).astype(np.float32)
    print(f"fused vs two kernels {name}", flush=True)

    def run():
        return (ctx.fused_loss_backward(params, targets, sigma, bgs, want_images=True),
                ctx.backward_from_grad(params, gin, sigma, bgs),
                ctx.fused_loss_backward(params, targets, sigma, bgs, deterministic=True),
                ctx.backward_from_grad(params, gin, sigma, bgs, deterministic=True))

    (fl, fg, fimg), ff, (fdl, fdg), fdf = run()
    monkeypatch.setenv("DRH_UNFUSED", "1")
    (ul, ug, uimg), uf, (udl, udg), udf = run()
    assert np.array_equal(fl, ul) and np.array_equal(fimg, uimg)
    assert grad_err(fg, ug) <= 1e-6 and grad_err(ff, uf) <= 1e-6
    assert np.array_equal(fdl, udl) and np.array_equal(fdg, udg) and np.array_equal(fdf, udf)
    assert np.array_equal(fdl, fl)
    cl, cg = orc.loss_backward_batch(params, targets, sigma, bgs)
    check_losses(ul, cl)
    assert_grads(ug, cg, label=f"two kernels {name}")
    assert_grads(uf, orc.backward_from_grad_batch(params, gin, sigma, bgs), label=f"two kernels from_grad {name}")


@pytest.mark.parametrize("mode", ["loss", "from_grad"])
def test_split_backward_matches_oracle(ctx, orc, mode):
    # Six 128x128 scenes of large triangles: 384 blocks, under six per compute
    # unit, so the backward splits the sweep of the heaviest quarter of blocks
    # over three waves per tile from the forward kernel's checkpoints (tiles
    # with up to ~60 recorded entries). Against the oracle, and against the
    # fixed-order mode, which never splits.
    B, H, W, T, sigma = 6, 128, 128, 128, 0.0015
    params = synth.batch("uniform", B, T, 41)
    bgs = synth.uniforms(47, B * 3).reshape(B, 3).astype(np.float32)
    print(f"split backward {mode}", flush=True)
    if mode == "loss":
        targets = orc.render_batch(synth.batch("uniform", B, T, 41, target_offset=1000), H, W, sigma, bgs[::-1].copy())
        gl, gg = ctx.fused_loss_backward(params, targets, sigma, bgs)
        dl, dg = ctx.fused_loss_backward(params, targets, sigma, bgs, deterministic=True)
        cl, cg = orc.loss_backward_batch(params, targets, sigma, bgs)
        check_losses(gl, cl)
        assert np.array_equal(gl, dl)
    else:
        gin = ((synth.uniforms(49, B * H * W * 3) - 0.5) * 1e-3).reshape(B, H, W, 3).astype(np.float32)
        gg = ctx.backward_from_grad(params, gin, sigma, bgs)
        dg = ctx.backward_from_grad(params, gin, sigma, bgs, deterministic=True)
        cg = orc.backward_from_grad_batch(params, gin, sigma, bgs)
    assert_grads(gg, cg, label=f"split {mode}")
    assert grad_err(gg, dg) <= 1e-6


def test_opaque_stack_and_clamped_alpha(ctx, orc):
    # alpha >= 1 makes w == 1 exactly deep inside: zero transmittance factors.
    params = synth.batch("uniform", 2, 20, 9)
    params[:, ::3, 9] = 1.0
    params[:, 1::3, 9] = 1.7
    params[:, 2::5, 9] = 0.999
    targets = np.stack([synth.blob_target(3 + b, 40, 44) for b in range(2)])
    gl, gg = ctx.fused_loss_backward(params, targets, 0.003)
    cl, cg = orc.loss_backward_batch(params, targets, 0.003)
    check_losses(gl, cl)
    assert_grads(gg, cg)
    pinned = params[..., 9] >= 1.0  # a clamped alpha gets no gradient (grad.rs:144-145)
    assert pinned.sum() > 10 and np.all(gg[..., 9][pinned] == 0.0)


def test_deep_stack_rescales_the_transmittance(ctx, orc):
    # 70 large triangles of alpha 0.8-0.95: where ~25 or more cover a pixel its
    # transmittance falls below 2^-64 and the kernels rescale it (10 and 6 of the
    # 30 tiles; those take the general transmittance path, the others the plain product)
    rng = np.random.default_rng(5)
    B, T, H, W = 2, 70, 40, 48
    ang = rng.uniform(0, 2 * np.pi, (B, T, 3))
    rad = rng.uniform(0.9, 1.6, (B, T, 3))
    params = np.zeros((B, T, 10), np.float32)
    params[..., 0:6:2] = 0.5 + rad * np.cos(ang)
    params[..., 1:6:2] = 0.5 + rad * np.sin(ang)
    params[..., 6:9] = rng.uniform(0, 1, (B, T, 3))
    params[..., 9] = rng.uniform(0.8, 0.95, (B, T))
    params[1, :, :6] = params[1, :, :6] * 0.5 + 0.25
    targets = np.stack([synth.blob_target(7 + b, H, W) for b in range(B)])
    for sigma in (0.003, 0.02):
        gl, gg = ctx.fused_loss_backward(params, targets, sigma)
        cl, cg = orc.loss_backward_batch(params, targets, sigma)
        check_losses(gl, cl)
        assert_grads(gg, cg)
        gi = (targets - 0.5).astype(np.float32) * 1e-3
        assert_grads(ctx.backward_from_grad(params, gi, sigma), orc.backward_from_grad_batch(params, gi, sigma))


def test_special_triangles(ctx, orc):
    nan = float("nan")
    params = synth.batch("uniform", 1, 12, 11)
    params[0, 0, :6] = [0.5, 0.5, 0.5, 0.5, 0.5, 0.5]          # point triangle
    params[0, 1, :6] = [0.1, 0.1, 0.5, 0.5, 0.9, 0.9]          # collinear
    params[0, 2, :6] = [5.0, 5.0, 6.0, 5.0, 5.5, 6.0]          # off-canvas
    params[0, 3, 0] = nan                                      # non-finite vertex
    params[0, 4, 9] = 0.0                                      # transparent
    params[0, 5, 9] = -0.5                                     # clamped to 0
    params[0, 6, :6] = [0.2, 0.2, 1e20, 0.2, 0.3, 0.4]         # bbox wraps: culled
    params[0, 7, 9] = 1e-7                                     # below MIN_WEIGHT everywhere
    target = synth.blob_target(4, 30, 34)[None]
    for sigma in (0.01, 0.002):
        g = ctx.render(params, 30, 34, sigma)
        c = orc.render_batch(params, 30, 34, sigma)
        assert np.abs(g - c).max() <= IMG_TOL
        gl, gg = ctx.fused_loss_backward(params, target, sigma)
        cl, cg = orc.loss_backward_batch(params, target, sigma)
        check_losses(gl, cl)
        assert_grads(gg, cg)
        assert np.all(gg[0, [2, 3, 4, 5, 6]] == 0.0)


def test_nan_alpha_follows_each_reference_path(ctx, orc):
    params = synth.batch("uniform", 1, 6, 12)
    params[0, 2, 9] = float("nan")
    g = ctx.render(params, 24, 24, 0.01)
    c = orc.render_batch(params, 24, 24, 0.01)
    assert np.array_equal(np.isnan(g), np.isnan(c)) and np.isnan(c).any()  # raster.rs:48-51
    ok = ~np.isnan(c)
    assert np.abs(g[ok] - c[ok]).max() <= IMG_TOL
    target = np.zeros((1, 24, 24, 3), np.float32)
    gl, gg = ctx.fused_loss_backward(params, target, 0.01)  # grad.rs:61-62 culls it
    cl, cg = orc.loss_backward_batch(params, target, 0.01)
    check_losses(gl, cl)
    assert_grads(gg, cg)
    assert np.all(gg[0, 2] == 0)


def test_empty_scene_and_empty_batch(ctx, orc):
    bg = np.array([[0.2, 0.4, 0.6]], np.float32)
    img = ctx.render(np.zeros((1, 0, 10), np.float32), 16, 16, 0.01, bg)
    assert np.all(img == bg[0])
    target = synth.blob_target(1, 16, 16)[None]
    losses, grads = ctx.fused_loss_backward(np.zeros((1, 0, 10), np.float32), target, 0.01, bg)
    assert grads.shape == (1, 0, 10)
    assert abs(losses[0] - orc.mse(img[0], target[0])) <= 1e-7
    assert ctx.render(np.zeros((0, 5, 10), np.float32), 8, 8, 0.01).shape == (0, 8, 8, 3)


def test_zero_loss_gives_zero_gradient(ctx):  # grad.rs:462-469
    params = synth.batch("uniform", 2, 16, 13)
    rendered = ctx.render(params, 32, 32, 0.01)
    losses, grads = ctx.fused_loss_backward(params, rendered, 0.01)
    assert np.all(losses == 0.0) and np.all(grads == 0.0)


def test_gradient_input_mode_matches_target_mode(ctx):  # crates/diffrast-gpu/src/lib.rs:1502-1533
    params = synth.batch("uniform", 3, 40, 14)
    targets = np.stack([synth.blob_target(20 + b, 36, 36) for b in range(3)])
    _, g_t, img = ctx.fused_loss_backward(params, targets, 0.004, want_images=True)
    gin = (np.float32(2.0 / (36 * 36 * 3)) * (img - targets)).astype(np.float32)
    g_g = ctx.backward_from_grad(params, gin, 0.004)
    assert grad_err(g_g, g_t) <= 1e-6


def test_results_are_bit_reproducible(ctx, orc):
    # DRH_DETERMINISTIC: per-block partial rows summed in a fixed order.
    params = synth.batch("uniform", 4, 128, 15)
    targets = np.stack([synth.blob_target(30 + b, 96, 96) for b in range(4)])
    a = ctx.fused_loss_backward(params, targets, 0.0015, deterministic=True)
    b = ctx.fused_loss_backward(params, targets, 0.0015, deterministic=True)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
    # the default (one float atomic per triangle parameter per block) agrees
    # with it, and with the oracle, to the gradient bar
    c = ctx.fused_loss_backward(params, targets, 0.0015)
    assert np.array_equal(a[0], c[0])
    assert grad_err(c[1], a[1]) <= 1e-6
    cl, cg = orc.loss_backward_batch(params, targets, 0.0015)
    check_losses(a[0], cl)
    assert_grads(a[1], cg)
    gin = ((synth.uniforms(6, 4 * 96 * 96 * 3) - 0.5) * 1e-3).reshape(4, 96, 96, 3).astype(np.float32)
    d1 = ctx.backward_from_grad(params, gin, 0.0015, deterministic=True)
    d2 = ctx.backward_from_grad(params, gin, 0.0015, deterministic=True)
    assert np.array_equal(d1, d2)
    assert grad_err(ctx.backward_from_grad(params, gin, 0.0015), d1) <= 1e-6


def test_pool_reuses_buffers_across_identical_calls(ctx):  # crates/diffrast-gpu/src/lib.rs:1420-1476
    params = synth.batch("uniform", 2, 6, 16)
    targets = np.full((2, 32, 32, 3), 0.4, np.float32)
    first = ctx.fused_loss_backward(params, targets, 0.02)
    s1 = ctx.pool_stats()
    second = ctx.fused_loss_backward(params, targets, 0.02)
    s2 = ctx.pool_stats()
    assert s2["misses"] == s1["misses"] and s2["hits"] > s1["hits"]
    # reused buffers give the same results: to the reference's bar
    # (crates/diffrast-gpu/src/lib.rs:1479-1484), as float atomics may sum in
    # another order; the losses are summed in a fixed order either way
    assert np.array_equal(first[0], second[0])
    assert grad_err(second[1], first[1]) <= 1e-4
    ctx.clear_pool()
    assert ctx.pool_stats()["bytes"] == 0


def test_backward_many_timed_reports_host_phases(ctx):  # crates/diffrast-gpu/src/lib.rs:96-114, 649-664
    from diffrast import _lib

    params = synth.batch("uniform", 4, 64, 17)
    targets = np.stack([synth.blob_target(70 + b, 96, 96) for b in range(4)])
    plain = ctx.fused_loss_backward(params, targets, 0.004, deterministic=True)
    losses, grads, ph = ctx.backward_many_timed(params, targets, 0.004)
    print("phases (ms):", {k: round(v, 3) for k, v in ph.items()}, flush=True)
    assert np.array_equal(losses, plain[0])
    assert grad_err(grads, plain[1]) <= 1e-6
    parts = ("pack_ms", "alloc_ms", "dispatch_ms", "readback_ms", "loss_ms")
    assert all(ph[k] >= 0.0 for k in parts) and ph["loss_ms"] == 0.0
    assert ph["dispatch_ms"] > 0.0 and ph["readback_ms"] > 0.0
    assert ph["total_ms"] == pytest.approx(sum(ph[k] for k in parts), rel=1e-12)
    # the phases stay those of the last timed call: an untimed call leaves them
    ctx.fused_loss_backward(params, targets, 0.004)
    assert _lib.Context.read_phases() == ph


def test_pool_buffers_move_between_streams(ctx):
    # Pooled buffers used on one stream, then on others (device pointers,
    # asynchronous calls): results identical to a single-stream run.
    import torch

    from diffrast import _lib

    dev = torch.device("cuda:0")
    B, H, W, T, sigma = 2, 40, 48, 20, 0.01
    params = torch.from_numpy(synth.batch("uniform", B, T, 21)).to(dev)
    targets = torch.from_numpy(np.stack([synth.blob_target(40 + b, H, W) for b in range(B)])).to(dev)
    bg = torch.zeros((B, 3), device=dev)

    def run(stream):
        losses = torch.empty(B, device=dev)
        grads = torch.empty((B, T, 10), device=dev)
        ctx.fused_ptr(params.data_ptr(), bg.data_ptr(), targets.data_ptr(), B, T, H, W, sigma,
                      losses.data_ptr(), grads.data_ptr(), None, stream.cuda_stream, _lib.DETERMINISTIC)
        return losses, grads

    ref = run(torch.cuda.current_stream(dev))
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(dev), torch.cuda.Stream(dev)
    outs = [run(s) for s in (s1, s2, s1, s2, torch.cuda.current_stream(dev))]
    torch.cuda.synchronize()
    for losses, grads in outs:
        assert torch.equal(losses, ref[0]) and torch.equal(grads, ref[1])


def test_concurrent_calls_on_one_context(ctx):
    # The reference's binding lets threads call one device concurrently
    # (crates/diffrast-py/src/lib.rs:47-65). Four host threads, three
    # host-array calls each on one context, different scenes per call: every
    # result equals the same call made alone (fixed-order sums: bit-equal).
    import threading

    B, H, W, T, sigma = 2, 48, 40, 24, 0.01
    jobs = [(synth.batch("uniform", B, T, 60 + j),
             np.stack([synth.blob_target(70 + j * B + b, H, W) for b in range(B)])) for j in range(12)]
    alone = [ctx.fused_loss_backward(p, t, sigma, deterministic=True) for p, t in jobs]
    got = [None] * len(jobs)
    errors = []

    def worker(k):
        try:
            for j in range(k, len(jobs), 4):
                got[j] = ctx.fused_loss_backward(jobs[j][0], jobs[j][1], sigma, deterministic=True)
        except Exception as e:  # reported below, not swallowed
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not errors, errors
    for (al, ag), (gl, gg) in zip(alone, got):
        assert np.array_equal(al, gl) and np.array_equal(ag, gg)


def test_adam_step_is_bit_exact(ctx, orc):  # optim.rs:40-60 + fit.rs:399-424
    n = 150
    p0 = synth.uniform_scene(17, 15).ravel().copy()
    g = ((synth.uniforms(18, n) - 0.5) * 0.2).astype(np.float32)
    lr = np.tile(np.array([0.004] * 6 + [0.02] * 3 + [0.01], np.float32), 15)
    pg, mg, vg = p0.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    pc = p0.copy()
    adam = orc.Adam(n)
    for step in range(1, 6):
        ctx.adam_project_step(pg, g * step, mg, vg, lr, step)
        adam.step(pc, g * step, lr)
        pc[:] = orc.project(pc)
        assert np.array_equal(pg, pc), step
        assert np.array_equal(mg, adam.m) and np.array_equal(vg, adam.v)


def test_device_fit_tracks_the_oracle(ctx, orc):  # fit.rs:166-288
    target = synth.blob_target(9, 40, 40)
    init, bg = synth.seed_scene(target, 12, 9)
    g = ctx.fit(target, init, bg, iters=60, patience=None)
    c = orc.fit(target, init, bg, iters=60, patience=None)
    assert g["stop_reason"] == c["stop_reason"] == "Completed"
    assert len(g["losses"]) == len(c["losses"]) == 60
    rel = np.abs(g["losses"] - c["losses"]) / c["losses"]
    print(f"fit 40x40 T=12: loss rel err first 20 {rel[:20].max():.2e}, all 60 {rel.max():.2e}; "
          f"best iter gpu {g['best_iter']} oracle {c['best_iter']}", flush=True)
    assert rel[:20].max() <= 1e-4
    assert rel.max() <= 1e-3
    assert g["best_loss"] == g["losses"][g["best_iter"]]
    # the snapshot is the scene the best loss was measured on (taken before the update)
    sig = orc.sigma_at(0.02, 0.0015, 60, g["best_iter"])
    again = orc.mse(orc.render(g["best_params"], 40, 40, sig, bg), target)
    assert abs(again - g["best_loss"]) <= 1e-4 * g["best_loss"]
    if g["best_iter"] == c["best_iter"]:
        d = np.abs(g["best_params"] - c["best_params"]).max()
        print(f"fit 40x40 T=12: best params max abs diff {d:.2e}", flush=True)
        assert d <= 1e-3


def test_device_fit_stop_reasons(ctx):
    flat = np.full((24, 24, 3), 0.4, np.float32)
    init, bg = synth.seed_scene(flat, 4, 0)
    r = ctx.fit(flat, init, bg, iters=1000, patience=5)  # fit.rs:530-540
    assert r["stop_reason"] == "Converged" and len(r["losses"]) < 1000
    r = ctx.fit(flat, init, bg, iters=0)  # fit.rs:628-635
    assert r["stop_reason"] == "Completed" and len(r["losses"]) == 0
    bad = flat.copy()
    bad[3, 4, 1] = float("nan")
    r = ctx.fit(bad, init, bg, iters=10)  # fit.rs:259-265
    assert r["stop_reason"] == "Diverged" and len(r["losses"]) == 0


def test_rebuild_path_past_the_recorded_entries(ctx, orc, monkeypatch):
    # Tiles keep at most DRH_MAX_TILE_ENTRIES recorded entries; past them the
    # backward kernel rebuilds and reclassifies the remaining chunks.
    params, bgs = make_case(2, 40, 48, 300, "small")
    targets = synth.batch("small", 2, 300, 900)
    targets = orc.render_batch(targets, 40, 48, 0.004, bgs)
    want_l, want_g = orc.loss_backward_batch(params, targets, 0.004, bgs)
    for cap in ("3", "40", "1"):
        monkeypatch.setenv("DRH_MAX_TILE_ENTRIES", cap)
        print(f"rebuild cap={cap}", flush=True)
        for det in (False, True):
            l, g = ctx.fused_loss_backward(params, targets, 0.004, bgs, deterministic=det)
            check_losses(l, want_l)
            assert_grads(g, want_g, label=f"rebuild cap={cap} det={det}")
        gi = np.random.default_rng(1).standard_normal((2, 40, 48, 3)).astype(np.float32) * 1e-3
        g2 = ctx.backward_from_grad(params, gi, 0.004, bgs)
        assert_grads(g2, orc.backward_from_grad_batch(params, gi, 0.004, bgs))


def test_channels_first_layout_gives_the_same_numbers(ctx):
    # DRH_CHANNELS_FIRST: images, targets and grad_images as B x 3 x H x W,
    # the torch op's layout; every result equals the B x H x W x 3 call's.
    import torch

    from diffrast import _lib

    B, H, W, T, sig = 3, 37, 29, 40, 0.004
    params, bgs = make_case(B, H, W, T, "uniform")
    dev = torch.device("cuda:0")
    p, bg = torch.from_numpy(params).to(dev), torch.from_numpy(bgs).to(dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    hwc = torch.empty((B, H, W, 3), device=dev)
    chw = torch.empty((B, 3, H, W), device=dev)
    ctx.render_ptr(p.data_ptr(), bg.data_ptr(), B, T, H, W, sig, hwc.data_ptr(), s)
    ctx.render_ptr(p.data_ptr(), bg.data_ptr(), B, T, H, W, sig, chw.data_ptr(), s, _lib.CHANNELS_FIRST)
    assert torch.equal(chw, hwc.permute(0, 3, 1, 2))
    tgt = torch.rand((B, H, W, 3), device=dev, generator=torch.Generator(device=dev).manual_seed(3))
    out = {}
    for name, t, flags in (("hwc", tgt, 0), ("chw", tgt.permute(0, 3, 1, 2).contiguous(), _lib.CHANNELS_FIRST)):
        l, g = torch.empty(B, device=dev), torch.empty((B, T, 10), device=dev)
        img = torch.empty_like(t)
        ctx.fused_ptr(p.data_ptr(), bg.data_ptr(), t.data_ptr(), B, T, H, W, sig, l.data_ptr(), g.data_ptr(),
                      img.data_ptr(), s, flags | _lib.DETERMINISTIC)
        gi = (t - 0.5) * 1e-3
        g2 = torch.empty((B, T, 10), device=dev)
        ctx.from_grad_ptr(p.data_ptr(), bg.data_ptr(), gi.data_ptr(), B, T, H, W, sig, g2.data_ptr(), s,
                          flags | _lib.DETERMINISTIC)
        out[name] = (l, g, img if flags == 0 else img.permute(0, 2, 3, 1), g2)
    torch.cuda.synchronize()
    for a, b in zip(out["hwc"], out["chw"]):
        assert torch.equal(a, b)


def random_case(i):
    """Seeded shape i of the sweep: B in [1, 4], H and W in [1, 300], T in [1, 1200]
    (cut so that the oracle sees at most 1.5e7 pixel-triangle pairs), sigma
    log-uniform in [1e-4, 0.05], one of the three scene kinds."""
    rng = np.random.default_rng(7000 + i)
    B = int(rng.integers(1, 5))
    H, W = (int(v) for v in rng.integers(1, 301, size=2))
    T = int(rng.integers(1, 1201))
    T = max(1, min(T, 15_000_000 // (B * H * W)))
    sigma = float(10.0 ** rng.uniform(-4.0, np.log10(0.05)))
    kind = ("uniform", "small", "random")[int(rng.integers(0, 3))]
    return B, H, W, T, sigma, kind


@pytest.mark.parametrize("i", range(16))
def test_random_shapes_match_oracle(ctx, orc, i, monkeypatch):
    # Every gradient path on a seeded random shape: the fast and exact fused
    # calls, the fixed-order sums and the two-kernel path (DRH_UNFUSED=1: the
    # split backward and the rebuild past the recorded entries where they
    # apply) against the oracle; the fixed-order and two-kernel losses equal
    # the default path's.
    B, H, W, T, sigma, kind = random_case(i)
    params, bgs = make_case(B, H, W, T, kind, seed=300 + 10 * i)
    targets = orc.render_batch(synth.batch(kind, B, T, 300 + 10 * i, target_offset=1000), H, W, sigma,
                               bgs[::-1].copy())
    print(f"random case {i}: B={B} H={H} W={W} T={T} sigma={sigma:.3g} kind={kind}", flush=True)
    cl, cg = orc.loss_backward_batch(params, targets, sigma, bgs)
    cimg = orc.render_batch(params, H, W, sigma, bgs)
    losses = {}
    for exact in (False, True):
        gl, gg, gimg = ctx.fused_loss_backward(params, targets, sigma, bgs, exact=exact, want_images=True)
        check_image(gimg, cimg, label=f"case {i} exact={exact}")
        check_losses(gl, cl, label=f"case {i} exact={exact}")
        assert_grads(gg, cg, label=f"case {i} exact={exact}")
        losses[exact] = gl
    dl, dg = ctx.fused_loss_backward(params, targets, sigma, bgs, deterministic=True)
    assert np.array_equal(dl, losses[False])
    assert_grads(dg, cg, label=f"case {i} fixed-order")
    # the fused kernels other than fused_seg_kernel (which small grids take by
    # default and which rounds its segment composite differently)
    monkeypatch.setenv("DRH_NO_SEGMENTS", "1")
    nl, ng = ctx.fused_loss_backward(params, targets, sigma, bgs)
    check_losses(nl, cl, label=f"case {i} no segments")
    assert_grads(ng, cg, label=f"case {i} no segments")
    monkeypatch.setenv("DRH_UNFUSED", "1")
    ul, ug = ctx.fused_loss_backward(params, targets, sigma, bgs)
    assert np.array_equal(ul, nl)
    assert_grads(ug, cg, label=f"case {i} two kernels")
