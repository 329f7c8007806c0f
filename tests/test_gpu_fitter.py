"""The step-wise fitter (Fitter, crates/diffrast/src/fit.rs:191-335) through the C
ABI, against the oracle's fit loop (fit.rs:166-288), and the forward record's
argument checks."""

import numpy as np
import pytest

from bars import check_image
from diffrast import _lib, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = _lib.Context()
    yield c
    c.close()


def test_stepping_tracks_the_oracle_fit(ctx, orc):  # fit.rs:239-288, 596-617
    target = synth.blob_target(11, 48, 40)
    init, bg = synth.seed_scene(target, 16, 11)
    iters = 40
    f = _lib.Fitter(ctx, target, init, bg, iters=iters, patience=None)
    assert f.status()["iter"] == 0 and not f.status()["done"]
    assert np.array_equal(f.scene(), init)
    steps = []
    while (s := f.step()) is not None:
        steps.append(s)
    c = orc.fit(target, init, bg, iters=iters, patience=None)
    assert [s["iter"] for s in steps] == list(range(iters))
    for s in steps:  # StepInfo.sigma is sigma_at(i) (fit.rs:343-349)
        assert s["sigma"] == np.float32(orc.sigma_at(0.02, 0.0015, iters, s["iter"]))
    losses = np.array([s["loss"] for s in steps], np.float32)
    assert np.array_equal(losses, f.losses())
    rel = np.abs(losses - c["losses"]) / c["losses"]
    print(f"fitter 48x40 T=16: loss rel err first 20 {rel[:20].max():.2e}, all {rel.max():.2e}", flush=True)
    assert rel[:20].max() <= 1e-4
    st = f.status()
    assert st["done"] and st["iter"] == iters and st["stop_reason"] == "Completed"
    assert st["sigma"] == np.float32(orc.sigma_at(0.02, 0.0015, iters, iters - 1))
    rep = f.into_report()
    assert rep["stop_reason"] == "Completed" and rep["best_loss"] == losses[rep["best_iter"]]
    # render_current: the current scene at sigma_end (fit.rs:320-324)
    check_image(f.render_current(), orc.render(f.scene(), 48, 40, 0.0015, bg), label="render_current")
    f.close()


def test_run_and_step_compose_like_the_batch_fit(ctx):  # fit.rs:166-181
    target = synth.blob_target(12, 32, 36)
    init, bg = synth.seed_scene(target, 10, 12)
    whole = ctx.fit(target, init, bg, iters=50, patience=None)
    f = _lib.Fitter(ctx, target, init, bg, iters=50, patience=None)
    assert f.run(17) == 17
    assert f.step()["iter"] == 17
    assert f.run(1000) == 32
    assert f.step() is None
    rep = f.into_report()
    # fixed-order sums: the same iterations give the same bits
    assert np.array_equal(rep["losses"], whole["losses"])
    assert np.array_equal(rep["best_params"], whole["best_params"])
    assert np.array_equal(f.scene(), whole["params"])
    f.close()


def test_patience_stops_with_a_last_step(ctx):  # fit.rs:277-281, 530-540
    flat = np.full((24, 24, 3), 0.4, np.float32)
    init, bg = synth.seed_scene(flat, 4, 0)
    f = _lib.Fitter(ctx, flat, init, bg, iters=1000, patience=5)
    n = 0
    while f.step() is not None:
        n += 1
    st = f.status()
    assert st["stop_reason"] == "Converged" and st["iter"] == n < 1000
    assert f.step() is None and f.status()["iter"] == n
    # the batch form stops at the same iteration without wasted iterations
    r = ctx.fit(flat, init, bg, iters=1000, patience=5)
    assert r["stop_reason"] == "Converged" and len(r["losses"]) == n
    f.close()


def test_patience_zero_stops_after_the_first_snapshot(ctx, orc):  # fit.rs:267-281
    # patience 0: the first iteration improves on an infinite best loss and, with
    # since = 0 >= 0, converges: the best scene is the initial one (snapshotted
    # before the update, in every block of parameter columns) and no update runs
    target = synth.blob_target(5, 24, 24)
    init, bg = synth.seed_scene(target, 30, 5)  # 300 parameters: several blocks of 64 columns
    r = ctx.fit(target, init, bg, iters=20, patience=0)
    c = orc.fit(target, init, bg, iters=20, patience=0)
    assert r["stop_reason"] == c["stop_reason"] == "Converged"
    assert len(r["losses"]) == len(c["losses"]) == 1 and r["best_iter"] == c["best_iter"] == 0
    assert np.array_equal(r["best_params"].reshape(-1), np.asarray(init, np.float32).reshape(-1))
    assert np.array_equal(r["params"].reshape(-1), np.asarray(init, np.float32).reshape(-1))
    assert abs(r["losses"][0] - c["losses"][0]) <= 1e-4 * abs(c["losses"][0])


def test_divergence_returns_none_before_recording(ctx):  # fit.rs:259-265
    bad = np.full((16, 16, 3), 0.4, np.float32)
    bad[3, 4, 1] = float("nan")
    init, bg = synth.seed_scene(np.full((16, 16, 3), 0.4, np.float32), 4, 1)
    f = _lib.Fitter(ctx, bad, init, bg, iters=10)
    assert f.step() is None
    st = f.status()
    assert st["stop_reason"] == "Diverged" and st["iter"] == 0 and len(f.losses()) == 0
    assert f.into_report()["stop_reason"] == "Diverged"
    f.close()


def test_a_stopped_fit_launches_no_work(ctx):
    # Iterations launched after the device stopped return at entry: the batch
    # fit of a flat target converging early costs far less than its budget.
    import time

    flat = np.full((64, 64, 3), 0.4, np.float32)
    init, bg = synth.seed_scene(flat, 30, 2)
    ctx.fit(flat, init, bg, iters=50, patience=None)
    t0 = time.perf_counter()
    r = ctx.fit(flat, init, bg, iters=5000, patience=3)
    stopped = time.perf_counter() - t0
    t0 = time.perf_counter()
    full = ctx.fit(flat, init, bg, iters=len(r["losses"]) + 64, patience=None)
    ran = time.perf_counter() - t0
    print(f"fit stopped after {len(r['losses'])} of 5000 iterations in {stopped * 1e3:.1f} ms; "
          f"{len(full['losses'])} iterations without stopping {ran * 1e3:.1f} ms", flush=True)
    assert r["stop_reason"] == "Converged" and len(r["losses"]) < 100
    assert stopped < 5 * ran


def test_backward_of_a_record_checks_its_arguments(ctx):
    import torch

    dev = torch.device("cuda:0")
    B, T, H, W, sig = 2, 12, 24, 20, 0.01
    p = torch.from_numpy(synth.batch("uniform", B, T, 3)).to(dev)
    bg = torch.zeros((B, 3), device=dev)
    img = torch.empty((B, H, W, 3), device=dev)
    nbytes = _lib.record_bytes(B, T, H, W)
    rec = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream(dev).cuda_stream
    ctx.render_record_ptr(p.data_ptr(), bg.data_ptr(), B, T, H, W, sig, img.data_ptr(), rec.data_ptr(), nbytes, s)
    gi = torch.full((B, H, W, 3), 1e-3, device=dev)
    g = torch.empty((B, T, 10), device=dev)
    ctx.backward_recorded_ptr(rec.data_ptr(), nbytes, gi.data_ptr(), B, T, H, W, sig, g.data_ptr(), s)
    with pytest.raises(_lib.DiffrastError) as e:
        ctx.backward_recorded_ptr(rec.data_ptr(), nbytes, gi.data_ptr(), B, T, H, W, 0.02, g.data_ptr(), s)
    assert e.value.code == 6 and "sigma" in str(e.value)
    with pytest.raises(_lib.DiffrastError) as e:
        ctx.backward_recorded_ptr(rec.data_ptr(), nbytes, gi.data_ptr(), B, T, H, W, sig, g.data_ptr(), s,
                                  _lib.EXACT_MATH)
    assert e.value.code == 6 and "EXACT_MATH" in str(e.value)
    # a context that did not make the record reads its head from the device
    other = _lib.Context()
    g2 = torch.empty((B, T, 10), device=dev)
    other.backward_recorded_ptr(rec.data_ptr(), nbytes, gi.data_ptr(), B, T, H, W, sig, g2.data_ptr(), s,
                                _lib.DETERMINISTIC)
    g3 = torch.empty((B, T, 10), device=dev)
    ctx.backward_recorded_ptr(rec.data_ptr(), nbytes, gi.data_ptr(), B, T, H, W, sig, g3.data_ptr(), s,
                              _lib.DETERMINISTIC)
    torch.cuda.synchronize()
    assert torch.equal(g2, g3)
    with pytest.raises(_lib.DiffrastError) as e:
        other.backward_recorded_ptr(rec.data_ptr(), nbytes, gi.data_ptr(), B, T, H, W, 0.5, g2.data_ptr(), s)
    assert e.value.code == 6
    # memory that no forward pass wrote is refused
    junk = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    with pytest.raises(_lib.DiffrastError) as e:
        other.backward_recorded_ptr(junk.data_ptr(), nbytes, gi.data_ptr(), B, T, H, W, sig, g2.data_ptr(), s)
    assert e.value.code == 6 and "drh_render_record" in str(e.value)
    other.close()
