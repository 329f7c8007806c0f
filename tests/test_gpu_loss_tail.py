"""The fused kernels' own loss sums (RasterArgs::loss_tail).

Outside the fixed-order mode the one-wave and segmented fused kernels store
their per-tile loss partials with device-scope atomic stores into slots that
setup_records marks pending, and the grid's last B workgroups, one per scene,
poll their scene's slots and add them in sum_losses' order. The losses must be
the bits of the two-kernel path (DRH_UNFUSED=1) and of the fixed-order mode,
whatever the number of scenes (one summing workgroup each), the size of a scene
(past 256 blocks the partials are read in a second pass instead of being held
in registers), a NaN among the partials, or the shape of the call before.
"""

import numpy as np
import pytest

from bars import check_losses
from diffrast import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    from diffrast import _lib

    c = _lib.Context()
    yield c
    c.close()


def make_case(orc, B, H, W, T, sigma, kind="uniform", seed=900):
    params = synth.batch(kind, B, T, seed)
    bgs = synth.uniforms(seed + 7, B * 3).reshape(B, 3).astype(np.float32)
    targets = orc.render_batch(synth.batch(kind, B, T, seed, target_offset=1000), H, W, sigma, bgs[::-1].copy())
    return params, bgs, targets


def losses_three_ways(ctx, params, targets, sigma, bgs, monkeypatch):
    tail = ctx.fused_loss_backward(params, targets, sigma, bgs)[0]
    fixed = ctx.fused_loss_backward(params, targets, sigma, bgs, deterministic=True)[0]
    monkeypatch.setenv("DRH_UNFUSED", "1")
    two = ctx.fused_loss_backward(params, targets, sigma, bgs)[0]
    monkeypatch.delenv("DRH_UNFUSED")
    return tail, fixed, two


# (name, B, H, W, T, sigma): the one-wave tile kernel's tail (more than 2048
# tiles); the last one has 38 x 33 blocks per scene (the two-pass sum)
CASES = [
    ("48-scenes", 48, 40, 56, 20, 0.004),
    ("1254-blocks", 1, 600, 520, 40, 0.002),
    ("odd-2-scenes", 2, 301, 333, 70, 0.003),
]


@pytest.mark.parametrize("name,B,H,W,T,sigma", CASES, ids=[c[0] for c in CASES])
def test_tail_losses_are_the_two_kernel_paths_bits(ctx, orc, name, B, H, W, T, sigma, monkeypatch):
    monkeypatch.setenv("DRH_NO_SEGMENTS", "1")
    params, bgs, targets = make_case(orc, B, H, W, T, sigma)
    print(f"loss tail {name}", flush=True)
    tail, fixed, two = losses_three_ways(ctx, params, targets, sigma, bgs, monkeypatch)
    assert np.array_equal(tail, two), name
    assert np.array_equal(tail, fixed), name
    check_losses(tail, orc.loss_backward_batch(params, targets, sigma, bgs)[0], label=name)


def test_segmented_kernels_tail(ctx, orc, monkeypatch):
    # two scenes of 64 tiles: fused_seg_kernel, whose losses are the other
    # fused kernels' bits
    params, bgs, targets = make_case(orc, 2, 64, 64, 32, 0.0015, seed=910)
    print("loss tail segmented", flush=True)
    tail, fixed, two = losses_three_ways(ctx, params, targets, 0.0015, bgs, monkeypatch)
    assert np.array_equal(tail, fixed) and np.array_equal(tail, two)
    monkeypatch.setenv("DRH_NO_SEGMENTS", "1")
    assert np.array_equal(ctx.fused_loss_backward(params, targets, 0.0015, bgs)[0], tail)
    check_losses(tail, orc.loss_backward_batch(params, targets, 0.0015, bgs)[0], label="segmented")


def test_nan_partial_gives_that_scenes_loss_nan_only(ctx, orc, monkeypatch):
    monkeypatch.setenv("DRH_NO_SEGMENTS", "1")
    B, H, W, T, sigma = 6, 96, 80, 24, 0.003
    params, bgs, targets = make_case(orc, B, H, W, T, sigma, seed=920)
    targets = targets.copy()
    targets[3, 17, 41, 1] = np.nan  # one pixel of scene 3: its tile's partial is NaN
    print("loss tail with a NaN partial", flush=True)
    tail, fixed, two = losses_three_ways(ctx, params, targets, sigma, bgs, monkeypatch)
    assert np.isnan(tail[3]) and np.isnan(two[3])
    keep = np.arange(B) != 3
    assert np.all(np.isfinite(tail[keep]))
    assert np.array_equal(tail[keep], two[keep]) and np.array_equal(tail[keep], fixed[keep])


def test_calls_of_different_shapes_in_a_row(ctx, orc, monkeypatch):
    # each call's setup marks its own slots pending: a larger call, then a
    # smaller one whose slots the first left written, then the first again
    monkeypatch.setenv("DRH_NO_SEGMENTS", "1")
    shapes = [(8, 128, 128, 40, 0.002), (3, 64, 96, 30, 0.004), (8, 128, 128, 40, 0.002)]
    print("loss tail, calls of different shapes", flush=True)
    for i, (B, H, W, T, sigma) in enumerate(shapes):
        params, bgs, targets = make_case(orc, B, H, W, T, sigma, seed=930 + i)
        tail, fixed, two = losses_three_ways(ctx, params, targets, sigma, bgs, monkeypatch)
        assert np.array_equal(tail, two) and np.array_equal(tail, fixed), i


def test_scenes_without_triangles(ctx, orc, monkeypatch):
    # T = 0: the losses of the backgrounds against the targets
    monkeypatch.setenv("DRH_NO_SEGMENTS", "1")
    B, H, W = 5, 70, 90
    bgs = synth.uniforms(940, B * 3).reshape(B, 3).astype(np.float32)
    params = np.zeros((B, 0, 10), np.float32)
    targets = synth.uniforms(941, B * H * W * 3).reshape(B, H, W, 3).astype(np.float32)
    print("loss tail, no triangles", flush=True)
    tail, fixed, two = losses_three_ways(ctx, params, targets, 0.002, bgs, monkeypatch)
    assert np.array_equal(tail, two) and np.array_equal(tail, fixed)
    check_losses(tail, orc.loss_backward_batch(params, targets, 0.002, bgs)[0], label="T = 0")
