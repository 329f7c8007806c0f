"""Forward-only renders at the reference's benchmark and export sizes, HIP vs the oracle.

The reference's GPU forward benchmark renders one `Scene::random(n, [0.1, 0.11, 0.14],
0.15)` scene at sigma 0.0015 for (size, triangles) = (128, 64), (256, 128), (512, 256),
(512, 1024) and reports the max |gpu - cpu| (crates/diffrast-gpu/src/bin/gpu_bench.rs:18-69;
docs/gpu-report.txt:163-167 quotes 6.3e-7 to 1.1e-6). The `fit` binary re-renders the fitted
scene with the longest side at --export (default 1024) and sigma scaled by the size ratio
(crates/diffrast/src/bin/fit.rs:95-99). Scenes come from `synth.random_scene` (same
distributions, our generator). Bar: max |gpu - cpu| <= 1e-5 (the image bar of this path).
"""

import numpy as np
import pytest

from diffrast import synth

pytestmark = pytest.mark.gpu

IMG_TOL = 1e-5
BENCH_BG = (0.1, 0.11, 0.14)  # gpu_bench.rs:20


@pytest.fixture(scope="module")
def ctx():
    from diffrast import _lib

    c = _lib.Context()
    yield c
    c.close()


@pytest.mark.parametrize("size,tris", [(128, 64), (256, 128), (512, 256), (512, 1024)])
def test_reference_forward_cells_match_oracle(ctx, orc, size, tris):
    params = synth.random_scene(11, tris)[None]
    print(f"render {size}x{size} T={tris}", flush=True)
    gpu = ctx.render(params, size, size, 0.0015, BENCH_BG)
    cpu = orc.render_batch(params, size, size, 0.0015, BENCH_BG)
    assert np.abs(gpu - cpu).max() <= IMG_TOL


@pytest.mark.parametrize("W,H", [(1024, 1024), (1024, 576), (683, 1024)])
def test_export_render_matches_oracle(ctx, orc, W, H):
    # a 150-triangle scene fitted at 176 px, re-rendered sharp: sigma_end * 176 / 1024
    params = synth.random_scene(12, 150, 0.18)[None]
    sigma = 0.0015 * 176 / max(W, H)
    bg = (0.2, 0.3, 0.4)
    print(f"export {W}x{H} sigma={sigma:.3g}", flush=True)
    gpu = ctx.render(params, H, W, sigma, bg)
    cpu = orc.render_batch(params, H, W, sigma, bg)
    assert gpu.shape == (1, H, W, 3)
    assert np.abs(gpu - cpu).max() <= IMG_TOL


def test_batched_forward_matches_oracle_per_item(ctx, orc):
    # a dataset-style batch: many small scenes, one background each (forward_batch.wgsl:18-20)
    B, H, W, T = 24, 96, 96, 40
    params = synth.batch("random", B, T, 300)
    bgs = synth.uniforms(301, B * 3).reshape(B, 3).astype(np.float32)
    gpu = ctx.render(params, H, W, 0.004, bgs)
    cpu = orc.render_batch(params, H, W, 0.004, bgs)
    assert np.abs(gpu - cpu).max() <= IMG_TOL
    # items are independent: rendering one alone gives the same pixels
    one = ctx.render(params[5:6], H, W, 0.004, bgs[5:6])
    assert np.array_equal(one[0], gpu[5])
