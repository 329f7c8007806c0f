"""sRGB bytes on the GPU (drh_encode_srgb / drh_decode_srgb) vs the oracle, bit for bit.

Byte work: the bar is bit-exact. Inputs cover each byte's threshold and its neighbouring
floats, the clamp (negatives, values above 1, infinities), NaN, and a large uniform
sample; the PNG helpers (Canvas::save_png / load_image, canvas.rs:61-86) are checked end
to end against the reference's own fit target.
"""

from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def ctx():
    from diffrast import _lib

    c = _lib.Context()
    yield c
    c.close()


def edge_values(orc):
    _, thr = orc.srgb_encode_scan()
    t = thr[1:]
    near = [t, np.nextafter(t, np.float32(-1)), np.nextafter(t, np.float32(2)),
            np.nextafter(np.nextafter(t, np.float32(-1)), np.float32(-1))]
    special = np.array([0.0, -0.0, 1.0, -1.0, 2.0, np.inf, -np.inf, np.nan, 1e-30, -1e-30,
                        0.0031308, np.nextafter(np.float32(0.0031308), np.float32(1)), 1.0000001,
                        np.nextafter(np.float32(1), np.float32(0)), 5e-45], np.float32)
    return np.concatenate(near + [special]).astype(np.float32)


def test_encode_matches_oracle_at_every_threshold(ctx, orc):
    v = edge_values(orc)
    assert np.array_equal(ctx.encode_srgb(v), orc.encode_srgb(v))


def test_encode_matches_oracle_on_a_large_sample(ctx, orc):
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.uniform(-0.1, 1.1, 3_000_000), rng.uniform(0, 0.01, 1_000_000)]).astype(np.float32)
    v = v.reshape(1000, 1000, 4)  # any shape: the call works on n values
    got = ctx.encode_srgb(v)
    assert got.shape == v.shape
    assert np.array_equal(got, orc.encode_srgb(v))


def test_decode_matches_oracle_for_every_byte(ctx, orc):
    b = np.tile(np.arange(256, dtype=np.uint8), 1000)
    assert np.array_equal(ctx.decode_srgb(b), orc.decode_srgb(b))
    assert ctx.encode_srgb(np.zeros(0, np.float32)).size == 0


def test_device_tensors_stay_on_the_device(orc):
    import torch

    from diffrast import scene_io

    x = torch.linspace(-0.5, 1.5, 100_003, device="cuda")
    b = scene_io.encode_srgb(x)
    assert b.is_cuda and b.dtype == torch.uint8
    assert np.array_equal(b.cpu().numpy(), orc.encode_srgb(x.cpu().numpy()))
    d = scene_io.decode_srgb(b)
    assert d.is_cuda and d.dtype == torch.float32
    assert np.array_equal(d.cpu().numpy(), orc.decode_srgb(b.cpu().numpy()))


def test_png_files_round_trip_the_reference_fit_target(tmp_path, orc):
    from diffrast import scene_io

    src = GOLDEN / "fit_target_176.png"
    lin = scene_io.load_png(src)
    raw = scene_io.read_png(src)
    assert lin.shape == (176, 176, 3) and lin.dtype == np.float32
    assert np.array_equal(lin, orc.decode_srgb(raw))
    out = tmp_path / "again.png"
    scene_io.save_png(out, lin)
    assert np.array_equal(scene_io.read_png(out), raw)  # decode then encode is the identity
    with pytest.raises(scene_io.FitError):
        scene_io.load_png(src, 64, 64)


def test_saved_render_matches_the_oracle_bytes(ctx, orc, tmp_path):
    from diffrast import scene_io, synth

    params = synth.random_scene(12, 150, 0.18)[None]
    img = ctx.render(params, 300, 400, 0.001, (0.2, 0.3, 0.4))[0]
    scene_io.save_png(tmp_path / "fit.png", img)
    cpu = orc.render_batch(params, 300, 400, 0.001, (0.2, 0.3, 0.4))[0]
    got = scene_io.read_png(tmp_path / "fit.png").astype(int)
    want = orc.encode_srgb(cpu).astype(int)
    # the images agree to 1e-5, so a byte can move only where a pixel sits on a threshold
    assert np.abs(got - want).max() <= 1
    assert np.array_equal(got, orc.encode_srgb(img))
