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


@pytest.mark.parametrize("size", [(64, 64), (100, 37), (176, 90), (301, 512), (176, 176)])
def test_load_png_resamples_like_the_oracle(orc, size):  # canvas.rs:71-87
    from diffrast import scene_io

    src = GOLDEN / "fit_target_176.png"
    raw = scene_io.read_png(src)
    lin = scene_io.load_png(src, *size)
    assert lin.shape == (size[1], size[0], 3)
    assert np.array_equal(lin, orc.decode_srgb(orc.resize_lanczos3(raw, *size)))


def test_load_target_keeps_the_aspect_ratio(orc, tmp_path):  # crates/diffrast/src/bin/fit.rs:186-196
    from diffrast import scene_io

    rng = np.random.default_rng(3)
    wide = rng.integers(0, 256, (120, 300, 3), dtype=np.uint8)
    scene_io.write_png(tmp_path / "wide.png", wide)
    t = scene_io.load_target(tmp_path / "wide.png", 176)
    assert t.shape == (70, 176, 3)  # fit_within(300, 120, 176)
    assert np.array_equal(t, orc.decode_srgb(orc.resize_lanczos3(wide, 176, 70)))
    small = scene_io.load_target(tmp_path / "wide.png", 1000)  # never scaled up
    assert np.array_equal(small, orc.decode_srgb(wide))
    with pytest.raises(scene_io.FitError):
        scene_io.load_target(tmp_path / "missing.png", 176)


@pytest.mark.parametrize("shape,size", [((480, 640, 3), (176, 132)), ((33, 47, 4), (141, 99)), ((64, 64, 1), (17, 5)),
                                        ((2000, 3, 3), (1, 700)), ((1, 1, 3), (9, 4)), ((70000, 2, 1), (3, 70001))])
def test_resize_matches_the_oracle(ctx, orc, shape, size):
    rng = np.random.default_rng(shape[0] + size[0])
    img = rng.integers(0, 256, shape, dtype=np.uint8)
    print(f"resize {shape} -> {size}", flush=True)
    assert np.array_equal(ctx.resize_lanczos3(img, *size), orc.resize_lanczos3(img, *size))


def test_resize_rejects_bad_arguments(ctx):
    from diffrast import _lib

    img = np.zeros((8, 8, 5), np.uint8)
    with pytest.raises(_lib.DiffrastError) as e:
        ctx.resize_lanczos3(img, 4, 4)
    assert e.value.code == 6
    with pytest.raises(_lib.DiffrastError) as e:
        ctx.resize_lanczos3(np.zeros((8, 8, 3), np.uint8), 0, 4)
    assert e.value.code == 6


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
