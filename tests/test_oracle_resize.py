"""Pins of the oracle's Lanczos3 resize (the resample of Canvas::load_image,
canvas.rs:71-79: image 0.25.10 imageops::resize with FilterType::Lanczos3).

The crate is absent from the reference tree and the reference's own tests only
load at the file's size (crates/diffrast/tests/integration.rs:120-134), so the
restatement is pinned by what the mathematics fixes:
  * each weight against the Lanczos3 window sin(pi x)/(pi x) * sin(pi x/3)/(pi x/3)
    in float64 at the centre (o + 0.5) * n_src / n_dst - 0.5, stretched by the
    ratio when shrinking, normalised to sum 1, over [centre - 3s, centre + 3s];
  * the whole resize against a float64 evaluation of the same separable sum
    (vertical pass first), rounded: equal except within 1e-3 of a .5 boundary;
  * invariants: the same size is a copy, a constant image stays constant,
    channels are independent, and odd integer upscales reproduce the input at
    the aligned outputs, where the window's other taps sit on its zeros.
"""

import numpy as np
import pytest


def window64(x):
    x = np.asarray(x, np.float64)
    out = np.where(x == 0, 1.0, np.sinc(x) * np.sinc(x / 3.0))
    return np.where(np.abs(x) < 3.0, out, 0.0)


def taps64(n_src, n_dst, o):
    ratio = n_src / n_dst
    s = max(ratio, 1.0)
    centre = (o + 0.5) * ratio
    lo = min(max(int(np.floor(centre - 3 * s)), 0), n_src - 1)
    hi = min(max(int(np.ceil(centre + 3 * s)), lo + 1), n_src)
    w = window64((np.arange(lo, hi) - (centre - 0.5)) / s)
    return lo, w / w.sum(), centre, s


def resize64(img, width, height):
    """The separable sum in float64: rows first, then columns, then clamp."""
    a = img.astype(np.float64)
    H, W, C = a.shape
    tmp = np.zeros((height, W, C))
    for oy in range(height):
        lo, w, _, _ = taps64(H, height, oy)
        tmp[oy] = np.tensordot(w, a[lo:lo + len(w)], axes=1)
    out = np.zeros((height, width, C))
    for ox in range(width):
        lo, w, _, _ = taps64(W, width, ox)
        out[:, ox] = np.tensordot(tmp[:, lo:lo + len(w)], w, axes=([1], [0]))
    return np.clip(out, 0, 255)


@pytest.mark.parametrize("n_src,n_dst", [(100, 50), (37, 11), (10, 30), (64, 64), (17, 16), (5, 1), (1, 7), (300, 176)])
def test_weights_are_the_normalised_lanczos3_window(orc, n_src, n_dst):
    checked = 0
    for o in range(n_dst):
        lo, w = orc.lanczos3_taps(n_src, n_dst, o)
        lo64, w64, centre, s = taps64(n_src, n_dst, o)
        edge = min(abs(centre - 3 * s - round(centre - 3 * s)), abs(centre + 3 * s - round(centre + 3 * s)))
        if 0 < edge < 1e-4:  # a float32 bound this close to an integer may round across it
            continue
        assert lo == lo64 and len(w) == len(w64), (o, lo, lo64)
        np.testing.assert_allclose(w, w64, atol=2e-5)  # f32 centre: ~1e-5 of position at o ~ 200
        assert abs(float(w.astype(np.float64).sum()) - 1.0) < 1e-5
        checked += 1
    assert checked >= n_dst - 2


def test_the_window_itself(orc):
    xs = np.linspace(-3.2, 3.2, 257, dtype=np.float32)
    got = np.array([orc.lanczos3(float(x)) for x in xs])
    np.testing.assert_allclose(got, window64(xs), atol=1e-6)
    assert orc.lanczos3(0.0) == 1.0 and orc.lanczos3(3.0) == 0.0 and orc.lanczos3(-3.0) == 0.0


@pytest.mark.parametrize("shape,size", [((40, 30, 3), (15, 20)), ((23, 41, 3), (64, 48)), ((50, 50, 4), (17, 29)),
                                        ((12, 9, 1), (30, 5)), ((64, 64, 3), (64, 32)), ((64, 64, 3), (32, 64))])
def test_resize_matches_the_float64_separable_sum(orc, shape, size):
    rng = np.random.default_rng(sum(shape) + sum(size))
    img = rng.integers(0, 256, shape, dtype=np.uint8)
    got = orc.resize_lanczos3(img, *size).astype(np.int64)
    want = resize64(img, *size)
    near_tie = np.abs(want - np.floor(want) - 0.5) < 1e-3
    exact = np.floor(want + 0.5)
    assert np.all(np.abs(got - exact) <= 1)
    assert np.array_equal(got[~near_tie], exact[~near_tie])


def test_invariants(orc):
    rng = np.random.default_rng(5)
    img = rng.integers(0, 256, (33, 47, 3), dtype=np.uint8)
    assert np.array_equal(orc.resize_lanczos3(img, 47, 33), img)
    for v in (0, 1, 128, 254, 255):
        flat = np.full((21, 34, 3), v, np.uint8)
        for size in ((7, 5), (34, 40), (100, 21), (1, 1)):
            assert np.all(orc.resize_lanczos3(flat, *size) == v), (v, size)
    # channels are independent: a 3-channel resize equals three 1-channel ones
    out = orc.resize_lanczos3(img, 20, 60)
    for c in range(3):
        assert np.array_equal(out[..., c], orc.resize_lanczos3(img[..., c:c + 1], 20, 60)[..., 0])
    # x3 upscale: output 3n + 1 sits on input n, the other taps on the window's zeros
    up = orc.resize_lanczos3(img, 47 * 3, 33 * 3)
    assert np.array_equal(up[1::3, 1::3], img)
