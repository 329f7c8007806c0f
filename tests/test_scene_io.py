"""Scene JSON, PNG container and the sRGB oracle (CPU).

JSON cases follow crates/diffrast/src/serial.rs:74-121 and python/test_runner.py:20-82;
sizes canvas.rs:143-150; the sRGB oracle is pinned by canvas.rs:120-136's tests, by
the sRGB standard's values and by an exhaustive monotonicity scan (which the GPU
encoding relies on). The PNG reader is checked against PIL on the reference's own
fit target and on files written with every filter type.
"""

from __future__ import annotations

import io
import json
import math
from pathlib import Path

import numpy as np
import pytest

from diffrast import scene_io
from diffrast.scene_io import FitError, Scene, Triangle, fit_within, load_scene, parse_scene, scene_to_json

GOLDEN = Path(__file__).resolve().parent / "golden"


def sample() -> Scene:  # serial.rs:79-83
    return Scene([0.1, 0.2, 0.3], [Triangle([[0.0, 0.0], [1.0, 0.0], [0.5, 1.0]], [1.0, 0.5, 0.25], 0.75)])


# ---------------------------------------------------------------- serial.rs


def test_emits_expected_fields():
    js = scene_to_json(sample())
    assert '"version": 1' in js
    assert '"background": [0.100000, 0.200000, 0.300000]' in js
    assert '"alpha": 0.750000' in js


def test_exact_text_of_the_sample():
    # serial.rs:21-46 laid out by hand: two-space indent, one triangle per line
    assert scene_to_json(sample()) == (
        '{\n  "version": 1,\n  "background": [0.100000, 0.200000, 0.300000],\n  "triangles": [\n'
        '    {"verts": [[0.000000, 0.000000], [1.000000, 0.000000], [0.500000, 1.000000]], '
        '"color": [1.000000, 0.500000, 0.250000], "alpha": 0.750000}\n  ]\n}\n')


def test_empty_scene_is_still_valid_json():
    js = scene_to_json(Scene([0.0, 0.0, 0.0]))
    assert '"triangles": [\n  ]' in js
    assert json.loads(js)["triangles"] == []


def test_non_finite_values_never_reach_the_output():
    s = sample()
    s.triangles[0].alpha = float("nan")
    s.triangles[0].verts[0][0] = float("inf")
    js = scene_to_json(s)
    assert "NaN" not in js and "inf" not in js and "nan" not in js
    assert json.loads(js)["triangles"][0]["alpha"] == 0.0


def test_triangle_count_matches_separator_count():
    s = sample()
    s.triangles += [s.triangles[0], s.triangles[0]]
    js = scene_to_json(s)
    assert js.count('"verts"') == 3
    assert js.count("},\n") == 2  # no trailing comma


def test_values_are_the_f32_rounded_to_six_decimals():
    # {v:.6} formats the f32's exact value, correctly rounded (ties to even)
    p = np.zeros((1, 10), np.float32)
    p[0, :6] = [0.1234565, 2.0 ** -7, -1e-9, 1.0000005, 123.456789, -0.0]
    p[0, 6:] = [1.0 / 3.0, 0.5, 0.999999, 0.3]
    verts = json.loads(scene_to_json(p))["triangles"][0]["verts"]
    text = scene_to_json(p)
    assert "0.007812" in text  # 2^-7 = 0.0078125 exactly: the tie goes to even
    assert "-0.000000" in text  # negative values that round to zero keep their sign
    for got, want in zip(np.asarray(verts).ravel(), p[0, :6]):
        assert abs(got - float(want)) <= 5e-7 + 1e-12


def test_json_round_trip_through_parse_scene():
    rng = np.random.default_rng(3)
    p = rng.uniform(-0.25, 1.25, (17, 10)).astype(np.float32)
    text = scene_to_json(p, (0.2, 0.4, 0.6))
    back = parse_scene(json.loads(text))
    assert len(back) == 17
    # six decimals (<= 5e-7), then the parsed decimal rounded to f32 (<= 6e-8 below 2)
    assert np.abs(back.params() - p).max() <= 5e-7 + 6e-8
    assert scene_to_json(back) == text  # a written scene reads back to the same text


# ---------------------------------------------------------------- runner.py

VALID_SCENE = {
    "version": 1,
    "background": [0.1, 0.2, 0.3],
    "triangles": [
        {"verts": [[0.0, 0.0], [1.0, 0.0], [0.5, 1.0]], "color": [1.0, 0.5, 0.25], "alpha": 0.75},
        {"verts": [[0.1, 0.1], [0.9, 0.2], [0.4, 0.8]], "color": [0.2, 0.4, 0.6], "alpha": 0.25},
    ],
}


def test_parses_a_valid_scene():
    scene = parse_scene(VALID_SCENE)
    assert len(scene) == 2
    assert scene.background == [0.1, 0.2, 0.3]
    assert scene.mean_alpha == pytest.approx(0.5)


def test_rejects_unknown_and_missing_versions():
    with pytest.raises(FitError, match="version"):
        parse_scene(dict(VALID_SCENE, version=99))
    with pytest.raises(FitError):
        parse_scene({k: v for k, v in VALID_SCENE.items() if k != "version"})


def test_rejects_malformed_triangles():
    with pytest.raises(FitError):
        parse_scene(dict(VALID_SCENE, triangles=[{"verts": [[0, 0]]}]))
    with pytest.raises(FitError):
        parse_scene(dict(VALID_SCENE, triangles=[{"verts": [[0, 0]], "color": [1, 1, 1], "alpha": 1}]))


def test_empty_scene_is_valid():
    scene = parse_scene({"version": 1, "background": [0, 0, 0], "triangles": []})
    assert len(scene) == 0 and scene.mean_alpha == 0.0
    assert scene.params().shape == (0, 10)


def test_load_scene_files(tmp_path):
    path = tmp_path / "scene.json"
    path.write_text(json.dumps(VALID_SCENE))
    assert len(load_scene(path)) == 2
    with pytest.raises(FitError):
        load_scene(tmp_path / "absent.json")
    bad = tmp_path / "broken.json"
    bad.write_text("{not json")
    with pytest.raises(FitError, match="valid JSON"):
        load_scene(bad)
    scene_io.save_scene(tmp_path / "out.json", parse_scene(VALID_SCENE))
    assert load_scene(tmp_path / "out.json").params().tolist() == parse_scene(VALID_SCENE).params().tolist()


# ---------------------------------------------------------------- canvas.rs sizes


def test_fit_within_preserves_aspect_and_never_upscales():
    assert fit_within(1000, 500, 200) == (200, 100)
    assert fit_within(500, 1000, 200) == (100, 200)
    assert fit_within(64, 32, 200) == (64, 32)
    assert fit_within(0, 0, 200) == (1, 1)
    assert fit_within(10_000, 1, 100) == (100, 1)
    assert fit_within(300, 100, 0) == (300, 100)
    assert fit_within(1000, 333, 100) == (100, 33)  # 33.3
    assert fit_within(600, 100, 400) == (400, 67)  # 66.67
    assert fit_within(800, 100, 400) == (400, 50)
    assert fit_within(1600, 1000, 1024) == (1024, 640)


# ---------------------------------------------------------------- PNG container


def test_png_round_trip_and_pil_agreement():
    from PIL import Image

    rng = np.random.default_rng(5)
    for h, w in ((1, 1), (3, 7), (64, 48), (17, 255)):
        a = rng.integers(0, 256, (h, w, 3), dtype=np.uint8)
        data = scene_io.encode_png(a)
        assert np.array_equal(scene_io.decode_png(data), a)
        assert np.array_equal(np.asarray(Image.open(io.BytesIO(data)).convert("RGB")), a)


@pytest.mark.parametrize("mode", ["RGB", "RGBA", "L", "LA", "P"])
def test_png_reader_matches_pil_on_every_filter_and_colour_type(mode):
    from PIL import Image

    rng = np.random.default_rng(7)
    # smooth content with noise so PIL's adaptive filtering uses all five filter types
    yy, xx = np.mgrid[0:40, 0:53]
    base = np.stack([(xx * 5) % 256, (yy * 7) % 256, ((xx + yy) * 3) % 256], -1)
    img = np.clip(base + rng.integers(-3, 4, base.shape), 0, 255).astype(np.uint8)
    pil = Image.fromarray(img, "RGB")
    pil = pil.convert(mode) if mode != "P" else pil.quantize(64)
    buf = io.BytesIO()
    pil.save(buf, format="PNG", optimize=False)
    want = np.asarray(Image.open(io.BytesIO(buf.getvalue())).convert("RGB"))
    assert np.array_equal(scene_io.decode_png(buf.getvalue()), want)


def _png_with_filter(img: np.ndarray, ftype: int) -> bytes:
    """An RGB PNG whose every row uses filter `ftype` (PNG spec section 9.2)."""
    import struct
    import zlib

    h, w, bpp = img.shape[0], img.shape[1], 3
    rows = img.reshape(h, w * bpp).astype(np.int64)
    out = bytearray()
    for y in range(h):
        prev = rows[y - 1] if y else np.zeros(w * bpp, np.int64)
        out.append(ftype)
        for x in range(w * bpp):
            a = rows[y, x - bpp] if x >= bpp else 0
            b = prev[x]
            c = prev[x - bpp] if x >= bpp else 0
            if ftype == 0:
                pred = 0
            elif ftype == 1:
                pred = a
            elif ftype == 2:
                pred = b
            elif ftype == 3:
                pred = (a + b) // 2
            else:
                p = a + b - c
                pa, pb, pc = abs(p - a), abs(p - b), abs(p - c)
                pred = a if pa <= pb and pa <= pc else (b if pb <= pc else c)
            out.append(int(rows[y, x] - pred) & 0xFF)

    def chunk(k, d):
        return struct.pack(">I", len(d)) + k + d + struct.pack(">I", zlib.crc32(k + d) & 0xFFFFFFFF)

    return (b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", struct.pack(">IIBBBBB", w, h, 8, 2, 0, 0, 0)) +
            chunk(b"IDAT", zlib.compress(bytes(out))) + chunk(b"IEND", b""))


@pytest.mark.parametrize("ftype", [0, 1, 2, 3, 4])
def test_png_reader_undoes_each_filter_type(ftype):
    from PIL import Image

    img = np.random.default_rng(ftype).integers(0, 256, (9, 11, 3), dtype=np.uint8)
    data = _png_with_filter(img, ftype)
    assert np.array_equal(np.asarray(Image.open(io.BytesIO(data)).convert("RGB")), img)
    assert np.array_equal(scene_io.decode_png(data), img)


def test_reference_fit_target_decodes_like_pil():
    from PIL import Image

    path = GOLDEN / "fit_target_176.png"
    a = scene_io.read_png(path)
    assert a.shape == (176, 176, 3)
    assert np.array_equal(a, np.asarray(Image.open(path).convert("RGB")))


def test_png_reader_rejects_corruption():
    data = bytearray(scene_io.encode_png(np.zeros((4, 4, 3), np.uint8)))
    data[20] ^= 0xFF  # inside IHDR: the CRC no longer matches
    with pytest.raises(FitError):
        scene_io.decode_png(bytes(data))
    with pytest.raises(FitError):
        scene_io.decode_png(b"GIF89a")


# ---------------------------------------------------------------- sRGB oracle


def test_oracle_srgb_reference_cases(orc):
    # canvas.rs:120-136
    for v in (0, 1, 17, 128, 200, 255):
        assert orc.encode_srgb(orc.decode_srgb(np.array([v], np.uint8)))[0] == v
    assert orc.encode_srgb(np.array([-1.0, 2.0, np.nan], np.float32)).tolist() == [0, 255, 0]


def test_oracle_srgb_standard_values(orc):
    # the sRGB transfer function (IEC 61966-2-1), computed here in float64
    def enc64(v):
        v = min(max(v, 0.0), 1.0)
        s = 12.92 * v if v <= 0.0031308 else 1.055 * v ** (1 / 2.4) - 0.055
        return int(s * 255 + 0.5)

    def dec64(b):
        v = b / 255
        return v / 12.92 if v <= 0.04045 else ((v + 0.055) / 1.055) ** 2.4

    dec = orc.decode_srgb(np.arange(256, dtype=np.uint8))
    assert dec[0] == 0.0 and dec[255] == 1.0
    assert np.abs(dec.astype(np.float64) - np.array([dec64(b) for b in range(256)])).max() < 2e-7
    assert np.all(np.diff(dec) > 0)
    xs = np.linspace(0, 1, 20001).astype(np.float32)
    e = orc.encode_srgb(xs).astype(int)
    e64 = np.array([enc64(float(x)) for x in xs])
    # f32 rounding may move a value sitting on a byte boundary by one
    assert np.abs(e - e64).max() <= 1 and (e != e64).mean() < 1e-3
    assert orc.encode_srgb(np.array([0.5], np.float32))[0] == 188


def test_oracle_srgb_round_trips_every_byte(orc):
    b = np.arange(256, dtype=np.uint8)
    assert np.array_equal(orc.encode_srgb(orc.decode_srgb(b)), b)


def test_oracle_srgb_encoding_is_monotonic_with_sorted_thresholds(orc):
    # every float in [2^-14, 1]: the GPU encodes by counting thresholds, which is
    # the reference's byte only if its encoding never steps down
    drops, thr = orc.srgb_encode_scan()
    assert drops == 0
    assert np.all(np.diff(thr) > 0)
    assert orc.encode_srgb(thr[1:]).tolist() == list(range(1, 256))
    below = np.nextafter(thr[1:], np.float32(-1))
    assert orc.encode_srgb(below).tolist() == list(range(0, 255))
