"""Scene JSON and sRGB PNG files: the artefacts of the reference's `fit` binary.

- `scene_to_json` writes crates/diffrast/src/serial.rs:21-72's format character for
  character (hand-rolled there, six decimals, non-finite values written as 0.0).
- `parse_scene` / `load_scene` read it back as python/diffrast/runner.py:204-236 does,
  with the same schema-version check and `FitError` on malformed input.
- `save_png` / `load_png` are Canvas::save_png / load_image (canvas.rs:61-86): the
  gamma (encode_srgb / decode_srgb, canvas.rs:100-115) runs on the GPU through
  `drh_encode_srgb` / `drh_decode_srgb`, bit-identical to the reference; the PNG
  container is written and read here over zlib (8-bit RGB out; 8-bit gray, RGB,
  palette, gray+alpha and RGBA in, alpha dropped as `to_rgb8` drops it).
  `load_png(path, width, height)` resamples to another size first, as `load_image`
  does, with image 0.25's Lanczos3 `resize_exact` on the GPU (`drh_resize_lanczos3`);
  `load_target` is the fit binary's target loading (aspect kept by `fit_within`).
"""

from __future__ import annotations

import json
import math
import struct
import zlib
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

N_PARAMS = 10


class FitError(RuntimeError):
    """A scene or image file could not be read (python/diffrast/runner.py:22-23)."""


@dataclass
class Triangle:
    verts: list
    color: list
    alpha: float


@dataclass
class Scene:
    background: list
    triangles: list = field(default_factory=list)

    def __len__(self) -> int:
        return len(self.triangles)

    @property
    def mean_alpha(self) -> float:
        """runner.py:41-45: 0.0 for an empty scene."""
        if not self.triangles:
            return 0.0
        return sum(t.alpha for t in self.triangles) / len(self.triangles)

    def params(self) -> np.ndarray:
        """(T, 10) float32 in the reference's order (scene.rs:81-92)."""
        out = np.zeros((len(self.triangles), N_PARAMS), np.float32)
        for i, t in enumerate(self.triangles):
            out[i, 0:6] = np.asarray(t.verts, np.float32).reshape(6)
            out[i, 6:9] = np.asarray(t.color, np.float32).reshape(3)
            out[i, 9] = t.alpha
        return out

    @classmethod
    def from_params(cls, params, background=(0.0, 0.0, 0.0)) -> "Scene":
        """scene.rs:94-101 set_params on a scene of len(params) triangles."""
        p = np.asarray(params, np.float32).reshape(-1, N_PARAMS)
        tris = [Triangle(verts=[[float(r[0]), float(r[1])], [float(r[2]), float(r[3])],
                                [float(r[4]), float(r[5])]],
                         color=[float(r[6]), float(r[7]), float(r[8])], alpha=float(r[9]))
                for r in p]
        return cls(background=[float(np.float32(b)) for b in background], triangles=tris)


# ---------------------------------------------------------------- JSON

def _fmt_f32(v) -> str:
    """serial.rs:63-72: `{v:.6}` of the f32 value, "0.0" when not finite.

    Both Rust's fixed-precision formatting and Python's are correctly rounded
    (ties to even) decimal conversions of the exact binary value, and the f32
    value widens to a double exactly.
    """
    v = float(np.float32(v))
    if not math.isfinite(v):
        return "0.0"
    return "%.6f" % v


def _push_array(vals) -> str:
    return "[" + ", ".join(_fmt_f32(v) for v in vals) + "]"


def scene_to_json(scene, background=None) -> str:
    """serial.rs:21-46. `scene` is a Scene, or (T, 10) parameters with `background`."""
    if not isinstance(scene, Scene):
        scene = Scene.from_params(scene, (0.0, 0.0, 0.0) if background is None else background)
    s = "{\n  \"version\": 1,\n  \"background\": " + _push_array(scene.background)
    s += ",\n  \"triangles\": [\n"
    n = len(scene.triangles)
    for i, t in enumerate(scene.triangles):
        s += "    {\"verts\": [" + ", ".join(_push_array(v) for v in t.verts) + "], \"color\": "
        s += _push_array(t.color) + ", \"alpha\": " + _fmt_f32(t.alpha) + "}"
        if i + 1 < n:
            s += ","
        s += "\n"
    return s + "  ]\n}\n"


def save_scene(path, scene, background=None) -> None:
    """fit.rs:102: the scene.json the fit binary writes."""
    Path(path).write_text(scene_to_json(scene, background))


def parse_scene(raw: dict) -> Scene:
    """runner.py:218-236: decoded JSON to a Scene, checking the schema version."""
    version = raw.get("version") if isinstance(raw, dict) else None
    if version != 1:
        raise FitError(f"unsupported scene version: {version!r}")
    try:
        triangles = []
        for t in raw["triangles"]:
            verts = np.asarray(t["verts"], np.float64)
            color = np.asarray(t["color"], np.float64)
            if verts.shape != (3, 2) or color.shape != (3,):
                raise ValueError(f"a triangle needs 3 vertices of 2 and 3 colour values, got {t!r}")
            triangles.append(Triangle(verts=t["verts"], color=t["color"], alpha=float(t["alpha"])))
        background = raw["background"]
        if np.asarray(background, np.float64).shape != (3,):
            raise ValueError(f"background needs 3 values, got {background!r}")
        return Scene(background=background, triangles=triangles)
    except (KeyError, TypeError, ValueError) as exc:
        raise FitError(f"malformed scene: {exc}") from exc


def load_scene(path) -> Scene:
    """runner.py:204-215."""
    path = Path(path)
    if not path.exists():
        raise FitError(f"no scene file at {path}")
    try:
        raw = json.loads(path.read_text())
    except json.JSONDecodeError as exc:
        raise FitError(f"{path} is not valid JSON: {exc}") from exc
    return parse_scene(raw)


# ---------------------------------------------------------------- sizes

def fit_within(w: int, h: int, max_side: int) -> tuple[int, int]:
    """canvas.rs:89-97: scale (w, h) down so neither side exceeds max_side, keeping the
    aspect ratio; never up, never to zero. f64::round rounds halves away from zero."""
    if max_side == 0 or w == 0 or h == 0 or (w <= max_side and h <= max_side):
        return max(w, 1), max(h, 1)
    scale = max_side / max(w, h)
    return max(int(math.floor(w * scale + 0.5)), 1), max(int(math.floor(h * scale + 0.5)), 1)


# ---------------------------------------------------------------- PNG container

_SIG = b"\x89PNG\r\n\x1a\n"


def _chunk(kind: bytes, data: bytes) -> bytes:
    return struct.pack(">I", len(data)) + kind + data + struct.pack(">I", zlib.crc32(kind + data) & 0xFFFFFFFF)


def encode_png(rgb8) -> bytes:
    """(H, W, 3) uint8 to an 8-bit RGB PNG (filter type 0 on every row)."""
    a = np.ascontiguousarray(rgb8, dtype=np.uint8)
    if a.ndim != 3 or a.shape[2] != 3 or a.shape[0] == 0 or a.shape[1] == 0:
        raise ValueError(f"expected a non-empty (H, W, 3) image, got {a.shape}")
    h, w = a.shape[0], a.shape[1]
    raw = np.zeros((h, 1 + 3 * w), np.uint8)
    raw[:, 1:] = a.reshape(h, 3 * w)
    ihdr = struct.pack(">IIBBBBB", w, h, 8, 2, 0, 0, 0)
    return _SIG + _chunk(b"IHDR", ihdr) + _chunk(b"IDAT", zlib.compress(raw.tobytes(), 6)) + _chunk(b"IEND", b"")


def write_png(path, rgb8) -> None:
    Path(path).write_bytes(encode_png(rgb8))


def _unfilter(data: bytes, h: int, stride: int, bpp: int) -> np.ndarray:
    """PNG filter types 0-4 (None, Sub, Up, Average, Paeth), row by row."""
    if len(data) < h * (stride + 1):
        raise FitError("truncated PNG image data")
    out = np.zeros((h, stride), np.uint8)
    prev = np.zeros(stride, np.int32)
    pos = 0
    for y in range(h):
        ft = data[pos]
        row = np.frombuffer(data, np.uint8, stride, pos + 1).astype(np.int32)
        pos += stride + 1
        if ft == 0:
            cur = row
        elif ft == 2:
            cur = (row + prev) & 0xFF
        elif ft in (1, 3, 4):
            cur = np.zeros(stride, np.int32)
            for x in range(stride):
                left = cur[x - bpp] if x >= bpp else 0
                up = prev[x]
                if ft == 1:
                    pred = left
                elif ft == 3:
                    pred = (left + up) >> 1
                else:
                    ul = prev[x - bpp] if x >= bpp else 0
                    p = left + up - ul
                    pa, pb, pc = abs(p - left), abs(p - up), abs(p - ul)
                    pred = left if (pa <= pb and pa <= pc) else (up if pb <= pc else ul)
                cur[x] = (row[x] + pred) & 0xFF
        else:
            raise FitError(f"unknown PNG filter type {ft}")
        out[y] = cur
        prev = cur
    return out


def decode_png(data: bytes) -> np.ndarray:
    """A non-interlaced 8-bit PNG to (H, W, 3) uint8 RGB."""
    if data[:8] != _SIG:
        raise FitError("not a PNG file")
    pos, ihdr, plte, idat = 8, None, None, []
    while pos + 8 <= len(data):
        n, kind = struct.unpack(">I4s", data[pos:pos + 8])
        body = data[pos + 8:pos + 8 + n]
        crc = struct.unpack(">I", data[pos + 8 + n:pos + 12 + n])[0]
        if zlib.crc32(kind + body) & 0xFFFFFFFF != crc:
            raise FitError(f"PNG chunk {kind!r} fails its CRC")
        if kind == b"IHDR":
            ihdr = struct.unpack(">IIBBBBB", body)
        elif kind == b"PLTE":
            plte = np.frombuffer(body, np.uint8).reshape(-1, 3)
        elif kind == b"IDAT":
            idat.append(body)
        elif kind == b"IEND":
            break
        pos += 12 + n
    if ihdr is None or not idat:
        raise FitError("PNG without IHDR or image data")
    w, h, depth, ctype, _comp, _filt, interlace = ihdr
    channels = {0: 1, 2: 3, 3: 1, 4: 2, 6: 4}.get(ctype)
    if depth != 8 or channels is None or interlace != 0:
        raise FitError(f"unsupported PNG: bit depth {depth}, colour type {ctype}, interlace {interlace}")
    px = _unfilter(zlib.decompress(b"".join(idat)), h, w * channels, channels).reshape(h, w, channels)
    if ctype == 3:
        if plte is None:
            raise FitError("palette PNG without PLTE")
        return plte[px[:, :, 0]]
    if ctype in (0, 4):
        return np.repeat(px[:, :, :1], 3, axis=2)
    return np.ascontiguousarray(px[:, :, :3])


def read_png(path) -> np.ndarray:
    return decode_png(Path(path).read_bytes())


# ---------------------------------------------------------------- gamma on the GPU

def _context():
    from . import torch_layer

    return torch_layer._context(torch_layer._gpu())


def encode_srgb(images):
    """Linear values to sRGB bytes, canvas.rs:100-105 per value, on the GPU. A torch
    tensor on the GPU stays there (uint8 tensor, current stream); anything else is
    copied through and returned as a numpy uint8 array of the same shape."""
    try:
        import torch
    except ImportError:  # pragma: no cover - torch is a dependency of the package
        torch = None
    if torch is not None and isinstance(images, torch.Tensor) and images.is_cuda:
        from . import torch_layer

        x = images.detach().to(torch.float32).contiguous()
        out = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
        torch_layer._context(x.device).encode_srgb_ptr(x.data_ptr(), x.numel(), out.data_ptr(),
                                                        torch_layer._stream(x.device))
        return out
    if torch is not None and isinstance(images, torch.Tensor):
        images = images.detach().numpy()
    return _context().encode_srgb(images)


def decode_srgb(data):
    """sRGB bytes to linear float32, canvas.rs:108-115 per byte, on the GPU."""
    try:
        import torch
    except ImportError:  # pragma: no cover
        torch = None
    if torch is not None and isinstance(data, torch.Tensor) and data.is_cuda:
        from . import torch_layer

        b = data.detach().to(torch.uint8).contiguous()
        out = torch.empty(b.shape, dtype=torch.float32, device=b.device)
        torch_layer._context(b.device).decode_srgb_ptr(b.data_ptr(), b.numel(), out.data_ptr(),
                                                        torch_layer._stream(b.device))
        return out
    if torch is not None and isinstance(data, torch.Tensor):
        data = data.detach().numpy()
    return _context().decode_srgb(data)


def save_png(path, image) -> None:
    """Canvas::save_png (canvas.rs:61-68): an (H, W, 3) linear image to an sRGB PNG."""
    shape = tuple(image.shape)
    if len(shape) != 3 or shape[2] != 3:
        raise ValueError(f"expected an (H, W, 3) image, got {shape}")
    b = encode_srgb(image)
    if not isinstance(b, np.ndarray):
        b = b.cpu().numpy()
    write_png(path, b)


def _read(path) -> np.ndarray:
    try:
        return read_png(path)
    except OSError as exc:
        raise FitError(f"cannot read {path}: {exc}") from exc


def _linear(rgb: np.ndarray, width: int, height: int):
    """Bytes resampled to width x height (image 0.25's Lanczos3 resize_exact, on the
    GPU via drh_resize_lanczos3; the same size is left as is), then decoded."""
    if width <= 0 or height <= 0:
        raise FitError(f"cannot resize to {width}x{height}")
    if (width, height) != (rgb.shape[1], rgb.shape[0]):
        rgb = _context().resize_lanczos3(rgb, width, height)
    return decode_srgb(rgb)


def load_png(path, width: int | None = None, height: int | None = None) -> np.ndarray:
    """Canvas::load_image (canvas.rs:70-86): an (H, W, 3) linear float32 image at
    width x height (default: the file's size)."""
    rgb = _read(path)
    h, w = rgb.shape[0], rgb.shape[1]
    return _linear(rgb, w if width is None else int(width), h if height is None else int(height))


def load_target(path, size: int) -> np.ndarray:
    """The fit binary's target loading (crates/diffrast/src/bin/fit.rs:186-196): the file
    scaled so neither side exceeds `size`, keeping its aspect ratio (fit_within)."""
    if not Path(path).exists():
        raise FitError(f"no such file: {path}")
    rgb = _read(path)
    return _linear(rgb, *fit_within(rgb.shape[1], rgb.shape[0], size))
