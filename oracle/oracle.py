"""numpy front end of the C oracle (test infrastructure only).

Shapes mirror the reference's Python boundary (crates/diffrast-py/src/lib.rs:10-13):
params (B, T, 10) float32, images (B, H, W, 3) float32, backgrounds (B, 3).
Single-scene helpers take params (T, 10) and images (H, W, 3).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"

_F = ctypes.POINTER(ctypes.c_float)
_SZ = ctypes.c_size_t


class Counts(ctypes.Structure):
    _fields_ = [("n_box", ctypes.c_uint64), ("n_contrib", ctypes.c_uint64)]


class FitConfig(ctypes.Structure):
    _fields_ = [
        ("iters", ctypes.c_size_t),
        ("sigma_start", ctypes.c_float),
        ("sigma_end", ctypes.c_float),
        ("lr_pos", ctypes.c_float),
        ("lr_color", ctypes.c_float),
        ("lr_alpha", ctypes.c_float),
        ("patience", ctypes.c_long),
        ("min_delta", ctypes.c_float),
    ]


class FitReport(ctypes.Structure):
    _fields_ = [
        ("n_losses", ctypes.c_size_t),
        ("best_iter", ctypes.c_size_t),
        ("best_loss", ctypes.c_float),
        ("stop_reason", ctypes.c_int),
    ]


STOP_REASONS = {0: "Completed", 1: "Converged", 2: "Diverged"}


def build() -> Path:
    """Compile liboracle.so with its Makefile (gcc, -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        C = ctypes.POINTER(Counts)
        L.orc_render.argtypes = [_F, _SZ, _F, _SZ, _SZ, ctypes.c_float, _F, C]
        L.orc_mse.argtypes = [_F, _F, _SZ]
        L.orc_mse.restype = ctypes.c_float
        L.orc_loss_backward.argtypes = [_F, _SZ, _F, _SZ, _SZ, ctypes.c_float, _F, _F, _F, C]
        L.orc_loss_backward.restype = ctypes.c_float
        L.orc_backward_from_grad_inverted.argtypes = [_F, _SZ, _F, _SZ, _SZ, ctypes.c_float, _F, _F]
        L.orc_backward_from_grad.argtypes = [_F, _SZ, _F, _SZ, _SZ, ctypes.c_float, _F, _F]
        L.orc_render_batch.argtypes = [_F, _SZ, _SZ, _F, _SZ, _SZ, ctypes.c_float, _F, ctypes.c_int, C]
        L.orc_loss_backward_batch.argtypes = [
            _F, _SZ, _SZ, _F, _SZ, _SZ, ctypes.c_float, _F, _F, _F, ctypes.c_int, C]
        L.orc_backward_from_grad_batch.argtypes = [
            _F, _SZ, _SZ, _F, _SZ, _SZ, ctypes.c_float, _F, _F, ctypes.c_int]
        L.orc_finite_difference.argtypes = [_F, _SZ, _F, _SZ, _SZ, ctypes.c_float, _F, ctypes.c_float, _F]
        L.orc_finite_difference.restype = ctypes.c_float
        L.orc_adam_step.argtypes = [_F, _F, _F, _F, _F, ctypes.POINTER(ctypes.c_uint32), _SZ,
                                    ctypes.c_float, ctypes.c_float, ctypes.c_float]
        L.orc_project.argtypes = [_F, _SZ]
        L.orc_sigma_at.argtypes = [ctypes.c_float, ctypes.c_float, _SZ, _SZ]
        L.orc_sigma_at.restype = ctypes.c_float
        L.orc_fit.argtypes = [_F, _SZ, _SZ, _F, _F, _SZ, ctypes.POINTER(FitConfig), _F, _F,
                              ctypes.POINTER(FitReport), C]
        L.orc_mean_color.argtypes = [_F, _SZ, _SZ, _F]
        L.orc_sample.argtypes = [_F, _SZ, _SZ, ctypes.c_float, ctypes.c_float, _F]
        L.orc_signed_distance.argtypes = [_F, ctypes.c_float, ctypes.c_float]
        L.orc_signed_distance.restype = ctypes.c_float
        L.orc_coverage.argtypes = [_F, ctypes.c_float, ctypes.c_float, ctypes.c_float]
        L.orc_coverage.restype = ctypes.c_float
        L.orc_coverage_with_grad.argtypes = [_F, ctypes.c_float, ctypes.c_float, ctypes.c_float, _F]
        L.orc_coverage_with_grad.restype = ctypes.c_float
        L.orc_pixel_bounds.argtypes = [_F, _SZ, _SZ, ctypes.c_float, ctypes.POINTER(ctypes.c_uint64)]
        L.orc_pixel_bounds.restype = ctypes.c_int
        _U8 = ctypes.POINTER(ctypes.c_uint8)
        L.orc_encode_srgb.argtypes = [_F, _SZ, _U8]
        L.orc_decode_srgb.argtypes = [_U8, _SZ, _F]
        L.orc_srgb_encode_scan.argtypes = [_F]
        L.orc_srgb_encode_scan.restype = ctypes.c_uint64
        L.orc_lanczos3.argtypes = [ctypes.c_float]
        L.orc_lanczos3.restype = ctypes.c_float
        L.orc_lanczos3_taps.argtypes = [_SZ, _SZ, _SZ, ctypes.POINTER(ctypes.c_size_t), _F, _SZ]
        L.orc_lanczos3_taps.restype = _SZ
        L.orc_resize_lanczos3.argtypes = [_U8, _SZ, _SZ, _SZ, _U8, _SZ, _SZ]
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a: np.ndarray):
    return a.ctypes.data_as(_F)


def _bgs(background, B: int) -> np.ndarray:
    bg = _f32(background)
    if bg.ndim == 1:
        bg = np.broadcast_to(bg, (B, 3))
    return _f32(bg.reshape(B, 3))


def render(params, height: int, width: int, sigma: float, background=(0, 0, 0), counts=None):
    """raster.rs:37-43 for one scene: params (T, 10) -> image (H, W, 3)."""
    p = _f32(params).reshape(-1, 10)
    bg = _f32(background)
    out = np.empty((height, width, 3), np.float32)
    lib().orc_render(_p(p), p.shape[0], _p(bg), width, height, sigma, _p(out),
                     ctypes.byref(counts) if counts is not None else None)
    return out


def render_batch(params, height: int, width: int, sigma: float, background=(0, 0, 0),
                 nthreads: int = 0, counts=None):
    p = _f32(params)
    B, T = p.shape[0], p.shape[1]
    bgs = _bgs(background, B)
    out = np.empty((B, height, width, 3), np.float32)
    lib().orc_render_batch(_p(p), B, T, _p(bgs), width, height, sigma, _p(out), nthreads,
                           ctypes.byref(counts) if counts is not None else None)
    return out


def mse(a, b) -> float:
    a, b = _f32(a), _f32(b)
    assert a.size == b.size
    return float(lib().orc_mse(_p(a), _p(b), a.size))


def loss_backward(params, target, sigma: float, background=(0, 0, 0), counts=None,
                  want_image: bool = False):
    """grad.rs:56-131 for one scene -> (loss, grads (T, 10)[, image])."""
    p = _f32(params).reshape(-1, 10)
    t = _f32(target)
    H, W = t.shape[0], t.shape[1]
    bg = _f32(background)
    g = np.empty_like(p)
    img = np.empty((H, W, 3), np.float32) if want_image else None
    loss = lib().orc_loss_backward(_p(p), p.shape[0], _p(bg), W, H, sigma, _p(t), _p(g),
                                   _p(img) if img is not None else None,
                                   ctypes.byref(counts) if counts is not None else None)
    return (float(loss), g, img) if want_image else (float(loss), g)


def loss_backward_batch(params, targets, sigma: float, background=(0, 0, 0), nthreads: int = 0,
                        counts=None):
    """grad.rs:192-207 backward_batch -> (losses (B,), grads (B, T, 10))."""
    p = _f32(params)
    t = _f32(targets)
    B, T = p.shape[0], p.shape[1]
    H, W = t.shape[1], t.shape[2]
    bgs = _bgs(background, B)
    losses = np.empty(B, np.float32)
    g = np.empty_like(p)
    lib().orc_loss_backward_batch(_p(p), B, T, _p(bgs), W, H, sigma, _p(t), _p(losses), _p(g),
                                  nthreads, ctypes.byref(counts) if counts is not None else None)
    return losses, g


def backward_from_grad(params, grad_image, sigma: float, background=(0, 0, 0),
                       inverted: bool = False):
    """Upstream-gradient backward for one scene -> grads (T, 10).

    inverted=False: dL/dpixel used as given (backward_batch_reduced.wgsl:143-156).
    inverted=True : the reference CPU binding's target reconstruction
                    (crates/diffrast-py/src/lib.rs:301-318).
    """
    p = _f32(params).reshape(-1, 10)
    gi = _f32(grad_image)
    H, W = gi.shape[0], gi.shape[1]
    bg = _f32(background)
    g = np.empty_like(p)
    fn = lib().orc_backward_from_grad_inverted if inverted else lib().orc_backward_from_grad
    fn(_p(p), p.shape[0], _p(bg), W, H, sigma, _p(gi), _p(g))
    return g


def backward_from_grad_batch(params, grad_images, sigma: float, background=(0, 0, 0),
                             nthreads: int = 0):
    p = _f32(params)
    gi = _f32(grad_images)
    B, T = p.shape[0], p.shape[1]
    H, W = gi.shape[1], gi.shape[2]
    bgs = _bgs(background, B)
    g = np.empty_like(p)
    lib().orc_backward_from_grad_batch(_p(p), B, T, _p(bgs), W, H, sigma, _p(gi), _p(g), nthreads)
    return g


def finite_difference(params, target, sigma: float, eps: float, background=(0, 0, 0)):
    """grad.rs:298-323 -> (loss, grads (T, 10))."""
    p = _f32(params).reshape(-1, 10)
    t = _f32(target)
    H, W = t.shape[0], t.shape[1]
    bg = _f32(background)
    g = np.empty_like(p)
    loss = lib().orc_finite_difference(_p(p), p.shape[0], _p(bg), W, H, sigma, _p(t), eps, _p(g))
    return float(loss), g


class Adam:
    """optim.rs:11-60 with flat state arrays."""

    def __init__(self, n: int, beta1=0.9, beta2=0.999, eps=1e-8):
        self.m = np.zeros(n, np.float32)
        self.v = np.zeros(n, np.float32)
        self.t = ctypes.c_uint32(0)
        self.beta1, self.beta2, self.eps = beta1, beta2, eps

    def step(self, params: np.ndarray, grads, lr) -> None:
        assert params.dtype == np.float32 and params.flags.c_contiguous
        g, lr = _f32(grads).ravel(), _f32(lr).ravel()
        lib().orc_adam_step(_p(params), _p(g), _p(lr), _p(self.m), _p(self.v),
                            ctypes.byref(self.t), params.size, self.beta1, self.beta2, self.eps)

    @property
    def steps_taken(self) -> int:
        return int(self.t.value)


def project(params) -> np.ndarray:
    """fit.rs:399-424 on a copy."""
    p = _f32(params).copy()
    lib().orc_project(_p(p), p.size)
    return p


def sigma_at(sigma_start: float, sigma_end: float, iters: int, i: int) -> float:
    return float(lib().orc_sigma_at(sigma_start, sigma_end, iters, i))


def mean_color(image) -> np.ndarray:
    img = _f32(image)
    out = np.empty(3, np.float32)
    lib().orc_mean_color(_p(img), img.shape[1], img.shape[0], _p(out))
    return out


def sample(image, x: float, y: float) -> np.ndarray:
    img = _f32(image)
    out = np.empty(3, np.float32)
    lib().orc_sample(_p(img), img.shape[1], img.shape[0], x, y, _p(out))
    return out


FIT_DEFAULTS = dict(iters=1500, sigma_start=0.02, sigma_end=0.0015, lr_pos=0.004,
                    lr_color=0.02, lr_alpha=0.01, patience=250, min_delta=1e-7)


def fit(target, init_params, background=None, counts=None, **cfg):
    """fit.rs:166-288 from a given initial scene.

    Returns dict(losses, best_params, best_iter, best_loss, stop_reason).
    `patience=None` disables early stopping (fit.rs:60-62). `counts` (a
    Counts) sums the box and contributing pairs of every iteration.
    """
    c = dict(FIT_DEFAULTS)
    c.update(cfg)
    t = _f32(target)
    H, W = t.shape[0], t.shape[1]
    p = _f32(init_params).reshape(-1, 10)
    bg = _f32(mean_color(t) if background is None else background)
    conf = FitConfig(c["iters"], c["sigma_start"], c["sigma_end"], c["lr_pos"], c["lr_color"],
                     c["lr_alpha"], -1 if c["patience"] is None else int(c["patience"]),
                     c["min_delta"])
    losses = np.empty(max(c["iters"], 1), np.float32)
    best = np.empty_like(p)
    rep = FitReport()
    lib().orc_fit(_p(t), W, H, _p(bg), _p(p), p.shape[0], ctypes.byref(conf), _p(losses),
                  _p(best), ctypes.byref(rep), ctypes.byref(counts) if counts is not None else None)
    return dict(losses=losses[: rep.n_losses].copy(), best_params=best, best_iter=rep.best_iter,
                best_loss=float(rep.best_loss), stop_reason=STOP_REASONS[rep.stop_reason])


def signed_distance(tri, x: float, y: float) -> float:
    """raster.rs:96-106 for one triangle record (10 floats)."""
    t = _f32(tri).ravel()
    return float(lib().orc_signed_distance(_p(t), x, y))


def coverage(tri, x: float, y: float, sigma: float) -> float:
    """raster.rs:74-76."""
    t = _f32(tri).ravel()
    return float(lib().orc_coverage(_p(t), x, y, sigma))


def coverage_with_grad(tri, x: float, y: float, sigma: float):
    """grad.rs:231-270 -> (cov, d cov / d verts as (3, 2))."""
    t = _f32(tri).ravel()
    d = np.zeros(6, np.float32)
    cov = lib().orc_coverage_with_grad(_p(t), x, y, sigma, _p(d))
    return float(cov), d.reshape(3, 2)


def pixel_bounds(tri, width: int, height: int, sigma: float):
    """raster.rs:144-168 -> (x0, y0, x1, y1) or None."""
    t = _f32(tri).ravel()
    out = (ctypes.c_uint64 * 4)()
    ok = lib().orc_pixel_bounds(_p(t), width, height, sigma, out)
    return tuple(int(v) for v in out) if ok else None


def cpu_count() -> int:
    return os.cpu_count() or 1


def encode_srgb(values) -> np.ndarray:
    """canvas.rs:100-105 per value."""
    v = _f32(values)
    out = np.empty(v.shape, np.uint8)
    lib().orc_encode_srgb(_p(v), v.size, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
    return out


def decode_srgb(data) -> np.ndarray:
    """canvas.rs:108-115 per byte."""
    b = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty(b.shape, np.float32)
    lib().orc_decode_srgb(b.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), b.size, _p(out))
    return out


def srgb_encode_scan():
    """(count of monotonicity breaks of encode_srgb over [2^-14, 1], thresholds[256])."""
    thr = np.zeros(256, np.float32)
    drops = lib().orc_srgb_encode_scan(_p(thr))
    return int(drops), thr


def lanczos3(x: float) -> float:
    """image 0.25.10 lanczos3_kernel in f32."""
    return float(lib().orc_lanczos3(x))


def lanczos3_taps(n_src: int, n_dst: int, o: int):
    """(left, weights) of output index o of one resize pass."""
    cap = 64 + int(6 * max(n_src / n_dst, 1.0))
    w = np.zeros(cap, np.float32)
    left = ctypes.c_size_t(0)
    n = lib().orc_lanczos3_taps(n_src, n_dst, o, ctypes.byref(left), _p(w), cap)
    assert n > 0
    return int(left.value), w[:n].copy()


def resize_lanczos3(img, width: int, height: int) -> np.ndarray:
    """Canvas::load_image's resize_exact(width, height, Lanczos3) of an (H, W, C) uint8 image."""
    a = np.ascontiguousarray(img, dtype=np.uint8)
    H, W, C = a.shape
    out = np.zeros((height, width, C), np.uint8)
    u8 = ctypes.POINTER(ctypes.c_uint8)
    lib().orc_resize_lanczos3(a.ctypes.data_as(u8), W, H, C, out.ctypes.data_as(u8), width, height)
    return out
