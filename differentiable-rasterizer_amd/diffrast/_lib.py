"""ctypes binding of libdiffrast_hip.so (the C ABI in include/diffrast_hip.h).

There is no CPU fallback: if the library is missing or no HIP device is
present, the calls raise. `Context` methods accept numpy arrays (host
pointers, synchronous) or, via the `*_ptr` forms, raw device pointers and a
stream handle (asynchronous), which is what the torch layer uses.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent.parent / "libdiffrast_hip.so"

DRH_OK = 0
ERR_NAMES = {
    1: "NoDevice",
    2: "Timeout",
    3: "Device",
    4: "Readback",
    5: "TooLarge",
    6: "InvalidArgument",
}
HOST_PTRS = 0x1
SYNC = 0x2
EXACT_MATH = 0x4
DETERMINISTIC = 0x8
CHANNELS_FIRST = 0x10
PHASES = 0x20

STOP_REASONS = {0: "Completed", 1: "Converged", 2: "Diverged"}
CONFIG_ERRORS = {1: "NoTriangles", 2: "NonPositiveSigma", 3: "SigmaNotDecreasing",
                 4: "NonPositiveLearningRate"}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_U32 = ctypes.c_uint32


class DiffrastError(RuntimeError):
    """A failed C ABI call; `code` is the drh status (1-6)."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{ERR_NAMES.get(code, code)}: {message}")
        self.code = code


class FitConfig(ctypes.Structure):
    _fields_ = [
        ("iters", ctypes.c_int64),
        ("sigma_start", ctypes.c_float),
        ("sigma_end", ctypes.c_float),
        ("lr_pos", ctypes.c_float),
        ("lr_color", ctypes.c_float),
        ("lr_alpha", ctypes.c_float),
        ("patience", ctypes.c_int64),
        ("min_delta", ctypes.c_float),
    ]


class FitReport(ctypes.Structure):
    _fields_ = [
        ("n_losses", ctypes.c_int64),
        ("best_iter", ctypes.c_int64),
        ("best_loss", ctypes.c_float),
        ("stop_reason", ctypes.c_int32),
    ]


class Timings(ctypes.Structure):
    _fields_ = [
        ("setup_ms", ctypes.c_double),
        ("raster_ms", ctypes.c_double),
        ("reduce_ms", ctypes.c_double),
        ("adam_ms", ctypes.c_double),
        ("setup_n", ctypes.c_int64),
        ("raster_n", ctypes.c_int64),
        ("reduce_n", ctypes.c_int64),
        ("adam_n", ctypes.c_int64),
        ("backward_ms", ctypes.c_double),
        ("backward_n", ctypes.c_int64),
    ]


class PhaseTimings(ctypes.Structure):
    _fields_ = [(name, ctypes.c_double) for name in
                ("pack_ms", "alloc_ms", "dispatch_ms", "readback_ms", "loss_ms", "total_ms")]


class StepInfo(ctypes.Structure):
    _fields_ = [("iter", ctypes.c_int64), ("loss", ctypes.c_float), ("sigma", ctypes.c_float)]


class FitStatus(ctypes.Structure):
    _fields_ = [
        ("iter", ctypes.c_int64),
        ("best_iter", ctypes.c_int64),
        ("best_loss", ctypes.c_float),
        ("sigma", ctypes.c_float),
        ("done", ctypes.c_int32),
        ("stop_reason", ctypes.c_int32),
    ]


# Every symbol include/diffrast_hip.h declares, with its ctypes signature.
SIGNATURES = {
    "drh_timing_enable": ([_P, ctypes.c_int], ctypes.c_int),
    "drh_timing_read": ([_P, ctypes.POINTER(Timings)], ctypes.c_int),
    "drh_phases_read": ([ctypes.POINTER(PhaseTimings)], ctypes.c_int),
    "drh_create": ([ctypes.POINTER(_P)], ctypes.c_int),
    "drh_destroy": ([_P], ctypes.c_int),
    "drh_last_error": ([], ctypes.c_char_p),
    "drh_device_info": ([_P, ctypes.c_char_p, ctypes.c_size_t], ctypes.c_int),
    "drh_is_discrete": ([_P], ctypes.c_int),
    "drh_params_per_triangle": ([], ctypes.c_int),
    "drh_pool_stats": ([_P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64),
                        ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "drh_clear_pool": ([_P], ctypes.c_int),
    "drh_render": ([_P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P, _P, _U32], ctypes.c_int),
    "drh_fused_loss_backward": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P, _P, _P, _P, _U32],
                                ctypes.c_int),
    "drh_fused_loss_backward_noalloc": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P, _P, _P, _P, _U32],
                                        ctypes.c_int),
    "drh_backward_from_grad": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P, _P, _U32], ctypes.c_int),
    "drh_adam_project_step": ([_P, _P, _P, _P, _P, _P, _I64, _U32, _F32, _F32, _F32, ctypes.c_int, _P, _U32],
                              ctypes.c_int),
    "drh_fit_validate": ([ctypes.POINTER(FitConfig), _I64], ctypes.c_int),
    "drh_fit": ([_P, _P, _I64, _I64, _P, _P, _I64, ctypes.POINTER(FitConfig), _P, _P, _P,
                 ctypes.POINTER(FitReport), _P, _U32], ctypes.c_int),
    "drh_fitter_create": ([_P, _P, _I64, _I64, _P, _P, _I64, ctypes.POINTER(FitConfig), _P, _U32,
                           ctypes.POINTER(_P)], ctypes.c_int),
    "drh_fitter_destroy": ([_P], ctypes.c_int),
    "drh_fitter_step": ([_P, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(StepInfo)], ctypes.c_int),
    "drh_fitter_run": ([_P, _I64, ctypes.POINTER(_I64)], ctypes.c_int),
    "drh_fitter_status": ([_P, ctypes.POINTER(FitStatus)], ctypes.c_int),
    "drh_fitter_scene": ([_P, _P, _U32], ctypes.c_int),
    "drh_fitter_losses": ([_P, _P, _I64, ctypes.POINTER(_I64), _U32], ctypes.c_int),
    "drh_fitter_render_current": ([_P, _P, _U32], ctypes.c_int),
    "drh_fitter_report": ([_P, _P, ctypes.POINTER(FitReport), _U32], ctypes.c_int),
    "drh_record_bytes": ([_I64, _I64, _I64, _I64, ctypes.POINTER(ctypes.c_uint64)], ctypes.c_int),
    "drh_render_record": ([_P, _P, _P, _I64, _I64, _I64, _I64, _F32, _P, _P, ctypes.c_uint64, _P, _U32],
                          ctypes.c_int),
    "drh_backward_recorded": ([_P, _P, ctypes.c_uint64, _P, _I64, _I64, _I64, _I64, _F32, _P, _P, _U32],
                              ctypes.c_int),
    "drh_encode_srgb": ([_P, _P, _I64, _P, _P, _U32], ctypes.c_int),
    "drh_decode_srgb": ([_P, _P, _I64, _P, _P, _U32], ctypes.c_int),
    "drh_resize_lanczos3": ([_P, _P, _I64, _I64, _I64, _P, _I64, _I64, _P, _U32], ctypes.c_int),
}

_lib = None
_lock = threading.Lock()


def _load_torch_runtime() -> None:
    """Load PyTorch's HIP runtime first, when PyTorch is installed.

    A process has one libamdhip64.so.7: PyTorch bundles its own and the library
    links the system one under the same soname, so whichever is loaded first
    serves both. PyTorch only works with its own, and the torch layer passes
    its device pointers and streams to this library, so it must come first.
    """
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def lib() -> ctypes.CDLL:
    """Load the HIP library; raises if it has not been built."""
    global _lib
    with _lock:
        if _lib is None:
            _load_torch_runtime()
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing; build it with `python build.py` "
                    "(or __graft_entry__.build()). There is no CPU fallback.")
            L = ctypes.CDLL(str(LIB_PATH))
            for name, (args, res) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.argtypes = args
                fn.restype = res
            _lib = L
    return _lib


def last_error() -> str:
    return lib().drh_last_error().decode(errors="replace")


def check(rc: int) -> None:
    if rc != DRH_OK:
        raise DiffrastError(rc, last_error())


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _bgs(background, B: int) -> np.ndarray:
    bg = _f32(background)
    if bg.ndim == 1:
        bg = np.broadcast_to(bg, (B, 3))
    return _f32(bg.reshape(B, 3))


class Context:
    """A drh_ctx bound to the current HIP device (GpuRasterizer::new)."""

    def __init__(self):
        h = ctypes.c_void_p()
        check(lib().drh_create(ctypes.byref(h)))
        self.handle = h

    def close(self) -> bool:
        if self.handle:
            lib().drh_destroy(self.handle)
            self.handle = None
            return True
        return False

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- introspection -----------------------------------------------------
    def device_info(self) -> str:
        buf = ctypes.create_string_buffer(512)
        check(lib().drh_device_info(self.handle, buf, 512))
        return buf.value.decode()

    def is_discrete(self) -> bool:
        return bool(lib().drh_is_discrete(self.handle))

    def pool_stats(self) -> dict:
        h, m, b = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        check(lib().drh_pool_stats(self.handle, ctypes.byref(h), ctypes.byref(m), ctypes.byref(b)))
        return dict(hits=h.value, misses=m.value, bytes=b.value)

    def clear_pool(self) -> None:
        check(lib().drh_clear_pool(self.handle))

    def timing(self, enable: bool) -> None:
        """Bracket every launched kernel with HIP events (BackwardTimings)."""
        check(lib().drh_timing_enable(self.handle, int(enable)))

    def read_timings(self) -> dict:
        """Accumulated kernel milliseconds and launch counts since the last read."""
        t = Timings()
        check(lib().drh_timing_read(self.handle, ctypes.byref(t)))
        return {name: getattr(t, name) for name, _ in Timings._fields_}

    @staticmethod
    def read_phases() -> dict:
        """Host phases of this thread's last call made with the PHASES flag."""
        t = PhaseTimings()
        check(lib().drh_phases_read(ctypes.byref(t)))
        return {name: getattr(t, name) for name, _ in PhaseTimings._fields_}

    # -- device-pointer forms (asynchronous on `stream`) ---------------------
    def render_ptr(self, params, bgs, B, T, H, W, sigma, out, stream=None, flags=0):
        check(lib().drh_render(self.handle, params, bgs, B, T, H, W, sigma, out, stream, flags))

    def fused_ptr(self, params, bgs, targets, B, T, H, W, sigma, losses, grads, images=None,
                  stream=None, flags=0):
        check(lib().drh_fused_loss_backward(self.handle, params, bgs, targets, B, T, H, W, sigma,
                                            losses, grads, images, stream, flags))

    def fused_noalloc_ptr(self, params, bgs, targets, B, T, H, W, sigma, losses, grads, images=None,
                          stream=None, flags=0):
        """drh_fused_loss_backward_noalloc: device pointers, no device allocation."""
        check(lib().drh_fused_loss_backward_noalloc(self.handle, params, bgs, targets, B, T, H, W, sigma,
                                                    losses, grads, images, stream, flags))

    def from_grad_ptr(self, params, bgs, grad_images, B, T, H, W, sigma, grads, stream=None, flags=0):
        check(lib().drh_backward_from_grad(self.handle, params, bgs, grad_images, B, T, H, W, sigma,
                                           grads, stream, flags))

    def render_record_ptr(self, params, bgs, B, T, H, W, sigma, out, record, record_bytes, stream=None,
                          flags=0):
        """drh_render that also fills `record` (record_bytes(B, T, H, W) bytes of device memory)."""
        check(lib().drh_render_record(self.handle, params, bgs, B, T, H, W, sigma, out, record, record_bytes,
                                      stream, flags))

    def backward_recorded_ptr(self, record, record_bytes, grad_images, B, T, H, W, sigma, grads, stream=None,
                              flags=0):
        """Gradients for the scenes of a render_record_ptr call, from its record."""
        check(lib().drh_backward_recorded(self.handle, record, record_bytes, grad_images, B, T, H, W, sigma,
                                          grads, stream, flags))

    def encode_srgb_ptr(self, values, n, out, stream=None, flags=0):
        check(lib().drh_encode_srgb(self.handle, values, n, out, stream, flags))

    def decode_srgb_ptr(self, data, n, out, stream=None, flags=0):
        check(lib().drh_decode_srgb(self.handle, data, n, out, stream, flags))

    def resize_lanczos3_ptr(self, src, H, W, C, dst, new_H, new_W, stream=None, flags=0):
        check(lib().drh_resize_lanczos3(self.handle, src, H, W, C, dst, new_H, new_W, stream, flags))

    # -- host (numpy) forms, synchronous --------------------------------------
    def resize_lanczos3(self, image, width: int, height: int) -> np.ndarray:
        """Canvas::load_image's resize_exact(width, height, Lanczos3) (canvas.rs:71-79) of an
        (H, W, C) uint8 image."""
        a = np.ascontiguousarray(image, dtype=np.uint8)
        if a.ndim != 3:
            raise ValueError(f"expected an (H, W, C) image, got shape {a.shape}")
        H, W, C = a.shape
        out = np.empty((height, width, C), np.uint8)
        self.resize_lanczos3_ptr(a.ctypes.data_as(ctypes.c_void_p), H, W, C, out.ctypes.data_as(ctypes.c_void_p),
                                 height, width, flags=HOST_PTRS)
        return out

    def encode_srgb(self, values) -> np.ndarray:
        """canvas.rs:100-105 per value: linear float32 to sRGB bytes, same shape."""
        v = _f32(values)
        out = np.empty(v.shape, np.uint8)
        self.encode_srgb_ptr(_ptr(v), v.size, out.ctypes.data_as(ctypes.c_void_p), flags=HOST_PTRS)
        return out

    def decode_srgb(self, data) -> np.ndarray:
        """canvas.rs:108-115 per byte: sRGB bytes to linear float32, same shape."""
        b = np.ascontiguousarray(data, dtype=np.uint8)
        out = np.empty(b.shape, np.float32)
        self.decode_srgb_ptr(b.ctypes.data_as(ctypes.c_void_p), b.size, _ptr(out), flags=HOST_PTRS)
        return out

    def render(self, params, height: int, width: int, sigma: float, background=(0, 0, 0),
               exact: bool = False) -> np.ndarray:
        p = _f32(params)
        B, T = p.shape[0], p.shape[1]
        bgs = _bgs(background, B)
        out = np.empty((B, height, width, 3), np.float32)
        self.render_ptr(_ptr(p), _ptr(bgs), B, T, height, width, sigma, _ptr(out),
                        flags=HOST_PTRS | (EXACT_MATH if exact else 0))
        return out

    def fused_loss_backward(self, params, targets, sigma: float, background=(0, 0, 0),
                            exact: bool = False, want_images: bool = False, deterministic: bool = False):
        p, t = _f32(params), _f32(targets)
        B, T = p.shape[0], p.shape[1]
        H, W = t.shape[1], t.shape[2]
        bgs = _bgs(background, B)
        losses = np.empty(B, np.float32)
        grads = np.empty((B, T, 10), np.float32)
        imgs = np.empty((B, H, W, 3), np.float32) if want_images else None
        self.fused_ptr(_ptr(p), _ptr(bgs), _ptr(t), B, T, H, W, sigma, _ptr(losses), _ptr(grads),
                       _ptr(imgs), flags=HOST_PTRS | (EXACT_MATH if exact else 0) |
                       (DETERMINISTIC if deterministic else 0))
        return (losses, grads, imgs) if want_images else (losses, grads)

    def backward_many_timed(self, params, targets, sigma: float, background=(0, 0, 0)):
        """fused_loss_backward with its host phases (GpuRasterizer::backward_many_timed,
        crates/diffrast-gpu/src/lib.rs:649-664): (losses, grads, phases). The stream is
        drained between phases, so the total bounds the untimed call from above."""
        p, t = _f32(params), _f32(targets)
        B, T = p.shape[0], p.shape[1]
        H, W = t.shape[1], t.shape[2]
        bgs = _bgs(background, B)
        losses = np.empty(B, np.float32)
        grads = np.empty((B, T, 10), np.float32)
        self.fused_ptr(_ptr(p), _ptr(bgs), _ptr(t), B, T, H, W, sigma, _ptr(losses), _ptr(grads),
                       None, flags=HOST_PTRS | PHASES)
        return losses, grads, self.read_phases()

    def backward_from_grad(self, params, grad_images, sigma: float, background=(0, 0, 0),
                           exact: bool = False, deterministic: bool = False) -> np.ndarray:
        p, g = _f32(params), _f32(grad_images)
        B, T = p.shape[0], p.shape[1]
        H, W = g.shape[1], g.shape[2]
        bgs = _bgs(background, B)
        grads = np.zeros((B, T, 10), np.float32)
        self.from_grad_ptr(_ptr(p), _ptr(bgs), _ptr(g), B, T, H, W, sigma, _ptr(grads),
                           flags=HOST_PTRS | (EXACT_MATH if exact else 0) |
                           (DETERMINISTIC if deterministic else 0))
        return grads

    def adam_project_step(self, params: np.ndarray, grads, m: np.ndarray, v: np.ndarray, lr,
                          step: int, beta1=0.9, beta2=0.999, eps=1e-8, project=True) -> None:
        """In place on params, m, v (float32 contiguous numpy arrays)."""
        g, l = _f32(grads), _f32(lr)
        for a in (params, m, v):
            assert a.dtype == np.float32 and a.flags.c_contiguous
        check(lib().drh_adam_project_step(self.handle, _ptr(params), _ptr(g), _ptr(m), _ptr(v), _ptr(l),
                                          params.size, step, beta1, beta2, eps, int(project), None,
                                          HOST_PTRS))

    def fit(self, target, init_params, background, iters=1500, sigma_start=0.02, sigma_end=0.0015,
            lr_pos=0.004, lr_color=0.02, lr_alpha=0.01, patience=250, min_delta=1e-7):
        """fit.rs:166-288 on the device from a given initial scene."""
        t = _f32(target)
        H, W = t.shape[0], t.shape[1]
        p = _f32(init_params).reshape(-1, 10)
        T = p.shape[0]
        bg = _f32(background).reshape(3)
        cfg = FitConfig(iters, sigma_start, sigma_end, lr_pos, lr_color, lr_alpha,
                        -1 if patience is None else int(patience), min_delta)
        losses = np.empty(max(iters, 1), np.float32)
        best = np.empty_like(p)
        last = np.empty_like(p)
        rep = FitReport()
        check(lib().drh_fit(self.handle, _ptr(t), H, W, _ptr(bg), _ptr(p), T, ctypes.byref(cfg),
                            _ptr(losses), _ptr(best), _ptr(last), ctypes.byref(rep), None, HOST_PTRS))
        return dict(losses=losses[: rep.n_losses].copy(), best_params=best, params=last,
                    best_iter=int(rep.best_iter), best_loss=float(rep.best_loss),
                    stop_reason=STOP_REASONS[rep.stop_reason])


FIT_DEFAULTS = dict(iters=1500, sigma_start=0.02, sigma_end=0.0015, lr_pos=0.004, lr_color=0.02,
                    lr_alpha=0.01, patience=250, min_delta=1e-7)  # FitConfig::default (fit.rs:67-89)


def _fit_config(**cfg) -> FitConfig:
    c = dict(FIT_DEFAULTS)
    c.update(cfg)
    return FitConfig(c["iters"], c["sigma_start"], c["sigma_end"], c["lr_pos"], c["lr_color"], c["lr_alpha"],
                     -1 if c["patience"] is None else int(c["patience"]), c["min_delta"])


class Fitter:
    """Fitter (fit.rs:191-335) on the device, from a given initial scene.

    `step()` runs one iteration and returns its StepInfo as a dict (None once
    the fit has stopped, for any reason); `run(n)` runs up to n iterations
    without waiting between them. The state lives on the device."""

    def __init__(self, ctx: Context, target, init_params, background, exact: bool = False, **cfg):
        t = _f32(target)
        self.H, self.W = t.shape[0], t.shape[1]
        p = _f32(init_params).reshape(-1, 10)
        self.T = p.shape[0]
        bg = _f32(background).reshape(3)
        self.cfg = _fit_config(**cfg)
        self._ctx = ctx  # the context must outlive the fitter
        h = ctypes.c_void_p()
        check(lib().drh_fitter_create(ctx.handle, _ptr(t), self.H, self.W, _ptr(bg), _ptr(p), self.T,
                                      ctypes.byref(self.cfg), None, HOST_PTRS | (EXACT_MATH if exact else 0),
                                      ctypes.byref(h)))
        self.handle = h

    def close(self) -> None:
        if self.handle:
            lib().drh_fitter_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def step(self):
        stepped = ctypes.c_int()
        info = StepInfo()
        check(lib().drh_fitter_step(self.handle, ctypes.byref(stepped), ctypes.byref(info)))
        if not stepped.value:
            return None
        return dict(iter=int(info.iter), loss=float(info.loss), sigma=float(info.sigma))

    def run(self, max_steps: int) -> int:
        ran = ctypes.c_int64()
        check(lib().drh_fitter_run(self.handle, max_steps, ctypes.byref(ran)))
        return int(ran.value)

    def status(self) -> dict:
        s = FitStatus()
        check(lib().drh_fitter_status(self.handle, ctypes.byref(s)))
        return dict(iter=int(s.iter), best_iter=int(s.best_iter), best_loss=float(s.best_loss),
                    sigma=float(s.sigma), done=bool(s.done),
                    stop_reason=None if s.stop_reason < 0 else STOP_REASONS[s.stop_reason])

    def scene(self) -> np.ndarray:
        out = np.empty((self.T, 10), np.float32)
        check(lib().drh_fitter_scene(self.handle, _ptr(out), HOST_PTRS))
        return out

    def losses(self) -> np.ndarray:
        n = ctypes.c_int64()
        out = np.empty(max(int(self.cfg.iters), 1), np.float32)
        check(lib().drh_fitter_losses(self.handle, _ptr(out), out.size, ctypes.byref(n), HOST_PTRS))
        return out[: n.value].copy()

    def render_current(self) -> np.ndarray:
        out = np.empty((self.H, self.W, 3), np.float32)
        check(lib().drh_fitter_render_current(self.handle, _ptr(out), HOST_PTRS))
        return out

    def into_report(self) -> dict:
        best = np.empty((self.T, 10), np.float32)
        rep = FitReport()
        check(lib().drh_fitter_report(self.handle, _ptr(best), ctypes.byref(rep), HOST_PTRS))
        return dict(best_params=best, losses=self.losses(), best_iter=int(rep.best_iter),
                    best_loss=float(rep.best_loss), stop_reason=STOP_REASONS[rep.stop_reason])


def validate_fit_config(T: int, **cfg) -> str | None:
    """FitConfig::validate (fit.rs:98-117): None when valid, else the error name."""
    conf = _fit_config(**cfg)
    rc = lib().drh_fit_validate(ctypes.byref(conf), T)
    return CONFIG_ERRORS.get(rc)


def record_bytes(B: int, T: int, H: int, W: int) -> int:
    """Device bytes drh_render_record keeps for B scenes of T triangles at H x W."""
    n = ctypes.c_uint64()
    check(lib().drh_record_bytes(B, T, H, W, ctypes.byref(n)))
    return int(n.value)


def params_per_triangle() -> int:
    return int(lib().drh_params_per_triangle())
