"""The rasterizer as a PyTorch operation — drop-in for the reference's
python/diffrast/torch_layer.py, running on MI355X through libdiffrast_hip.so.

    params = model(image)                    # (B, T, 10)
    render = rasterize(params, 128, 128)     # (B, 3, H, W)
    loss = F.mse_loss(render, image)
    loss.backward()                          # gradients reach `model`

Same functions, argument meanings and ValueError cases as the reference
(torch_layer.py:37-303, crates/diffrast-py/src/lib.rs:85-195). What differs:

* Tensors already on the GPU stay there: the op hands device pointers and
  torch's current stream to the C ABI, with no host copy (the reference
  copies every call to CPU numpy, torch_layer.py:46, 58-59, 123-124).
  CPU tensors are moved to the current GPU and results are returned on the
  caller's device, as the reference returns them.
* When autograd will need it, `rasterize` keeps its forward pass's record
  (a device tensor of `_lib.record_bytes(B, T, H, W)` bytes, held until the
  graph is freed) and its backward runs only the backward kernel; the
  reference's backward renders the batch again (torch_layer.py:55-66).
* There is no CPU backend. `device="gpu"`, `"cuda"` and `"auto"` run the HIP
  kernels; `device="cpu"` raises ValueError instead of silently running
  something else, and a missing library or GPU raises rather than falling
  back. `last_device()` therefore reports "gpu" after every call.
"""

from __future__ import annotations

import atexit
import math
import threading

import torch
from torch import Tensor

from . import _lib

#: Parameters per triangle: 6 position + 3 color + 1 alpha.
N_PARAMS: int = _lib.params_per_triangle()

_contexts: dict[int, _lib.Context] = {}
_ctx_lock = threading.Lock()
_last_device = "cpu"


def _parse_device(name: str) -> None:
    """crates/diffrast-py/src/lib.rs:85-94, minus the CPU backend."""
    if name in ("gpu", "cuda", "auto"):
        return
    if name == "cpu":
        raise ValueError(
            'device="cpu" is not available: the rasterizer runs only on the GPU '
            '(use "gpu" or "auto")')
    raise ValueError(f'unknown device {name!r} — expected "cpu", "gpu" or "auto"')


def _check_sigma(sigma: float) -> None:
    if not (isinstance(sigma, (int, float)) and math.isfinite(sigma) and sigma > 0):
        raise ValueError("sigma must be positive and finite")


def _gpu() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("no HIP device is visible; there is no CPU path")
    return torch.device("cuda", torch.cuda.current_device())


def _context(dev: torch.device) -> _lib.Context:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    with _ctx_lock:
        ctx = _contexts.get(idx)
        if ctx is None:
            with torch.cuda.device(idx):
                ctx = _lib.Context()
            _contexts[idx] = ctx
    return ctx


def _stream(dev: torch.device):
    return torch.cuda.current_stream(dev).cuda_stream


def _on_gpu(t: Tensor, dev: torch.device) -> Tensor:
    return t.detach().to(device=dev, dtype=torch.float32).contiguous()


_bg_cache: dict = {}


def _backgrounds(background, B: int, dev: torch.device) -> Tensor:
    """The (B, 3) device array of one background colour, cached: a host-to-device
    copy of pageable memory per call would wait for the stream's queued work."""
    if isinstance(background, Tensor):
        bg = background.detach().to(dtype=torch.float32)
        if bg.numel() != 3:
            raise ValueError("background must have 3 components")
        return bg.reshape(1, 3).expand(B, 3).to(dev).contiguous()
    vals = tuple(float(v) for v in background)
    if len(vals) != 3:
        raise ValueError("background must have 3 components")
    key = (dev.index, B, vals)
    with _ctx_lock:
        bg = _bg_cache.get(key)
    if bg is None:
        bg = torch.tensor(vals, dtype=torch.float32).reshape(1, 3).expand(B, 3).contiguous().to(dev)
        torch.cuda.current_stream(dev).synchronize()  # usable from any stream from now on
        with _ctx_lock:
            if len(_bg_cache) >= 64:
                _bg_cache.clear()
            _bg_cache[key] = bg
    return bg


def _note_gpu() -> None:
    global _last_device
    _last_device = "gpu"


def _render(params: Tensor, height: int, width: int, sigma: float, background, channels_first: bool) -> Tensor:
    """(B, 3, H, W) or (B, H, W, 3), written in that layout by the kernel."""
    dev = _gpu()
    p = _on_gpu(params, dev)
    B, T = p.shape[0], p.shape[1]
    bg = _backgrounds(background, B, dev)
    shape = (B, 3, height, width) if channels_first else (B, height, width, 3)
    out = torch.empty(shape, device=dev, dtype=torch.float32)
    _context(dev).render_ptr(p.data_ptr(), bg.data_ptr(), B, T, height, width, float(sigma),
                             out.data_ptr(), _stream(dev), _lib.CHANNELS_FIRST if channels_first else 0)
    _note_gpu()
    return out


def _render_record(params: Tensor, height: int, width: int, sigma: float, background,
                   channels_first: bool) -> tuple[Tensor, Tensor]:
    """_render that also returns the forward record the backward pass reads."""
    dev = _gpu()
    p = _on_gpu(params, dev)
    B, T = p.shape[0], p.shape[1]
    bg = _backgrounds(background, B, dev)
    shape = (B, 3, height, width) if channels_first else (B, height, width, 3)
    out = torch.empty(shape, device=dev, dtype=torch.float32)
    nbytes = _lib.record_bytes(B, T, height, width)
    record = torch.empty((nbytes,), device=dev, dtype=torch.uint8)
    _context(dev).render_record_ptr(p.data_ptr(), bg.data_ptr(), B, T, height, width, float(sigma),
                                    out.data_ptr(), record.data_ptr(), nbytes, _stream(dev),
                                    _lib.CHANNELS_FIRST if channels_first else 0)
    _note_gpu()
    return out, record


class _Rasterize(torch.autograd.Function):
    """Forward renders, backward maps dL/dimage to dL/dparams (torch_layer.py:36-66)."""

    @staticmethod
    def forward(ctx, params: Tensor, height: int, width: int, sigma: float, background, device,
                channels_first: bool, keep_record: bool):
        if keep_record:
            images, record = _render_record(params, height, width, sigma, background, channels_first)
            ctx.save_for_backward(params, record)
        else:
            images = _render(params, height, width, sigma, background, channels_first)
            ctx.save_for_backward(params)
        ctx.sigma = sigma
        ctx.background = background
        ctx.device = device
        ctx.channels_first = channels_first
        ctx.size = (height, width)
        return images

    @staticmethod
    def backward(ctx, grad_images: Tensor):
        params, *kept = ctx.saved_tensors
        dev = _gpu()
        g = _on_gpu(grad_images, dev)
        B, T = params.shape[0], params.shape[1]
        H, W = ctx.size
        flags = _lib.CHANNELS_FIRST if ctx.channels_first else 0
        grads = torch.empty((B, T, N_PARAMS), device=dev, dtype=torch.float32)
        if kept:
            (record,) = kept
            _context(dev).backward_recorded_ptr(record.data_ptr(), record.numel(), g.data_ptr(), B, T, H, W,
                                                float(ctx.sigma), grads.data_ptr(), _stream(dev), flags)
        else:
            p = _on_gpu(params, dev)
            bg = _backgrounds(ctx.background, B, dev)
            _context(dev).from_grad_ptr(p.data_ptr(), bg.data_ptr(), g.data_ptr(), B, T, H, W,
                                        float(ctx.sigma), grads.data_ptr(), _stream(dev), flags)
        _note_gpu()
        return grads.to(params.device, params.dtype), None, None, None, None, None, None, None


def rasterize(
    params: Tensor,
    height: int,
    width: int,
    sigma: float = 0.0015,
    background: tuple[float, float, float] = (0.0, 0.0, 0.0),
    channels_first: bool = True,
    device: str = "auto",
) -> Tensor:
    """Render a batch of triangle scenes, differentiably (torch_layer.py:69-108).

    Args:
        params: `(B, T, 10)` — `[x0, y0, x1, y1, x2, y2, r, g, b, a]` per
            triangle, in normalized image coordinates.
        height, width: output resolution.
        sigma: edge softness in normalized units.
        background: color the canvas is cleared to.
        channels_first: return `(B, 3, H, W)` rather than `(B, H, W, 3)`.
        device: `"gpu"`, `"cuda"` or `"auto"` (all run the HIP kernels).

    Returns:
        The rendered batch, in linear light, on `params.device`.
    """
    if params.dim() != 3 or params.shape[-1] != N_PARAMS:
        raise ValueError(f"expected params of shape (B, T, {N_PARAMS}), got {tuple(params.shape)}")
    if height <= 0 or width <= 0:
        raise ValueError("height and width must be positive")
    if not (sigma > 0):
        raise ValueError("sigma must be positive")
    _check_sigma(sigma)
    _parse_device(device)

    keep_record = torch.is_grad_enabled() and params.requires_grad
    images = _Rasterize.apply(params, height, width, sigma, background, device, bool(channels_first),
                              keep_record)
    return images.to(params.device, params.dtype)


def _fused(params: Tensor, targets: Tensor, sigma: float, background, channels_first: bool = False):
    """(losses (B,), grads (B, T, 10)) on the GPU, float32; targets (B, H, W, 3), or
    (B, 3, H, W) when channels_first (read in place, no transposing copy)."""
    dev = _gpu()
    p = _on_gpu(params, dev)
    t = _on_gpu(targets, dev)
    B, T = p.shape[0], p.shape[1]
    if t.shape[0] != B:
        raise ValueError(f"batch mismatch: {B} parameter rows but {t.shape[0]} targets")
    if t.shape[1 if channels_first else 3] != 3:
        raise ValueError("targets must have 3 channels")
    H, W = (t.shape[2], t.shape[3]) if channels_first else (t.shape[1], t.shape[2])
    if H == 0 or W == 0:
        raise ValueError("height and width must be non-zero")
    bg = _backgrounds(background, B, dev)
    losses = torch.empty((B,), device=dev, dtype=torch.float32)
    grads = torch.empty((B, T, N_PARAMS), device=dev, dtype=torch.float32)
    _context(dev).fused_ptr(p.data_ptr(), bg.data_ptr(), t.data_ptr(), B, T, H, W, float(sigma),
                            losses.data_ptr(), grads.data_ptr(), None, _stream(dev),
                            _lib.CHANNELS_FIRST if channels_first else 0)
    _note_gpu()
    return losses, grads


class _FusedMSE(torch.autograd.Function):
    """Photometric MSE against a target in one render (torch_layer.py:111-138)."""

    @staticmethod
    def forward(ctx, params: Tensor, targets: Tensor, sigma: float, background, device):
        losses, grads = _fused(params, targets, sigma, background, channels_first=True)
        ctx.save_for_backward(grads.to(params.device, params.dtype))
        ctx.batch = len(params)
        return losses.mean().to(params.device, params.dtype)

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        (grads,) = ctx.saved_tensors
        # the kernel differentiates the sum of per-item MSE; the forward
        # returns their mean, hence the 1/B.
        return grad_out * grads / ctx.batch, None, None, None, None


def fused_mse(
    params: Tensor,
    targets: Tensor,
    sigma: float = 0.0015,
    background: tuple[float, float, float] = (0.0, 0.0, 0.0),
    device: str = "auto",
) -> Tensor:
    """Mean squared error between the rendered scenes and `targets`
    (torch_layer.py:141-168); one render per step instead of two.

    Args:
        params: `(B, T, 10)` scene parameters.
        targets: `(B, 3, H, W)`, matching what `rasterize` returns.
    """
    if params.dim() != 3 or params.shape[-1] != N_PARAMS:
        raise ValueError(f"expected params of shape (B, T, {N_PARAMS}), got {tuple(params.shape)}")
    if targets.dim() != 4 or targets.shape[1] != 3:
        raise ValueError(f"expected targets of shape (B, 3, H, W), got {tuple(targets.shape)}")
    if not (sigma > 0):
        raise ValueError("sigma must be positive")
    _check_sigma(sigma)
    _parse_device(device)

    return _FusedMSE.apply(params, targets, sigma, background, device)


def gpu_adapter() -> str | None:
    """Name of the GPU the extension uses, or `None` if there is none."""
    if not torch.cuda.is_available():
        return None
    return _context(_gpu()).device_info()


def last_device() -> str:
    """Device the most recent call ran on (torch_layer.py:176-184)."""
    return _last_device


def shutdown_gpu() -> bool:
    """Release the rasterizer's device state now (torch_layer.py:187-193).

    Returns True if a context was released. A later call creates a new one.
    """
    with _ctx_lock:
        released = bool(_contexts)
        for ctx in _contexts.values():
            ctx.close()
        _contexts.clear()
        _bg_cache.clear()
    return released


atexit.register(shutdown_gpu)


# Pixel x triangle evaluations per call from which a discrete MI355X beats
# this host's CPU on the fused loss + backward with host arrays in and out.
# Measured on MI355X against 16 EPYC cores (batch 1-16, 16-256 pixels square,
# 2-512 triangles): the CPU wins up to 32,768 evaluations (0.07x-0.88x), the
# GPU from 131,072 on (2.5x-113x), single scenes included (1 x 64x64 x 32:
# 2.5x; 1 x 128x128 x 64: 16.9x). Its fixed cost is ~0.17-0.2 ms per call
# (copies, launch, wait) whatever the batch, so the rule has no batch term;
# the floor sits at the log-midpoint of the crossover interval.
MI355X_WORK_FLOOR = 65_536


def policy_prefers_gpu(batch: int, triangles: int, pixels: int, discrete: bool | None = None) -> bool:
    """`device="auto"`'s size rule (crates/diffrast-py/src/lib.rs:113-147), re-derived for MI355X.

    Discrete GPUs (the default): the GPU is worth it from `MI355X_WORK_FLOOR`
    pixel x triangle evaluations per call, with no batch condition; the
    reference's rule (batch >= 2 and >= 250,000, measured on an RTX 4090)
    would send single scenes to the CPU that this GPU runs 2.5-17x faster.
    Integrated GPUs keep the reference's rule (no integrated part was
    measured here). The rule is advisory in this build: it has no CPU backend,
    so `auto` runs on the GPU whatever the rule says.
    """
    if discrete is None:
        discrete = True
    if not discrete:
        return batch >= 4 and batch * triangles * pixels >= 1_000_000_000
    return batch >= 1 and batch * triangles * pixels >= MI355X_WORK_FLOOR


def _rtx4090_rule(batch: int, triangles: int, pixels: int) -> bool:
    """The reference's discrete-GPU rule (crates/diffrast-py/src/lib.rs:138-147), for comparison."""
    return batch >= 2 and batch * triangles * pixels >= 250_000


def fused_loss(
    params: Tensor,
    targets: Tensor,
    sigma: float = 0.0015,
    background: tuple[float, float, float] = (0.0, 0.0, 0.0),
    device: str = "auto",
) -> tuple[Tensor, Tensor]:
    """Per-item MSE and parameter gradients in one call, without autograd
    (torch_layer.py:218-253).

    Returns:
        `(losses, grads)` — `(B,)` and `(B, T, 10)`, on `params.device`.
    """
    if targets.dim() != 4:
        raise ValueError(f"expected targets of shape (B, H, W, 3), got {tuple(targets.shape)}")
    if params.dim() != 3 or params.shape[-1] != N_PARAMS:
        raise ValueError(f"expected last parameter dimension {N_PARAMS}, got {tuple(params.shape)}")
    _check_sigma(sigma)
    _parse_device(device)
    losses, grads = _fused(params, targets, sigma, background)
    return losses.to(params.device), grads.to(params.device, params.dtype)


def random_params(
    batch: int,
    triangles: int,
    *,
    device: torch.device | str = "cpu",
    generator: torch.Generator | None = None,
) -> Tensor:
    """Small triangles scattered over the canvas (torch_layer.py:256-279)."""
    centers = torch.rand(batch, triangles, 1, 2, device=device, generator=generator)
    offsets = (torch.rand(batch, triangles, 3, 2, device=device, generator=generator) - 0.5) * 0.3
    verts = (centers + offsets).reshape(batch, triangles, 6)
    colors = torch.rand(batch, triangles, 3, device=device, generator=generator)
    alphas = torch.rand(batch, triangles, 1, device=device, generator=generator) * 0.4 + 0.3
    return torch.cat([verts, colors, alphas], dim=-1)


def clamp_params(params: Tensor) -> Tensor:
    """Project parameters back into their valid ranges (torch_layer.py:282-291)."""
    verts = params[..., :6].clamp(-0.25, 1.25)
    colors = params[..., 6:9].clamp(0.0, 1.0)
    alpha = params[..., 9:10].clamp(1e-3, 0.999)
    return torch.cat([verts, colors, alpha], dim=-1)


def psnr(a: Tensor, b: Tensor, max_value: float = 1.0) -> Tensor:
    """Peak signal-to-noise ratio in dB (torch_layer.py:294-303)."""
    mse = torch.mean((a - b) ** 2)
    if mse == 0:
        return torch.tensor(float("inf"), device=a.device)
    return 10.0 * torch.log10(max_value**2 / mse)
