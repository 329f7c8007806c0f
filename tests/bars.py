"""Parity bars of the HIP path against the CPU oracle, shared by the GPU tests.

  images     max |gpu - cpu| <= 1e-5
  losses     |gpu - cpu| <= 1e-4 |cpu| (+ 1e-7 absolute, for losses near zero)
  gradients  per scene, max |gpu - cpu| / ||cpu||_2 <= 1e-4, over the whole scene
             (the reference's own normalisation, crates/diffrast-gpu/src/lib.rs:1249-1254)
             AND separately over each parameter group: vertices (params 0-5), colours
             (6-8) and alpha (9), so that a group whose gradients are small against the
             scene's norm cannot hide an error under it
The GPU sums per-pixel contributions in another order than the CPU's serial f32
loops, so gradients are compared to a tolerance, not bitwise.
"""

from __future__ import annotations

import numpy as np

IMG_TOL = 1e-5
LOSS_RTOL = 1e-4
GRAD_RTOL = 1e-4
GROUPS = {"vertices": slice(0, 6), "colours": slice(6, 9), "alpha": slice(9, 10)}


def _per_scene(a) -> np.ndarray:
    a = np.asarray(a, np.float64)
    return a.reshape(a.shape[0], -1, 10) if a.size else a.reshape(a.shape[0] if a.ndim else 0, 0, 10)


def grad_err(gpu, cpu) -> float:
    """Per-scene max |d| / ||g_cpu||_2, worst over the batch."""
    worst = 0.0
    for a, b in zip(_per_scene(gpu), _per_scene(cpu)):
        if a.size == 0:
            continue
        n = max(np.linalg.norm(b), 1e-30)
        worst = max(worst, float(np.abs(a - b).max()) / n)
    return worst


def grad_err_groups(gpu, cpu) -> dict:
    """Per-scene, per-group max |d| / ||g_cpu group||_2, worst over the batch.

    A group whose oracle gradients are all exactly zero (every alpha clamped, say)
    is measured against the scene's norm instead, so it must then be zero on the
    GPU too up to the whole-scene bar."""
    out = {name: 0.0 for name in GROUPS}
    for a, b in zip(_per_scene(gpu), _per_scene(cpu)):
        if a.size == 0:
            continue
        scene = max(np.linalg.norm(b), 1e-30)
        for name, sl in GROUPS.items():
            n = np.linalg.norm(b[:, sl])
            d = float(np.abs(a[:, sl] - b[:, sl]).max())
            out[name] = max(out[name], d / (n if n > 0 else scene))
    return out


def assert_grads(gpu, cpu, tol: float = GRAD_RTOL, label: str = "") -> dict:
    """The whole-scene and per-group gradient bars; prints the measured errors."""
    whole = grad_err(gpu, cpu)
    groups = grad_err_groups(gpu, cpu)
    print(f"{label} grad err: scene {whole:.2e}  " +
          "  ".join(f"{k} {v:.2e}" for k, v in groups.items()), flush=True)
    assert whole <= tol, f"{label}: gradient error {whole:.3e} over the scene norm > {tol}"
    for k, v in groups.items():
        assert v <= tol, f"{label}: {k} gradient error {v:.3e} over the group norm > {tol}"
    return dict(scene=whole, **groups)


def check_losses(gpu, cpu, label: str = "") -> float:
    gpu, cpu = np.asarray(gpu, np.float64), np.asarray(cpu, np.float64)
    err = float(np.max(np.abs(gpu - cpu) / np.maximum(np.abs(cpu), 1e-30))) if cpu.size else 0.0
    if label:
        print(f"{label} loss rel err {err:.2e}", flush=True)
    assert np.all(np.abs(gpu - cpu) <= LOSS_RTOL * np.abs(cpu) + 1e-7), (gpu, cpu)
    return err


def check_image(gpu, cpu, label: str = "") -> float:
    err = float(np.abs(np.asarray(gpu) - np.asarray(cpu)).max()) if np.size(cpu) else 0.0
    if label:
        print(f"{label} image max abs err {err:.2e}", flush=True)
    assert err <= IMG_TOL, f"{label}: image error {err:.3e} > {IMG_TOL}"
    return err
