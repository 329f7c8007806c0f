"""Seeded synthetic inputs for the benchmark workloads.

One documented generator feeds the HIP path, the tests and the CPU baseline,
so every consumer sees the same bytes for the same seed.

Generator: SplitMix64 (Steele, Lea & Flood, "Fast splittable pseudorandom
number generators", OOPSLA 2014). Each 64-bit output `z` gives one uniform
float `u = (z >> 40) * 2**-24` in [0, 1), exact in float32. `uniform(a, b)` is
`a + (b - a) * u` evaluated in float64 and rounded once to float32.

Workloads (all float32; background (0, 0, 0) unless stated):
  uniform scenes : per triangle, in draw order, x0 y0 x1 y1 x2 y2 ~ U[0,1),
                   r g b ~ U[0,1), alpha ~ U[0.3, 0.9)
  small scenes   : per triangle cx cy ~ U[0,1), then per vertex
                   (cx + U[-0.05,0.05), cy + U[-0.05,0.05)), then rgb, alpha
  blob target    : background rgb ~ U[0,1); then 8 blobs, each centre ~ U[0,1)^2,
                   radius ~ U[0.05, 0.2), colour ~ U[0,1)^3, painted in order
                   as img += (colour - img) * 0.9 * exp(-|p - centre|^2 / (2 r^2))
                   at pixel centres ((x + .5)/W, (y + .5)/H)
  fit init       : the reference's seed_scene (fit.rs:356-367) driven by this
                   generator instead of rand::StdRng: Scene::random(T, bg, 0.18)
                   (scene.rs:58-78: cx cy, 3 x (dx dy) ~ U[-0.18,0.18), rgb,
                   alpha ~ U[0.3,0.8)) for every triangle, then per triangle the
                   colour sampled at the centroid and alpha ~ U[0.3,0.7)
Seeds: item b of a batch uses scene seed `seed + b` and target seed
`seed + 1000 + b`.
"""

from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """The first n outputs of SplitMix64 seeded with `seed` (uint64)."""
    with np.errstate(over="ignore"):
        s = np.uint64(seed & 0xFFFFFFFFFFFFFFFF)
        k = np.arange(1, n + 1, dtype=np.uint64)
        z = s + k * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        z = z ^ (z >> np.uint64(31))
    return z


def uniforms(seed: int, n: int) -> np.ndarray:
    """n floats in [0, 1) with 24-bit resolution (float64 holding exact values)."""
    return (splitmix64(seed, n) >> np.uint64(40)).astype(np.float64) * (2.0 ** -24)


def _rng_range(u: np.ndarray, a: float, b: float) -> np.ndarray:
    return (a + (b - a) * u).astype(np.float32)


def uniform_scene(seed: int, T: int) -> np.ndarray:
    """(T, 10) scene: vertices U[0,1)^2, rgb U[0,1), alpha U[0.3,0.9)."""
    u = uniforms(seed, T * 10).reshape(T, 10)
    out = np.empty((T, 10), np.float32)
    out[:, :9] = u[:, :9].astype(np.float32)
    out[:, 9] = _rng_range(u[:, 9], 0.3, 0.9)
    return out


def small_scene(seed: int, T: int, spread: float = 0.05) -> np.ndarray:
    """(T, 10) scene of small triangles: centre U[0,1)^2 plus offsets U[-s, s)."""
    u = uniforms(seed, T * 12).reshape(T, 12)
    out = np.empty((T, 10), np.float32)
    cx, cy = u[:, 0], u[:, 1]
    for v in range(3):
        out[:, 2 * v] = (cx + (-spread + 2 * spread * u[:, 2 + 2 * v])).astype(np.float32)
        out[:, 2 * v + 1] = (cy + (-spread + 2 * spread * u[:, 3 + 2 * v])).astype(np.float32)
    out[:, 6:9] = u[:, 8:11].astype(np.float32)
    out[:, 9] = _rng_range(u[:, 11], 0.3, 0.9)
    return out


def random_scene(seed: int, T: int, seed_scale: float = 0.15) -> np.ndarray:
    """(T, 10) scene shaped like the reference's `Scene::random` (scene.rs:58-76): per
    triangle a centre U[0,1)^2, three vertices centre + U[-s, s)^2, rgb U[0,1), alpha
    U[0.3,0.8). Same distributions, our own generator (the reference draws from StdRng)."""
    u = uniforms(seed, T * 12).reshape(T, 12)
    out = np.empty((T, 10), np.float32)
    cx, cy = u[:, 0].astype(np.float32), u[:, 1].astype(np.float32)
    s = np.float32(seed_scale)
    for v in range(3):
        out[:, 2 * v] = cx + _rng_range(u[:, 2 + 2 * v], -s, s)
        out[:, 2 * v + 1] = cy + _rng_range(u[:, 3 + 2 * v], -s, s)
    out[:, 6:9] = u[:, 8:11].astype(np.float32)
    out[:, 9] = _rng_range(u[:, 11], 0.3, 0.8)
    return out


def batch(kind: str, B: int, T: int, seed: int, target_offset: int = 0) -> np.ndarray:
    """(B, T, 10) with item b drawn from seed + target_offset + b."""
    fn = {"uniform": uniform_scene, "small": small_scene, "random": random_scene}[kind]
    return np.stack([fn(seed + target_offset + b, T) for b in range(B)])


def blob_target(seed: int, H: int, W: int, blobs: int = 8) -> np.ndarray:
    """(H, W, 3) smooth target: a flat background with painted Gaussian blobs."""
    u = uniforms(seed, 3 + blobs * 6)
    img = np.empty((H, W, 3), np.float64)
    img[:] = u[:3]
    ys = (np.arange(H) + 0.5) / H
    xs = (np.arange(W) + 0.5) / W
    px, py = np.meshgrid(xs, ys)
    for j in range(blobs):
        cx, cy, r = u[3 + 6 * j], u[4 + 6 * j], 0.05 + 0.15 * u[5 + 6 * j]
        col = u[6 + 6 * j: 9 + 6 * j]
        g = 0.9 * np.exp(-((px - cx) ** 2 + (py - cy) ** 2) / (2 * r * r))
        img += (col[None, None, :] - img) * g[..., None]
    return img.astype(np.float32)


def mean_color(image: np.ndarray) -> np.ndarray:
    """fit.rs:369-378: per-channel mean accumulated in float64."""
    img = np.asarray(image, np.float32).reshape(-1, 3).astype(np.float64)
    n = np.float32(img.shape[0])
    return (img.sum(axis=0, dtype=np.float64) / np.float64(n)).astype(np.float32)


def sample(image: np.ndarray, x: float, y: float) -> np.ndarray:
    """fit.rs:381-385 nearest-pixel sample, clamped to the canvas."""
    H, W = image.shape[0], image.shape[1]

    def index(v: float, n: int) -> int:
        # Rust's `as isize`: truncates toward zero, saturates, NaN -> 0
        f = np.float32(v) * np.float32(n)
        return 0 if np.isnan(f) else int(np.clip(np.trunc(f), 0, n - 1))

    return np.asarray(image[index(y, H), index(x, W)], np.float32).copy()


def seed_scene(target: np.ndarray, T: int, seed: int, seed_scale: float = 0.18):
    """fit.rs:356-367 with this module's generator; returns (params (T,10), background)."""
    bg = mean_color(target)
    u = uniforms(seed, T * 12 + T)
    tri = u[: T * 12].reshape(T, 12)
    out = np.empty((T, 10), np.float32)
    cx, cy = tri[:, 0], tri[:, 1]
    for v in range(3):
        out[:, 2 * v] = (cx + (-seed_scale + 2 * seed_scale * tri[:, 2 + 2 * v])).astype(np.float32)
        out[:, 2 * v + 1] = (cy + (-seed_scale + 2 * seed_scale * tri[:, 3 + 2 * v])).astype(np.float32)
    alphas = _rng_range(u[T * 12:], 0.3, 0.7)
    for k in range(T):
        x0, x1, x2 = out[k, 0], out[k, 2], out[k, 4]
        y0, y1, y2 = out[k, 1], out[k, 3], out[k, 5]
        ccx = np.float32(np.float32(np.float32(x0 + x1) + x2) / np.float32(3.0))
        ccy = np.float32(np.float32(np.float32(y0 + y1) + y2) / np.float32(3.0))
        out[k, 6:9] = sample(target, ccx, ccy)
        out[k, 9] = alphas[k]
    return out, bg


# The benchmark workloads, by name. sigma is the drop-in default (0.0015,
# python/diffrast/torch_layer.py:73).
CONFIGS = {
    "c0": dict(B=1, H=64, W=64, T=32, kind="uniform"),
    "c1": dict(B=16, H=128, W=128, T=128, kind="uniform"),
    "c2": dict(B=16, H=256, W=256, T=128, kind="uniform"),
    "c3": dict(B=8, H=256, W=256, T=512, kind="small"),
    "c4": dict(B=1, H=176, W=176, T=150, kind="fit", iters=800),
}
