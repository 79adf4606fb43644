"""Seeded synthetic event windows for the event-transport workloads.

The reference ships no event simulator (its ``atl/data`` package is absent), so the workloads define their
own scenes.  Units follow the reference (atl/motion/base.py:1-12): time is normalised to [0, 1] per window,
velocities are pixels per window (v_px/s * T).  Every window is built by NumPy ``default_rng(seed)`` and
returned as fp32/int64 arrays that the GPU path and the CPU oracle consume unchanged.

Scenes
------
* ``segments``: a fraction ``1 - noise`` of the events lies within 1 px (normal offset U(-1, 1)) of
  ``n_segments`` random line segments (endpoints uniform in the sensor); each scene point moves with the
  motion, x(t) = x0 + v(x0) t; the rest is uniform noise.  Positions are rounded to the pixel grid as a
  sensor reports them; events that leave the sensor are redrawn.
* ``blobs``: a fraction ``1 - noise`` of the events in ``n_blobs`` isotropic Gaussian blobs (sigma
  ``blob_sigma`` px, centres uniform), the rest uniform noise (the contention workload).

Polarity is +-1 equiprobable; t ~ U[0, 1] sorted ascending.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np

F32 = np.float32


@dataclass
class Window:
    """One packed event window (numpy) plus the motion that generated it."""
    xy: np.ndarray              # (N, 2) f32, pixel coordinates (x, y)
    t: np.ndarray               # (N,) f32 in [0, 1], ascending within each batch entry
    p: np.ndarray               # (N,) f32 in {-1, +1}
    b: np.ndarray               # (N,) int64 batch index (sorted by (b, t))
    height: int
    width: int
    batch_size: int = 1
    duration: float = 1.0       # seconds per window
    motion: dict = field(default_factory=dict)

    @property
    def n(self) -> int:
        return int(self.t.shape[0])


def smooth_flow(rng, H, W, sigma=40.0, vmax=20.0, B=1):
    """(B, 2, H, W) f32 smooth random field: N(0, 1) Gaussian-filtered (scipy.ndimage, mode='reflect',
    truncate=4) per channel, scaled so that max ||v|| = vmax px/window."""
    from scipy.ndimage import gaussian_filter
    g = rng.standard_normal((B, 2, H, W))
    out = np.empty_like(g)
    for k in range(B):
        for c in range(2):
            out[k, c] = gaussian_filter(g[k, c], sigma=sigma, mode="reflect", truncate=4.0)
    out *= vmax / np.sqrt((out ** 2).sum(1)).max()
    return out.astype(F32)


def _bilinear_np(field, x, y):
    """Bilinear lookup of a (C, H, W) field at float positions (clamped to the grid): (N, C) float64."""
    H, W = field.shape[-2:]
    x = np.clip(x, 0, W - 1)
    y = np.clip(y, 0, H - 1)
    x0 = np.minimum(np.floor(x), W - 2).astype(np.int64)
    y0 = np.minimum(np.floor(y), H - 2).astype(np.int64)
    ax, ay = x - x0, y - y0
    f = field.astype(np.float64)
    return ((1 - ax) * (1 - ay) * f[:, y0, x0] + ax * (1 - ay) * f[:, y0, x0 + 1] +
            (1 - ax) * ay * f[:, y0 + 1, x0] + ax * ay * f[:, y0 + 1, x0 + 1]).T


def _velocity(motion, x, y, W, H):
    kind = motion["kind"]
    if kind == "translation":
        th = motion["theta"]
        return np.broadcast_to(np.asarray(th[:2], np.float64), (x.shape[0], 2))
    if kind == "dense":
        return _bilinear_np(motion["grid"][0], x / (W - 1) * (motion["grid"].shape[-1] - 1),
                            y / (H - 1) * (motion["grid"].shape[-2] - 1))
    if kind == "sim2":
        tx, ty, s, w = motion["theta"]
        cx, cy = (W - 1) / 2.0, (H - 1) / 2.0
        dx, dy = x - cx, y - cy
        return np.stack([tx + s * dx - w * dy, ty + w * dx + s * dy], 1)
    raise ValueError(kind)


def _scene_points(rng, n, W, H, kind, n_objects, blob_sigma):
    if kind == "segments":
        A = rng.uniform([0, 0], [W - 1, H - 1], size=(n_objects, 2))
        Bp = rng.uniform([0, 0], [W - 1, H - 1], size=(n_objects, 2))
        seg = rng.integers(0, n_objects, n)
        u = rng.uniform(0, 1, n)
        d = Bp[seg] - A[seg]
        nrm = np.stack([-d[:, 1], d[:, 0]], 1) / np.maximum(np.linalg.norm(d, axis=1, keepdims=True), 1e-9)
        return A[seg] + u[:, None] * d + nrm * rng.uniform(-1, 1, n)[:, None]
    if kind == "blobs":
        C = rng.uniform([0, 0], [W - 1, H - 1], size=(n_objects, 2))
        k = rng.integers(0, n_objects, n)
        return C[k] + rng.standard_normal((n, 2)) * blob_sigma
    raise ValueError(kind)


def make_window(n, H, W, motion, scene="segments", n_objects=20, noise=0.3, blob_sigma=8.0, seed=0,
                duration=1.0, rng: Optional[np.random.Generator] = None) -> Window:
    """One window of ``n`` events moving under ``motion`` (dict with ``kind`` in translation/dense/sim2)."""
    rng = np.random.default_rng(seed) if rng is None else rng
    n_sig = int(round(n * (1 - noise)))
    xs, ts = [], []
    need = n_sig
    while need > 0:                                    # scene events, redrawn while outside the sensor
        m = int(need * 1.3) + 16
        x0 = _scene_points(rng, m, W, H, scene, n_objects, blob_sigma)
        t = rng.uniform(0, 1, m)
        x = x0 + _velocity(motion, x0[:, 0], x0[:, 1], W, H) * t[:, None]
        x = np.round(x)
        ok = (x[:, 0] >= 0) & (x[:, 0] <= W - 1) & (x[:, 1] >= 0) & (x[:, 1] <= H - 1)
        x, t = x[ok][:need], t[ok][:need]
        xs.append(x); ts.append(t)
        need -= x.shape[0]
    n_noise = n - n_sig
    xs.append(np.stack([rng.integers(0, W, n_noise), rng.integers(0, H, n_noise)], 1).astype(np.float64))
    ts.append(rng.uniform(0, 1, n_noise))
    x = np.concatenate(xs)
    t = np.concatenate(ts).astype(F32)
    order = np.argsort(t, kind="stable")
    p = np.where(rng.uniform(0, 1, n) < 0.5, 1.0, -1.0).astype(F32)
    return Window(xy=np.ascontiguousarray(x[order].astype(F32)), t=np.ascontiguousarray(t[order]), p=p,
                  b=np.zeros(n, np.int64), height=H, width=W, duration=duration, motion=motion)


# ------------------------------------------------------------------------------------------- workloads
def plumbing_translation(seed=0, n=100_000) -> Window:
    """240x180 sensor, 100k events over 50 ms, 20 segments + 30% noise, constant flow (40, -25) px/s,
    i.e. theta = (2.0, -1.25) px/window."""
    T = 0.05
    motion = {"kind": "translation", "theta": np.array([40 * T, -25 * T], F32)}
    return make_window(n, 180, 240, motion, "segments", 20, 0.3, seed=seed, duration=T)


def dense_flow_window(seed=0, n=1_000_000, H=480, W=640) -> Window:
    """640x480 sensor, 1M events over 100 ms, 50 segments + 30% noise, smooth random dense flow
    (N(0,1) Gaussian-filtered with sigma = 40 px, max 200 px/s = 20 px/window) on a full-resolution grid."""
    T = 0.1
    rng = np.random.default_rng(seed)
    grid = smooth_flow(rng, H, W, sigma=40.0, vmax=200 * T)
    motion = {"kind": "dense", "grid": grid}
    return make_window(n, H, W, motion, "segments", 50, 0.3, duration=T, rng=rng)


def blob_window(seed=0, n=4_000_000, H=480, W=640) -> Window:
    """640x480, 4M events over 100 ms: 90% in 5 Gaussian blobs (sigma 8 px), 10% uniform noise; Sim2 motion
    with divergence 2/s and rotation 1 rad/s, theta = (0, 0, 0.1, 0.1) per window."""
    T = 0.1
    motion = {"kind": "sim2", "theta": np.array([0.0, 0.0, 1.0 * T, 1.0 * T], F32)}
    return make_window(n, H, W, motion, "blobs", 5, 0.1, blob_sigma=8.0, seed=seed, duration=T)


def small_window(seed=0, n=3000, H=40, W=48, vmax=6.0, B=1, scene="segments") -> Window:
    """A small dense-flow window (tests): B batch entries of n events each, packed and sorted by (b, t)."""
    rng = np.random.default_rng(seed)
    grid = smooth_flow(rng, H, W, sigma=6.0, vmax=vmax, B=B)
    parts = []
    for k in range(B):
        parts.append(make_window(n, H, W, {"kind": "dense", "grid": grid[k:k + 1]}, scene, 6, 0.3, rng=rng))
    xy = np.concatenate([w.xy for w in parts])
    t = np.concatenate([w.t for w in parts])
    p = np.concatenate([w.p for w in parts])
    b = np.concatenate([np.full(w.n, k, np.int64) for k, w in enumerate(parts)])
    return Window(xy=xy, t=t, p=p, b=b, height=H, width=W, batch_size=B, motion={"kind": "dense", "grid": grid})


def trajectory_coeffs(rng, B, K, H, W, sigma_px=40.0, dmax=5.0):
    """(B, 2K, H, W) f32 per-pixel trajectory coefficients (control points) [y_1..y_K, x_1..x_K]: every channel
    N(0, 1) Gaussian-filtered (sigma = sigma_px, mode='reflect'), scaled so that the largest coefficient
    displacement norm is dmax px."""
    from scipy.ndimage import gaussian_filter
    g = rng.standard_normal((B, 2 * K, H, W))
    for k in range(B):
        for c in range(2 * K):
            g[k, c] = gaussian_filter(g[k, c], sigma=sigma_px, mode="reflect", truncate=4.0)
    g *= dmax / np.sqrt(g[:, :K] ** 2 + g[:, K:] ** 2).max()
    return np.ascontiguousarray(g.astype(F32))


def _trajectory_window(rng, n, H, W, coef, K, scene="segments", n_objects=50, noise=0.3, duration=0.025):
    """One window of n events on per-pixel B-spline trajectories: scene points p at t = 0 (segments), each event
    at q(p, t) = p + sum_k c_k(p) N_k(t) (coefficients bilinear at p, border clamp), rounded to the pixel grid,
    redrawn while outside the sensor; uniform noise events on top."""
    from .motion.trajectories import basis_table
    n_sig = int(round(n * (1 - noise)))
    xs, ts = [], []
    need = n_sig
    while need > 0:
        m = int(need * 1.3) + 16
        p = _scene_points(rng, m, W, H, scene, n_objects, 8.0)
        t = rng.uniform(0, 1, m)
        c = _bilinear_np(coef, p[:, 0], p[:, 1])                 # (m, 2K) control points at p
        g, _ = basis_table(t, K, "bspline")
        x = p + np.stack([(c[:, K:] * g).sum(1), (c[:, :K] * g).sum(1)], 1)
        x = np.round(x)
        ok = (x[:, 0] >= 0) & (x[:, 0] <= W - 1) & (x[:, 1] >= 0) & (x[:, 1] <= H - 1)
        xs.append(x[ok][:need])
        ts.append(t[ok][:need])
        need -= xs[-1].shape[0]
    n_noise = n - n_sig
    xs.append(np.stack([rng.integers(0, W, n_noise), rng.integers(0, H, n_noise)], 1).astype(np.float64))
    ts.append(rng.uniform(0, 1, n_noise))
    x, t = np.concatenate(xs), np.concatenate(ts).astype(F32)
    order = np.argsort(t, kind="stable")
    pol = np.where(rng.uniform(0, 1, n) < 0.5, 1.0, -1.0).astype(F32)
    return x[order].astype(F32), t[order], pol


def bspline_windows(seed=0, B=4, n=500_000, H=480, W=640, K=10) -> Window:
    """Continuous-time trajectory workload: B windows of n events (640x480, 25 ms each, 50 segments + 30%
    noise) packed in one packet sorted by (b, t), moving on per-pixel cubic B-spline trajectories with K = 10
    control points per axis (the start pinned), (B, 2K, H, W) smooth random control points (sigma 40 px) of
    largest displacement 5 px = 200 px/s over 25 ms (``motion["coeffs"]``)."""
    rng = np.random.default_rng(seed)
    coef = trajectory_coeffs(rng, B, K, H, W)
    parts = [_trajectory_window(rng, n, H, W, coef[k], K) for k in range(B)]
    return Window(xy=np.ascontiguousarray(np.concatenate([w[0] for w in parts])),
                  t=np.ascontiguousarray(np.concatenate([w[1] for w in parts])),
                  p=np.concatenate([w[2] for w in parts]),
                  b=np.concatenate([np.full(n, k, np.int64) for k in range(B)]), height=H, width=W, batch_size=B,
                  duration=0.025, motion={"kind": "bspline", "coeffs": coef, "K": K})
