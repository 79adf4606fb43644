"""Autonomous velocity fields with the linear (CMax) warp x' = x + v(x) (t' - t) (atl/motion/parametric.py).

Only ``mode="linear"`` is on the hot path (the exact pair kernel requires it, atl/objectives/ats.py:77-78);
the reference's ``mode="exact"`` integrators are outside this library's scope and raise.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from ..ops.functional import sample_grid_hip
from .base import Motion, as_time


class VectorFieldMotion(Motion):
    n_params: int = 0

    @property
    def linear_at_event(self) -> bool:
        return self.mode == "linear"

    def __init__(self, batch_size: int, height: int, width: int, mode: str = "linear",
                 init: Optional[torch.Tensor] = None):
        super().__init__()
        if mode != "linear":
            raise NotImplementedError("only the linear warp x + v(x) dt is implemented")
        self.H, self.W, self.mode = height, width, mode
        self.c = torch.tensor([(width - 1) / 2.0, (height - 1) / 2.0])
        theta = torch.zeros(batch_size, self.n_params) if init is None else init.clone().float()
        self.theta = nn.Parameter(theta)

    def field(self, xy: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError

    def velocity(self, xy, t, b):
        return self.field(xy, b)

    def transport(self, xy, t, t_dst, b):
        """x + v(x) (t_dst - t) (atl/motion/parametric.py:53-56)."""
        dt = as_time(t_dst, t) - t
        return xy + self.field(xy, b) * dt[:, None]


def per_event(theta: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """theta[b] (per-event copy of the per-batch parameters).  Its gradient is a sum over the events of each
    batch item: with one item an expand (the backward is one reduction), otherwise index_select (index_add in
    the backward); advanced indexing would instead backpropagate through an accumulating index_put, which
    serialises over the repeated indices."""
    if theta.shape[0] == 1:
        return theta.expand(b.shape[0], theta.shape[1])
    return theta.index_select(0, b)


class Translation(VectorFieldMotion):
    """v = (tx, ty) (atl/motion/parametric.py:87-97)."""
    n_params = 2

    def field(self, xy, b):
        return per_event(self.theta, b)


class Sim2(VectorFieldMotion):
    """v = t + s (x - c) + w J (x - c): translation, divergence, rotation (atl/motion/parametric.py:128-144)."""
    n_params = 4

    def field(self, xy, b):
        th = per_event(self.theta, b)
        d = xy - self.c.to(xy)
        vx = th[:, 0] + (th[:, 2] * d[:, 0] - th[:, 3] * d[:, 1])
        vy = th[:, 1] + (th[:, 3] * d[:, 0] + th[:, 2] * d[:, 1])
        return torch.stack([vx, vy], 1)


class DenseLinearFlow(VectorFieldMotion):
    """Dense velocity grid (B, 2, Hg, Wg) spanning the image, bilinearly interpolated
    (atl/motion/parametric.py:196-232).  On device the lookup runs on the HIP flow sampler."""

    def __init__(self, batch_size, height, width, grid=(1, 1), mode="linear", init=None):
        Motion.__init__(self)
        if mode != "linear":
            raise NotImplementedError("only the linear warp x + v(x) dt is implemented")
        self.H, self.W, self.mode = height, width, mode
        self.c = torch.tensor([(width - 1) / 2.0, (height - 1) / 2.0])
        g = torch.zeros(batch_size, 2, *grid) if init is None else init.clone().float()
        self.grid = nn.Parameter(g)

    @property
    def theta(self):
        return self.grid

    def field(self, xy, b):
        Hg, Wg = self.grid.shape[-2:]
        if xy.is_cuda:
            return sample_grid_hip(self.grid, xy, b, img_hw=(self.H, self.W))
        gx = xy[:, 0] / max(self.W - 1, 1) * (Wg - 1)
        gy = xy[:, 1] / max(self.H - 1, 1) * (Hg - 1)
        return sample_grid(self.grid, torch.stack([gx, gy], 1), b)


def sample_grid(field: torch.Tensor, gpos: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Bilinear, border-clamped sample of a (B, C, Hg, Wg) field at grid coordinates (N, 2), returns (N, C)
    (atl/motion/parametric.py:235-251).  Device tensors use the HIP sampler."""
    if gpos.is_cuda:
        return sample_grid_hip(field, gpos, b)
    B, C, Hg, Wg = field.shape
    gx = gpos[:, 0].clamp(0, Wg - 1)
    gy = gpos[:, 1].clamp(0, Hg - 1)
    x0 = torch.floor(gx).clamp(max=max(Wg - 2, 0))
    y0 = torch.floor(gy).clamp(max=max(Hg - 2, 0))
    ax, ay = gx - x0, gy - y0
    x0, y0 = x0.long(), y0.long()
    x1, y1 = (x0 + 1).clamp(max=Wg - 1), (y0 + 1).clamp(max=Hg - 1)
    f = field.permute(0, 2, 3, 1).reshape(-1, C)
    base = b * (Hg * Wg)

    def at(yy, xx):
        return f[base + yy * Wg + xx]

    return (at(y0, x0) * ((1 - ax) * (1 - ay))[:, None] + at(y0, x1) * (ax * (1 - ay))[:, None] +
            at(y1, x0) * ((1 - ax) * ay)[:, None] + at(y1, x1) * (ax * ay)[:, None])
