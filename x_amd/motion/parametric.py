"""Velocity-field motions with the linear warp x' = x + v(x) (t' - t) (atl/motion/parametric.py).

Only the linear warp is on the hot path: the exact pair sums need motion linear at the event
(atl/objectives/ats.py:77-78).  The reference's "exact" integrators (ODE transport) are outside this library and
refused.  Parameters are per window (theta (B, n_params), or the dense grid (B, 2, Hg, Wg)); the centre c of the
affine models is the sensor centre ((W-1)/2, (H-1)/2).
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import nn

from ..ops.functional import sample_grid_hip
from .base import Motion, as_time


def per_event(theta: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """theta[b], the per-window parameters of every event.  One window: a broadcast view (its gradient is one
    reduction); several: index_select (index_add in the backward) rather than advanced indexing, whose backward
    is an accumulating index_put that serialises over repeated indices."""
    return theta.expand(b.shape[0], theta.shape[1]) if theta.shape[0] == 1 else theta.index_select(0, b)


class VectorFieldMotion(Motion):
    """Autonomous velocity field v(x; theta), transported by the linear warp."""
    n_params: int = 0

    def __init__(self, batch_size: int, height: int, width: int, mode: str = "linear", rk4_steps: int = 8,
                 init: Optional[torch.Tensor] = None):
        super().__init__()                        # rk4_steps: the reference's integrator setting, unused here
        self._set_geometry(height, width, mode)
        start = torch.zeros(batch_size, self.n_params) if init is None else init.clone().float()
        self.theta = nn.Parameter(start)

    def _set_geometry(self, height, width, mode):
        if mode != "linear":
            raise NotImplementedError("only the linear warp x + v(x) dt is implemented (mode='linear')")
        self.H, self.W, self.mode = height, width, mode
        self.c = torch.tensor([(width - 1) / 2.0, (height - 1) / 2.0])

    @property
    def linear_at_event(self) -> bool:
        return self.mode == "linear"

    def field(self, xy: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError(f"{type(self).__name__} defines no field")

    def velocity(self, xy, t, b):
        return self.field(xy, b)

    def transport(self, xy, t, t_dst, b):
        """x + v(x) (t_dst - t) (atl/motion/parametric.py:53-56): subtract, multiply, add, in that order."""
        step = as_time(t_dst, t) - t
        return xy + self.field(xy, b) * step[:, None]


class Translation(VectorFieldMotion):
    """v = (tx, ty) per window (atl/motion/parametric.py:87-97)."""
    n_params = 2

    def field(self, xy, b):
        return per_event(self.theta, b)


class Sim2(VectorFieldMotion):
    """v = (tx, ty) + s (x - c) + w J (x - c) with J the rotation by 90 degrees: translation, divergence s and
    in-plane rotation w per window (atl/motion/parametric.py:128-144)."""
    n_params = 4

    def field(self, xy, b):
        th = per_event(self.theta, b)
        d = xy - self.c.to(xy)
        s, w = th[:, 2], th[:, 3]
        return torch.stack([th[:, 0] + (s * d[:, 0] - w * d[:, 1]), th[:, 1] + (w * d[:, 0] + s * d[:, 1])], 1)


class DenseLinearFlow(VectorFieldMotion):
    """Velocity grid (B, 2, Hg, Wg) spanning the sensor, bilinearly interpolated with a border clamp
    (atl/motion/parametric.py:196-232): pixel (0, 0) sits on node (0, 0) and pixel (W-1, H-1) on node
    (Wg-1, Hg-1).  On device the look-up is the HIP flow sampler."""

    def __init__(self, batch_size, height, width, grid=(1, 1), mode="linear", init=None, rk4_steps=4):
        Motion.__init__(self)
        self._set_geometry(height, width, mode)
        start = torch.zeros(batch_size, 2, *grid) if init is None else init.clone().float()
        self.grid = nn.Parameter(start)

    @property
    def theta(self):
        """The grid, under the parameter name of the parametric models."""
        return self.grid

    def field(self, xy, b):
        if xy.is_cuda:
            return sample_grid_hip(self.grid, xy, b, img_hw=(self.H, self.W))
        Hg, Wg = self.grid.shape[-2:]
        node = torch.stack([xy[:, 0] / max(self.W - 1, 1) * (Wg - 1), xy[:, 1] / max(self.H - 1, 1) * (Hg - 1)], 1)
        return sample_grid(self.grid, node, b)

    def upsample(self, factor: int = 2):
        """Refine the grid by ``factor`` per axis (bilinear, corners aligned) for coarse-to-fine fitting."""
        Hg, Wg = self.grid.shape[-2:]
        with torch.no_grad():
            fine = torch.nn.functional.interpolate(self.grid, size=(Hg * factor, Wg * factor), mode="bilinear",
                                                   align_corners=True)
        self.grid = nn.Parameter(fine)
        return self

    def regulariser_fields(self, B, H, W):
        return self.grid


def sample_grid(field: torch.Tensor, gpos: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """(N, C) bilinear sample of a (B, C, Hg, Wg) field at grid coordinates gpos (N, 2), clamped to the border
    (atl/motion/parametric.py:235-251); device tensors use the HIP sampler.  The fp32 operations (clamp, floor
    capped at the last interior node, weights (1-a)(1-a') ..., the four products added corner (0,0), (0,1),
    (1,0), (1,1) in that order) are the reference's, because the device sampler and the oracle reproduce them
    bit for bit."""
    if gpos.is_cuda:
        return sample_grid_hip(field, gpos, b)
    B, C, Hg, Wg = field.shape
    g = torch.stack([gpos[:, 0].clamp(0, Wg - 1), gpos[:, 1].clamp(0, Hg - 1)], 1)
    lo = torch.minimum(torch.floor(g), g.new_tensor([max(Wg - 2, 0), max(Hg - 2, 0)]))
    a = g - lo
    i0 = lo.long()
    i1 = torch.minimum(i0 + 1, i0.new_tensor([Wg - 1, Hg - 1]))
    rows = field.permute(0, 2, 3, 1).reshape(B * Hg * Wg, C)
    base = b * (Hg * Wg)
    one = 1 - a
    out = rows[base + i0[:, 1] * Wg + i0[:, 0]] * (one[:, 0] * one[:, 1])[:, None]
    out = out + rows[base + i0[:, 1] * Wg + i1[:, 0]] * (a[:, 0] * one[:, 1])[:, None]
    out = out + rows[base + i1[:, 1] * Wg + i0[:, 0]] * (one[:, 0] * a[:, 1])[:, None]
    return out + rows[base + i1[:, 1] * Wg + i1[:, 0]] * (a[:, 0] * a[:, 1])[:, None]
