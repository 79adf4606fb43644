"""Dense continuous-time pixel trajectories (atl/motion/trajectories.py:1-120).

A coefficient grid C (B, 2K, H, W), channels [y_1..y_K, x_1..x_K], holds one trajectory per ``tile`` x ``tile``
patch, starting at the patch centre p at t = 0:

    q(p, t) = p + sum_k c_k(p) g_k(t),   g_k(t) = basis_k(t) - basis_k(0)

with the polynomial basis t^k or the degree-K Bernstein basis with the first control point pinned to the start.
The coefficients at continuous positions are the bilinear (border-clamped) interpolation between tile centres,
so every coefficient lookup is the flow-grid sampler (the HIP kernel on device, differentiable w.r.t. both the
coefficients and the positions).  An event (x, t) is transported by first solving p + d(p, t) = x by
fixed-point iteration (``assign="invert"``), then evaluating q(p, t').
"""
from __future__ import annotations

import math

import torch

from .base import Motion, as_time
from ..ops.functional import TRAJ_MAX_K, traj_displacement
from .parametric import sample_grid


def basis(t: torch.Tensor, K: int, kind: str = "polynomial") -> torch.Tensor:
    """(..., K) values g_k(t) = basis_k(t) - basis_k(0), k = 1..K (atl/motion/trajectories.py:26-37)."""
    tt = t[..., None]
    k = torch.arange(1, K + 1, device=t.device, dtype=t.dtype)
    if kind == "polynomial":
        return tt ** k
    if kind == "bezier":
        binom = torch.tensor([float(math.comb(K, j)) for j in range(1, K + 1)], device=t.device, dtype=t.dtype)
        return binom * tt ** k * (1 - tt) ** (K - k)
    raise ValueError(f"unknown basis {kind!r}")


class PixelTrajectories(Motion):
    """One continuous-time trajectory per tile (atl/motion/trajectories.py:40-120).

    ``coeff_grid`` (B, 2K, H, W) is typically a network output; gradients flow to it through every lookup."""

    def __init__(self, coeff_grid: torch.Tensor, K: int, basis_kind: str = "polynomial", tile: int = 4,
                 assign: str = "invert", n_fixed_point: int = 6):
        super().__init__()
        B, C, H, W = coeff_grid.shape
        if C != 2 * K:
            raise ValueError(f"coefficient grid has {C} channels, expected 2K = {2 * K}")
        if assign != "invert":
            raise NotImplementedError("only the fixed-point inversion assigns events to trajectories")
        self.coeff_grid, self.K, self.basis_kind, self.tile = coeff_grid, K, basis_kind, tile
        self.assign, self.n_fp = assign, n_fixed_point
        self.B, self.H, self.W = B, H, W
        s = tile // 2
        self.tile_c = coeff_grid[:, :, s::tile, s::tile]   # coefficients at the tile centres (B, 2K, Hq, Wq)
        self.Hq, self.Wq = self.tile_c.shape[-2:]
        self.offset = float(s)
        self.linear_at_event = K == 1 and basis_kind == "polynomial"

    def _coeff_at(self, p: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        """(N, K, 2) coefficients (x, y) at continuous pixel positions."""
        c = sample_grid(self.tile_c, (p - self.offset) / self.tile, b)
        return torch.stack([c[:, self.K:], c[:, :self.K]], -1)

    def displacement(self, p: torch.Tensor, b: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
        """q(p, t) - p for trajectories starting at ``p`` (on the device: one fused kernel)."""
        if p.is_cuda and self.K <= TRAJ_MAX_K and not t.requires_grad:
            return traj_displacement(self.tile_c, (p - self.offset) / self.tile, b, t, self.K, self.basis_kind)
        return (self._coeff_at(p, b) * basis(t, self.K, self.basis_kind)[..., None]).sum(1)

    def origin(self, xy: torch.Tensor, t: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        """Start p of the trajectory through (xy, t): fixed point of p = xy - d(p, t)."""
        p = xy
        for _ in range(self.n_fp):
            p = xy - self.displacement(p, b, t)
        return p

    def transport(self, xy, t, t_dst, b):
        p = self.origin(xy, t, b)
        return p + self.displacement(p, b, as_time(t_dst, t))

    def velocity(self, xy, t, b):
        if not self.linear_at_event:
            raise NotImplementedError("per-event velocity only for the degree-1 polynomial basis")
        return self._coeff_at(self.origin(xy, t, b), b)[:, 0]

    def tile_trajectories(self, times: torch.Tensor) -> torch.Tensor:
        """(B, n_t, Hq*Wq, 2) positions (x, y) of every tile trajectory at ``times``."""
        dev = self.tile_c.device
        ys = torch.arange(self.Hq, device=dev, dtype=torch.float32) * self.tile + self.offset
        xs = torch.arange(self.Wq, device=dev, dtype=torch.float32) * self.tile + self.offset
        gy, gx = torch.meshgrid(ys, xs, indexing="ij")
        start = torch.stack([gx, gy], -1).reshape(1, 1, -1, 2)
        c = self.tile_c.reshape(self.B, 2, self.K, self.Hq * self.Wq)
        cxy = torch.stack([c[:, 1], c[:, 0]], -1)           # (B, K, n, 2) in (x, y)
        g = basis(times, self.K, self.basis_kind)            # (n_t, K)
        return start + (g[None, :, :, None, None] * cxy[:, None]).sum(2)

    def flow_field(self, B, H, W, t0=0.0, t1=1.0):
        """Dense displacement t0 -> t1: tile displacements upsampled bilinearly (align_corners=False)."""
        times = torch.tensor([t0, t1], device=self.tile_c.device, dtype=torch.float32)
        tr = self.tile_trajectories(times)
        f = (tr[:, 1] - tr[:, 0]).reshape(self.B, self.Hq, self.Wq, 2).permute(0, 3, 1, 2)
        return torch.nn.functional.interpolate(f, size=(H, W), mode="bilinear", align_corners=False)

    def regulariser_fields(self, B, H, W):
        return self.tile_c
