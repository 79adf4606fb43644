"""Continuous-time pixel trajectories: the motion model of atl/motion/trajectories.py (MotionPriorCMax layout).

Model.  A coefficient grid (B, 2K, H, W), channels [y_1..y_K, x_1..x_K], defines one trajectory per tile centre
p of a ``tile`` x ``tile`` partition of the sensor (p at offset tile // 2 inside its tile):

    q(p, t) = p + d(p, t),   d(p, t) = sum_{k=1..K} c_k(p) g_k(t),   g_k(0) = 0, so q(p, 0) = p.

Bases g (``basis_kind``):
  * "polynomial"  g_k(t) = t^k;
  * "bezier"      g_k(t) = binom(K, k) t^k (1 - t)^(K - k): the degree-K Bernstein basis whose control point 0
                  is pinned to the start p;
  * "bspline"     g_k(t) = N_k(t): the clamped uniform B-spline basis of degree P = min(3, K) with K + 1
                  functions N_0..N_K over L = K + 1 - P equal spans of [0, 1].  N_0 carries the pinned start
                  (N_k(0) = 0 for k >= 1).  Control points c_k = v * xi_k at the Greville abscissae xi_k give
                  the straight trajectory p + v t exactly (linear precision), and K = 1 is the linear warp.
Between tile centres the 2K coefficients are the bilinear, border-clamped interpolation of the centres' values,
i.e. one flow-grid lookup of 2K channels (the HIP sampler on device, differentiable in the grid and the
position).  An event (x, t) lies on the trajectory whose start p solves q(p, t) = x; the model finds p by
n_fixed_point Picard steps p <- x - d(p, t) from p = x (the reference's assign="invert").
"""
from __future__ import annotations

import math

import numpy as np
import torch

from ..ops.functional import TRAJ_BASES, TRAJ_MAX_K, _tile_plan_ok, traj_displacement, traj_origin
from .base import Motion, as_time
from .parametric import sample_grid


# --------------------------------------------------------------------------------------------- bases
def _bspline_shape(K: int):
    """Degree P and span count L of the K-coefficient clamped uniform B-spline basis."""
    P = min(3, K)
    return P, K + 1 - P


def _bspline_torch(t: torch.Tensor, K: int) -> torch.Tensor:
    """(..., K) values N_1..N_K(t) by the triangular Cox-de Boor recursion on the span of t (the span index
    clamped to [0, L-1], so the end polynomials continue outside [0, 1]); the fp32 operation order of the
    device kernel, so both give the same bits."""
    P, L = _bspline_shape(K)
    fl = float(L)
    j = torch.clamp(torch.floor(t * fl), 0, L - 1).long()

    def knot(i):                                   # u_i = clamp(i - P, 0, L) / L
        return torch.clamp(i - P, 0, L).to(t.dtype) / fl

    nb = [torch.ones_like(t)]
    lefts, rights = [None], [None]
    for d in range(1, P + 1):
        lefts.append(t - knot(j + (P + 1 - d)))
        rights.append(knot(j + (P + d)) - t)
        saved = torch.zeros_like(t)
        for r in range(d):
            tmp = nb[r] / (rights[r + 1] + lefts[d - r])
            nb[r] = saved + rights[r + 1] * tmp
            saved = lefts[d - r] * tmp
        nb.append(saved)
    full = t.new_zeros(t.shape + (K + 1,))        # N_0..N_K; N_{j + r} = nb[r]
    for r in range(P + 1):
        full.scatter_(-1, (j + r)[..., None], nb[r][..., None])
    return full[..., 1:]


def basis(t: torch.Tensor, K: int, kind: str = "polynomial") -> torch.Tensor:
    """(..., K) values g_k(t), k = 1..K, of a trajectory basis (atl/motion/trajectories.py:26-37, plus the
    B-spline basis)."""
    if kind not in TRAJ_BASES:
        raise ValueError(f"unknown basis {kind!r}")
    if kind == "bspline":
        return _bspline_torch(t, K)
    powers = torch.stack([t ** k for k in range(1, K + 1)], -1)
    if kind == "polynomial":
        return powers
    one_minus = torch.stack([(1 - t) ** (K - k) for k in range(1, K + 1)], -1)
    binoms = t.new_tensor([float(math.comb(K, k)) for k in range(1, K + 1)])
    return binoms * powers * one_minus


def basis_table(times, K: int, kind: str):
    """Float64 values and time derivatives of g_1..g_K at the given times: two (n, K) arrays.  Used for the
    slice-centre tables of the trajectory pair sums (evaluated once per call, on the host)."""
    t = np.asarray(times, np.float64)[:, None]
    k = np.arange(1, K + 1, dtype=np.float64)[None, :]
    if kind == "polynomial":
        return t ** k, k * t ** (k - 1)
    if kind == "bezier":
        tt = t[:, 0]

        def bern(n, i):                            # B_{i,n}(t), zero outside 0 <= i <= n
            return math.comb(n, i) * tt ** i * (1 - tt) ** (n - i) if 0 <= i <= n else np.zeros_like(tt)
        val = np.stack([bern(K, i) for i in range(1, K + 1)], 1)
        der = np.stack([K * (bern(K - 1, i - 1) - bern(K - 1, i)) for i in range(1, K + 1)], 1)
        return val, der
    if kind != "bspline":
        raise ValueError(f"unknown basis {kind!r}")
    P, L = _bspline_shape(K)
    knots = np.clip(np.arange(K + P + 2) - P, 0, L) / L
    j = np.clip(np.floor(t[:, 0] * L), 0, L - 1).astype(np.int64)

    def degree(p):                                 # all N_{i,p}(t), i = 0..K+P-p, on the clamped span
        n = np.zeros((t.shape[0], K + P + 1))
        n[np.arange(t.shape[0]), j + P] = 1.0
        for q in range(1, p + 1):
            nxt = np.zeros_like(n)
            for i in range(K + P + 1 - q):
                a = knots[i + q] - knots[i]
                c = knots[i + q + 1] - knots[i + 1]
                if a > 0:
                    nxt[:, i] += (t[:, 0] - knots[i]) / a * n[:, i]
                if c > 0:
                    nxt[:, i] += (knots[i + q + 1] - t[:, 0]) / c * n[:, i + 1]
            n = nxt
        return n

    val = degree(P)[:, 1:K + 1]
    low = degree(P - 1)
    der = np.zeros_like(val)
    for i in range(1, K + 1):
        a = knots[i + P] - knots[i]
        c = knots[i + P + 1] - knots[i + 1]
        term = np.zeros(t.shape[0])
        if a > 0:
            term += low[:, i] / a
        if c > 0:
            term -= low[:, i + 1] / c
        der[:, i - 1] = P * term
    return val, der


def greville(K: int) -> np.ndarray:
    """Greville abscissae xi_1..xi_K of the B-spline basis (control points c_k = v xi_k give q = p + v t)."""
    P, L = _bspline_shape(K)
    knots = np.clip(np.arange(K + P + 2) - P, 0, L) / L
    return np.array([knots[k + 1:k + P + 1].mean() for k in range(1, K + 1)])


# --------------------------------------------------------------------------------------------- model
class PixelTrajectories(Motion):
    """One continuous-time trajectory per tile (atl/motion/trajectories.py:40-109); ``coeff_grid`` is usually a
    network output and receives the gradients of every lookup.  ``tile=1`` gives one trajectory per pixel."""

    def __init__(self, coeff_grid: torch.Tensor, K: int, basis_kind: str = "polynomial", tile: int = 4,
                 assign: str = "invert", n_fixed_point: int = 6):
        super().__init__()
        if coeff_grid.dim() != 4 or coeff_grid.shape[1] != 2 * K:
            raise ValueError(f"coefficient grid must be (B, 2K = {2 * K}, H, W), got {tuple(coeff_grid.shape)}")
        if basis_kind not in TRAJ_BASES:
            raise ValueError(f"unknown basis {basis_kind!r}")
        if assign != "invert":
            raise NotImplementedError("events are assigned to trajectories by fixed-point inversion only")
        if tile < 1:
            raise ValueError("tile must be >= 1")
        self.coeff_grid, self.K, self.basis_kind = coeff_grid, int(K), basis_kind
        self.tile, self.assign, self.n_fp = int(tile), assign, int(n_fixed_point)
        self.B, _, self.H, self.W = coeff_grid.shape
        off = self.tile // 2
        # the coefficients at the tile centres (a strided view: gradients reach the full grid)
        self.tile_c = coeff_grid if self.tile == 1 else coeff_grid[:, :, off::self.tile, off::self.tile]
        self.Hq, self.Wq = self.tile_c.shape[-2:]
        self.offset = float(off)
        self.linear_at_event = self.K == 1           # every basis has g_1(t) = t when K = 1

    # positions in pixels <-> grid coordinates of the tile-centre grid
    def _grid_coords(self, p: torch.Tensor) -> torch.Tensor:
        return p if self.tile == 1 else (p - self.offset) / self.tile

    def coeff_rows(self, p: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        """(N, 2K) coefficients at pixel positions ``p`` in the grid's channel order [y_1..y_K, x_1..x_K]."""
        return sample_grid(self.tile_c, self._grid_coords(p), b)

    def displacement(self, p: torch.Tensor, b: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
        """d(p, t) = q(p, t) - p, (N, 2) in (x, y); on the device one fused kernel."""
        if p.is_cuda and self.K <= TRAJ_MAX_K and not t.requires_grad:
            return traj_displacement(self.tile_c, self._grid_coords(p), b, t, self.K, self.basis_kind)
        c = self.coeff_rows(p, b).view(-1, 2, self.K)          # [:, 0] y coefficients, [:, 1] x coefficients
        d = (c * basis(t, self.K, self.basis_kind)[:, None, :]).sum(-1)
        return d.flip(-1)

    def origin(self, xy: torch.Tensor, t: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        """Start p of the trajectory through (xy, t): n_fixed_point Picard steps on p = xy - d(p, t).  On the
        device, B-spline trajectories take the steps as one autograd node (traj_origin: one coefficient-grid
        accumulation for all steps in the backward)."""
        if self._one_node(xy, t):
            return traj_origin(self.tile_c, xy, b, t, self.K, "bspline", self.n_fp, self.offset, self.tile)
        p = xy
        for _ in range(self.n_fp):
            p = xy - self.displacement(p, b, t)
        return p

    def _one_node(self, xy, t) -> bool:
        """Device B-spline trajectories: origin (and transport) run as one autograd node (traj_origin)."""
        return (xy.is_cuda and self.basis_kind == "bspline" and 3 <= self.K <= TRAJ_MAX_K and not t.requires_grad
                and self.n_fp >= 1 and _tile_plan_ok(*self.tile_c.shape))

    def transport(self, xy, t, t_dst, b):
        td = as_time(t_dst, t)
        if self._one_node(xy, t) and not td.requires_grad:
            return traj_origin(self.tile_c, xy, b, t, self.K, "bspline", self.n_fp, self.offset, self.tile, t_dst=td)
        p = self.origin(xy, t, b)
        return p + self.displacement(p, b, td)

    def velocity(self, xy, t, b):
        """dq/dt at the event; defined here for K = 1 only (straight trajectories: the motion is linear at the
        event, as the exact pair sums require)."""
        if not self.linear_at_event:
            raise NotImplementedError("per-event velocity only for K = 1 (straight trajectories)")
        return self.coeff_rows(self.origin(xy, t, b), b).flip(-1)

    def slice_tables(self, n_slices: int, device) -> torch.Tensor:
        """(S, 2K) float32 table of the basis at the slice centres c_s = (s + 1/2) / S (fp32, as the pair kernels
        compute them): row s = [g_1..g_K(c_s), g_1'..g_K'(c_s)], evaluated in float64."""
        cs = (np.arange(n_slices, dtype=np.float32) + np.float32(0.5)) * np.float32(1.0 / n_slices)
        val, der = basis_table(cs.astype(np.float64), self.K, self.basis_kind)
        return torch.as_tensor(np.concatenate([val, der], 1).astype(np.float32), device=device)

    def tile_trajectories(self, times: torch.Tensor) -> torch.Tensor:
        """Positions (B, n_t, Hq*Wq, 2) in (x, y) of every tile trajectory at ``times`` (the look-up table of
        MotionPriorCMax)."""
        dev, K = self.tile_c.device, self.K
        cy = torch.arange(self.Hq, device=dev, dtype=torch.float32) * self.tile + self.offset
        cx = torch.arange(self.Wq, device=dev, dtype=torch.float32) * self.tile + self.offset
        start = torch.cartesian_prod(cy, cx).flip(-1)                   # (Hq*Wq, 2) in (x, y), row-major
        coef = self.tile_c.reshape(self.B, 2, K, -1).flip(1)            # (B, [x, y], K, n)
        g = basis(times.to(torch.float32), K, self.basis_kind)          # (n_t, K)
        disp = torch.einsum("tk,bckn->btnc", g, coef)
        return start[None, None] + disp

    def flow_field(self, B, H, W, t0=0.0, t1=1.0):
        """(B, 2, H, W) displacement from t0 to t1: the tile trajectories' displacements, upsampled bilinearly
        (align_corners=False), as MotionPriorCMax evaluates its flow."""
        times = torch.tensor([t0, t1], device=self.tile_c.device, dtype=torch.float32)
        pos = self.tile_trajectories(times)
        f = (pos[:, 1] - pos[:, 0]).transpose(1, 2).reshape(self.B, 2, self.Hq, self.Wq)
        return torch.nn.functional.interpolate(f, size=(H, W), mode="bilinear", align_corners=False)

    def regulariser_fields(self, B, H, W):
        return self.tile_c
