"""Anchored transport score: every raw event (anchor) is scored by the density of the other events transported
to its own timestamp (atl/objectives/ats.py:1-105).

    S(theta) = mean_i log(eps + rho_{-i}(x_i)),
    rho_{-i}(x) = (1 / W_i) sum_{j != i, |t_i - t_j| <= tau} K_h(x - Phi_{t_j -> t_i}(x_j)),

with a Gaussian kernel K_h cut at cut * h, W_i the number of same-batch events within +-tau scaled by the
visible fraction (exposure correction), uniform dequantisation of every source and Gaussian smoothing N(0, h^2)
of every anchor.

* :class:`AnchoredExact`        motion linear at the event, Phi = x_j + v_j (t_i - t_j): the exact pair sums.
* :class:`AnchoredTrajectories` pixel trajectories (no counterpart in the reference, whose exact score refuses
                                motion that is not linear at the event): Phi is the source's trajectory linearised
                                at the anchor's time-slice centre (x_amd.ops.ats_pair_sums_traj), exact for
                                straight trajectories.

On device the whole chain runs on HIP kernels (noise, flow or trajectory look-ups, pair sums, window counts,
visible fraction, epilogue and mean); on CPU tensors the same chain runs on torch ops.
"""
from __future__ import annotations

import math
import os
from typing import Optional

import torch

from ..core.events import EventPacket
from ..ops import (anchored_log_scores, anchored_score_mean, ats_pair_sums, ats_pair_sums_flow, ats_pair_sums_traj,
                   event_noise, layout_scope, traj_visible_fraction, visible_fraction_linear, window_counts)
from .base import Objective


# --------------------------------------------------------------------------------------------- exposure
def _bin_counts_cpu(ev: EventPacket, n_check: int) -> torch.Tensor:
    """Events per (batch, time bin) of n_check equal bins of [0, 1] (bin of t: floor(t n_check), clamped)."""
    sl = torch.clamp((ev.t * n_check).long(), 0, n_check - 1)
    flat = torch.bincount(ev.b * n_check + sl, minlength=ev.batch_size * n_check)
    return flat.to(ev.t.dtype).view(ev.batch_size, n_check)


@torch.no_grad()
def visible_fraction(motion, xa, ta, ba, ev: EventPacket, tau: float, n_check: int = 16) -> torch.Tensor:
    """Share of each anchor's +-tau source mass recorded while its scene content was inside the field of view
    (atl/objectives/ats.py:31-50): the anchor is transported to the n_check bin centres c_k; bin k counts with
    weight (events of the anchor's batch in bin k) * [|t_a - c_k| <= tau]; the result is the weighted share of
    centres where the transported anchor is inside the sensor, at least 1e-3.

    Device tensors with motion linear at the event run one fused kernel; trajectory motion finds each anchor's
    trajectory start once and evaluates the trajectory at every centre; any other motion is transported per
    centre."""
    if xa.is_cuda and getattr(motion, "linear_at_event", False):
        va = motion.velocity(xa, ta, ba)
        return visible_fraction_linear(xa, va, ta, ba, ev.t, ev.b, ev.batch_size, ev.height, ev.width, tau, n_check,
                                       assume_sorted=bool(ev.meta.get("sorted")))
    from ..motion import PixelTrajectories
    from ..ops.functional import TRAJ_MAX_K
    if (xa.is_cuda and type(motion) is PixelTrajectories and motion.K <= TRAJ_MAX_K and motion.assign == "invert"
            and motion.tile_c.is_cuda):             # start, one coefficient look-up, every centre: one pass
        return traj_visible_fraction(motion.tile_c, motion.K, motion.basis_kind, motion.n_fp, motion.offset,
                                     motion.tile, xa, ta, ba, ev.t, ev.b, ev.batch_size, ev.height, ev.width, tau,
                                     n_check, assume_sorted=bool(ev.meta.get("sorted")))
    edges = torch.linspace(0, 1, n_check + 1, device=ev.device)
    centres = (0.5 * (edges[:-1] + edges[1:])).tolist()           # one host transfer
    counts = _bin_counts_cpu(ev, n_check) if not xa.is_cuda else None
    if counts is None:
        from ..ops.functional import bin_counts
        counts = bin_counts(ev.t, ev.b, ev.batch_size, n_check, assume_sorted=bool(ev.meta.get("sorted")))
    start = motion.origin(xa, ta, ba) if hasattr(motion, "origin") else None
    vis, tot = torch.zeros_like(ta), torch.zeros_like(ta)
    for k, c in enumerate(centres):
        if start is not None:
            y = start + motion.displacement(start, ba, torch.full_like(ta, c))
        else:
            y = motion.transport(xa, ta, c, ba)
        seen = ((y[:, 0] >= 0) & (y[:, 0] <= ev.width - 1) & (y[:, 1] >= 0) & (y[:, 1] <= ev.height - 1))
        w = counts[ba, k] * ((ta - c).abs() <= tau).to(ta.dtype)
        vis += w * seen.to(ta.dtype)
        tot += w
    return (vis / tot.clamp(min=1)).clamp(min=1e-3)


# --------------------------------------------------------------------------------------------- shared base
class _Anchored(Objective):
    """Anchors, noise and epilogue shared by the anchored scores.  Noise: ``rng="cpu"`` draws it from a CPU
    ``torch.Generator`` in the reference's order (dequantisation, then smoothing; then a copy to the device);
    ``rng="device"`` draws on the device (different numbers for the same seed), with every event an anchor as
    one fused Philox pass (both draws and both adds)."""
    reference_frame = False

    def __init__(self, h, tau, eps_frac, n_anchors, n_slices, cut, seed, smooth_anchors, dequantize, visibility,
                 anchor_margin, rng):
        if rng not in ("cpu", "device"):
            raise ValueError(f"rng must be 'cpu' or 'device', got {rng!r}")
        self.__dict__.update(h=h, tau=tau, eps_frac=eps_frac, n_anchors=n_anchors, n_slices=n_slices, cut=cut,
                             seed=seed, smooth_anchors=smooth_anchors, dequantize=dequantize,
                             visibility=visibility, anchor_margin=anchor_margin, rng=rng)
        self.gen = None if seed is None else torch.Generator().manual_seed(seed)
        self._dev_gen = None          # torch device generator (noise for anchor subsets)
        self._philox = None           # (seed, draws so far) of the fused device noise

    def set_bandwidth(self, h: float):
        """Kernel width h (bandwidth annealing)."""
        self.h = float(h)

    def _anchors(self, ev: EventPacket) -> Optional[torch.Tensor]:
        """Sorted anchor indices, or None for every event in order (then no index array is built or used)."""
        idx = None
        if self.n_anchors is not None and self.n_anchors < ev.n:
            idx = torch.sort(torch.randperm(ev.n, generator=self.gen, device="cpu")[:self.n_anchors]).values
            idx = idx.to(ev.device)
        if self.anchor_margin > 0:    # selection on raw positions: independent of the motion
            if idx is None:
                idx = torch.arange(ev.n, device=ev.device)
            idx = idx[ev.inside(ev.xy[idx], margin=-self.anchor_margin)]
        return idx

    def _fresh_seed(self) -> int:
        return self.seed if self.seed is not None else int.from_bytes(os.urandom(8), "little")

    def _noise(self, ev: EventPacket, anchors):
        """(xs, xa): dequantised source positions and smoothed anchor positions."""
        xy = ev.xy
        on_device = self.rng == "device" and xy.is_cuda
        if on_device and anchors is None and not xy.requires_grad and (self.dequantize or self.smooth_anchors):
            if self._philox is None:
                self._philox = [self._fresh_seed(), 0]
            xs, xa = event_noise(xy, self._philox[0], self._philox[1], self.h, self.dequantize, self.smooth_anchors)
            self._philox[1] += 1
            return xs, (xs if xa is None else xa)

        def draw(shape, normal):
            if on_device:
                if self._dev_gen is None:
                    self._dev_gen = torch.Generator(device=xy.device).manual_seed(self._fresh_seed())
                out = torch.empty(shape, device=xy.device, dtype=xy.dtype)
                return out.normal_(0.0, 1.0, generator=self._dev_gen) if normal else \
                    out.uniform_(0.0, 1.0, generator=self._dev_gen)
            f = torch.randn if normal else torch.rand
            return f(shape, generator=self.gen).to(xy)

        xs = xy + (draw(xy.shape, False) - 0.5) if self.dequantize else xy
        xa = xs if anchors is None else xs[anchors]
        if self.smooth_anchors:
            xa = xa + self.h * draw(xa.shape, True)
        return xs, xa

    def _pair_sums(self, ev, motion, xs, xa, anchors):
        raise NotImplementedError

    def _check_motion(self, motion):
        pass

    def _terms(self, ev: EventPacket, motion, anchors: Optional[torch.Tensor] = None):
        """(S, window counts, visible fraction or None, eps) of the given or the drawn anchors."""
        self._check_motion(motion)
        if anchors is None:
            anchors = self._anchors(ev)
        xs, xa = self._noise(ev, anchors)
        S = self._pair_sums(ev, motion, xs, xa, anchors)
        ta = ev.t if anchors is None else ev.t[anchors]
        ba = ev.b if anchors is None else ev.b[anchors]
        wc = window_counts(ev.t, ev.b, anchors, self.tau, assume_sorted=ev.meta.get("sorted"))
        vis = visible_fraction(motion, xa.detach(), ta, ba, ev, self.tau) if self.visibility else None
        return (S, wc, vis, self.eps_frac / (ev.height * ev.width)), anchors

    def log_scores(self, ev: EventPacket, motion, anchors: Optional[torch.Tensor] = None):
        """Per-anchor log predictive densities log(eps + S / (W 2 pi h^2)) and the anchor indices
        (atl/objectives/ats.py:75-96)."""
        with layout_scope():          # the motion's field is sampled at the sources and at the anchors
            (S, wc, vis, eps), anchors = self._terms(ev, motion, anchors)
        if anchors is None:
            anchors = torch.arange(ev.n, device=ev.device)
        if ev.xy.is_cuda:
            return anchored_log_scores(S, wc, vis, self.h, eps), anchors
        Wn = wc.clamp(min=1) if vis is None else wc.clamp(min=1) * vis
        return torch.log(eps + S / (Wn * 2 * math.pi * self.h ** 2)), anchors

    def __call__(self, ev, motion):
        if ev.xy.is_cuda:                  # epilogue, mean and negation in one launch
            with layout_scope():
                (S, wc, vis, eps), _ = self._terms(ev, motion)
            loss, score = anchored_score_mean(S, wc, vis, self.h, eps)
            return {"loss": loss, "score": score}
        s = self.log_scores(ev, motion)[0].mean()
        return {"loss": -s, "score": s.detach()}


# --------------------------------------------------------------------------------------------- objectives
class AnchoredExact(_Anchored):
    """Anchored score with the exact pair sums for motion linear at the event (atl/objectives/ats.py:60-105);
    same constructor, plus ``rng`` ("cpu": the reference's CPU-generator noise; "device": drawn on the GPU)."""
    name = "ats_exact"

    def __init__(self, h: float = 1.0, tau: float = 1.0, eps_frac: float = 1e-2, n_anchors: Optional[int] = 20000,
                 n_slices: int = 16, cut: float = 3.0, seed: Optional[int] = None, smooth_anchors: bool = True,
                 dequantize: bool = True, visibility: bool = True, anchor_margin: float = 0.0, rng: str = "cpu"):
        super().__init__(h, tau, eps_frac, n_anchors, n_slices, cut, seed, smooth_anchors, dequantize, visibility,
                         anchor_margin, rng)

    def _check_motion(self, motion):
        if not getattr(motion, "linear_at_event", False):
            raise ValueError("AnchoredExact needs a motion that is linear at the event (use AnchoredTrajectories "
                             "for trajectories)")

    def _pair_sums(self, ev, motion, xs, xa, anchors):
        from ..motion import DenseLinearFlow
        if ev.xy.is_cuda and type(motion) is DenseLinearFlow:   # the flow's gradient straight from the pair sums
            return ats_pair_sums_flow(motion.grid, xs, ev.t, ev.b, ev.batch_size, ev.height, ev.width, anchors,
                                      self.h, self.tau, self.cut, self.n_slices, anchor_xy=xa)
        v = motion.velocity(xs, ev.t, ev.b)
        return ats_pair_sums(xs, ev.t, v, ev.b, ev.batch_size, ev.height, ev.width, anchors, self.h, self.tau,
                             self.cut, self.n_slices, anchor_xy=xa)


class AnchoredTrajectories(_Anchored):
    """Anchored score for PixelTrajectories.  Each source j is put on its trajectory (start p_j by the model's
    fixed-point inversion at (xs_j, t_j), coefficients looked up at p_j); seen from anchor i of slice s it sits
    at q_j(c_s) + q_j'(c_s) (t_i - c_s), its trajectory linearised at the slice centre (|t_i - c_s| <= 1 / 2S).
    Straight trajectories (K = 1, or control points on a line) give AnchoredExact's sums.  The gradient reaches
    the coefficient grid through the pair sums, the coefficient look-up and the inversion.  Same constructor
    as AnchoredExact."""
    name = "ats_trajectories"

    def __init__(self, h: float = 1.0, tau: float = 1.0, eps_frac: float = 1e-2, n_anchors: Optional[int] = 20000,
                 n_slices: int = 16, cut: float = 3.0, seed: Optional[int] = None, smooth_anchors: bool = True,
                 dequantize: bool = True, visibility: bool = True, anchor_margin: float = 0.0, rng: str = "cpu"):
        super().__init__(h, tau, eps_frac, n_anchors, n_slices, cut, seed, smooth_anchors, dequantize, visibility,
                         anchor_margin, rng)

    def _check_motion(self, motion):
        if not (hasattr(motion, "origin") and hasattr(motion, "coeff_rows") and hasattr(motion, "slice_tables")):
            raise ValueError("AnchoredTrajectories needs a trajectory motion (PixelTrajectories)")

    def _pair_sums(self, ev, motion, xs, xa, anchors):
        start = motion.origin(xs, ev.t, ev.b)
        coef = motion.coeff_rows(start, ev.b)
        table = motion.slice_tables(self.n_slices, ev.device)
        return ats_pair_sums_traj(start, coef, ev.t, ev.b, ev.batch_size, ev.height, ev.width, anchors, self.h,
                                  self.tau, self.cut, self.n_slices, anchor_xy=xa, K=motion.K, table=table)
