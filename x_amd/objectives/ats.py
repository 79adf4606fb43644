"""Anchored transport score (atl/objectives/ats.py:1-105).

    S(theta) = mean_i log(eps + rho_{-i}(x_i)),
    rho_{-i}(x) = (1 / W_i) sum_{j != i, |t_i - t_j| <= tau} K_h(x - (x_j + v_j (t_i - t_j)))

Every raw event (anchor) is scored by the Gaussian density of all other events transported to its own
timestamp, with leave-one-out, dequantisation jitter of the sources, smoothed anchors and an exposure
correction.  On device the whole chain runs on HIP kernels: flow lookup, pair sums, window counts,
visible fraction and the log-score epilogue.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from ..core.events import EventPacket
from ..ops import anchored_log_scores, ats_pair_sums, visible_fraction_linear, window_counts
from .base import Objective


@torch.no_grad()
def visible_fraction(motion, xa, ta, ba, ev: EventPacket, tau: float, n_check: int = 16) -> torch.Tensor:
    """Fraction of the sources within +-tau of each anchor recorded while the anchor's scene content was inside
    the field of view (atl/objectives/ats.py:31-50)."""
    if xa.is_cuda and getattr(motion, "linear_at_event", False):
        with torch.no_grad():
            va = motion.velocity(xa, ta, ba)
        return visible_fraction_linear(xa, va, ta, ba, ev.t, ev.b, ev.batch_size, ev.height, ev.width, tau, n_check)
    edges = torch.linspace(0, 1, n_check + 1, device=ev.device)
    centres = 0.5 * (edges[:-1] + edges[1:])
    sl = torch.clamp((ev.t * n_check).long(), 0, n_check - 1)
    counts = torch.zeros(ev.batch_size, n_check, device=ev.device)
    counts.index_put_((ev.b, sl), torch.ones_like(ev.t), accumulate=True)
    vis = torch.zeros_like(ta)
    tot = torch.zeros_like(ta)
    for k in range(n_check):
        c = float(centres[k])
        near = ((ta - c).abs() <= tau).to(ta.dtype)
        y = motion.transport(xa, ta, c, ba)
        inside = ((y[:, 0] >= 0) & (y[:, 0] <= ev.width - 1) & (y[:, 1] >= 0) & (y[:, 1] <= ev.height - 1)).to(ta.dtype)
        w = counts[ba, k] * near
        vis += w * inside
        tot += w
    return (vis / tot.clamp(min=1)).clamp(min=1e-3)


def _pick_anchors(ev: EventPacket, n_anchors: Optional[int], gen: Optional[torch.Generator]) -> torch.Tensor:
    if n_anchors is None or n_anchors >= ev.n:
        return torch.arange(ev.n, device=ev.device)
    idx = torch.randperm(ev.n, generator=gen, device="cpu")[:n_anchors].to(ev.device)
    return torch.sort(idx).values


class AnchoredExact(Objective):
    """Anchored transport score with the exact pair sums (motion must be linear at the event).

    Same constructor as atl/objectives/ats.py:65-73, plus ``rng``: ``"cpu"`` draws the dequantisation and
    smoothing noise from a CPU ``torch.Generator`` exactly like the reference (then copies it to the device);
    ``"device"`` draws it on the device (no host round trip; different random numbers for the same seed)."""
    name = "ats_exact"
    reference_frame = False

    def __init__(self, h: float = 1.0, tau: float = 1.0, eps_frac: float = 1e-2, n_anchors: Optional[int] = 20000,
                 n_slices: int = 16, cut: float = 3.0, seed: Optional[int] = None, smooth_anchors: bool = True,
                 dequantize: bool = True, visibility: bool = True, anchor_margin: float = 0.0, rng: str = "cpu"):
        self.visibility, self.anchor_margin = visibility, anchor_margin
        self.h, self.tau, self.eps_frac, self.n_anchors, self.n_slices, self.cut = h, tau, eps_frac, n_anchors, n_slices, cut
        self.smooth_anchors, self.dequantize = smooth_anchors, dequantize
        self.seed, self.rng = seed, rng
        self.gen = torch.Generator().manual_seed(seed) if seed is not None else None
        self._dgen = None

    def _noise(self, shape, like: torch.Tensor, kind: str) -> torch.Tensor:
        if self.rng == "device" and like.is_cuda:
            if self._dgen is None:
                self._dgen = torch.Generator(device=like.device)
                self._dgen.manual_seed(self.seed if self.seed is not None else torch.seed())
            f = torch.rand if kind == "uniform" else torch.randn
            return f(shape, generator=self._dgen, device=like.device, dtype=like.dtype)
        f = torch.rand if kind == "uniform" else torch.randn
        return f(shape, generator=self.gen).to(like)

    def log_scores(self, ev: EventPacket, motion, anchors: Optional[torch.Tensor] = None):
        """Per-anchor log predictive densities and the anchor indices (atl/objectives/ats.py:75-96)."""
        if not getattr(motion, "linear_at_event", False):
            raise ValueError("AnchoredExact needs a motion that is linear at the event")
        if anchors is None:
            anchors = _pick_anchors(ev, self.n_anchors, self.gen)
            if self.anchor_margin > 0:
                anchors = anchors[ev.inside(ev.xy[anchors], margin=-self.anchor_margin)]
        xs = ev.xy
        if self.dequantize:
            xs = xs + (self._noise(xs.shape, xs, "uniform") - 0.5)
        xa = xs[anchors]
        if self.smooth_anchors:
            xa = xa + self.h * self._noise(xa.shape, xa, "normal")
        v = motion.velocity(xs, ev.t, ev.b)
        S = ats_pair_sums(xs, ev.t, v, ev.b, ev.batch_size, ev.height, ev.width, anchors, self.h, self.tau,
                          self.cut, self.n_slices, anchor_xy=xa)
        eps = self.eps_frac / (ev.height * ev.width)
        if ev.xy.is_cuda:
            wc = window_counts(ev.t, ev.b, anchors, self.tau, assume_sorted=ev.meta.get("sorted"))
            vis = (visible_fraction(motion, xa.detach(), ev.t[anchors], ev.b[anchors], ev, self.tau)
                   if self.visibility else None)
            return anchored_log_scores(S, wc, vis, self.h, eps), anchors
        Wn = window_counts(ev.t, ev.b, anchors, self.tau).clamp(min=1)
        if self.visibility:
            Wn = Wn * visible_fraction(motion, xa.detach(), ev.t[anchors], ev.b[anchors], ev, self.tau)
        return torch.log(eps + S / (Wn * 2 * math.pi * self.h ** 2)), anchors

    def set_bandwidth(self, h: float):
        self.h = float(h)

    def __call__(self, ev, motion):
        ls, _ = self.log_scores(ev, motion)
        s = ls.mean()
        return {"loss": -s, "score": s.detach()}
