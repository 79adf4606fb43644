"""Anchored transport score (atl/objectives/ats.py:1-200).

    S(theta) = mean_i log(eps + rho_{-i}(x_i)),
    rho_{-i}(x) = (1 / W_i) sum_{j != i, |t_i - t_j| <= tau} K_h(x - (x_j + v_j (t_i - t_j)))

Every raw event (anchor) is scored by the Gaussian density of all other events transported to its own
timestamp, with leave-one-out, dequantisation jitter of the sources, smoothed anchors and an exposure
correction.  On device the whole chain runs on HIP kernels: flow lookup, pair sums, window counts,
visible fraction and the log-score epilogue.

* :class:`AnchoredExact`: exact pair sums, for motion that is linear at the event.
* :class:`AnchoredSliced`: any motion (e.g. pixel trajectories).  The anchors of time slice s are scored
  against a Gaussian splat of all sources transported to the slice centre c_s, at the anchors moved from their
  own time to c_s, plus the exact log|det| of that small step.
"""
from __future__ import annotations

import math
import os
from typing import Optional

import torch

from ..core.events import EventPacket
from ..ops import (anchored_log_scores, anchored_score_mean, ats_pair_sums, event_noise, gather, splat,
                   visible_fraction_linear, window_counts)
from .base import Objective


@torch.no_grad()
def visible_fraction(motion, xa, ta, ba, ev: EventPacket, tau: float, n_check: int = 16) -> torch.Tensor:
    """Fraction of the sources within +-tau of each anchor recorded while the anchor's scene content was inside
    the field of view (atl/objectives/ats.py:31-50)."""
    if xa.is_cuda and getattr(motion, "linear_at_event", False):
        with torch.no_grad():
            va = motion.velocity(xa, ta, ba)
        return visible_fraction_linear(xa, va, ta, ba, ev.t, ev.b, ev.batch_size, ev.height, ev.width, tau, n_check,
                                       assume_sorted=bool(ev.meta.get("sorted")))
    edges = torch.linspace(0, 1, n_check + 1, device=ev.device)
    centres = 0.5 * (edges[:-1] + edges[1:])
    sl = torch.clamp((ev.t * n_check).long(), 0, n_check - 1)
    counts = torch.zeros(ev.batch_size, n_check, device=ev.device)
    counts.index_put_((ev.b, sl), torch.ones_like(ev.t), accumulate=True)
    vis = torch.zeros_like(ta)
    tot = torch.zeros_like(ta)
    for k, c in enumerate(centres.tolist()):     # one host transfer for the bin centres
        near = ((ta - c).abs() <= tau).to(ta.dtype)
        y = motion.transport(xa, ta, c, ba)
        inside = ((y[:, 0] >= 0) & (y[:, 0] <= ev.width - 1) & (y[:, 1] >= 0) & (y[:, 1] <= ev.height - 1)).to(ta.dtype)
        w = counts[ba, k] * near
        vis += w * inside
        tot += w
    return (vis / tot.clamp(min=1)).clamp(min=1e-3)


def _pick_anchors(ev: EventPacket, n_anchors: Optional[int], gen: Optional[torch.Generator]):
    """Anchor indices, or None for every event in order (no index array is then built or gathered through)."""
    if n_anchors is None or n_anchors >= ev.n:
        return None
    idx = torch.randperm(ev.n, generator=gen, device="cpu")[:n_anchors].to(ev.device)
    return torch.sort(idx).values


class AnchoredExact(Objective):
    """Anchored transport score with the exact pair sums (motion must be linear at the event).

    Same constructor as atl/objectives/ats.py:65-73, plus ``rng``: ``"cpu"`` draws the dequantisation and
    smoothing noise from a CPU ``torch.Generator`` exactly like the reference (then copies it to the device);
    ``"device"`` draws it on the device (no host round trip; different random numbers for the same seed); with
    every event as anchor both draws and both adds are one pass (``event_noise``, Philox4x32-10)."""
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
        self._dseed, self._draws = None, 0          # fused device noise: Philox key and call counter

    def _noise(self, shape, like: torch.Tensor, kind: str, scale: float = 1.0) -> torch.Tensor:
        """Dequantisation noise U(-1/2, 1/2) (kind "uniform") or smoothing noise N(0, scale^2) ("normal").  From
        the CPU generator the reference's ops are kept (rand - 0.5, scale * randn); on the device each draw is
        one in-place fill of the target distribution."""
        if self.rng == "device" and like.is_cuda:
            if self._dgen is None:
                self._dgen = torch.Generator(device=like.device)
                self._dgen.manual_seed(self.seed if self.seed is not None else torch.seed())
            out = torch.empty(shape, device=like.device, dtype=like.dtype)
            if kind == "uniform":
                return out.uniform_(-0.5, 0.5, generator=self._dgen)
            return out.normal_(0.0, scale, generator=self._dgen)
        if kind == "uniform":
            return torch.rand(shape, generator=self.gen).to(like) - 0.5
        return scale * torch.randn(shape, generator=self.gen).to(like)

    def _device_seed(self) -> int:
        if self._dseed is None:
            self._dseed = self.seed if self.seed is not None else int.from_bytes(os.urandom(8), "little")
        return self._dseed

    def log_scores(self, ev: EventPacket, motion, anchors: Optional[torch.Tensor] = None):
        """Per-anchor log predictive densities and the anchor indices (atl/objectives/ats.py:75-96)."""
        parts, anchors = self._terms(ev, motion, anchors)
        if anchors is None:
            anchors = torch.arange(ev.n, device=ev.device)
        if ev.xy.is_cuda:
            S, wc, vis, eps = parts
            return anchored_log_scores(S, wc, vis, self.h, eps), anchors
        return parts, anchors

    def _terms(self, ev: EventPacket, motion, anchors: Optional[torch.Tensor] = None):
        """On device: (S, window counts, visible fraction or None, eps) for the epilogue; on the CPU the log
        scores themselves."""
        if not getattr(motion, "linear_at_event", False):
            raise ValueError("AnchoredExact needs a motion that is linear at the event")
        if anchors is None:
            anchors = _pick_anchors(ev, self.n_anchors, self.gen)
            if self.anchor_margin > 0:
                if anchors is None:
                    anchors = torch.arange(ev.n, device=ev.device)
                anchors = anchors[ev.inside(ev.xy[anchors], margin=-self.anchor_margin)]
        pick = (lambda a: a) if anchors is None else (lambda a: a[anchors])   # None: every event, in order
        xs = ev.xy
        if (self.rng == "device" and xs.is_cuda and anchors is None and not xs.requires_grad
                and (self.dequantize or self.smooth_anchors)):
            # both draws and both adds in one pass over the events
            xs, xa = event_noise(xs, self._device_seed(), self._draws, self.h, self.dequantize, self.smooth_anchors)
            self._draws += 1
            xa = xs if xa is None else xa
        else:
            if self.dequantize:
                xs = xs + self._noise(xs.shape, xs, "uniform")
            xa = pick(xs)
            if self.smooth_anchors:
                xa = xa + self._noise(xa.shape, xa, "normal", self.h)
        v = motion.velocity(xs, ev.t, ev.b)
        S = ats_pair_sums(xs, ev.t, v, ev.b, ev.batch_size, ev.height, ev.width, anchors, self.h, self.tau,
                          self.cut, self.n_slices, anchor_xy=xa)
        eps = self.eps_frac / (ev.height * ev.width)
        if ev.xy.is_cuda:
            wc = window_counts(ev.t, ev.b, anchors, self.tau, assume_sorted=ev.meta.get("sorted"))
            vis = (visible_fraction(motion, xa.detach(), pick(ev.t), pick(ev.b), ev, self.tau)
                   if self.visibility else None)
            return (S, wc, vis, eps), anchors
        Wn = window_counts(ev.t, ev.b, anchors, self.tau).clamp(min=1)
        if self.visibility:
            Wn = Wn * visible_fraction(motion, xa.detach(), pick(ev.t), pick(ev.b), ev, self.tau)
        return torch.log(eps + S / (Wn * 2 * math.pi * self.h ** 2)), anchors

    def set_bandwidth(self, h: float):
        self.h = float(h)

    def __call__(self, ev, motion):
        parts, _ = self._terms(ev, motion)
        if ev.xy.is_cuda:                          # epilogue, mean and negation in one launch
            loss, score = anchored_score_mean(*parts[:3], self.h, parts[3])
            return {"loss": loss, "score": score}
        s = parts.mean()
        return {"loss": -s, "score": s.detach()}


def _noise_from(gen, dgen_holder, rng, seed, shape, like, kind):
    """Dequantisation / smoothing noise: from a CPU generator as the reference draws it (``rng="cpu"``), or
    drawn on the device (``"device"``: no host round trip, other numbers for the same seed)."""
    f = torch.rand if kind == "uniform" else torch.randn
    if rng == "device" and like.is_cuda:
        if dgen_holder[0] is None:
            dgen_holder[0] = torch.Generator(device=like.device)
            dgen_holder[0].manual_seed(seed if seed is not None else torch.seed())
        return f(shape, generator=dgen_holder[0], device=like.device, dtype=like.dtype)
    return f(shape, generator=gen).to(like)


def _splat_value_at(a: torch.Tensor, y: torch.Tensor, sigma: float, H: int, W: int, truncate: bool) -> torch.Tensor:
    """Bilinear look-up at ``a`` of one event's own Gaussian splat centred at ``y`` (normalised by 2 pi sigma^2;
    with ``truncate``, zero beyond the splat's radius ceil(3 sigma) around round(y), as the splat kernel)."""
    R = int(math.ceil(3 * sigma))
    x0, y0 = torch.floor(a[:, 0]), torch.floor(a[:, 1])
    ax, ay = a[:, 0] - x0, a[:, 1] - y0
    cx, cy = torch.round(y[:, 0]), torch.round(y[:, 1])
    norm = 1.0 / (2 * math.pi * sigma * sigma)
    s = torch.zeros_like(ax)
    for dy, wy in ((0, 1 - ay), (1, ay)):
        for dx, wx in ((0, 1 - ax), (1, ax)):
            px, py = x0 + dx, y0 + dy
            ok = (px >= 0) & (px < W) & (py >= 0) & (py < H)
            if truncate:
                ok = ok & ((px - cx).abs() <= R) & ((py - cy).abs() <= R)
            d2 = (px - y[:, 0]) ** 2 + (py - y[:, 1]) ** 2
            s = s + wx * wy * ok.to(a.dtype) * norm * torch.exp(-d2 / (2 * sigma * sigma))
    return s


def cross_term(a, y, sigma, H, W):
    """The anchor's own source copy at y, seen from the moved anchor a (atl/objectives/ats.py:186-202)."""
    return _splat_value_at(a, y, sigma, H, W, truncate=True)


def self_term(y, sigma, H, W):
    """An event's own splat at its own position (atl/objectives/cmax.py:125-137)."""
    return _splat_value_at(y, y, sigma, H, W, truncate=False)


class AnchoredSliced(Objective):
    """Anchored transport score for any motion model (atl/objectives/ats.py:108-183): per time slice, a
    Gaussian splat of the sources transported to the slice centre, looked up at the anchors moved to it, with
    the log|det| of the move, leave-one-out by subtracting the anchor's own splat, and the exposure correction.
    Same constructor, plus ``rng`` as in :class:`AnchoredExact`."""
    name = "ats_sliced"
    reference_frame = False

    def __init__(self, n_slices: int = 10, slices_per_step: Optional[int] = None, sigma: float = 1.0,
                 tau: float = 1.0, eps_frac: float = 1e-2, n_anchors_per_slice: Optional[int] = None,
                 logdet: bool = True, seed: Optional[int] = None, smooth_anchors: bool = True,
                 dequantize: bool = True, visibility: bool = True, rng: str = "cpu"):
        self.S, self.sps, self.sigma, self.tau, self.eps_frac = n_slices, slices_per_step, sigma, tau, eps_frac
        self.nap, self.logdet = n_anchors_per_slice, logdet
        self.smooth_anchors, self.dequantize, self.visibility = smooth_anchors, dequantize, visibility
        self.seed, self.rng = seed, rng
        self.gen = torch.Generator().manual_seed(seed) if seed is not None else None
        self._dgen = [None]

    def log_scores(self, ev: EventPacket, motion, anchor_mask: Optional[torch.Tensor] = None,
                   source_mask: Optional[torch.Tensor] = None):
        """Per-anchor log predictive densities over the scored slices, and the anchor indices."""
        S = self.S
        delta = 1.0 / S
        slice_of = torch.clamp(torch.floor(ev.t / delta), 0, S - 1).long()
        slices = list(range(S))
        if self.sps is not None and self.sps < S:
            slices = torch.randperm(S, generator=self.gen)[: self.sps].tolist()
        eps = self.eps_frac / (ev.height * ev.width)
        noise = lambda shape, like, kind: _noise_from(self.gen, self._dgen, self.rng, self.seed, shape, like, kind)
        xs = ev.xy
        if self.dequantize:
            xs = xs + (noise(xs.shape, xs, "uniform") - 0.5)
        xsm = xs + self.sigma * noise(xs.shape, xs, "normal") if self.smooth_anchors else xs
        if self.nap is None:
            return self._scores_all_slices(ev, motion, xs, xsm, slices, slice_of, delta, eps, anchor_mask,
                                           source_mask)
        scores, picked = [], []
        for s in slices:
            c = (s + 0.5) * delta
            src = (ev.t - c).abs() <= self.tau + delta / 2
            if source_mask is not None:
                src = src & source_mask
            anc = slice_of == s
            if anchor_mask is not None:
                anc = anc & anchor_mask
            ai = torch.nonzero(anc).squeeze(1)
            if ai.numel() == 0:
                continue
            if self.nap is not None and ai.numel() > self.nap:
                ai = ai[torch.randperm(ai.numel(), generator=self.gen)[: self.nap].to(ai.device)]
            si = torch.nonzero(src).squeeze(1)
            y = motion.transport(xs[si], ev.t[si], c, ev.b[si])
            img = splat(y, torch.ones_like(ev.t[si]), ev.b[si], ev.batch_size, ev.height, ev.width, kernel="gauss",
                        sigma=self.sigma)
            if self.logdet:
                a, ld = motion.transport_logdet(xsm[ai], ev.t[ai], c, ev.b[ai])
            else:
                a, ld = motion.transport(xsm[ai], ev.t[ai], c, ev.b[ai]), 0.0
            val = gather(img, a, ev.b[ai])
            in_src = src[ai].to(val.dtype)
            if self.smooth_anchors:           # the anchor's own source copy sits at transport(xs_i)
                y_own = motion.transport(xs[ai], ev.t[ai], c, ev.b[ai])
                own = in_src * cross_term(a, y_own, self.sigma, ev.height, ev.width)
            else:
                own = in_src * self_term(a, self.sigma, ev.height, ev.width)
            nsrc = torch.bincount(ev.b[si], minlength=ev.batch_size).to(val.dtype)[ev.b[ai]] - in_src
            if self.visibility:
                nsrc = nsrc * visible_fraction(motion, xsm[ai].detach(), ev.t[ai], ev.b[ai], ev, self.tau)
            rho = (val - own).clamp(min=0) / nsrc.clamp(min=1)
            scores.append(torch.log(eps + rho) + ld)
            picked.append(ai)
        if not scores:
            z = ev.t.new_zeros(0)
            return z, z.long()
        return torch.cat(scores), torch.cat(picked)

    def _scores_all_slices(self, ev, motion, xs, xsm, slices, slice_of, delta, eps, anchor_mask, source_mask):
        """Every scored slice at once: the per-slice terms of the loop in ``log_scores`` (the reference's loop,
        atl/objectives/ats.py:133-176), each computed once over all slices.  Slice j's splats are images
        j*B .. j*B + B - 1 of one splat; the anchors' moves, look-ups, leave-one-out terms and exposure
        correction are elementwise, so they run over every anchor together.  Scores come slice by slice in the
        order of ``slices``, anchors in event order within a slice, as the loop appends them.  (Each slice's
        targets are per-element times, so a motion's transport must accept a tensor ``t_dst``.)"""
        dev, B, H, W = ev.device, ev.batch_size, ev.height, ev.width
        nsl = len(slices)
        # the slice centres in the events' dtype, as the loop's Python-float centre enters each op
        cen = torch.tensor([(s + 0.5) * delta for s in slices], dtype=ev.t.dtype, device=dev)
        src = (ev.t[None, :] - cen[:, None]).abs() <= self.tau + delta / 2          # (slices, N)
        if source_mask is not None:
            src = src & source_mask[None, :]
        slot = torch.full((self.S,), -1, dtype=torch.long, device=dev)
        slot[torch.tensor(slices, dtype=torch.long, device=dev)] = torch.arange(nsl, device=dev)
        aslot = slot[slice_of]
        anc = aslot >= 0
        if anchor_mask is not None:
            anc = anc & anchor_mask
        ai = torch.nonzero(anc).squeeze(1)
        if ai.numel() == 0:
            z = ev.t.new_zeros(0)
            return z, z.long()
        ai = ai[torch.argsort(aslot[ai], stable=True)]                                 # slice-major
        ja = aslot[ai]
        js, si = torch.nonzero(src, as_tuple=True)                                     # slice-major pairs
        y = motion.transport(xs[si], ev.t[si], cen[js], ev.b[si])
        img = splat(y, torch.ones_like(ev.t[si]), js * B + ev.b[si], nsl * B, H, W, kernel="gauss",
                    sigma=self.sigma)
        ca, ta, ba = cen[ja], ev.t[ai], ev.b[ai]
        if self.logdet:
            a, ld = motion.transport_logdet(xsm[ai], ta, ca, ba)
        else:
            a, ld = motion.transport(xsm[ai], ta, ca, ba), 0.0
        ia = ja * B + ba
        val = gather(img, a, ia)
        in_src = src[ja, ai].to(val.dtype)
        if self.smooth_anchors:
            own = in_src * cross_term(a, motion.transport(xs[ai], ta, ca, ba), self.sigma, H, W)
        else:
            own = in_src * self_term(a, self.sigma, H, W)
        nsrc = torch.bincount(js * B + ev.b[si], minlength=nsl * B).to(val.dtype)[ia] - in_src
        if self.visibility:
            nsrc = nsrc * visible_fraction(motion, xsm[ai].detach(), ta, ba, ev, self.tau)
        rho = (val - own).clamp(min=0) / nsrc.clamp(min=1)
        return torch.log(eps + rho) + ld, ai

    def set_bandwidth(self, h: float):
        self.sigma = float(h)

    def __call__(self, ev, motion):
        ls, _ = self.log_scores(ev, motion)
        s = ls.mean() if ls.numel() else ev.t.new_zeros(())
        return {"loss": -s, "score": s.detach()}
