"""Packed event batches: the container every kernel of the path reads (atl/core/events.py:23-120).

A batch of B event windows is stored as flat per-event arrays plus a batch index, sorted by (b, t), so that a
kernel needs no per-window bookkeeping and the events of one window (and of one time range) are contiguous:

    xy (N, 2) float32   column x and row y in pixels (pixel centres at integers)
    t  (N,)   float32   time, normalised to [0, 1] per window
    p  (N,)   float32   polarity +-1
    b  (N,)   int64     window index in [0, batch_size)

``duration`` holds the seconds per window, ``meta`` free-form flags (``"sorted": True`` when the (b, t) order is
known to hold, which lets the device window counts skip their check).
"""
from __future__ import annotations

import dataclasses
from dataclasses import dataclass, field
from typing import Optional, Sequence

import numpy as np
import torch

_PER_EVENT = ("xy", "t", "p", "b")


def _tensor(a, dtype, device) -> torch.Tensor:
    if torch.is_tensor(a):
        return a.to(device=device, dtype=dtype)
    return torch.as_tensor(np.asarray(a), dtype=dtype, device=device)


@dataclass
class EventPacket:
    xy: torch.Tensor
    t: torch.Tensor
    p: torch.Tensor
    b: torch.Tensor
    batch_size: int
    height: int
    width: int
    duration: Optional[torch.Tensor] = None
    meta: dict = field(default_factory=dict)

    # ------------------------------------------------------------------------------------------ builders
    @staticmethod
    def from_arrays(x, y, t, p, height: int, width: int, duration: float | None = None,
                    normalize_time: bool = True, device="cpu") -> "EventPacket":
        """One window from raw arrays (atl/core/events.py:38-54): time rescaled to [0, 1] by its own range (in
        float64, then float32) when ``normalize_time``, events put in time order (stable), polarity mapped to
        +-1 by its sign."""
        tt = _tensor(t, torch.float64, device)
        if normalize_time and tt.numel():
            lo, hi = tt.min(), tt.max()
            tt = (tt - lo) / torch.clamp(hi - lo, min=1e-12)
        tt = tt.to(torch.float32)
        order = torch.argsort(tt, stable=True)
        xy = torch.stack([_tensor(x, torch.float32, device), _tensor(y, torch.float32, device)], 1)
        pol = torch.where(_tensor(p, torch.float32, device) > 0, 1.0, -1.0)
        dur = None if duration is None else torch.tensor([float(duration)], device=device)
        return EventPacket(xy[order], tt[order], pol[order], torch.zeros_like(order), 1, height, width, dur)

    @staticmethod
    def from_window(win, device="cpu") -> "EventPacket":
        """Packet from a :class:`x_amd.synth.Window` (already sorted by (b, t), time already normalised)."""
        return EventPacket(torch.as_tensor(win.xy, device=device), torch.as_tensor(win.t, device=device),
                           torch.as_tensor(win.p, device=device), torch.as_tensor(win.b, device=device),
                           win.batch_size, win.height, win.width,
                           torch.full((win.batch_size,), float(win.duration), device=device), {"sorted": True})

    @staticmethod
    def collate(samples: Sequence["EventPacket"]) -> "EventPacket":
        """Pack single-window packets into one batch; window k of the result is samples[k]
        (atl/core/events.py:57-68).  Windows without a duration count as 1 s."""
        if not samples:
            raise ValueError("collate needs at least one packet")
        first = samples[0]
        for s in samples:
            if s.batch_size != 1 or (s.height, s.width) != (first.height, first.width):
                raise ValueError("collate takes single-window packets of one sensor size")
        sizes = torch.tensor([s.n for s in samples], device=first.device)
        cat = {f: torch.cat([getattr(s, f) for s in samples]) for f in ("xy", "t", "p")}
        b = torch.repeat_interleave(torch.arange(len(samples), device=first.device), sizes)
        dur = torch.cat([s.duration if s.duration is not None else torch.ones(1, device=s.device) for s in samples])
        return EventPacket(cat["xy"], cat["t"], cat["p"], b, len(samples), first.height, first.width, dur)

    # ------------------------------------------------------------------------------------------ views
    @property
    def n(self) -> int:
        return int(self.t.numel())

    @property
    def device(self):
        return self.t.device

    @property
    def offsets(self) -> torch.Tensor:
        """(B + 1,) start of every window's events (the packet is sorted by b) and the total."""
        per = torch.zeros(self.batch_size, dtype=torch.long, device=self.device)
        per.scatter_add_(0, self.b, torch.ones_like(self.b))
        return torch.nn.functional.pad(torch.cumsum(per, 0), (1, 0))

    def _replace(self, **kw) -> "EventPacket":
        return dataclasses.replace(self, meta=dict(kw.pop("meta", self.meta)), **kw)

    def to(self, device) -> "EventPacket":
        moved = {f: getattr(self, f).to(device) for f in _PER_EVENT}
        return self._replace(duration=None if self.duration is None else self.duration.to(device), **moved)

    def select(self, mask_or_index: torch.Tensor) -> "EventPacket":
        """Events kept by a boolean mask (order preserved) or picked by an index (which may reorder them, so the
        "sorted" flag is dropped)."""
        meta = dict(self.meta)
        if mask_or_index.dtype != torch.bool:
            meta.pop("sorted", None)
        return self._replace(meta=meta, **{f: getattr(self, f)[mask_or_index] for f in _PER_EVENT})

    def split(self, frac: float, generator: Optional[torch.Generator] = None):
        """Random (first, second) split: each event joins the first part with probability ``frac`` (uniform
        draws from a CPU generator)."""
        first = torch.rand(self.n, generator=generator, device="cpu").to(self.device) < frac
        return self.select(first), self.select(~first)

    def subsample(self, k: int, generator: Optional[torch.Generator] = None) -> "EventPacket":
        """k events drawn without replacement (a CPU random permutation), kept in their original order."""
        if self.n <= k:
            return self
        pick = torch.randperm(self.n, generator=generator, device="cpu")[:k]
        return self.select(torch.sort(pick).values.to(self.device))

    def inside(self, xy: Optional[torch.Tensor] = None, margin: float = 0.0) -> torch.Tensor:
        """True where a position lies in the sensor [0, W-1] x [0, H-1] grown by ``margin`` px."""
        q = self.xy if xy is None else xy
        lo = -margin
        return ((q[:, 0] >= lo) & (q[:, 0] <= self.width - 1 + margin) &
                (q[:, 1] >= lo) & (q[:, 1] <= self.height - 1 + margin))

    def __repr__(self):
        return (f"EventPacket(n={self.n}, B={self.batch_size}, HxW={self.height}x{self.width}, "
                f"device={self.device})")
