"""Objective interface and the image-of-warped-events builder (atl/objectives/base.py:14-60)."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from ..core.events import EventPacket
from ..ops import blur, splat


class Objective:
    """Callable ``(events, motion) -> {'loss': ...}``; ``loss`` is minimised."""
    name = "objective"
    reference_frame = True

    def __call__(self, ev: EventPacket, motion) -> dict:
        raise NotImplementedError


@dataclass
class IWEConfig:
    kernel: str = "bilinear"            # "bilinear" vote (+ optional Gaussian blur) or "gauss" splat
    sigma: float = 1.0
    polarity: str = "pooled"            # "pooled" | "split"
    mask_border: bool = True
    scale_by_dt: bool = False


def make_iwe(ev: EventPacket, xy_ref: torch.Tensor, t_ref, cfg: IWEConfig,
             extra_weight: Optional[torch.Tensor] = None) -> torch.Tensor:
    """IWE of events transported to ``t_ref``: (B, H, W), or (2B, H, W) with split polarity
    (atl/objectives/base.py:40-60)."""
    w = torch.ones_like(ev.t)
    if extra_weight is not None:
        w = w * extra_weight
    if cfg.scale_by_dt:
        tr = t_ref if torch.is_tensor(t_ref) else torch.tensor(float(t_ref), device=ev.device)
        w = w * (1 - (ev.t - tr).abs().clamp(0, 1)).detach()
    if cfg.mask_border:
        w = w * ev.inside(xy_ref).to(w.dtype).detach()
    b, nb = ev.b, ev.batch_size
    if cfg.polarity == "split":
        b = ev.b * 2 + (ev.p < 0).long()
        nb = 2 * ev.batch_size
    if cfg.kernel == "gauss":
        return splat(xy_ref, w, b, nb, ev.height, ev.width, kernel="gauss", sigma=cfg.sigma)
    img = splat(xy_ref, w, b, nb, ev.height, ev.width, kernel="bilinear")
    return blur(img, cfg.sigma) if cfg.sigma > 0 else img
