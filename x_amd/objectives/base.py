"""Objective interface and the image of warped events (IWE) (atl/objectives/base.py:14-60).

An objective is a callable ``obj(events, motion) -> dict`` whose ``"loss"`` entry is minimised.  The IWE is the
splat of the events transported to a reference time, weighted by the options of :class:`IWEConfig`.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from ..core.events import EventPacket
from ..ops import blur, gather, image_variance, layout_scope, splat, warp_splat_gather


class Objective:
    """Callable ``(events, motion) -> {"loss": ..., diagnostics}``; ``reference_frame`` is True for objectives
    evaluated at warped positions (an IWE at a reference time) and False for the anchored scores, which
    evaluate at raw events."""
    name = "objective"
    reference_frame = True

    def __call__(self, ev: EventPacket, motion) -> dict:
        raise NotImplementedError(f"{type(self).__name__} defines no loss")

    def __repr__(self):
        return f"{type(self).__name__}({self.name})"


@dataclass
class IWEConfig:
    """IWE options (field names and defaults of the reference's config):
    kernel "bilinear" (then a Gaussian blur of width sigma if sigma > 0) or "gauss" (truncated Gaussian splat of
    width sigma); polarity "pooled" or "split" (one image per polarity, batch entries 2b and 2b + 1);
    mask_border drops events transported outside the sensor; scale_by_dt weights each event by
    1 - |t - t_ref| (clamped to [0, 1])."""
    kernel: str = "bilinear"
    sigma: float = 1.0
    polarity: str = "pooled"
    mask_border: bool = True
    scale_by_dt: bool = False


def _iwe_weights(ev: EventPacket, xy_ref: torch.Tensor, t_ref, cfg: IWEConfig,
                 extra_weight: Optional[torch.Tensor]) -> torch.Tensor:
    """Per-event splat weight: the product of the optional extra weight, the time weight and the in-sensor
    mask.  The time weight and the mask carry no gradient."""
    factors = []
    if extra_weight is not None:
        factors.append(extra_weight)
    with torch.no_grad():
        if cfg.scale_by_dt:
            tr = torch.as_tensor(t_ref, dtype=ev.t.dtype, device=ev.device)
            factors.append(1 - (ev.t - tr).abs().clamp(0, 1))
        if cfg.mask_border:
            factors.append(ev.inside(xy_ref).to(ev.t.dtype))
    w = torch.ones_like(ev.t)
    for f in factors:
        w = w * f
    return w


def make_iwe(ev: EventPacket, xy_ref: torch.Tensor, t_ref, cfg: IWEConfig,
             extra_weight: Optional[torch.Tensor] = None) -> torch.Tensor:
    """IWE (B, H, W) of the events at their transported positions ``xy_ref`` (time ``t_ref``), or (2B, H, W)
    with split polarity (atl/objectives/base.py:40-60)."""
    w = _iwe_weights(ev, xy_ref, t_ref, cfg, extra_weight)
    if cfg.polarity == "split":
        b, nb = 2 * ev.b + (ev.p < 0).long(), 2 * ev.batch_size
    elif cfg.polarity == "pooled":
        b, nb = ev.b, ev.batch_size
    else:
        raise ValueError(f"polarity must be 'pooled' or 'split', got {cfg.polarity!r}")
    if cfg.kernel == "gauss":
        return splat(xy_ref, w, b, nb, ev.height, ev.width, kernel="gauss", sigma=cfg.sigma)
    if cfg.kernel != "bilinear":
        raise ValueError(f"kernel must be 'bilinear' or 'gauss', got {cfg.kernel!r}")
    img = splat(xy_ref, w, b, nb, ev.height, ev.width, kernel="bilinear")
    return blur(img, cfg.sigma) if cfg.sigma > 0 else img


def sobel(img: torch.Tensor):
    """Horizontal and vertical Sobel derivatives of a (B, H, W) image, zero padding (atl/objectives/base.py:63-68):
    the x kernel is the outer product of the smoothing [1, 2, 1] (rows) and the difference [-1, 0, 1] (columns),
    the y kernel its transpose."""
    smooth = img.new_tensor([1.0, 2.0, 1.0])
    diff = img.new_tensor([-1.0, 0.0, 1.0])
    kx = torch.outer(smooth, diff)
    k = torch.stack([kx, kx.t()])[:, None]                    # (2, 1, 3, 3): x then y
    g = torch.nn.functional.conv2d(img[:, None], k, padding=1)
    return g[:, 0], g[:, 1]


def iwe_at_events(ev: EventPacket, motion, t_ref: float, cfg: Optional[IWEConfig] = None):
    """The IWE at ``t_ref`` and its bilinear values at the transported events: ``(img, vals)``, both
    differentiable with respect to the motion (the reference composes transport, make_iwe and gather:
    atl/motion/parametric.py:53-56, atl/objectives/base.py:40-60, atl/ops/functional.py:67-87).  A dense flow on
    the device with a plain bilinear IWE (sigma 0, pooled polarity, no time weight) runs the fused
    warp -> splat -> gather launches; anything else composes the three ops."""
    cfg = cfg or IWEConfig(kernel="bilinear", sigma=0.0)
    from ..motion import DenseLinearFlow, Translation
    plain = (ev.device.type == "cuda" and cfg.kernel == "bilinear" and cfg.sigma == 0 and cfg.polarity == "pooled"
             and not cfg.scale_by_dt)
    if plain and isinstance(motion, DenseLinearFlow):
        return warp_splat_gather(motion.grid, ev.xy, ev.t, ev.b, t_ref, ev.height, ev.width, cfg.mask_border)
    if plain and type(motion) is Translation:
        # a translation is the constant field of a one-node grid (B, 2, 1, 1): its bilinear sample is theta_b
        # exactly (weight 1 on the node), so the fused launches give the composed warp's bits
        grid = motion.theta.view(motion.theta.shape[0], 2, 1, 1)
        return warp_splat_gather(grid, ev.xy, ev.t, ev.b, t_ref, ev.height, ev.width, cfg.mask_border)
    xy_ref = motion.transport(ev.xy, ev.t, t_ref, ev.b)
    img = make_iwe(ev, xy_ref, t_ref, cfg)
    return img, gather(img, xy_ref, ev.b)


def iwe_variance(ev: EventPacket, motion, t_ref: float, cfg: Optional[IWEConfig] = None) -> torch.Tensor:
    """Contrast of the IWE at ``t_ref``: its per-image variance over the pixels, averaged over the images (the
    variance metric of the reference's contrast maximisation, atl/objectives/cmax.py:23-25)."""
    cfg = cfg or IWEConfig(kernel="bilinear", sigma=0.0)
    with layout_scope():
        img = make_iwe(ev, motion.transport(ev.xy, ev.t, t_ref, ev.b), t_ref, cfg)
    return image_variance(img).mean()
