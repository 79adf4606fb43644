"""Motion interface (atl/motion/base.py:21-61): ``transport(xy, t, t_dst, b) -> xy'``; models linear at the
event also give ``velocity(xy, t, b)`` and set ``linear_at_event``.  Times are normalised to [0, 1] per
window, velocities are pixels per window."""
from __future__ import annotations

import torch
from torch import nn


class Motion(nn.Module):
    linear_at_event: bool = False

    def transport(self, xy: torch.Tensor, t: torch.Tensor, t_dst, b: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError

    def velocity(self, xy: torch.Tensor, t: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError(f"{type(self).__name__} has no per-event velocity")


def as_time(t_dst, like: torch.Tensor) -> torch.Tensor:
    """Scalar or tensor target time broadcast to ``like`` (atl/motion/base.py:57-61)."""
    if torch.is_tensor(t_dst):
        return t_dst.to(like.dtype).expand_as(like) if t_dst.dim() == 0 else t_dst.to(like.dtype)
    return torch.full_like(like, float(t_dst))
