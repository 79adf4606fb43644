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

    def flow_field(self, B: int, H: int, W: int, t0: float = 0.0, t1: float = 1.0) -> torch.Tensor:
        """(B, 2, H, W) displacement (x, y) of every pixel transported from t0 to t1
        (atl/motion/base.py:33-43)."""
        params = list(self.parameters())
        dev = params[0].device if params else torch.device("cpu")
        ys, xs = torch.meshgrid(torch.arange(H, device=dev, dtype=torch.float32),
                                torch.arange(W, device=dev, dtype=torch.float32), indexing="ij")
        xy = torch.stack([xs, ys], -1).reshape(1, H * W, 2).expand(B, -1, -1).reshape(-1, 2)
        b = torch.arange(B, device=dev).repeat_interleave(H * W)
        t = torch.full((xy.shape[0],), float(t0), device=dev)
        return (self.transport(xy, t, float(t1), b) - xy).view(B, H, W, 2).permute(0, 3, 1, 2)

    def transport_logdet(self, xy, t, t_dst, b, delta: float = 0.5):
        """Transport and log|det| of its Jacobian in xy, by central differences with step ``delta``
        (atl/motion/base.py:45-52)."""
        y = self.transport(xy, t, t_dst, b)
        dx = xy.new_tensor([delta, 0.0])
        dy = xy.new_tensor([0.0, delta])
        jx = (self.transport(xy + dx, t, t_dst, b) - self.transport(xy - dx, t, t_dst, b)) / (2 * delta)
        jy = (self.transport(xy + dy, t, t_dst, b) - self.transport(xy - dy, t, t_dst, b)) / (2 * delta)
        det = jx[:, 0] * jy[:, 1] - jx[:, 1] * jy[:, 0]
        return y, torch.log(det.abs().clamp(min=1e-12))

    def regulariser_fields(self, B: int, H: int, W: int):
        """Field for smoothness regularisers, or None (atl/motion/base.py:54-56)."""
        return None


def as_time(t_dst, like: torch.Tensor) -> torch.Tensor:
    """Scalar or tensor target time broadcast to ``like`` (atl/motion/base.py:57-61)."""
    if torch.is_tensor(t_dst):
        return t_dst.to(like.dtype).expand_as(like) if t_dst.dim() == 0 else t_dst.to(like.dtype)
    return torch.full_like(like, float(t_dst))
