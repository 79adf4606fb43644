"""The motion interface the objectives see (atl/motion/base.py:21-61).

A motion maps an event (xy, t) of window b to its position at another time, ``transport(xy, t, t_dst, b)``.
Models linear at the event (x + v (t' - t)) also give the per-event velocity and set ``linear_at_event``,
which the exact pair sums require.  Time is normalised to [0, 1] per window and velocities are pixels per
window.
"""
from __future__ import annotations

import torch
from torch import nn


def as_time(t_dst, like: torch.Tensor) -> torch.Tensor:
    """A target time (a number, a 0-d tensor or one per event) as a tensor shaped and typed like ``like``
    (atl/motion/base.py:57-61)."""
    if not torch.is_tensor(t_dst):
        return torch.full_like(like, float(t_dst))
    t_dst = t_dst.to(like.dtype)
    return t_dst.expand_as(like) if t_dst.dim() == 0 else t_dst


def pixel_events(B: int, H: int, W: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    """Every pixel centre of B windows as events: positions (B*H*W, 2) in (x, y), window by window in row-major
    order, and their window index."""
    rows = torch.arange(H, device=device, dtype=torch.float32)
    cols = torch.arange(W, device=device, dtype=torch.float32)
    xy = torch.cartesian_prod(rows, cols).flip(-1).repeat(B, 1)
    b = torch.arange(B, device=device).repeat_interleave(H * W)
    return xy, b


class Motion(nn.Module):
    linear_at_event: bool = False

    def transport(self, xy: torch.Tensor, t: torch.Tensor, t_dst, b: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError(f"{type(self).__name__} defines no transport")

    def velocity(self, xy: torch.Tensor, t: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        raise NotImplementedError(f"{type(self).__name__} has no per-event velocity")

    def _device(self):
        for prm in self.parameters():
            return prm.device
        return torch.device("cpu")

    def flow_field(self, B: int, H: int, W: int, t0: float = 0.0, t1: float = 1.0) -> torch.Tensor:
        """(B, 2, H, W) displacement (x, y) of every pixel transported from t0 to t1 (atl/motion/base.py:33-43)."""
        xy, b = pixel_events(B, H, W, self._device())
        moved = self.transport(xy, torch.full_like(xy[:, 0], float(t0)), float(t1), b)
        return (moved - xy).view(B, H, W, 2).permute(0, 3, 1, 2)

    def transport_logdet(self, xy, t, t_dst, b, delta: float = 0.5):
        """Transported positions and log|det| of the transport's Jacobian in xy, by central differences of step
        ``delta`` (atl/motion/base.py:45-52); the five evaluations run as one batched transport."""
        n = xy.shape[0]
        steps = xy.new_tensor([[0.0, 0.0], [delta, 0.0], [-delta, 0.0], [0.0, delta], [0.0, -delta]])
        q = self.transport((xy[None] + steps[:, None]).reshape(5 * n, 2), t.repeat(5),
                           as_time(t_dst, t).repeat(5) if torch.is_tensor(t_dst) else t_dst, b.repeat(5))
        q = q.view(5, n, 2)
        jx = (q[1] - q[2]) / (2 * delta)
        jy = (q[3] - q[4]) / (2 * delta)
        det = jx[:, 0] * jy[:, 1] - jx[:, 1] * jy[:, 0]
        return q[0], torch.log(det.abs().clamp(min=1e-12))

    def regulariser_fields(self, B: int, H: int, W: int):
        """The field a smoothness regulariser acts on, or None (atl/motion/base.py:54-56)."""
        return None
