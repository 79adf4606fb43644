"""x_amd: the event-transport hot path of atl (splat, gather, anchored pair sums) on MI355X HIP kernels."""
from . import ops
from .core import EventPacket

__all__ = ["ops", "EventPacket"]
