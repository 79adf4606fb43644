from .events import EventPacket

__all__ = ["EventPacket"]
