"""Callers of the hot path: the anchored transport score and the image-of-warped-events builder."""
from .ats import AnchoredExact, visible_fraction
from .base import IWEConfig, Objective, make_iwe

__all__ = ["AnchoredExact", "visible_fraction", "IWEConfig", "Objective", "make_iwe"]
