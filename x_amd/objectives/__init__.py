"""Callers of the hot path: the anchored transport scores and the image-of-warped-events builder."""
from .ats import AnchoredExact, AnchoredSliced, cross_term, self_term, visible_fraction
from .base import IWEConfig, Objective, make_iwe

__all__ = ["AnchoredExact", "AnchoredSliced", "cross_term", "self_term", "visible_fraction", "IWEConfig", "Objective",
           "make_iwe"]
