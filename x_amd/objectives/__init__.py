"""Callers of the hot path: the anchored transport scores and the image-of-warped-events builder."""
from .ats import AnchoredExact, AnchoredTrajectories, visible_fraction
from .base import IWEConfig, Objective, iwe_at_events, iwe_variance, make_iwe, sobel
from .mpcm import MotionPriorCMaxLoss, charbonnier_tv, knn_indices

__all__ = ["AnchoredExact", "AnchoredTrajectories", "visible_fraction", "IWEConfig", "Objective", "make_iwe", "iwe_at_events",
           "iwe_variance", "sobel", "MotionPriorCMaxLoss", "charbonnier_tv", "knn_indices"]
