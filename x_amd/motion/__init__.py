"""Motion models on the hot path: where an event at (x, t) is transported at another time."""
from .base import Motion, as_time
from .parametric import DenseLinearFlow, Sim2, Translation, VectorFieldMotion, sample_grid
from .trajectories import PixelTrajectories, basis

__all__ = ["Motion", "as_time", "VectorFieldMotion", "Translation", "Sim2", "DenseLinearFlow", "sample_grid",
           "PixelTrajectories", "basis"]
