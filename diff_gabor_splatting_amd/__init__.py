"""MI355X-native differentiable Gabor-surface rasterization (gfx950 HIP kernels)."""

from .rendering import rasterize_gabors, rasterize_neural_gabors

__all__ = ["rasterize_gabors", "rasterize_neural_gabors"]
