"""MI355X-native differentiable Gabor-surface rasterization (gfx950 HIP kernels).

The public renderers load ``libgabor_hip.so`` on first use (importing the
package alone does not, so ``diff_gabor_splatting_amd.build`` can rebuild a
stale library). There is no CPU fallback: a missing library raises.
"""

__all__ = ["rasterize_gabors", "rasterize_neural_gabors", "fixed_capacity", "single_map_storage"]


def __getattr__(name):
    if name in __all__:
        from . import rendering

        return getattr(rendering, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
