"""Drop-in import name of the reference package, served by the HIP backend.

``import gabor_splatting`` and ``gabor_splatting.rendering`` resolve to the
modules of ``diff_gabor_splatting_amd``, so code (and monkeypatches) written
against the reference's module paths act on the HIP implementation.
"""

import sys

from diff_gabor_splatting_amd import rendering
from diff_gabor_splatting_amd.rendering import rasterize_gabors, rasterize_neural_gabors

sys.modules[__name__ + ".rendering"] = rendering

__all__ = ["rasterize_gabors", "rasterize_neural_gabors"]
