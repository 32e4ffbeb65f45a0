"""Planted violations of the renderer's value contracts, with known answers.

Each case mutates a valid scene from ``scenes.make_inputs`` and names the
messages the reference's check_values (rendering.py:88-153) must report,
worked out from the contract itself: |x - t| <= atol + rtol |t| with
1e-4/1e-4 for norms, sums, orthonormality and determinants and the
torch.isclose defaults (1e-8/1e-5) for the last rows. Boundary cases sit a
clear margin inside or outside each tolerance.
"""

from __future__ import annotations

import math

import torch

from scenes import make_inputs

FINITE = "{} must contain only finite values"
SCALES = "scales must be strictly positive"
OPACITIES = "opacities must lie in [0, 1]"
QUATERNIONS = "quaternions must be unit wxyz vectors"
VIEW_ROW = "view_matrices must have last row [0, 0, 0, 1]"
K_ROW = "intrinsics must have last row [0, 0, 1]"
FOCAL = "intrinsics fx and fy must be positive"
ORTHONORMAL = "view_matrices rotations must be orthonormal"
DETERMINANT = "view_matrices rotations must have determinant +1"
WEIGHTS = "frequency_weights must be nonnegative"
MAGNITUDES = "frequency_magnitudes must be nonnegative"
WEIGHT_SUM = "frequency_weights must sum to one"


def _set(name, index, value):
    def mutate(values):
        values[name][index] = value
    return mutate


def _scale(name, index, factor):
    def mutate(values):
        values[name][index] *= factor
    return mutate


def _all(*mutations):
    def mutate(values):
        for m in mutations:
            m(values)
    return mutate


def _nan_cases(method):
    # (tensor, index, messages besides its own finiteness message for a NaN,
    # and for +inf, which passes the one-sided bounds)
    spots = [
        ("means", (0, 1, 2), [], []),
        ("quaternions", (0, 2, 1), [QUATERNIONS], [QUATERNIONS]),
        ("scales", (0, 0, 1), [SCALES], []),
        ("opacities", (0, 2), [OPACITIES], [OPACITIES]),
        ("view_matrices", (0, 1, 0, 3), [], []),
        ("intrinsics", (0, 0, 0, 2), [], []),
        ("backgrounds", (0, 1, 2), [], []),
    ]
    if method == "classic":
        spots += [
            ("colors", (0, 1, 0), [], []),
            ("secondary_colors", (0, 2, 2), [], []),
            ("frequency_weights", (0, 0, 3), [WEIGHTS, WEIGHT_SUM], [WEIGHT_SUM]),
            ("frequency_magnitudes", (0, 1, 1), [MAGNITUDES], []),
            ("phases", (0, 2, 0), [], []),
        ]
    else:
        spots += [
            ("input_weights", (0, 1, 2, 3), [], []),
            ("input_biases", (0, 0, 5), [], []),
            ("output_weights", (0, 2, 1, 4), [], []),
            ("output_biases", (0, 1, 2), [], []),
        ]
    cases = []
    for name, index, nan_extra, inf_extra in spots:
        cases.append((f"nan-{name}", _set(name, index, math.nan),
                      [FINITE.format(name)] + nan_extra))
        cases.append((f"inf-{name}", _set(name, index, math.inf),
                      [FINITE.format(name)] + inf_extra))
    # A NaN in a rotation entry or focal length also fails the derived contracts.
    cases.append(("nan-rotation", _set("view_matrices", (0, 0, 1, 1), math.nan),
                  [FINITE.format("view_matrices"), ORTHONORMAL, DETERMINANT]))
    cases.append(("nan-focal", _set("intrinsics", (0, 1, 1, 1), math.nan),
                  [FINITE.format("intrinsics"), FOCAL]))
    return cases


def _rotation_scale(factor):
    def mutate(values):
        values["view_matrices"][0, 1, :3, :3] *= factor
    return mutate


def _reflect(values):
    values["view_matrices"][0, 0, :3, 0] *= -1


def _shear(values):
    values["view_matrices"][0, 2, 0, 1] += 1e-3


def _value_cases(method):
    cases = [
        ("valid", lambda values: None, []),
        ("negative-scale", _set("scales", (0, 1, 0), -0.1), [SCALES]),
        ("zero-scale", _set("scales", (0, 2, 1), 0.0), [SCALES]),
        ("opacity-above-one", _set("opacities", (0, 0), 1.01), [OPACITIES]),
        ("opacity-below-zero", _set("opacities", (0, 1), -0.01), [OPACITIES]),
        ("opacity-bounds", _all(_set("opacities", (0, 0), 0.0), _set("opacities", (0, 1), 1.0)),
         []),
        ("quaternion-inside", _scale("quaternions", (0, 1), math.sqrt(1 + 1.5e-4)), []),
        ("quaternion-outside", _scale("quaternions", (0, 1), math.sqrt(1 + 3e-4)),
         [QUATERNIONS]),
        ("view-row-inside", _set("view_matrices", (0, 1, 3, 3), 1 + 5e-6), []),
        ("view-row-outside", _set("view_matrices", (0, 1, 3, 3), 1 + 2e-5), [VIEW_ROW]),
        ("view-row-zero-inside", _set("view_matrices", (0, 0, 3, 0), 5e-9), []),
        ("view-row-zero-outside", _set("view_matrices", (0, 0, 3, 0), 3e-8), [VIEW_ROW]),
        ("k-row-inside", _set("intrinsics", (0, 2, 2, 2), 1 + 5e-6), []),
        ("k-row-outside", _set("intrinsics", (0, 2, 2, 2), 1 + 2e-5), [K_ROW]),
        ("k-row-zero-outside", _set("intrinsics", (0, 0, 2, 1), 3e-8), [K_ROW]),
        ("k-transposed", lambda v: v.__setitem__(
            "intrinsics", v["intrinsics"].transpose(-1, -2).contiguous()), [K_ROW]),
        ("fx-zero", _set("intrinsics", (0, 1, 0, 0), 0.0), [FOCAL]),
        ("fy-negative", _set("intrinsics", (0, 2, 1, 1), -1.0), [FOCAL]),
        ("rotation-inside", _rotation_scale(1 + 3e-5), []),
        ("rotation-outside", _rotation_scale(1 + 2e-4), [ORTHONORMAL, DETERMINANT]),
        ("reflection", _reflect, [DETERMINANT]),
        ("shear", _shear, [ORTHONORMAL]),
        ("several", _all(_set("scales", (0, 0, 0), -1.0), _set("opacities", (0, 2), 2.0),
                         _set("intrinsics", (0, 0, 0, 0), -5.0)),
         [SCALES, OPACITIES, FOCAL]),
    ]
    if method == "classic":
        def negative_weight(values):
            values["frequency_weights"][0, 1] = torch.tensor([-0.1, 0.35, 0.5, 0.25])

        cases += [
            ("negative-weight", negative_weight, [WEIGHTS]),
            ("negative-magnitude", _set("frequency_magnitudes", (0, 2, 3), -0.5), [MAGNITUDES]),
            ("weight-sum-inside", _set("frequency_weights", (0, 0, 0), 0.25 + 1.5e-4), []),
            ("weight-sum-outside", _set("frequency_weights", (0, 0, 0), 0.25 + 3e-4),
             [WEIGHT_SUM]),
        ]
    else:
        # Neural appearance has no frequency contracts: negative values pass.
        cases.append(("neural-negative-weights", _set("input_weights", (0, 0, 0, 0), -3.0), []))
    return cases


def contract_cases(method):
    """(label, mutate(values) in place, expected messages in reference order)."""
    return _nan_cases(method) + _value_cases(method)


def planted_inputs(method, mutate):
    """A valid 1-scene, 3-camera, 3-surfel scene with one mutation applied."""
    values = make_inputs(method, scenes=1, cameras=3, primitives=3)
    mutate(values)
    return values


def check_arguments(values, method):
    """Positional arguments of check_values for a dict of renderer inputs."""
    tensors = {name: (value, tuple(value.shape)) for name, value in values.items()}
    names = (("colors", "secondary_colors", "frequency_weights", "frequency_magnitudes",
              "phases") if method == "classic" else
             ("input_weights", "input_biases", "output_weights", "output_biases"))
    appearance = tuple(values[name] for name in names)
    return (tensors, values["quaternions"], values["scales"], values["opacities"],
            values["view_matrices"], values["intrinsics"], appearance, method == "neural")
