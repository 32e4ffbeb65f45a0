"""CPU restatement of the renderer's value contracts - TEST INFRASTRUCTURE ONLY.

Follows check_values (reference src/gabor_splatting/rendering.py:88-153):
each tensor finite (:95-96), scales > 0 (:97), opacities in [0, 1]
(:98-100), unit quaternions with tolerance 1e-4/1e-4 (:101-106), view and
intrinsics last rows at torch.isclose defaults (:107-118), positive focal
lengths (:119-124), orthonormal rotations and determinant +1 at 1e-4/1e-4
(:125-138), and for classic appearance nonnegative frequency weights and
magnitudes and weights summing to one (:139-148). Float32 throughout, as in
the reference. Returns the messages of every violated contract in that
order; the reference joins them with "; " into one ValueError.

Pinned in tests/test_oracle_validate.py by known answers: valid scenes pass,
each planted violation yields exactly its own message(s), and inputs a
margin inside and outside every tolerance land on the side the closed-form
bound |x - t| <= atol + rtol |t| puts them.
"""

from __future__ import annotations

import torch

UNIT = dict(atol=1e-4, rtol=1e-4)


def _close(value: torch.Tensor, target, **tolerances) -> bool:
    target = torch.as_tensor(target, dtype=value.dtype)
    return bool(torch.isclose(value, target.expand_as(value), **tolerances).all())


def value_violations(tensors: dict, quaternions, scales, opacities, view_matrices, intrinsics,
                     appearance, neural: bool) -> list[str]:
    """Messages of the violated value contracts, in the reference's order.

    Arguments as the reference's check_values: ``tensors`` maps each input
    name to (tensor, shape); ``appearance`` holds the appearance tensors in
    argument order (classic: colors, secondary colors, frequency weights,
    magnitudes, phases)."""
    messages = [f"{name} must contain only finite values"
                for name, (value, _) in tensors.items() if not bool(torch.isfinite(value).all())]
    rotation = view_matrices[..., :3, :3]
    checks = [
        ("scales must be strictly positive", bool((scales > 0).all())),
        ("opacities must lie in [0, 1]", bool(((opacities >= 0) & (opacities <= 1)).all())),
        ("quaternions must be unit wxyz vectors",
         _close((quaternions * quaternions).sum(-1), 1.0, **UNIT)),
        ("view_matrices must have last row [0, 0, 0, 1]",
         _close(view_matrices[..., 3, :], [0.0, 0.0, 0.0, 1.0])),
        ("intrinsics must have last row [0, 0, 1]",
         _close(intrinsics[..., 2, :], [0.0, 0.0, 1.0])),
        ("intrinsics fx and fy must be positive",
         bool(((intrinsics[..., 0, 0] > 0) & (intrinsics[..., 1, 1] > 0)).all())),
        ("view_matrices rotations must be orthonormal",
         _close(rotation.transpose(-1, -2) @ rotation, torch.eye(3), **UNIT)),
        ("view_matrices rotations must have determinant +1",
         _close(torch.linalg.det(rotation), 1.0, **UNIT)),
    ]
    if not neural:
        weights, magnitudes = appearance[2], appearance[3]
        checks += [
            ("frequency_weights must be nonnegative", bool((weights >= 0).all())),
            ("frequency_magnitudes must be nonnegative", bool((magnitudes >= 0).all())),
            ("frequency_weights must sum to one", _close(weights.sum(-1), 1.0, **UNIT)),
        ]
    return messages + [message for message, ok in checks if not ok]
