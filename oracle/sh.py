"""Real spherical-harmonic colours (reference: spherical_harmonics.cu:11-85).

Colour = max(0.5 + sum_k Y_k(d) c_k, 0) for both colour sets, with the real
SH basis in the Gaussian-splatting ordering and sign convention. The basis is
written here as products of the Cartesian monomials of each degree.
"""

from __future__ import annotations

import math

import torch

# Normalisation constants sqrt((2l+1)/(4 pi) (l-|m|)!/(l+|m|)!) times the
# polynomial factors of each real harmonic.
_C0 = 0.5 / math.sqrt(math.pi)
_C1 = math.sqrt(3.0 / (4.0 * math.pi))
_C2 = (
    0.5 * math.sqrt(15.0 / math.pi),
    0.25 * math.sqrt(5.0 / math.pi),
    0.25 * math.sqrt(15.0 / math.pi),
)
_C3 = (
    0.25 * math.sqrt(35.0 / (2.0 * math.pi)),
    0.5 * math.sqrt(105.0 / math.pi),
    0.25 * math.sqrt(21.0 / (2.0 * math.pi)),
    0.25 * math.sqrt(7.0 / math.pi),
    0.25 * math.sqrt(105.0 / math.pi),
)


def sh_basis(directions: torch.Tensor, degree: int) -> torch.Tensor:
    """Basis values [..., (degree+1)**2] at (not necessarily unit) directions."""
    x, y, z = directions.unbind(-1)
    terms = [torch.full_like(x, _C0)]
    if degree >= 1:
        terms += [-_C1 * y, _C1 * z, -_C1 * x]
    if degree >= 2:
        a, b, c = _C2
        terms += [
            a * x * y,
            -a * y * z,
            b * (2 * z * z - x * x - y * y),
            -a * x * z,
            c * (x * x - y * y),
        ]
    if degree >= 3:
        a, b, c, d, e = _C3
        terms += [
            -a * y * (3 * x * x - y * y),
            b * x * y * z,
            -c * y * (4 * z * z - x * x - y * y),
            d * z * (2 * z * z - 3 * x * x - 3 * y * y),
            -c * x * (4 * z * z - x * x - y * y),
            e * z * (x * x - y * y),
            -a * x * (x * x - 3 * y * y),
        ]
    return torch.stack(terms, -1)


def sh_colors(first: torch.Tensor, second: torch.Tensor, directions: torch.Tensor,
              degree: int) -> torch.Tensor:
    """Both colours [S,C,N,6] from coefficients [S,N,K,3] and directions [S,C,N,3]."""
    basis = sh_basis(directions, degree)                           # [S,C,N,K]
    out = []
    for coefficients in (first, second):
        raw = 0.5 + (basis[..., None] * coefficients[:, None]).sum(-2)  # [S,C,N,3]
        out.append(raw.clamp_min(0.0))
    return torch.cat(out, -1)
