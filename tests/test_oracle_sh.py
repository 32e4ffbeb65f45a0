"""Pins oracle/sh.py against the reference test's polynomial and SH orthonormality."""

import math

import numpy as np
import pytest
import torch

from oracle.sh import sh_basis, sh_colors


def polynomial_sh(degree, coefficients, d):
    """Real SH expanded as polynomials with the constants printed in the
    reference's SH test (tests/test_spherical_harmonics.py:10-69)."""
    x, y, z = d[..., 0:1], d[..., 1:2], d[..., 2:3]
    c = coefficients
    out = 0.28209479177387814 * c[..., 0, :] + 0 * x  # broadcast over cameras
    if degree >= 1:
        k = 0.4886025119029199
        out = out - k * y * c[..., 1, :] + k * z * c[..., 2, :] - k * x * c[..., 3, :]
    if degree >= 2:
        out = out + 1.0925484305920792 * (x * y) * c[..., 4, :]
        out = out - 1.0925484305920792 * (y * z) * c[..., 5, :]
        out = out + 0.31539156525252005 * (2 * z * z - x * x - y * y) * c[..., 6, :]
        out = out - 1.0925484305920792 * (x * z) * c[..., 7, :]
        out = out + 0.5462742152960396 * (x * x - y * y) * c[..., 8, :]
    if degree >= 3:
        out = out - 0.5900435899266435 * y * (3 * x * x - y * y) * c[..., 9, :]
        out = out + 2.890611442640554 * (x * y * z) * c[..., 10, :]
        out = out - 0.4570457994644658 * y * (4 * z * z - x * x - y * y) * c[..., 11, :]
        out = out + 0.3731763325901154 * z * (2 * z * z - 3 * x * x - 3 * y * y) * c[..., 12, :]
        out = out - 0.4570457994644658 * x * (4 * z * z - x * x - y * y) * c[..., 13, :]
        out = out + 1.445305721320277 * z * (x * x - y * y) * c[..., 14, :]
        out = out - 0.5900435899266435 * x * (x * x - 3 * y * y) * c[..., 15, :]
    return (out + 0.5).clamp_min(0.0)


@pytest.mark.parametrize("degree", [0, 1, 2, 3])
@pytest.mark.parametrize("cameras", [1, 3])
def test_matches_reference_polynomials(degree, cameras):
    g = torch.Generator().manual_seed(31)
    k = (degree + 1) ** 2
    first = torch.randn(2, 7, k, 3, generator=g, dtype=torch.float64)
    second = torch.randn(2, 7, k, 3, generator=g, dtype=torch.float64)
    d = torch.randn(2, cameras, 7, 3, generator=g, dtype=torch.float64)
    d = d / d.norm(dim=-1, keepdim=True)
    actual = sh_colors(first, second, d, degree)
    expected = torch.cat([polynomial_sh(degree, c[:, None], d) for c in (first, second)], -1)
    torch.testing.assert_close(actual, expected, atol=1e-13, rtol=0)


def test_basis_is_orthonormal_on_the_sphere():
    # Gauss-Legendre in cos(theta) x uniform phi integrates degree <= 6 exactly.
    nodes, weights = np.polynomial.legendre.leggauss(8)
    phi = np.arange(16) * (2 * np.pi / 16)
    ct, ph = np.meshgrid(nodes, phi, indexing="ij")
    st = np.sqrt(1 - ct**2)
    d = torch.tensor(np.stack([st * np.cos(ph), st * np.sin(ph), ct], -1))
    w = torch.tensor(np.repeat(weights[:, None], 16, 1) * (2 * np.pi / 16))
    Y = sh_basis(d, 3)                                       # [8,16,16]
    gram = torch.einsum("ab,abi,abj->ij", w, Y, Y)
    torch.testing.assert_close(gram, torch.eye(16, dtype=torch.float64), atol=1e-12, rtol=0)


def test_degree_zero_closed_form_and_clamp():
    c = torch.tensor([[[[2.0, -3.0, 0.1]]]], dtype=torch.float64, requires_grad=True)
    d = torch.tensor([[[[0.0, 0.0, 1.0]]]], dtype=torch.float64)
    out = sh_colors(c, c, d, 0)
    raw = 0.5 / math.sqrt(math.pi) * c.detach()[0, 0, 0] + 0.5
    expected = raw.clamp_min(0).repeat(2)
    torch.testing.assert_close(out[0, 0, 0], expected)
    out.sum().backward()
    # The clamped (negative) channel gets no gradient.
    assert c.grad[0, 0, 0, 1] == 0 and c.grad[0, 0, 0, 0] > 0
