"""CPU parity oracle for the Gabor tile rasterizer - TEST INFRASTRUCTURE ONLY.

This package restates, from scratch and on the CPU, what the reference
rasterizer (luisrodolfo10/diff_gabor_splatting v0.1.1) computes on its hot
path, so the HIP implementation can be checked against it:

  projection.py  rendering.py:156-218 (quaternion rotation, projected plane
                 T, conic centre, extent, facing normal, direction, radii)
  sh.py          spherical_harmonics.cu:11-85 (real SH colours, clamp)
  binning.py     rasterize.cu:24-69 (tile rectangles, counts, keys, stable
                 sort, tile ranges) and rendering.py:362-364 (packing) in
                 numpy with float32 arithmetic for bit-exact integer results
  composite.py   rasterize.cu:71-281 (ray/plane sample, low-pass filter,
                 appearance, front-to-back compositing, early termination),
                 vectorised over tiles; gradients come from torch autograd
  render.py      rendering.py:241-400 (record layout, packing, meta)
  validate.py    rendering.py:88-153 (value contracts and their messages)

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
reported CPU baseline. The product (``diff_gabor_splatting_amd``) never
imports it and has no CPU fallback.

Pinning (each function is checked against an independent formulation in
``tests/test_oracle_*.py``): quaternion rotations against the axis-angle
form and orthonormality; projection against closed forms for fronto-parallel
surfels; SH against the reference test's polynomial form and numerical
orthonormality on the sphere; binning against brute force over every tile;
the compositor against a per-pixel float64 evaluation that solves the ray/
plane system with ``torch.linalg.solve`` (as the reference's own test does),
against closed forms (single opaque surfel, zero opacity, early stop) and
against pairwise distortion; gradients against central finite differences;
the value contracts against planted violations with known answers.
No function is "parity unpinned" except the equal-depth tie order, which the
reference specifies (stable sort by pair index) but none of its tests pins.
"""
