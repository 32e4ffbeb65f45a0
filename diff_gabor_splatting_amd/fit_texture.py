"""Fit a stripe texture on one surface through the renderer: an end-to-end training loop.

The workload of the reference's example (examples/fit_texture.py:12-72): one
0.7 x 0.7 surface three units in front of a 32 x 32 pinhole camera, whose
classic appearance (colours, magnitudes, phases; frequency weights fixed at
[1, 0, 0, 0]) or SIREN weights are fitted by Adam (lr 0.01) to the stripes
0.5 + 0.4 cos(0.7 x) masked by the rendered alpha, with magnitudes clamped
nonnegative after each classic step. Every step renders forward and backward
through the HIP path.

Initial parameters are drawn on the CPU from a seeded generator, so the same
problem can be handed to any renderer with the public signature (the tests
run it through the float64 oracle as well and compare the loss curves).

    python -m diff_gabor_splatting_amd.fit_texture --method both --steps 100 \\
        --output texture.png
"""

from __future__ import annotations

import argparse
import math
import struct
import zlib
from pathlib import Path

import torch

SIZE = 32


def texture_problem(method: str, device="cuda", dtype=torch.float32, seed: int = 3):
    """(fixed inputs, fitted parameters, target stripes [1, H, W, 3])."""
    gen = torch.Generator().manual_seed(seed)

    def tensor(values):
        return torch.tensor(values, dtype=dtype).to(device)

    fixed = {
        "means": tensor([[0.0, 0.0, 3.0]]),
        "quaternions": tensor([[1.0, 0.0, 0.0, 0.0]]),
        "scales": tensor([[0.7, 0.7]]),
        "opacities": tensor([0.9]),
        "view_matrices": torch.eye(4, dtype=dtype, device=device)[None],
        "intrinsics": tensor([[[40.0, 0.0, 15.5], [0.0, 40.0, 15.5], [0.0, 0.0, 1.0]]]),
    }
    if method == "classic":
        fixed["frequency_weights"] = tensor([[1.0, 0.0, 0.0, 0.0]])
        fitted = {
            "colors": tensor([[0.6, 0.4, 0.5]]),
            "secondary_colors": tensor([[0.3, 0.5, 0.4]]),
            "frequency_magnitudes": torch.ones(1, 4, dtype=dtype, device=device),
            "phases": torch.zeros(1, 4, dtype=dtype, device=device),
        }
    elif method == "neural":
        def uniform(shape, bound):
            return ((torch.rand(shape, generator=gen) * 2 - 1) * bound).to(dtype).to(device)

        fitted = {
            "input_weights": uniform((1, 6, 5), 1 / 5),
            "input_biases": torch.zeros(1, 6, dtype=dtype, device=device),
            "output_weights": uniform((1, 3, 6), 1 / 30),
            "output_biases": torch.zeros(1, 3, dtype=dtype, device=device),
        }
    else:
        raise ValueError(f"unknown method {method!r}")
    for value in fitted.values():
        value.requires_grad_()
    x = torch.arange(SIZE, dtype=dtype, device=device)
    target = (0.5 + 0.4 * torch.cos(0.7 * x))[None, None, :, None].expand(1, SIZE, SIZE, 3)
    return fixed, fitted, target.contiguous()


def _public_renderer(method):
    from .rendering import rasterize_gabors, rasterize_neural_gabors

    return rasterize_gabors if method == "classic" else rasterize_neural_gabors


def fit_texture(method: str, steps: int, device="cuda", dtype=torch.float32, render=None,
                verbose: bool = False) -> dict:
    """Run the fit; returns per-step losses and target/initial/final renders [H, W, 3]."""
    render = render or _public_renderer(method)
    fixed, fitted, target = texture_problem(method, device, dtype)
    arguments = dict(width=SIZE, height=SIZE)
    with torch.no_grad():
        initial, alpha, _ = render(**fixed, **fitted, **arguments)
        masked_target = target * alpha
    optimizer = torch.optim.Adam(list(fitted.values()), lr=0.01)
    losses = []
    for step in range(steps):
        optimizer.zero_grad(set_to_none=True)
        rgb, alpha, _ = render(**fixed, **fitted, **arguments)
        loss = (rgb - target * alpha.detach()).square().mean()
        loss.backward()
        optimizer.step()
        if method == "classic":
            with torch.no_grad():
                fitted["frequency_magnitudes"].clamp_min_(0)
        losses.append(loss.item())
        if verbose and (step == 0 or step == steps - 1):
            print(f"{method} step={step + 1} loss={losses[-1]:.6f}", flush=True)
    if not all(math.isfinite(value) for value in losses):
        raise RuntimeError("optimization produced non-finite losses")
    with torch.no_grad():
        final, _, _ = render(**fixed, **fitted, **arguments)
    return {
        "losses": losses,
        "target": masked_target[0].cpu(),
        "initial": initial[0].cpu(),
        "final": final[0].cpu(),
    }


def write_png(path: Path, image: torch.Tensor) -> None:
    """Write an [H, W, 3] image in [0, 1] as an 8-bit RGB PNG (zlib, no dependencies)."""
    pixels = (image.clamp(0, 1) * 255).round().to(torch.uint8).contiguous()
    height, width, _ = pixels.shape
    raw = b"".join(b"\x00" + bytes(row.flatten().tolist()) for row in pixels)

    def chunk(kind, data):
        body = kind + data
        return struct.pack(">I", len(data)) + body + struct.pack(">I", zlib.crc32(body))

    header = struct.pack(">IIBBBBB", width, height, 8, 2, 0, 0, 0)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_bytes(b"\x89PNG\r\n\x1a\n" + chunk(b"IHDR", header)
                     + chunk(b"IDAT", zlib.compress(raw, 9)) + chunk(b"IEND", b""))


def main(argv=None) -> dict:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--method", choices=["classic", "neural", "both"], default="classic")
    parser.add_argument("--steps", type=int, default=100)
    parser.add_argument("--output", type=Path,
                        help="save target | initial | fitted panels, one row per method, as PNG")
    args = parser.parse_args(argv)
    if args.steps < 1:
        parser.error("--steps must be positive")
    methods = ["classic", "neural"] if args.method == "both" else [args.method]
    results = {method: fit_texture(method, args.steps, verbose=True) for method in methods}
    if args.output:
        rows = [torch.cat([r["target"], r["initial"], r["final"]], 1) for r in results.values()]
        panels = torch.cat(rows, 0)
        write_png(args.output, panels.repeat_interleave(4, 0).repeat_interleave(4, 1))
        print(f"saved {args.output}")
    return results


if __name__ == "__main__":
    main()
