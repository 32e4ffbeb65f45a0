"""Writes the golden fixtures in this directory from the CPU oracle.

The reference ships no fixture files, so these vectors come from this
repository's own float64 oracle (itself pinned by tests/test_oracle_*.py).
Inputs are stored as float32 (what the GPU path consumes), expected maps and
gradients as float64, discrete outputs as integers.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path[:0] = [str(HERE.parent), str(HERE.parents[1])]

from oracle import binning  # noqa: E402
from oracle import render as oracle_render  # noqa: E402
from scenes import make_inputs, oracle_reference, perturbation_sensitivity, random_scene  # noqa: E402

CASES = {
    "classic_tile": dict(method="classic", builder=lambda: make_inputs("classic"), width=9, height=9),
    "neural_tile": dict(method="neural", builder=lambda: make_inputs("neural"), width=9, height=9),
    "classic_sh2_multitile": dict(
        method="classic",
        builder=lambda: random_scene("classic", cameras=2, n=40, width=40, height=33, seed=4, sh=2),
        width=40, height=33, sh_degree=2,
    ),
    "neural_multitile_packed": dict(
        method="neural",
        builder=lambda: random_scene("neural", scenes=2, cameras=1, n=30, width=35, height=20, seed=9),
        width=35, height=20, packed=True,
    ),
}


def weights_for(shape):
    return torch.linspace(-0.5, 0.8, int(np.prod(shape)), dtype=torch.float64).reshape(shape)


def render_case(spec, values):
    leaves = {k: torch.from_numpy(v).double().requires_grad_() for k, v in values.items()}
    rest = dict(leaves)
    backgrounds = rest.pop("backgrounds")
    fn = oracle_render.rasterize_gabors if spec["method"] == "classic" else oracle_render.rasterize_neural_gabors
    options = {k: spec[k] for k in ("sh_degree", "packed") if k in spec}
    maps, meta, aux = fn(**rest, width=spec["width"], height=spec["height"],
                         backgrounds=backgrounds, **options)
    grads = torch.autograd.grad((maps * weights_for(maps.shape)).sum(), list(leaves.values()),
                                allow_unused=True)
    grads = {f"grad_{k}": (torch.zeros_like(v) if g is None else g).numpy()
             for (k, v), g in zip(leaves.items(), grads)}
    # Float32-scale conditioning of every map value (see scenes.perturbation_sensitivity).
    names = list(values)

    def maps_of(*tensors):
        inputs = dict(zip(names, tensors))
        bg = inputs.pop("backgrounds")
        return fn(**inputs, width=spec["width"], height=spec["height"], backgrounds=bg,
                  radii=meta["radii"] if not options.get("packed") else None, **options)[0]

    sensitivity = perturbation_sensitivity(maps_of, [torch.from_numpy(values[k]) for k in names])[0]
    _, _, grad_sensitivity = oracle_reference(
        lambda backgrounds, **kw: fn(**kw, width=spec["width"], height=spec["height"],
                                      backgrounds=backgrounds, **options),
        {k: torch.from_numpy(v) for k, v in values.items()}, weights_for(maps.shape),
    )
    return {
        "maps": maps.detach().numpy(),
        "maps_sensitivity": sensitivity.numpy(),
        **{f"gradsens_{k}": v.numpy() for k, v in grad_sensitivity.items()},
        "radii": meta["radii"].numpy(),
        "point_list": np.asarray(aux["point_list"], np.int32),
        "ranges": np.asarray(aux["ranges"], np.int32),
        "contributors": aux["contributors"],
        **grads,
    }


def binning_case():
    rng = np.random.default_rng(123)
    q, width, height, images = 200, 50, 40, 2
    geometry = rng.normal(size=(q, 17)).astype(np.float32)
    geometry[:, 9] = rng.uniform(-30, width + 30, q)
    geometry[:, 10] = rng.uniform(-30, height + 30, q)
    geometry[:, 8] = rng.choice(rng.uniform(0.3, 9, 50).astype(np.float32), q)
    radii = rng.integers(-1, 25, q).astype(np.int32)
    image_ids = rng.integers(0, images, q).astype(np.int64)
    keys, point_list, ranges = binning.bin_pairs(geometry, radii, image_ids, images, width, height)
    return dict(geometry=geometry, radii=radii, image_ids=image_ids,
                meta=np.array([width, height, images]), sorted_keys=keys,
                point_list=point_list, ranges=ranges)


def main():
    for name, spec in CASES.items():
        values = {k: v.numpy().astype(np.float32) for k, v in spec["builder"]().items()}
        expected = render_case(spec, values)
        np.savez_compressed(HERE / f"{name}.npz", **{f"in_{k}": v for k, v in values.items()},
                            **{f"out_{k}": v for k, v in expected.items()})
    np.savez_compressed(HERE / "binning_random.npz", **binning_case())
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
