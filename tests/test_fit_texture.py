"""End-to-end training through the renderer: the texture fit.

The reference's validation states that both synthetic optimisation examples
reduce their losses over 30 steps (docs/validation.md:26). Here the same
problem runs through the float64 oracle on the CPU (which pins the problem
itself: the loss must fall) and through the HIP path, whose loss curve must
follow the oracle's step for step.
"""

import pytest
import torch

from diff_gabor_splatting_amd.fit_texture import fit_texture, texture_problem, write_png
from oracle import render as oracle_render

STEPS = 30


def oracle_renderer(method):
    function = (oracle_render.rasterize_gabors if method == "classic"
                else oracle_render.rasterize_neural_gabors)

    def render(**arguments):
        maps, meta, _ = function(**arguments)
        return maps[..., :3], maps[..., 3:4], meta
    return render


_ORACLE_FITS = {}


def oracle_fit(method):
    if method not in _ORACLE_FITS:
        _ORACLE_FITS[method] = fit_texture(method, STEPS, device="cpu", dtype=torch.float64,
                                           render=oracle_renderer(method))
    return _ORACLE_FITS[method]


@pytest.mark.parametrize("method", ["classic", "neural"])
def test_oracle_fit_reduces_the_loss(method):
    losses = oracle_fit(method)["losses"]
    assert len(losses) == STEPS
    assert losses[-1] < losses[0], losses


def test_problem_matches_the_reference_example():
    fixed, fitted, target = texture_problem("classic", device="cpu")
    assert fixed["intrinsics"][0].tolist() == [[40.0, 0.0, 15.5], [0.0, 40.0, 15.5],
                                                [0.0, 0.0, 1.0]]
    assert set(fitted) == {"colors", "secondary_colors", "frequency_magnitudes", "phases"}
    assert target.shape == (1, 32, 32, 3)
    torch.testing.assert_close(target[0, 5, 3], torch.full((3,), 0.5 + 0.4 * torch.cos(
        torch.tensor(2.1)).item()))
    _, neural, _ = texture_problem("neural", device="cpu")
    assert neural["input_weights"].abs().max() <= 0.2 and neural["output_weights"].abs().max() <= 1 / 30


def test_png_writer_produces_a_valid_file(tmp_path):
    import zlib

    path = tmp_path / "panel.png"
    image = torch.zeros(2, 3, 3)
    image[1, 2] = torch.tensor([1.0, 0.5, 0.0])
    write_png(path, image)
    data = path.read_bytes()
    assert data[:8] == b"\x89PNG\r\n\x1a\n"
    idat = data.index(b"IDAT")
    length = int.from_bytes(data[idat - 4:idat], "big")
    raw = zlib.decompress(data[idat + 4:idat + 4 + length])
    assert len(raw) == 2 * (1 + 3 * 3)
    assert raw[-3:] == bytes([255, 128, 0])


@pytest.mark.gpu
@pytest.mark.skipif(not torch.cuda.is_available(), reason="needs a GPU")
@pytest.mark.parametrize("method", ["classic", "neural"])
def test_hip_fit_follows_the_oracle(method):
    hip = fit_texture(method, STEPS)
    expected = oracle_fit(method)
    torch.testing.assert_close(torch.tensor(hip["losses"], dtype=torch.float64),
                               torch.tensor(expected["losses"], dtype=torch.float64), rtol=2e-3,
                               atol=1e-6)
    torch.testing.assert_close(hip["final"].double(), expected["final"], atol=2e-3, rtol=0)
    assert hip["losses"][-1] < hip["losses"][0]
