"""Host unit test of the range checks the binning kernels apply to sort
outputs (csrc/index_guard.hpp): the header is compiled with g++ and its
contract exercised on the CPU."""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_index_guard_on_the_host(tmp_path):
    binary = tmp_path / "index_guard_check"
    source = ROOT / "tests" / "native" / "index_guard_check.cpp"
    include = ROOT / "diff_gabor_splatting_amd" / "csrc"
    build = subprocess.run(
        ["g++", "-std=c++17", "-O1", "-Wall", "-Werror", f"-I{include}", str(source), "-o",
         str(binary)],
        capture_output=True, text=True,
    )
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(binary)], capture_output=True, text=True)
    assert run.returncode == 0 and run.stdout.strip() == "ok", run.stdout + run.stderr


def test_status_bits_match_the_header():
    header = (ROOT / "include" / "gabor_hip.h").read_text()
    assert "#define GS_BIN_OVERFLOW 1u" in header
    assert "#define GS_BIN_BAD_INDEX 2u" in header
