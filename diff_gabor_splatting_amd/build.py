"""Build the gfx950 HIP library ``libgabor_hip.so`` in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object under ``_build/`` and the
objects are linked into ``diff_gabor_splatting_amd/libgabor_hip.so``. With
``diagnostics=True`` the same sources are compiled with ``-DGS_DIAGNOSTICS``
under ``_build/diagnostics/`` into ``libgabor_hip_diag.so``, whose compositors
also record per-tile times and active-lane counts (gs_diagnostics_set). The
library links the HIP runtime by its SONAME (``libamdhip64.so.7``), so when it
is loaded after ``import torch`` it binds to the runtime torch already loaded
and shares torch's streams and allocations.

The renderer's host functions (``csrc/host.cpp``) are a Python extension
module, ``diff_gabor_splatting_amd/_host*.so``, compiled with the host C++
compiler against the installed torch (:func:`build_host`); it calls the HIP
library's C ABI through function addresses handed over at import.

Run ``python -m diff_gabor_splatting_amd.build`` or call :func:`build_library`
and :func:`build_host`.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
SOURCE_DIR = PACKAGE_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
BUILD_DIR = REPO_DIR / "_build"
LIBRARY = PACKAGE_DIR / "libgabor_hip.so"
DIAGNOSTICS_LIBRARY = PACKAGE_DIR / "libgabor_hip_diag.so"
HOST_SOURCE = SOURCE_DIR / "host.cpp"
HOST_EXTENSION = PACKAGE_DIR / ("_host" + sysconfig.get_config_var("EXT_SUFFIX"))
ROCM_DIR = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = os.environ.get("GABOR_HIP_ARCH", "gfx950")

COMPILE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # Hardware float atomics (global_atomic_add_f32) on device memory.
    "-munsafe-fp-atomics",
    # Keep the compiler from forming packed-FP32 VALU instructions.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; the HIP library cannot be built")
    return found


def _quiet(text: str) -> str:
    # hipcc's host pass does not know the device-only feature flag.
    return "\n".join(
        line for line in text.splitlines() if "is not a recognized feature" not in line
    )


def _compile(source: Path, verbose: bool, directory: Path, defines: list[str]) -> Path:
    obj = directory / (source.stem + ".o")
    cmd = [_hipcc(), *COMPILE_FLAGS, *defines, f"-I{INCLUDE_DIR}", f"-I{SOURCE_DIR}", "-c",
           str(source)]
    cmd += ["-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    messages = _quiet(result.stdout + result.stderr)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{messages}")
    if verbose and messages.strip():
        print(messages, file=sys.stderr)
    return obj


def build_library(verbose: bool = False, diagnostics: bool = False) -> Path:
    """Compile every HIP source for gfx950 and link the shared library (the
    diagnostics build with ``diagnostics``)."""
    directory = BUILD_DIR / "diagnostics" if diagnostics else BUILD_DIR
    library = DIAGNOSTICS_LIBRARY if diagnostics else LIBRARY
    defines = ["-DGS_DIAGNOSTICS"] if diagnostics else []
    directory.mkdir(parents=True, exist_ok=True)
    sources = sorted(SOURCE_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {SOURCE_DIR}")
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objects = list(pool.map(lambda s: _compile(s, verbose, directory, defines), sources))
    temporary = library.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects)]
    cmd += ["-o", str(temporary)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{_quiet(result.stdout + result.stderr)}")
    os.replace(temporary, library)
    if verbose:
        print(f"built {library}", file=sys.stderr)
    return library


def build_host(verbose: bool = False) -> Path:
    """Compile the renderer's C++ host functions into the ``_host`` extension
    module (no device code: the host compiler and torch's headers)."""
    import torch
    from torch.utils import cpp_extension

    compiler = shutil.which("g++") or shutil.which("c++")
    if compiler is None:
        raise RuntimeError("no host C++ compiler found; the _host extension cannot be built")
    torch_libraries = cpp_extension.library_paths()
    includes = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"],
                str(ROCM_DIR / "include"), str(INCLUDE_DIR)]
    temporary = HOST_EXTENSION.with_name(HOST_EXTENSION.name + ".tmp")
    cmd = [
        compiler, "-O2", "-std=c++17", "-fPIC", "-shared", "-fvisibility=hidden",
        f"-D_GLIBCXX_USE_CXX11_ABI={int(torch.compiled_with_cxx11_abi())}",
        "-DTORCH_EXTENSION_NAME=_host", "-DTORCH_API_INCLUDE_EXTENSION_H",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *(f"-I{path}" for path in includes),
        str(HOST_SOURCE), "-o", str(temporary),
        *(f"-L{path}" for path in torch_libraries),
        *(f"-Wl,-rpath,{path}" for path in torch_libraries),
        "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lamdhip64",
    ]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"{compiler} failed on {HOST_SOURCE.name}:\n{result.stdout}{result.stderr}")
    os.replace(temporary, HOST_EXTENSION)
    if verbose:
        print(f"built {HOST_EXTENSION}", file=sys.stderr)
    return HOST_EXTENSION


if __name__ == "__main__":
    build_library(verbose=True)
    build_host(verbose=True)
    if "--diagnostics" in sys.argv[1:]:
        build_library(verbose=True, diagnostics=True)
