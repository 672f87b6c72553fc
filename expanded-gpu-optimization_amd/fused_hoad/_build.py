"""In-tree build of the gfx950 kernels and the ``fused_hoad._C`` extension.

Two artefacts, both written next to this file so they travel with the source tree:

* ``libfused_hoad_hip.so``: the HIP kernels and the C ABI of ``include/fused_hoad.h``, built
  with ``hipcc --offload-arch=gfx950``;
* ``_C<ext-suffix>``: the pybind11 torch extension (the reference's ``fused_hoad._C``, from
  ``csrc/bindings.cpp``), a host-only C++ file linked against the library above with an
  ``$ORIGIN`` rpath.

Replaces the reference's ``CUDAExtension`` build (/root/reference/setup.py:9-27). Run as
``python -m fused_hoad._build`` with ``expanded-gpu-optimization_amd`` on ``sys.path``;
``--phase-clock`` builds only the measurement copy of the library that ``phase_clock.py`` runs.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_ROOT = PACKAGE_DIR.parent
CSRC = SOURCE_ROOT / "csrc"
INCLUDE = SOURCE_ROOT.parent / "include"
LIBRARY_NAME = "libfused_hoad_hip.so"
LIBRARY = PACKAGE_DIR / LIBRARY_NAME
PHASE_CLOCK_LIBRARY = PACKAGE_DIR / "libfused_hoad_hip_phase_clock.so"
ARCH = "gfx950"

# -packed-fp32-ops keeps hipcc from forming v_pk_*_f32 instructions from scalar float code.
# -amdgpu-mfma-vgpr-form has MFMAs write their results to VGPRs where registers allow, so the
# VALU work that consumes them (tanh jet and adjoint) needs fewer AGPR-to-VGPR copies: in the
# backward kernel, 364 copies instead of 764 and 10 % fewer VALU instructions.
HIP_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
    "-fPIC",
    "-shared",
]


def extension_path() -> Path:
    return PACKAGE_DIR / f"_C{sysconfig.get_config_var('EXT_SUFFIX')}"


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            f"build step failed ({result.returncode}): {' '.join(cmd)}\n{result.stdout}{result.stderr}"
        )


def _hipcc() -> str:
    return os.environ.get("HIPCC") or shutil.which("hipcc") or "/opt/rocm/bin/hipcc"


def build_library(verbose: bool = False, phase_clock: bool = False) -> Path:
    """Compile the HIP kernels and the C ABI into ``libfused_hoad_hip.so``.

    ``phase_clock`` builds the measurement copy instead, ``libfused_hoad_hip_phase_clock.so``
    (``-DFHOAD_PHASE_CLOCK``: the backward kernel times its phases; see ``phase_clock.py``).
    Nothing in the package loads it.
    """
    library = PHASE_CLOCK_LIBRARY if phase_clock else LIBRARY
    tmp = library.with_suffix(".so.tmp")
    _run(
        [
            _hipcc(),
            *HIP_FLAGS,
            *(["-DFHOAD_PHASE_CLOCK"] if phase_clock else []),
            f"-I{INCLUDE}",
            f"-I{CSRC}",
            str(CSRC / "fused_hoad_kernels.hip"),
            "-o",
            str(tmp),
        ],
        verbose,
    )
    tmp.replace(library)
    return library


def build_extension(verbose: bool = False) -> Path:
    """Compile ``csrc/bindings.cpp`` into the ``fused_hoad._C`` torch extension."""
    import torch
    from torch.utils import cpp_extension

    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    includes = [*cpp_extension.include_paths(device_type="cuda"), sysconfig.get_paths()["include"]]
    libraries = cpp_extension.library_paths(device_type="cuda")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    out = extension_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [
        os.environ.get("CXX", "g++"),
        "-O2",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-D__HIP_PLATFORM_AMD__=1",
        "-DUSE_ROCM=1",
        "-DTORCH_EXTENSION_NAME=_C",
        "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        *(f"-I{path}" for path in includes),
        f"-I{INCLUDE}",
        f"-I{rocm}/include",
        str(CSRC / "bindings.cpp"),
        "-o",
        str(tmp),
        *(f"-L{path}" for path in libraries),
        f"-L{PACKAGE_DIR}",
        "-l:" + LIBRARY_NAME,
        "-lc10",
        "-lc10_hip",
        "-ltorch",
        "-ltorch_cpu",
        "-ltorch_python",
        f"-L{rocm}/lib",
        "-lamdhip64",
        "-Wl,-rpath,$ORIGIN",
    ]
    _run(cmd, verbose)
    tmp.replace(out)
    return out


def build(verbose: bool = False) -> None:
    build_library(verbose)
    build_extension(verbose)


if __name__ == "__main__":
    if "--phase-clock" in sys.argv:
        build_library(verbose="-q" not in sys.argv, phase_clock=True)
    else:
        build(verbose="-q" not in sys.argv)
