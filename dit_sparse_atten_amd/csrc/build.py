"""Build libdsa.so (all HIP kernels + the C-ABI) for gfx950 with hipcc.

Usage: ``python -m dit_sparse_atten_amd.csrc.build`` or ``build_library()``.
The library is written next to the package (``dit_sparse_atten_amd/libdsa.so``)
so it travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PACKAGE = CSRC.parent
INCLUDE = PACKAGE.parent / "include"
LIBRARY = PACKAGE / "libdsa.so"
SOURCES = (
    "dsa_api.hip",
    "bsa_fwd.hip",
    "block_mass.hip",
    "tile_stats.hip",
    "route.hip",
    "routing.hip",
    "tile_route.hip",
    "permute.hip",
    "dit_ops.hip",
)

# Packed FP32 VALU forms are disabled: the device code relies on scalar and
# float2 arithmetic only.  hipcc's host pass warns that it does not know the
# feature; that warning is expected.  MFMA results stay in architectural
# VGPRs (-amdgpu-mfma-vgpr-form): at one wave per SIMD the register allocator
# would otherwise place S accumulators in AGPRs and copy every element back
# with v_accvgpr_read before the softmax reads it.
HIPCC_FLAGS = (
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
)


def hipcc_path() -> str:
    candidates = [os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")]
    for candidate in candidates:
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def build_library(verbose: bool = False) -> Path:
    """Compile every HIP source into one shared library and return its path."""
    sources = [str(CSRC / name) for name in SOURCES]
    tmp = LIBRARY.with_suffix(".so.tmp")
    command = [hipcc_path(), *HIPCC_FLAGS, "-I", str(CSRC), "-I", str(INCLUDE), "-o", str(tmp), *sources]
    if verbose:
        print(" ".join(command), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    messages = [line for line in (result.stdout + result.stderr).splitlines()
                if noise not in line]
    if result.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(messages))
    if verbose and messages:
        print("\n".join(messages), flush=True)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
