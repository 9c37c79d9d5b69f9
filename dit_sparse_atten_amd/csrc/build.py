"""Build libdsa.so (all HIP kernels + the C-ABI) for gfx950 with hipcc.

Usage: ``python -m dit_sparse_atten_amd.csrc.build`` or ``build_library()``.
Every source is compiled to its own object in parallel (the kernels of one
file never call device code of another), then the objects are linked into
``dit_sparse_atten_amd/libdsa.so`` next to the package, so the library
travels with the source tree.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PACKAGE = CSRC.parent
INCLUDE = PACKAGE.parent / "include"
LIBRARY = PACKAGE / "libdsa.so"
OBJECTS = PACKAGE / "_build"
SOURCES = (
    "dsa_api.hip",
    "bsa_fwd.hip",
    "bsa_fwd_f16.hip",
    "bsa_fwd_f32.hip",
    "block_mass.hip",
    "tile_stats.hip",
    "sampled_mass.hip",
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
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
)
_NOISE = "is not a recognized feature for this target"


def hipcc_path() -> str:
    candidates = [os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")]
    for candidate in candidates:
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; set HIPCC or install ROCm")


def _run(command, verbose):
    if verbose:
        print(" ".join(command), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    messages = [line for line in (result.stdout + result.stderr).splitlines()
                if _NOISE not in line]
    if result.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(messages))
    if verbose and messages:
        print("\n".join(messages), flush=True)


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source into one shared library and return its path."""
    hipcc = hipcc_path()
    OBJECTS.mkdir(exist_ok=True)
    objects = [OBJECTS / (Path(name).stem + ".o") for name in SOURCES]
    commands = [[hipcc, *HIPCC_FLAGS, "-I", str(CSRC), "-I", str(INCLUDE), "-c",
                 str(CSRC / name), "-o", str(obj)] for name, obj in zip(SOURCES, objects)]
    jobs = jobs or min(len(commands), max(1, min(16, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for future in [pool.submit(_run, command, verbose) for command in commands]:
            future.result()
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objects)], verbose)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
