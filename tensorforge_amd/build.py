"""Build the gfx950 C-ABI library ``libtensorforge_amd.so`` in-tree.

Every ``csrc/*.hip`` translation unit is compiled with hipcc for gfx950 only
and linked into ``tensorforge_amd/lib/libtensorforge_amd.so``.  The library
exports the ``extern "C"`` entry points declared in
``include/tensorforge_amd.h`` and links against the HIP runtime that the host
process already loaded (torch's ``libamdhip64.so.7`` when imported after
torch).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR / "csrc"
LIBRARY_DIR = PACKAGE_DIR / "lib"
LIBRARY_PATH = LIBRARY_DIR / "libtensorforge_amd.so"
BUILD_DIR = PACKAGE_DIR.parent / "_build"
ARCH = "gfx950"

# Packed-fp32 VALU forms are disabled for every device compile; the compiler
# then emits scalar fp32 arithmetic only.
DEVICE_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
)


# Translation units whose MFMA accumulators the compiler otherwise keeps in
# AGPRs and copies to VGPRs around every VALU use (the online softmax's
# rescale, the split-K epilogue): the VGPR form of the MFMA instructions
# (gfx950 reads and writes C/D in VGPRs) removes those copies.
VGPR_MFMA_SOURCES = {"tf_prefill_attention.hip", "tf_linear_splitk.hip"}
VGPR_MFMA_FLAGS = ("-mllvm", "-amdgpu-mfma-vgpr-form")


def hipcc() -> str:
    candidate = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(candidate).exists():
        raise RuntimeError("hipcc was not found; the gfx950 library cannot be built")
    return candidate


def _compile(source: Path, compiler: str) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    extra = VGPR_MFMA_FLAGS if source.name in VGPR_MFMA_SOURCES else ()
    cmd = [compiler, *DEVICE_FLAGS, *extra, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr}")
    warnings = [
        line
        for line in result.stderr.splitlines()
        if line.strip() and "packed-fp32-ops" not in line
    ]
    if warnings:
        print("\n".join(warnings), file=sys.stderr)
    return obj


def build(verbose: bool = False) -> Path:
    """Compile all kernels for gfx950 and link the shared library."""

    compiler = hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIBRARY_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(SOURCE_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {SOURCE_DIR}")
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda src: _compile(src, compiler), sources))
    tmp = LIBRARY_PATH.with_suffix(".so.tmp")
    cmd = [
        compiler,
        f"--offload-arch={ARCH}",
        "-shared",
        "-fPIC",
        "-o",
        str(tmp),
        *map(str, objects),
    ]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, LIBRARY_PATH)
    if verbose:
        print(f"built {LIBRARY_PATH}")
    return LIBRARY_PATH


if __name__ == "__main__":
    build(verbose=True)
