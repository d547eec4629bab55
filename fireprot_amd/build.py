"""Build the gfx950 HIP library in-tree: ``fireprot_amd/_lib/libfireprot_amd.so``.

Plain ``hipcc`` per source file (objects compiled in parallel), then one
shared-library link.  The result lives inside the package so it travels with
the source tree and is what ``fireprot_amd._native`` loads.
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PACKAGE = pathlib.Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = ROOT / "include"
LIB_DIR = PACKAGE / "_lib"
LIB_PATH = LIB_DIR / "libfireprot_amd.so"
SOURCES = ("attention.hip", "attention_split.hip", "projection.hip", "bf16.hip",
           "elementwise.hip", "trimul.hip", "transition.hip", "capi.hip")
ARCH = "gfx950"

HIPCC_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Keep the compiler from forming packed FP32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Keep MFMA accumulators in ordinary VGPRs (gfx950 reads/writes them
    # directly): no v_accvgpr_read/write shuffles in the attention loop.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
)


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and pathlib.Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the gfx950 library cannot be built")


def _compile(hipcc: str, source: pathlib.Path, obj: pathlib.Path, verbose: bool) -> None:
    cmd = [hipcc, *HIPCC_FLAGS, "-I", str(INCLUDE), "-I", str(CSRC), "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if verbose or result.returncode:
        sys.stderr.write(result.stderr)
    if result.returncode:
        raise RuntimeError(f"hipcc failed for {source.name} (exit {result.returncode})")


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every HIP source for gfx950 and link the shared library."""
    hipcc = _hipcc()
    obj_dir = LIB_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    sources = [CSRC / name for name in SOURCES]
    objects = [obj_dir / (s.stem + ".o") for s in sources]
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(sources)) as pool:
        list(pool.map(lambda so: _compile(hipcc, so[0], so[1], verbose), zip(sources, objects)))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode:
        sys.stderr.write(result.stderr)
        raise RuntimeError("linking libfireprot_amd.so failed")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
