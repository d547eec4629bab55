"""The FP32-matrix-core kernels behind ``FPX_ATTENTION_MFMA=f32``.

The library reads the variable once per process (fp32_matrix_cores_selected,
attention.hip): set, the block's projections and attention, the strided
(OpenFold3) attention, the triangle multiplication and the pair transition
run on v_mfma_f32_32x32x2_f32 with plain FP32 operands instead of the
fp16-plane kernels.  This test runs the parity suites of those paths in one
child process whose environment sets the variable from the start: the block
(small sizes, C2 in full, C3/C4 sampled rows, golden fixtures, residual
forms), the FP32-accuracy bar against the float64 oracle, the strided
attention, the triangle multiplication and the pair transition.  Suites that
decode the fp16-plane workspace layout (test_gpu_planes.py) or cover the
BF16 block are not meant for this path and are left out.
"""
from __future__ import annotations

import os
import pathlib
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = pathlib.Path(__file__).resolve().parents[1]
SUITES = (
    "tests/test_gpu_block.py",
    "tests/test_gpu_fp32_accuracy.py",
    "tests/test_gpu_openfold3.py",
    "tests/test_gpu_tile_skip.py",
    "tests/test_gpu_trimul.py",
    "tests/test_gpu_transition.py",
    "tests/test_gpu_fp16_scaling.py",
)


def test_fp32_matrix_core_kernels_pass_the_parity_suites():
    import torch

    torch.cuda.empty_cache()  # leave the child the device memory
    env = dict(os.environ, FPX_ATTENTION_MFMA="f32")
    cmd = [sys.executable, "-u", "-m", "pytest", *SUITES, "-q", "-x", "-m", "gpu",
           "-p", "no:cacheprovider"]
    print(f"child: FPX_ATTENTION_MFMA=f32 {' '.join(cmd[2:])}", flush=True)
    proc = subprocess.run(cmd, cwd=ROOT, env=env, capture_output=True, text=True, timeout=180)
    tail = "\n".join((proc.stdout + proc.stderr).strip().splitlines()[-25:])
    print(tail, flush=True)
    assert proc.returncode == 0, f"FP32-matrix-core suites failed:\n{tail}"
    assert " passed" in tail and "failed" not in tail
