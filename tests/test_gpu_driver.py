"""The C++ host driver (ubridge_amd/driver/ub_drive.cpp): the reference's call
sequences issued through the C ABI alone -- GGUF QMatMul by name-keyed launch
against the fused GEMV, matmul_bf16_4bit against dequant_bf16 + matmul_bf16,
the MoE chain against the status-returning topsaten_* names, and a K-split
GEMM's scratch from the library pool against a hipMallocAsync caller
allocator, eager and inside a HIP graph."""
import json
import os
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

DRIVER = os.path.join(ROOT, "ubridge_amd", "lib", "ub_drive")


def test_driver_sequences_agree(dev):
    if not os.path.exists(DRIVER):
        pytest.fail("ub_drive is not built (python ubridge_amd/build.py)")
    r = subprocess.run([DRIVER, "--quick", "--reps", "3"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]
    seq = {l["sequence"]: l for l in lines if "sequence" in l}
    assert set(seq) == {"qmatmul", "w4a16", "moe", "workspace"}
    assert seq["qmatmul"]["rel_err"] < 2e-2 and seq["w4a16"]["rel_err"] < 1e-2
    assert lines[-1] == {"checks_failed": 0}
