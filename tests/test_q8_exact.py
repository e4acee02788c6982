"""The device Q8_0 quantiser's two shortcuts (q8_quant4, kernels/common.hpp)
against the plain formula of the reference's quantize_q8_avx2
(quant_q8_avx2.cpp:33-84): amax/127 by an fma-corrected product, checked on
every non-negative finite float, and the int8 of rint(v * 127/amax) read from
the low byte of RN(v*id) + 1.5*2^23 without saturation, checked on random
blocks, blocks with products on and next to halves, and an all-zero block.
The device code itself is pinned by the GPU tests that compare its Q8_0
blocks bit for bit (K/V rows, attention output blocks, GEMV prologues)."""
import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "cpp" / "q8_exact.c"


@pytest.mark.slow
@pytest.mark.timeout(600)
def test_q8_quantiser_shortcuts_are_exact(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "q8_exact"
    subprocess.run(["gcc", "-O2", "-mfma", "-ffp-contract=off", "-fopenmp", str(SRC), "-o", str(exe),
                    "-lm"], check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=580)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
