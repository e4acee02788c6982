"""Runs the C++ plugin-interface test (tests/cpp/test_backend_hip.cpp, built by
llm_core_amd.build) on the GPU: registry lookup, synchronous transfers,
RMS_NORM and MATMUL through IBackend/IKernel."""
import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parent.parent / "llm_core_amd" / "_build" / "test_backend_hip"


@pytest.mark.gpu
def test_cpp_backend_program():
    assert EXE.exists(), f"{EXE} missing: run python -m llm_core_amd.build"
    proc = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "PASSED (0 failures)" in proc.stdout
