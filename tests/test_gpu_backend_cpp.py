"""Runs the C++ plugin-interface test (tests/cpp/test_backend_hip.cpp, built by
llm_core_amd.build) on the GPU: registry lookup, synchronous transfers,
RMS_NORM and MATMUL through IBackend/IKernel.  The same test is run a second
time as llm_core_amd/_build/test_backend_dropin: the plugin compiled in its
drop-in mode against the reference's own headers, BackendRegistry, Tensor and
AttributeMap (tests/cpp/build_dropin.py, built where the reference tree
exists)."""
import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parent.parent / "llm_core_amd" / "_build" / "test_backend_hip"
DROPIN = EXE.parent / "test_backend_dropin"


@pytest.mark.gpu
def test_cpp_backend_program():
    assert EXE.exists(), f"{EXE} missing: run python -m llm_core_amd.build"
    proc = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "PASSED (0 failures)" in proc.stdout


@pytest.mark.gpu
def test_cpp_backend_program_against_the_reference_api():
    if not DROPIN.exists():
        pytest.skip("test_backend_dropin is built only where the reference tree exists")
    proc = subprocess.run([str(DROPIN)], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "PASSED (0 failures)" in proc.stdout
