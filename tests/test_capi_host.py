"""C-ABI library checks that need no GPU: libaxf_hip.so loads, exports every
function include/axf_hip.h declares, rejects null handles with
AXF_ERR_INVALID_ARG before touching a device, and its host-side helpers (row
sizes, the RoPE table, the synthetic generators) behave.  No kernel is
launched here."""
import ctypes as C
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from llm_core_amd import _ffi, hip
from oracle import oracle as O

ROOT = Path(__file__).resolve().parent.parent
HEADER = (ROOT / "include" / "axf_hip.h").read_text()
DECLARED = sorted(set(re.findall(r"^[A-Za-z_][\w *]*?\b(axf_\w+)\(", HEADER, re.M)))

AXF_ERR_INVALID_ARG = -1


def test_header_parse_found_the_api():
    assert len(DECLARED) >= 40
    for name in ("axf_hip_create", "axf_hip_gemv_q4k_q8", "axf_hip_gemv_q6k_q8",
                 "axf_hip_dequant_q4k", "axf_hip_quantize_q8_0", "axf_llama_generate"):
        assert name in DECLARED


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(str(_ffi.LIB_PATH))
    missing = [n for n in DECLARED if not hasattr(lib, n)]
    assert not missing, missing


def test_ffi_signatures_match_header():
    assert set(_ffi.SIGNATURES) == set(DECLARED)


def test_version():
    a, b, c = C.c_int(-1), C.c_int(-1), C.c_int(-1)
    assert _ffi.lib.axf_hip_version(C.byref(a), C.byref(b), C.byref(c)) == 0
    assert min(a.value, b.value, c.value) >= 0


def _zero_args(argtypes):
    out = []
    for t in argtypes:
        if t in (C.c_float, C.c_double):
            out.append(0.0)
        elif t in (C.c_int, C.c_int64, C.c_size_t, C.c_uint64, C.c_int32, C.c_uint32):
            out.append(0)
        else:
            out.append(None)
    return out


NULL_HANDLE_FUNCS = [n for n in DECLARED
                     if (n.startswith("axf_hip_") or n.startswith("axf_llama_"))
                     and n not in ("axf_hip_last_error", "axf_hip_version", "axf_hip_device_count",
                                   "axf_hip_create", "axf_hip_destroy", "axf_llama_destroy",
                                   "axf_llama_device_bytes")]


@pytest.mark.parametrize("name", NULL_HANDLE_FUNCS)
def test_null_handle_is_rejected(name):
    fn = getattr(_ffi.lib, name)
    rc = fn(*_zero_args(fn.argtypes))
    assert rc == AXF_ERR_INVALID_ARG
    assert _ffi.last_error()


def test_destroy_null_is_ok():
    assert _ffi.lib.axf_hip_destroy(None) == 0
    assert _ffi.lib.axf_llama_destroy(None) == 0
    assert _ffi.lib.axf_llama_device_bytes(None) == 0


def test_row_bytes():
    assert hip.row_bytes(12, 256) == 144 and hip.row_bytes(12, 512) == 288  # test_gguf_reader.cpp:366-368
    assert hip.row_bytes(14, 4096) == 16 * 210
    assert hip.row_bytes(0, 10) == 40
    assert hip.row_bytes(99, 256) == 0


def test_rope_table_matches_oracle_bitexact():
    for hd, theta, n in ((128, 10000.0, 300), (64, 1e6, 40), (256, 500000.0, 9)):
        c, s = hip.rope_table(hd, theta, n)
        oc, os_ = O.rope_table(hd, theta, n)
        assert np.array_equal(c.view(np.uint32), oc.view(np.uint32))
        assert np.array_equal(s.view(np.uint32), os_.view(np.uint32))


def test_synth_normal_deterministic_and_distributed():
    a = hip.synth_normal(1 << 16, seed=3)
    assert np.array_equal(a, hip.synth_normal(1 << 16, seed=3))
    assert not np.array_equal(a, hip.synth_normal(1 << 16, seed=4))
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1) < 0.02
    b = hip.synth_normal(1000, seed=3, mean=1.0, std=0.5)
    assert abs(b.mean() - 1) < 0.1


@pytest.mark.parametrize("qt,rel", [(12, 0.12), (14, 0.03)])
def test_synth_quantize_round_trip(qt, rel):
    x = hip.synth_normal(256 * 64, seed=9, std=0.02)
    blk = hip.synth_quantize(qt, x)
    y = O.dequant(qt, blk)
    assert np.all(np.isfinite(y))
    assert np.sqrt(np.mean((y - x) ** 2)) <= rel * np.sqrt(np.mean(x ** 2))


def test_synth_weight_is_row_blocks():
    W = hip.synth_weight(12, 3, 512, seed=1)
    assert W.size == 3 * 288
    assert np.array_equal(W, hip.synth_weight(12, 3, 512, seed=1))


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one" in r.stderr.lower()


def test_graft_entry_exports():
    sys.path.insert(0, str(ROOT))
    import __graft_entry__ as g

    assert callable(g.build) and callable(g.smoke)
