"""The CPU oracle against the reference's own kernels, through the committed
golden vectors (tests/golden/ref_kernels.npz, written by
tests/golden/make_golden.py from oracle/_ref, the reference's x86 kernel
sources compiled in place).  Every comparison is bit for bit: the oracle
restates the reference kernels' lane structure and reduction order."""
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

G = np.load(Path(__file__).resolve().parent / "golden" / "ref_kernels.npz", allow_pickle=False)
ROWS, COLS, T = (int(v) for v in G["shape"])
SETS = ["", "r"]  # realistic scales / any finite fp16 scale


def same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_fixture_is_well_formed():
    for k in G.files:
        if G[k].dtype == np.float32:
            assert np.all(np.isfinite(G[k])), k
    assert G["W_q4"].size == ROWS * COLS // 256 * 144
    assert G["W_q6"].size == ROWS * COLS // 256 * 210


def test_quantize_q8_0_matches_reference():
    assert np.array_equal(O.quantize_q8_0(G["x"]), G["xq8"])
    assert np.array_equal(O.quantize_q8_0(G["X"].reshape(-1)), G["XQ8"])
    assert np.array_equal(O.quantize_q8_0(G["x_edge"]), G["x_edge_q8"])


@pytest.mark.parametrize("s", SETS)
@pytest.mark.parametrize("qt,name", [(O.Q4K, "q4"), (O.Q6K, "q6")])
def test_dequant_matches_reference(qt, name, s):
    got = O.dequant(qt, G[f"W_{name}{s}"]).reshape(ROWS, COLS)
    want = G[f"deq_{name}{s}"]
    # the golden comes out of a one-hot GEMV, which cannot carry the sign of zero
    assert np.array_equal(got, want)
    nz = want != 0
    assert same_bits(got[nz], want[nz])


@pytest.mark.parametrize("s", SETS)
@pytest.mark.parametrize("qt,name", [(O.Q4K, "q4"), (O.Q6K, "q6")])
def test_gemv_f32_matches_reference(qt, name, s):
    got = O.gemv_f32(qt, G[f"W_{name}{s}"], G["x"], ROWS, COLS)
    assert same_bits(got, G[f"y_f32_{name}{s}"])


@pytest.mark.parametrize("s", SETS)
def test_gemv_q4k_q8_matches_reference(s):
    got = O.gemv_q8(O.Q4K, G[f"W_q4{s}"], G["xq8"], ROWS, COLS)
    assert same_bits(got, G[f"y_q8_avx2_q4{s}"])
    assert same_bits(got, G[f"y_r8_avx2_q4{s}"])
    if int(G["has_vnni"][0]):
        assert same_bits(got, G[f"y_q8_vnni_q4{s}"])
        assert same_bits(got, G[f"y_r8_vnni_q4{s}"])


@pytest.mark.parametrize("s", SETS)
def test_gemv_q6k_q8_matches_reference(s):
    got = O.gemv_q8(O.Q6K, G[f"W_q6{s}"], G["xq8"], ROWS, COLS)
    assert same_bits(got, G[f"y_q8_q6{s}"])


@pytest.mark.parametrize("s", SETS)
def test_repack_r8_matches_reference(s):
    assert np.array_equal(O.repack_r8(G[f"W_q4{s}"], ROWS, COLS), G[f"r8_q4{s}"])


@pytest.mark.parametrize("s", SETS)
def test_gemm_q4k_q8_matches_reference(s):
    got = O.gemm_q4k_q8(G[f"W_q4{s}"], G["XQ8"], ROWS, T, COLS)
    assert same_bits(got, G[f"Y_gemm_avx2_q4{s}"])
    if int(G["has_vnni"][0]):
        assert same_bits(got, G[f"Y_gemm_vnni_q4{s}"])
