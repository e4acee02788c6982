"""Oracle restatements of the other weight types' GEMVs (Q8_0, Q5_0 and F16
weights; llama_model.cpp:154-293, gemv_f16_avx2.cpp), pinned: F16 against the
reference's own kernel compiled from source (oracle/_ref), Q8_0 / Q5_0 by
blocks built bit by bit and one-hot activations.  CPU only."""
import struct

import numpy as np
import pytest

from oracle import oracle as O


def f16_bits(v: float) -> int:
    return int(np.array(v, np.float16).view(np.uint16))


def q8_0_block(d: float, q) -> bytes:
    return struct.pack("<H", f16_bits(d)) + np.asarray(q, np.int8).tobytes()


def q5_0_block(d: float, q) -> bytes:
    """q: 32 values in [0, 31]; element i keeps its low nibble in byte i % 16
    (low half for i < 16, high half otherwise) and bit 4 in bit i of qh."""
    q = np.asarray(q, np.uint32)
    qh = 0
    qs = bytearray(16)
    for i in range(32):
        qh |= int(q[i] >> 4 & 1) << i
        if i < 16:
            qs[i] |= int(q[i] & 15)
        else:
            qs[i - 16] |= int(q[i] & 15) << 4
    return struct.pack("<HI", f16_bits(d), qh) + bytes(qs)


def test_q8_0_known_blocks_and_one_hot():
    rng = np.random.default_rng(0)
    ds = [0.5, -0.0625, 1.5, 2.0 ** -10]
    qs = [rng.integers(-128, 128, 32) for _ in ds]
    qs[0][:4] = [-128, 127, 0, -1]
    row = b"".join(q8_0_block(d, q) for d, q in zip(ds, qs))
    want = np.concatenate([np.float32(d) * np.asarray(q, np.float32) for d, q in zip(ds, qs)])
    W = np.frombuffer(row, np.uint8)
    np.testing.assert_array_equal(O.dequant_row(8, W, 128), want)
    for i in (0, 1, 33, 127):
        x = np.zeros(128, np.float32)
        x[i] = 1.0
        assert O.gemv_misc(8, W, x, 1, 128)[0] == want[i]


def test_q8_0_q8_activation_exact_integer_dot():
    """With d_x = 1 and d_w = 1 the result is the exact integer dot (extremes
    included: 32 * 128 * 127 per block, well inside fp32's exact range)."""
    q = np.full(32, -128, np.int8)
    row = q8_0_block(1.0, q) * 2
    xq8 = (struct.pack("<f", 1.0) + np.full(32, 127, np.int8).tobytes()) * 2
    y = O.gemv_q8_0w_q8(np.frombuffer(row, np.uint8), np.frombuffer(xq8, np.uint8), 1, 64)
    assert y[0] == 2 * 32 * -128 * 127
    # one-hot: d_w * d_x * q * x
    qw = np.arange(-16, 16, dtype=np.int8)
    xq = np.zeros(32, np.int8)
    xq[5] = 3
    y = O.gemv_q8_0w_q8(np.frombuffer(q8_0_block(0.25, qw), np.uint8),
                        np.frombuffer(struct.pack("<f", 0.5) + xq.tobytes(), np.uint8), 1, 32)
    assert y[0] == np.float32(0.25 * 0.5) * (qw[5] * 3)


def test_q5_0_known_blocks_and_one_hot():
    rng = np.random.default_rng(1)
    ds = [0.5, -1.25, 2.0 ** -8]
    qs = [rng.integers(0, 32, 32) for _ in ds]
    qs[0][:4] = [0, 31, 16, 15]
    row = b"".join(q5_0_block(d, q) for d, q in zip(ds, qs))
    want = np.concatenate([np.float32(d) * (np.asarray(q, np.float32) - 16) for d, q in zip(ds, qs)])
    W = np.frombuffer(row, np.uint8)
    np.testing.assert_array_equal(O.dequant_row(6, W, 96), want)
    for i in (0, 1, 15, 16, 17, 31, 95):
        x = np.zeros(96, np.float32)
        x[i] = 1.0
        assert O.gemv_misc(6, W, x, 1, 96)[0] == want[i]


def test_f16_dequant_exact():
    v = np.array([0.0, -0.0, 1.0, -2.5, 65504.0, 6e-8, np.inf], np.float16)
    np.testing.assert_array_equal(O.dequant_row(1, v.view(np.uint8), v.size), v.astype(np.float32))


@pytest.mark.skipif(O.ref is None, reason="oracle/_ref not built (reference sources absent)")
@pytest.mark.parametrize("rows,cols", [(1, 8), (3, 16), (4, 24), (7, 40), (9, 4096), (5, 4099),
                                       (8, 1000), (13, 13)])
@pytest.mark.parametrize("with_bias", [False, True])
def test_f16_matches_compiled_reference(rows, cols, with_bias):
    """Bit for bit against gemv_f16_avx2_range compiled from the reference's
    source: 4-row tiles, the remaining rows, 16/8-element steps, scalar tails
    and the bias path."""
    rng = np.random.default_rng(rows * 1000 + cols)
    W = rng.standard_normal((rows, cols)).astype(np.float16)
    x = rng.standard_normal(cols).astype(np.float32)
    b = rng.standard_normal(rows).astype(np.float32) if with_bias else None
    want = np.zeros(rows, np.float32)
    O.ref.ref_gemv_f16_f32(O._ptr(want), O._ptr(W), O._ptr(x), None if b is None else O._ptr(b),
                           0, rows, cols)
    got = O.gemv_misc(1, W, x, rows, cols, b)
    np.testing.assert_array_equal(got, want)
