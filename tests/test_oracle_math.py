"""Pins of the CPU oracle by what the mathematics fixes: known-answer blocks
built bit by bit here (GGML super-block layouts), invariants of Q8_0,
float64 brute force with error bounds, closed forms of RMSNorm / RoPE /
attention / SwiGLU, and tie rules.  Each check is chosen so that a plausible
slip in the oracle (a dropped min term, a wrong nibble or scale index, a sign,
a transposed operand) fails it."""
import numpy as np
import pytest

from oracle import oracle as O

from qblocks import F16_HALF, F16_ONE, F16_QUARTER, pack_q4k, pack_q6k, unpack_q8  # noqa: F401


def test_q4k_known_answer_including_high_scale_bits():
    rng = np.random.default_rng(1)
    sc = [1, 2, 63, 17, 33, 45, 62, 7]      # j >= 4 entries use the high-bit path
    mn = [0, 3, 63, 8, 40, 2, 61, 31]
    q = rng.integers(0, 16, 256)
    blk = pack_q4k(F16_ONE, F16_HALF, sc, mn, q)
    assert blk.size == 144
    want = np.array([1.0 * sc[i // 32] * q[i] - 0.5 * mn[i // 32] for i in range(256)], np.float32)
    assert np.array_equal(O.dequant(O.Q4K, blk), want)


def test_q6k_known_answer_negative_scales():
    rng = np.random.default_rng(2)
    sc = [1, -1, 127, -128, 5, -7, 64, 33, -2, 3, 100, -100, 9, 0, -64, 12]
    q = rng.integers(0, 64, 256)
    blk = pack_q6k(F16_QUARTER, sc, q)
    assert blk.size == 210
    want = np.array([0.25 * sc[i // 16] * (int(q[i]) - 32) for i in range(256)], np.float32)
    assert np.array_equal(O.dequant(O.Q6K, blk), want)


def test_zero_blocks_dequant_to_zero():
    assert not np.any(O.dequant(O.Q4K, np.zeros(144, np.uint8)))
    # Q6_K: q == 32 everywhere is zero whatever the scales
    blk = pack_q6k(F16_ONE, [5] * 16, np.full(256, 32))
    assert not np.any(O.dequant(O.Q6K, blk))


def test_fp16_conversion_special_values():
    for h, v in ((0x3C00, 1.0), (0xC000, -2.0), (0x0001, 2.0 ** -24), (0x7BFF, 65504.0),
                 (0x0000, 0.0), (0x8000, -0.0), (0x3555, float(np.float16(1 / 3)))):
        assert O.orc.orc_fp16_to_fp32(h) == v
    assert np.isinf(O.orc.orc_fp16_to_fp32(0x7C00))


# ---------------------------------------------------------------------------
# Q8_0 (block_q8_0: q8_block.hpp:8-15; quantize: quant_q8_avx2.cpp:33-84)
# ---------------------------------------------------------------------------

def test_q8_0_invariants():
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32 * 64) * rng.choice([1e-3, 1.0, 50.0], 32 * 64)).astype(np.float32)
    d, q = unpack_q8(O.quantize_q8_0(x))
    xb = x.reshape(-1, 32)
    amax = np.max(np.abs(xb), axis=1)
    assert np.array_equal(d, (amax / np.float32(127)).astype(np.float32))
    assert np.all(np.abs(q) <= 127)
    # the amax element maps to +-127
    i = np.argmax(np.abs(xb), axis=1)
    assert np.all(np.abs(q[np.arange(len(i)), i]) == 127)
    err = np.abs(xb - d[:, None] * q)
    assert np.all(err <= d[:, None] * 0.5 * (1 + 1e-5) + 1e-30)


def test_q8_0_round_half_to_even_and_zero_block():
    x = np.zeros(64, np.float32)
    x[:32] = np.arange(-15.5, 16.5, 1.0)   # .5 ties with id = 127/127 = 1
    x[31] = 127.0
    d, q = unpack_q8(O.quantize_q8_0(x))
    assert d[0] == 1.0
    assert list(q[0, :31]) == [int(np.rint(v)) for v in x[:31]]  # rint: half to even
    assert d[1] == 0.0 and not np.any(q[1])


# ---------------------------------------------------------------------------
# GEMV / GEMM against float64 brute force
# ---------------------------------------------------------------------------

def rand_blocks(qt, n, seed):
    rng = np.random.default_rng(seed)
    bb = O.BLOCK_BYTES[qt]
    blk = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
    h = rng.uniform(1e-3, 1e-2, size=(n, 2)).astype(np.float16).view(np.uint16)
    hb = np.ascontiguousarray(h).view(np.uint8).reshape(n, 4)
    if qt == O.Q4K:
        blk[:, 0:4] = hb
    else:
        blk[:, 208:210] = hb[:, :2]
    return blk.reshape(-1)


@pytest.mark.parametrize("qt", [O.Q4K, O.Q6K])
def test_gemv_f32_vs_float64(qt):
    rows, cols = 37, 1024
    W = rand_blocks(qt, rows * cols // 256, 4)
    x = np.random.default_rng(5).standard_normal(cols).astype(np.float32)
    D = O.dequant(qt, W).reshape(rows, cols).astype(np.float64)
    want = D @ x.astype(np.float64)
    got = O.gemv_f32(qt, W, x, rows, cols)
    bound = 4 * cols * np.finfo(np.float32).eps * (np.abs(D) @ np.abs(x.astype(np.float64)))
    assert np.all(np.abs(got - want) <= bound + 1e-30)


@pytest.mark.parametrize("qt", [O.Q4K, O.Q6K])
def test_gemv_q8_vs_float64(qt):
    """Q8 GEMV == float64 dot of the dequantised weights with the dequantised
    activations (pins the integer dot, the scale and the min/32 corrections)."""
    rows, cols = 29, 2048
    W = rand_blocks(qt, rows * cols // 256, 6)
    x = np.random.default_rng(7).standard_normal(cols).astype(np.float32)
    xq = O.quantize_q8_0(x)
    d, q = unpack_q8(xq)
    xd = (d[:, None].astype(np.float64) * q).reshape(-1)
    D = O.dequant(qt, W).reshape(rows, cols).astype(np.float64)
    want = D @ xd
    got = O.gemv_q8(qt, W, xq, rows, cols)
    bound = 8 * cols * np.finfo(np.float32).eps * (np.abs(D) @ np.abs(xd))
    assert np.all(np.abs(got - want) <= bound + 1e-30)


def test_gemm_rows_equal_gemv_within_tolerance():
    rows, cols, T = 24, 1024, 5
    W = rand_blocks(O.Q4K, rows * cols // 256, 8)
    X = np.random.default_rng(9).standard_normal((T, cols)).astype(np.float32)
    XQ = O.quantize_q8_0(X.reshape(-1))
    Y = O.gemm_q4k_q8(W, XQ, rows, T, cols)
    for t in range(T):
        y = O.gemv_q8(O.Q4K, W, XQ[t * cols // 32 * 36:(t + 1) * cols // 32 * 36], rows, cols)
        assert np.allclose(Y[t], y, rtol=1e-3, atol=1e-4)  # north-star GEMV tolerance


def test_repack_r8_layout():
    """r8: per (8 rows x block) 1152 B: d[8] @0, dmin[8] @16, scales[8][12] @32,
    qs chunk c of row r at 128 + 256c + 32r (gemv_q4k_r8_avx2.cpp:102-136)."""
    rows, cols = 16, 512
    W = rand_blocks(O.Q4K, rows * cols // 256, 10)
    R = O.repack_r8(W, rows, cols)
    nb = cols // 256
    Wb = W.reshape(rows, nb, 144)
    for g in range(rows // 8):
        for b in range(nb):
            t = R[(g * nb + b) * 1152:(g * nb + b + 1) * 1152]
            for r in range(8):
                src = Wb[8 * g + r, b]
                assert np.array_equal(t[2 * r:2 * r + 2], src[0:2])
                assert np.array_equal(t[16 + 2 * r:18 + 2 * r], src[2:4])
                assert np.array_equal(t[32 + 12 * r:44 + 12 * r], src[4:16])
                for c in range(4):
                    o = 128 + 256 * c + 32 * r
                    assert np.array_equal(t[o:o + 32], src[16 + 32 * c:48 + 32 * c])


# ---------------------------------------------------------------------------
# decode-step ops (llama_model.cpp:319-451, 1031-1080, 1169-1272)
# ---------------------------------------------------------------------------

def test_rmsnorm_reference_closed_form():
    # tests/test_backend_x86.cpp:84-116 of the reference: x = 1..8, w = 1
    x = np.arange(1, 9, dtype=np.float32)
    y = O.rmsnorm(x, np.ones(8, np.float32), 1e-5)
    assert np.allclose(y, x / np.sqrt(25.5 + 1e-5), rtol=1e-4)


def test_rmsnorm_vs_float64():
    rng = np.random.default_rng(11)
    x = rng.standard_normal(4096).astype(np.float32) * 3
    w = rng.standard_normal(4096).astype(np.float32)
    y = O.rmsnorm(x, w, 1e-6)
    x64 = x.astype(np.float64)
    want = w * x64 / np.sqrt(np.mean(x64 * x64) + 1e-6)
    assert np.allclose(y, want, rtol=2e-6, atol=1e-7)


def test_rope_table_formula():
    hd, theta, n = 128, 10000.0, 257
    c, s = O.rope_table(hd, theta, n)
    i = np.arange(hd // 2)
    ang = np.arange(n)[:, None] * (1.0 / theta ** (2.0 * i / hd))[None, :]
    assert np.allclose(c.reshape(n, -1), np.cos(ang), atol=2e-5)
    assert np.allclose(s.reshape(n, -1), np.sin(ang), atol=2e-5)
    assert np.all(c[:hd // 2] == 1.0) and np.all(s[:hd // 2] == 0.0)


def test_rope_identity_pairs_and_norm():
    hd, H = 64, 3
    c, s = O.rope_table(hd, 10000.0, 50)
    x = np.random.default_rng(12).standard_normal(H * hd).astype(np.float32)
    assert np.array_equal(O.rope(x, 0, H, hd, c, s), x)
    y = O.rope(x, 37, H, hd, c, s)
    xh, yh = x.reshape(H, 2, hd // 2), y.reshape(H, 2, hd // 2)
    # rotate-half: pair (i, i + hd/2) keeps its norm
    assert np.allclose(np.hypot(yh[:, 0], yh[:, 1]), np.hypot(xh[:, 0], xh[:, 1]), rtol=1e-5)
    # a single non-zero at i only moves into i and i + hd/2, with the table's angle
    e = np.zeros(hd, np.float32)
    e[5] = 1.0
    r = O.rope(e, 37, 1, hd, c, s)
    nz = set(np.nonzero(r)[0])
    assert nz <= {5, 5 + hd // 2}
    assert r[5] == c[37 * hd // 2 + 5] and r[5 + hd // 2] == s[37 * hd // 2 + 5]


def test_rope_exact_rotations_and_rounding_bound():
    """apply_rope (llama_model.cpp:1046-1080) on tables whose products are exact:
    a quarter turn maps (x0, x1) to (-x1, x0), a half turn negates, and the
    bilinear form (x0 c - x1 s, x0 s + x1 c) with c = 0.5, s = 0.75 on small
    integers is exact whether or not the compiler contracts it into FMAs.  On
    the real table the result is within one rounding of each product of the
    float64 rotation.  Which FMA contraction GCC applies to the reference's
    expression cannot be observed here (llama_model.cpp does not build); the
    two candidates differ by at most one ulp of the larger product, and the GPU
    kernels follow the oracle's choice bit for bit."""
    hd, H = 16, 2
    half = hd // 2
    rng = np.random.default_rng(21)
    x = rng.integers(-1000, 1000, H * hd).astype(np.float32)
    xh = x.reshape(H, 2, half)
    for cv, sv, want0, want1 in ((0.0, 1.0, -xh[:, 1], xh[:, 0]),
                                 (-1.0, 0.0, -xh[:, 0], -xh[:, 1]),
                                 (0.5, 0.75, 0.5 * xh[:, 0] - 0.75 * xh[:, 1],
                                  0.75 * xh[:, 0] + 0.5 * xh[:, 1])):
        c = np.ones(2 * half, np.float32)
        s = np.zeros(2 * half, np.float32)
        c[half:] = cv
        s[half:] = sv
        y = O.rope(x, 1, H, hd, c, s).reshape(H, 2, half)
        assert np.array_equal(y[:, 0], want0.astype(np.float32))
        assert np.array_equal(y[:, 1], want1.astype(np.float32))
    c, s = O.rope_table(64, 10000.0, 300)
    xr = rng.standard_normal(4 * 64).astype(np.float32)
    for pos in (1, 77, 299):
        y = O.rope(xr, pos, 4, 64, c, s).astype(np.float64).reshape(4, 2, 32)
        cr = c[pos * 32:(pos + 1) * 32].astype(np.float64)
        sr = s[pos * 32:(pos + 1) * 32].astype(np.float64)
        a, b = xr.astype(np.float64).reshape(4, 2, 32)[:, 0], xr.astype(np.float64).reshape(4, 2, 32)[:, 1]
        bound = 2.0 ** -23 * (np.abs(a * cr) + np.abs(b * sr) + np.abs(a * sr) + np.abs(b * cr))
        assert np.all(np.abs(y[:, 0] - (a * cr - b * sr)) <= bound)
        assert np.all(np.abs(y[:, 1] - (a * sr + b * cr)) <= bound)


def attn64(q, K, V, H, KVH, hd):
    G = H // KVH
    out = np.zeros((H, hd))
    for h in range(H):
        kv = h // G
        k = K[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        v = V[:, kv * hd:(kv + 1) * hd].astype(np.float64)
        sc = k @ q[h * hd:(h + 1) * hd].astype(np.float64) / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        out[h] = (p / p.sum()) @ v
    return out.reshape(-1)


@pytest.mark.parametrize("H,KVH", [(4, 4), (8, 2), (16, 2)])
def test_attention_vs_float64_and_gqa_mapping(H, KVH):
    hd, seq = 64, 77
    rng = np.random.default_rng(13)
    q = rng.standard_normal(H * hd).astype(np.float32)
    K = rng.standard_normal((seq, KVH * hd)).astype(np.float32)
    V = rng.standard_normal((seq, KVH * hd)).astype(np.float32)
    got = O.attention(q, K, V, seq, H, KVH, hd)
    assert np.allclose(got, attn64(q, K, V, H, KVH, hd), rtol=1e-5, atol=1e-6)


def test_attention_closed_forms():
    hd, H, KVH = 32, 4, 2
    rng = np.random.default_rng(14)
    K = rng.standard_normal((9, KVH * hd)).astype(np.float32)
    V = rng.standard_normal((9, KVH * hd)).astype(np.float32)
    q = rng.standard_normal(H * hd).astype(np.float32)
    # seq == 1: softmax of one score is 1, out = V row 0 of the head's kv head
    got = O.attention(q, K, V, 1, H, KVH, hd).reshape(H, hd)
    for h in range(H):
        assert np.array_equal(got[h], V[0, (h // 2) * hd:(h // 2 + 1) * hd])
    # q == 0: uniform weights, out = mean of V
    got = O.attention(np.zeros_like(q), K, V, 9, H, KVH, hd).reshape(H, hd)
    for h in range(H):
        assert np.allclose(got[h], V[:, (h // 2) * hd:(h // 2 + 1) * hd].mean(0), rtol=1e-5,
                           atol=1e-6)


def test_swiglu_vs_float64():
    g = np.concatenate([np.linspace(-90, 90, 2001), [0.0, -0.0, 1e-30, -1e-30]]).astype(np.float32)
    u = np.random.default_rng(15).standard_normal(g.size).astype(np.float32)
    got = O.swiglu(g, u)
    g64 = g.astype(np.float64)
    want = g64 / (1 + np.exp(-g64)) * u
    assert np.allclose(got, want, rtol=2e-6, atol=1e-30)
    assert got[-4] == 0.0


def test_exp_polynomial_vs_exp():
    x = np.linspace(-87, 88, 100001).astype(np.float32)
    got = np.array([O.orc.orc_exp_cephes(float(v)) for v in x[::97]], np.float64)
    want = np.exp(x[::97].astype(np.float64))
    assert np.all(np.abs(got - want) <= 4e-7 * want)


def test_argmax_first_index_and_margin():
    x = np.array([1.0, 3.0, -np.inf, 3.0, 2.0], np.float32)
    assert O.argmax(x) == 1
    assert O.argmax(np.full(7, -np.inf, np.float32)) == 0
    assert O.top2_margin(np.array([1.0, 4.0, 2.5], np.float32)) == 1.5
