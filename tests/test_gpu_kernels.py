"""GPU parity of every kernel of the path against the CPU oracle (which is
itself bit-exact against the reference's compiled x86 kernels, see
test_oracle_ref.py).  Integer/byte work and dequantisation are compared bit
for bit; fp32 reductions within |gpu - ref| <= 1e-4 + 1e-3*|ref| (the
north-star GEMV tolerance) unless a tighter bound is stated."""
import ctypes as C

import functools

import numpy as np
import pytest

from llm_core_amd._ffi import call

from oracle import oracle as O

pytestmark = pytest.mark.gpu

Q4K, Q6K = 12, 14
RTOL, ATOL = 1e-3, 1e-4


def close(gpu, ref, rtol=RTOL, atol=ATOL):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(gpu - ref) - (atol + rtol * np.abs(ref))
    return bool(np.all(err <= 0)), float(np.max(np.abs(gpu - ref)) if gpu.size else 0.0)


def weights(qtype, rows, cols, seed):
    from llm_core_amd import hip
    return hip.synth_weight(qtype, rows, cols, seed)


def finite_random_blocks(qtype, nblocks, seed):
    """Random bytes with finite fp16 scales (zero, subnormal and normal)."""
    rng = np.random.default_rng(seed)
    bb = O.BLOCK_BYTES[qtype]
    blk = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    h = rng.integers(0, 0x7c00, size=(nblocks, 2), dtype=np.uint16)  # exponent < 31
    h |= (rng.integers(0, 2, size=(nblocks, 2), dtype=np.uint16) << 15)
    h[0] = 0
    hb = h.view(np.uint8).reshape(nblocks, 4)
    if qtype == Q4K:
        blk[:, 0:4] = hb
    else:
        blk[:, 208:210] = hb[:, 0:2]
    return blk.reshape(-1)


# ---------------------------------------------------------------------------
# dequantisation / quantisation (bit-exact)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("qtype", [Q4K, Q6K])
@pytest.mark.parametrize("kind", ["synthetic", "random_bytes"])
def test_dequant_bitexact(ctx, qtype, kind):
    nb = 1031
    blk = weights(qtype, nb, 256, 3) if kind == "synthetic" else finite_random_blocks(qtype, nb, 4)
    W = ctx.upload(blk)
    y = ctx.alloc(nb * 256 * 4)
    ctx.dequant(qtype, y, W, nb)
    got = ctx.download(y, np.float32, nb * 256)
    want = O.dequant(qtype, blk)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_quantize_q8_0_bitexact(ctx):
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(4096) * rng.choice([1e-30, 1e-3, 1.0, 1e3], 4096)).astype(np.float32)
    # edge blocks: all zero; exact .5 ties (amax 127 -> id == 1); one large outlier
    x[:32] = 0
    x[32:64] = np.arange(-15.5, 16.5, 1.0, dtype=np.float32)
    x[63] = 127.0
    x[64:96] = 1e-3
    x[64] = 1e6
    # tiny blocks: 127/amax overflows to +inf below amax = 127/FLT_MAX (every
    # value -128, as the reference's cvtps_epi32 + packs), just above it, and
    # subnormal values, each with zeros beside them
    lim = np.float32(127.0) / np.finfo(np.float32).max
    for b, m in enumerate([lim * np.float32(0.5), np.nextafter(lim, np.float32(1)),
                           np.float32(1e-39), np.float32(3e-37)]):
        blk = x[96 + 32 * b:128 + 32 * b]
        blk[:] = 0
        blk[1::3] = m
        blk[2::3] = -m * np.float32(0.5)
    xd = ctx.upload(x)
    q = ctx.alloc(4096 // 32 * 36)
    ctx.quantize_q8_0(q, xd, 4096)
    got = ctx.download(q, np.uint8, 4096 // 32 * 36)
    assert np.array_equal(got, O.quantize_q8_0(x))


def test_q8_0_zero_length_and_bad_n(ctx):
    from llm_core_amd._ffi import AxfError
    xd = ctx.alloc(256)
    ctx.quantize_q8_0(xd, xd, 0)  # no-op
    with pytest.raises(AxfError):
        ctx.quantize_q8_0(xd, xd, 33)


# ---------------------------------------------------------------------------
# GEMV
# ---------------------------------------------------------------------------

GEMV_SHAPES = [
    (Q4K, 4096, 4096),   # config 1
    (Q4K, 1, 256),
    (Q4K, 37, 512),
    (Q4K, 100, 2048),
    (Q4K, 75, 11008),    # 43 blocks per row
    (Q4K, 33, 16384),
    (Q4K, 21, 2304),     # half-block units: 18 per row, 14 idle lanes of 32
    (Q4K, 1001, 4096),   # half-block units, last workgroup partly past the rows
    (Q6K, 1, 256),
    (Q6K, 37, 2048),
    (Q6K, 1, 2048),      # 1680-byte rows: Q8_0 GEMV rows staged in LDS, one row
    (Q6K, 70, 2048),     # ... three workgroups, the last with 6 of its 32 rows
    (Q6K, 64, 4096),
    (Q6K, 23, 2304),     # half-block units on 1890-byte rows (odd rows 2-byte aligned)
    (Q6K, 77, 3072),
    (Q6K, 101, 11008),   # 9030-byte rows: odd rows start 2 bytes past a dword
    (Q6K, 17, 14336),
    # half-block units of 16 lanes (5-8 blocks per row): 10 of 16 lanes live at
    # 5 blocks, 2-byte-aligned Q6_K rows of 1050 and 1470 bytes, ragged row counts
    (Q4K, 45, 1280),
    (Q6K, 9, 1280),
    (Q6K, 33, 1792),
]


@pytest.mark.parametrize("qtype,rows,cols", GEMV_SHAPES)
def test_gemv_q8(ctx, qtype, rows, cols):
    W = weights(qtype, rows, cols, rows + cols)
    x = (np.random.default_rng(rows).standard_normal(cols)).astype(np.float32)
    xq = O.quantize_q8_0(x)
    want = O.gemv_q8(qtype, W, xq, rows, cols)
    dW, dx, dy = ctx.upload(W), ctx.upload(xq), ctx.alloc(rows * 4)
    ctx.gemv_q8(qtype, dy, dW, dx, rows, cols, O.row_bytes(qtype, cols))
    ok, err = close(ctx.download(dy, np.float32, rows), want)
    assert ok, f"max abs err {err}"


@pytest.mark.parametrize("qtype,rows,cols", [s for s in GEMV_SHAPES if s[2] <= 11008])
def test_gemv_f32(ctx, qtype, rows, cols):
    W = weights(qtype, rows, cols, 3 * rows + cols)
    x = (np.random.default_rng(cols).standard_normal(cols)).astype(np.float32)
    want = O.gemv_f32(qtype, W, x, rows, cols)
    dW, dx, dy = ctx.upload(W), ctx.upload(x), ctx.alloc(rows * 4)
    ctx.gemv_f32(qtype, dy, dW, dx, rows, cols, O.row_bytes(qtype, cols))
    got = ctx.download(dy, np.float32, rows)
    ok, err = close(got, want)
    assert ok, f"max abs err {err}"
    # and against a float64 product of the bit-exact dequantised weights
    d = O.dequant(qtype, W).reshape(rows, cols).astype(np.float64)
    ok, err = close(got, d @ x.astype(np.float64))
    assert ok, f"vs float64: {err}"


@pytest.mark.parametrize("qtype", [Q4K, Q6K])
def test_gemv_accumulate(ctx, qtype):
    rows, cols = 300, 2048
    W = weights(qtype, rows, cols, 9)
    x = np.random.default_rng(1).standard_normal(cols).astype(np.float32)
    y0 = np.random.default_rng(2).standard_normal(rows).astype(np.float32)
    xq = O.quantize_q8_0(x)
    dW, dx, dy = ctx.upload(W), ctx.upload(xq), ctx.upload(y0)
    ctx.gemv_q8(qtype, dy, dW, dx, rows, cols, O.row_bytes(qtype, cols), accumulate=True)
    want = y0 + O.gemv_q8(qtype, W, xq, rows, cols)
    ok, err = close(ctx.download(dy, np.float32, rows), want)
    assert ok, err


def test_gemv_rejects_bad_arguments(ctx):
    from llm_core_amd._ffi import AXF_ERR_INVALID_ARG, AXF_ERR_UNSUPPORTED, AxfError
    W = ctx.alloc(1 << 20)
    x = ctx.alloc(1 << 16)
    y = ctx.alloc(1 << 16)
    with pytest.raises(AxfError) as e:  # cols not a multiple of 256
        ctx.gemv_q8(Q4K, y, W, x, 4, 300, 144)
    assert e.value.code == AXF_ERR_INVALID_ARG
    with pytest.raises(AxfError) as e:  # Q4_K weights must be 16-byte aligned
        ctx.gemv_q8(Q4K, y, W.at(8), x, 4, 256, 144)
    assert e.value.code == AXF_ERR_INVALID_ARG
    with pytest.raises(AxfError) as e:  # row_bytes below one row
        ctx.gemv_q8(Q6K, y, W, x, 4, 512, 210)
    assert e.value.code == AXF_ERR_INVALID_ARG
    with pytest.raises(AxfError) as e:  # above the largest supported K
        ctx.gemv_q8(Q4K, y, W, x, 1, 33024, 129 * 144)
    assert e.value.code == AXF_ERR_UNSUPPORTED
    with pytest.raises(AxfError) as e:  # F32 activation too large for LDS staging
        ctx.gemv_f32(Q6K, y, W, x, 1, 16384, 64 * 210)
    assert e.value.code == AXF_ERR_UNSUPPORTED
    ctx.gemv_q8(Q4K, y, W, x, 0, 256, 144)  # empty: no-op


# ---------------------------------------------------------------------------
# batched Q4_K x Q8_0
# ---------------------------------------------------------------------------

GEMM_CASES = [(11008, 4096, 1), (11008, 4096, 4), (1024, 4096, 16), (512, 4096, 64),
              (11008, 4096, 16), (11008, 4096, 64),  # config 4 at full size
              (75, 11008, 5), (33, 256, 9), (40, 512, 17), (300, 1024, 33), (64, 768, 130),
              # the fp16 matrix-core kernel (65+ tokens): ragged 128-row and 64-token tiles
              # (32-row tiles below 256 workgroups of 64 rows)
              (300, 1024, 200), (520, 2048, 65), (1100, 4096, 96),
              # rows % 4 != 0: the epilogue's per-row stores instead of 16-byte ones
              (301, 1024, 70), (1026, 2048, 96),
              # 64-row tiles (fewer than 256 workgroups of 128 rows)
              (1536, 1024, 512)]


@functools.lru_cache(maxsize=2)
def gemm_case_data(rows, cols, T):
    """Weights, Q8_0 activations and the oracle's product, shared by the four paths."""
    W = weights(Q4K, rows, cols, 4)
    X = np.random.default_rng(T).standard_normal(T * cols).astype(np.float32)
    XQ = O.quantize_q8_0(X)
    return W, XQ, O.gemm_q4k_q8(W, XQ, rows, T, cols)


@pytest.mark.parametrize("path", [None, 1, 2, 3], ids=["auto", "dot4", "mfma", "stream"])
@pytest.mark.parametrize("rows,cols,T", GEMM_CASES)
def test_gemm_q4k_q8(ctx, rows, cols, T, path):
    W, XQ, want = gemm_case_data(rows, cols, T)
    dW, dX, dY = ctx.upload(W), ctx.upload(XQ), ctx.alloc(T * rows * 4)
    ctx.write(dY, np.full(T * rows, np.nan, np.float32))  # every output must be written
    ctx.gemm_q4k_q8(dY, dW, dX, rows, T, cols, O.row_bytes(Q4K, cols), path=path)
    got = ctx.download(dY, np.float32, T * rows).reshape(T, rows)
    ok, err = close(got, want)
    assert ok, err
    # row t of the batched product equals the GEMV of token t (the matrix-core
    # kernel sums in another order: same tolerance scale as float reordering)
    t = T // 2
    dy = ctx.alloc(rows * 4)
    ctx.gemv_q8(Q4K, dy, dW, dX.at(t * cols // 32 * 36), rows, cols, O.row_bytes(Q4K, cols))
    tol = dict(rtol=1e-5, atol=1e-6) if path not in (2, 3) and not (path is None and T >= 2) else \
        dict(rtol=1e-4, atol=1e-5)
    ok, err = close(got[t], ctx.download(dy, np.float32, rows), **tol)
    assert ok, err


def test_gemm_q4k_q8_wide_kernel_matches_int8_kernel(ctx):
    """The fp16 matrix-core kernel (65+ tokens) computes the int8 kernel's
    sums (sc * S exact in both): token t's row depends on token t alone, so
    the first 64 rows of a 130-token product match the 64-token product (int8
    kernel) up to the order of the sub-block sums (the int8 kernel splits a
    tile's sub-blocks over two waves at 64 tokens): fp32 rounding only."""
    rows, cols = 300, 2048
    W = weights(Q4K, rows, cols, 9)
    X = np.random.default_rng(130).standard_normal(130 * cols).astype(np.float32)
    XQ = O.quantize_q8_0(X)
    dW, dX = ctx.upload(W), ctx.upload(XQ)
    rb = O.row_bytes(Q4K, cols)
    out = {}
    for T in (130, 64):
        dY = ctx.alloc(T * rows * 4)
        ctx.gemm_q4k_q8(dY, dW, dX, rows, T, cols, rb, path=2)
        out[T] = ctx.download(dY, np.float32, T * rows).reshape(T, rows)
    np.testing.assert_allclose(out[130][:64], out[64], rtol=1e-5, atol=1e-5)


GEMM6_CASES = [(4096, 4096, 1), (4096, 11008, 4), (512, 11008, 9), (2048, 2048, 17),
               (40, 512, 8), (300, 1024, 33), (256, 2048, 64), (64, 768, 130), (75, 512, 12),
               (90, 768, 24), (6, 256, 8),
               # the wider tiles: 64x64 (ragged rows and tokens), 32x32, 16x16
               (4096, 768, 256), (4100, 768, 250), (2048, 1280, 128), (2040, 1280, 120),
               # the 7B down projection at config-4 token counts
               (4096, 11008, 16), (4096, 11008, 64),
               # the fp16 kernel (128 x 64 tiles, taken from 256 such tiles):
               # exactly 256 tiles, ragged rows and tokens, one super-block
               (4096, 2048, 512), (4100, 1024, 520), (16384, 256, 70)]


def _gemm6_want(W, XQ, rows, cols, T):
    bpt = cols // 32 * 36
    return np.stack([O.gemv_q8(Q6K, W, XQ[t * bpt:(t + 1) * bpt], rows, cols) for t in range(T)])


@pytest.mark.parametrize("path", [None, 1, 2], ids=["auto", "dot4", "mfma"])
@pytest.mark.parametrize("rows,cols,T", GEMM6_CASES)
def test_gemm_q6k_q8(ctx, rows, cols, T, path):
    """Batched Q6_K: row t equals the oracle's per-token GEMV of token t (the
    reference's gemm_wt_q8 runs gemv_q6k_q8 per token for Q6_K weights).  The
    matrix sits at the 4-byte-aligned offset that makes it end on a 16-byte
    boundary, so the matrix-core kernel runs for path 2 (and auto from 8 tokens)
    also where W itself is not 16-byte aligned."""
    W = weights(Q6K, rows, cols, 6)
    X = np.random.default_rng(T + 1).standard_normal(T * cols).astype(np.float32)
    XQ = O.quantize_q8_0(X)
    want = _gemm6_want(W, XQ, rows, cols, T)
    off = -W.size % 16
    assert off % 4 == 0
    dW = ctx.alloc(off + W.size)
    ctx.write(dW.at(off), W)
    dX, dY = ctx.upload(XQ), ctx.alloc(T * rows * 4)
    ctx.write(dY, np.full(T * rows, np.nan, np.float32))  # every output must be written
    ctx.gemm_q6k_q8(dY, dW.at(off), dX, rows, T, cols, O.row_bytes(Q6K, cols), path=path)
    got = ctx.download(dY, np.float32, T * rows).reshape(T, rows)
    ok, err = close(got, want)
    assert ok, err


@pytest.mark.parametrize("lead", [0, 8, 12])
def test_gemm_q6k_q8_unaligned_end(ctx, lead):
    """A Q6_K matrix whose end is not 16-byte aligned takes the dot4 kernel on
    every path (the matrix-core kernel's aligned spans would read past it):
    still exact against the oracle, with the matrix ending at its allocation's
    last byte."""
    rows, cols, T = 75, 512, 16   # 75 rows x 420 B: 31500 B, 12 mod 16
    W = weights(Q6K, rows, cols, 7)
    assert (lead + W.size) % 16 != 0
    X = np.random.default_rng(3).standard_normal(T * cols).astype(np.float32)
    XQ = O.quantize_q8_0(X)
    want = _gemm6_want(W, XQ, rows, cols, T)
    dW = ctx.alloc(lead + W.size)
    ctx.write(dW.at(lead), W)
    dX, dY = ctx.upload(XQ), ctx.alloc(T * rows * 4)
    for path in (None, 2):
        ctx.write(dY, np.full(T * rows, np.nan, np.float32))
        ctx.gemm_q6k_q8(dY, dW.at(lead), dX, rows, T, cols, O.row_bytes(Q6K, cols), path=path)
        got = ctx.download(dY, np.float32, T * rows).reshape(T, rows)
        ok, err = close(got, want)
        assert ok, (path, err)


# ---------------------------------------------------------------------------
# decode-step operations
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 2, 255, 256, 257, 32000, 151936])
def test_argmax_first_index(ctx, n):
    rng = np.random.default_rng(n)
    x = rng.standard_normal(n).astype(np.float32)
    if n > 10:
        x[n // 3] = x[n - 2] = x.max() + 1.0  # tie: the first index wins
    dx, di = ctx.upload(x), ctx.alloc(4)
    ctx.argmax(di, dx, n)
    assert int(ctx.download(di, np.int32, 1)[0]) == O.argmax(x) == int(np.argmax(x))


def test_argmax_all_equal_and_neg_inf(ctx):
    x = np.full(5000, -np.inf, np.float32)
    x[4000:] = -1.0
    dx, di = ctx.upload(x), ctx.alloc(4)
    ctx.argmax(di, dx, x.size)
    assert int(ctx.download(di, np.int32, 1)[0]) == 4000


@pytest.mark.parametrize("n", [32, 2048, 4096, 11008])
def test_rmsnorm(ctx, n):
    x = np.random.default_rng(n).standard_normal(n).astype(np.float32) * 3
    w = (1 + 0.1 * np.random.default_rng(n + 1).standard_normal(n)).astype(np.float32)
    dx, dw, dy, dq = ctx.upload(x), ctx.upload(w), ctx.alloc(n * 4), ctx.alloc(n // 32 * 36)
    ctx.rmsnorm(dy, dq, dx, dw, n, 1e-6)
    got = ctx.download(dy, np.float32, n)
    ok, err = close(got, O.rmsnorm(x, w, 1e-6), rtol=2e-6, atol=1e-7)
    assert ok, err
    # the fused Q8_0 output is the Q8_0 of the fused f32 output
    assert np.array_equal(ctx.download(dq, np.uint8, n // 32 * 36), O.quantize_q8_0(got))


def test_rmsnorm_closed_form(ctx):
    # reference tests/test_backend_x86.cpp:84-116: x = 1..8 (tiled), w = 1
    x = np.tile(np.arange(1, 9, dtype=np.float32), 4)
    w = np.ones(32, np.float32)
    dx, dw, dy = ctx.upload(x), ctx.upload(w), ctx.alloc(128)
    ctx.rmsnorm(dy, None, dx, dw, 32, 1e-5)
    want = x / np.sqrt(np.float32(204.0 / 8.0 + 1e-5))
    assert np.allclose(ctx.download(dy, np.float32, 32), want, rtol=1e-6, atol=0)


@pytest.mark.parametrize("hd,n_heads", [(128, 16), (64, 4), (128, 2)])
def test_rope_bitexact(ctx, hd, n_heads):
    from llm_core_amd import hip
    max_pos = 300
    c, s = hip.rope_table(hd, 1e6, max_pos)
    oc, os_ = O.rope_table(hd, 1e6, max_pos)
    assert np.array_equal(c, oc) and np.array_equal(s, os_)
    dc, ds = ctx.upload(c), ctx.upload(s)
    x = np.random.default_rng(hd).standard_normal(n_heads * hd).astype(np.float32)
    dx, dy = ctx.upload(x), ctx.alloc(x.nbytes)
    for pos in (0, 1, 17, max_pos - 1):
        ctx.rope(dy, dx, pos, n_heads, hd, dc, ds)
        got = ctx.download(dy, np.float32, x.size)
        assert np.array_equal(got, O.rope(x, pos, n_heads, hd, oc, os_))
    ctx.rope(dx, dx, 5, n_heads, hd, dc, ds)  # in place
    assert np.array_equal(ctx.download(dx, np.float32, x.size), O.rope(x, 5, n_heads, hd, oc, os_))


@pytest.mark.parametrize("seq,H,KVH,hd", [(1, 16, 2, 128), (5, 16, 2, 128), (64, 4, 4, 64),
                                          (65, 8, 2, 128), (1024, 16, 2, 128), (2048, 32, 32, 128),
                                          (300, 4, 1, 256),
                                          # more splits than one pass of the combine's threads
                                          # (32 at head dim 128, 64 at 64)
                                          (3000, 8, 2, 128), (4200, 4, 4, 64)])
def test_attention(ctx, seq, H, KVH, hd):
    rng = np.random.default_rng(seq + H)
    q = rng.standard_normal(H * hd).astype(np.float32)
    kc = rng.standard_normal(seq * KVH * hd).astype(np.float32)
    vc = rng.standard_normal(seq * KVH * hd).astype(np.float32)
    dq, dk, dv = ctx.upload(q), ctx.upload(kc), ctx.upload(vc)
    do, dq8 = ctx.alloc(H * hd * 4), ctx.alloc(H * hd // 32 * 36)
    ctx.attn_decode(do, dq8, dq, dk, dv, seq, H, KVH, hd)
    got = ctx.download(do, np.float32, H * hd)
    want = O.attention(q, kc, vc, seq, H, KVH, hd)
    ok, err = close(got, want, rtol=1e-5, atol=1e-6)
    assert ok, err
    if seq == 1:  # a single position returns V of its kv head exactly
        assert np.array_equal(got.reshape(H, hd), np.repeat(vc.reshape(KVH, hd), H // KVH, 0))
    assert np.array_equal(ctx.download(dq8, np.uint8, H * hd // 32 * 36), O.quantize_q8_0(got))


@pytest.mark.parametrize("hd,H,KVH,T,pos0", [(128, 32, 32, 64, 0), (128, 16, 2, 48, 100),
                                             (64, 8, 4, 37, 5), (256, 8, 8, 20, 40),
                                             (128, 14, 2, 70, 0), (128, 32, 32, 256, 256),
                                             (64, 8, 2, 1, 0), (128, 16, 2, 9, 3000),
                                             # 12 kv heads, one query head each
                                             (64, 12, 12, 33, 7)])
def test_attn_prefill(ctx, hd, H, KVH, T, pos0):
    """Causal multi-row attention (bias and RoPE of q inside): the matrix-core
    kernel and the split/combine token grid against the oracle's per-row
    attention; Q8_0 blocks bit-exact against the oracle's quantiser."""
    n = pos0 + T
    rng = np.random.default_rng(T * 7 + pos0 + hd)
    q = rng.standard_normal((T, H * hd)).astype(np.float32)
    bq = (rng.standard_normal(H * hd) * 0.1).astype(np.float32)
    kc = rng.standard_normal(n * KVH * hd).astype(np.float32)
    vc = rng.standard_normal(n * KVH * hd).astype(np.float32)
    cos_t, sin_t = O.rope_table(hd, 10000.0, n)
    want = np.stack([O.attention(O.rope(q[t] + bq, pos0 + t, H, hd, cos_t, sin_t), kc, vc,
                                 pos0 + t + 1, H, KVH, hd) for t in range(T)])
    dq, dbq, dk, dv = ctx.upload(q), ctx.upload(bq), ctx.upload(kc), ctx.upload(vc)
    dc, ds = ctx.upload(cos_t), ctx.upload(sin_t)
    do, dq8 = ctx.alloc(T * H * hd * 4), ctx.alloc(T * H * hd // 32 * 36)
    for path in (0, 1):
        ctx.write(do, np.full(T * H * hd, np.nan, np.float32))
        call("axf_hip_attn_prefill", ctx.handle, do.ptr, dq8.ptr, dq.ptr, H * hd, dbq.ptr, dk.ptr,
             dv.ptr, pos0, T, H, KVH, hd, dc.ptr, ds.ptr, path)
        got = ctx.download(do, np.float32, T * H * hd).reshape(T, H * hd)
        ok, err = close(got, want, rtol=1e-5, atol=1e-6)
        assert ok, (path, err)
        assert np.array_equal(ctx.download(dq8, np.uint8, T * H * hd // 32 * 36),
                              O.quantize_q8_0(got.reshape(-1))), path


@pytest.mark.parametrize("n", [32, 11008])
def test_swiglu_bitexact(ctx, n):
    rng = np.random.default_rng(n)
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    g[:4] = [0.0, -0.0, 100.0, -100.0]
    u = rng.standard_normal(n).astype(np.float32)
    dg, du, do, dq = ctx.upload(g), ctx.upload(u), ctx.alloc(n * 4), ctx.alloc(n // 32 * 36)
    ctx.swiglu(do, dq, dg, du, n)
    got = ctx.download(do, np.float32, n)
    assert np.array_equal(got, O.swiglu(g, u))
    assert np.array_equal(ctx.download(dq, np.uint8, n // 32 * 36), O.quantize_q8_0(got))


@pytest.mark.parametrize("qtype", [Q4K, Q6K])
def test_embed_row_bitexact(ctx, qtype):
    rows, cols = 50, 2048
    W = weights(qtype, rows, cols, 12)
    dW, do = ctx.upload(W), ctx.alloc(cols * 4)
    for tok in (0, 7, rows - 1):
        ctx.embed(do, qtype, dW, tok, rows, cols)
        want = O.dequant(qtype, W).reshape(rows, cols)[tok]
        assert np.array_equal(ctx.download(do, np.float32, cols), want)
    from llm_core_amd._ffi import AxfError
    with pytest.raises(AxfError):
        ctx.embed(do, qtype, dW, rows, rows, cols)


def test_add(ctx):
    a = np.arange(1000, dtype=np.float32)
    b = np.ones(1000, np.float32) * 0.5
    da, db, dy = ctx.upload(a), ctx.upload(b), ctx.alloc(4000)
    ctx.add(dy, da, db, 1000)
    assert np.array_equal(ctx.download(dy, np.float32, 1000), a + b)
