"""The other weight types' GEMVs and embedding rows on the device (Q8_0, Q5_0,
F16; kernels/gemv_misc.hip) against the oracle (tests/test_oracle_misc.py pins
it): GEMVs within the north-star tolerance, embedding rows bit-exact."""
import numpy as np
import pytest

from llm_core_amd import hip
from llm_core_amd._ffi import AXF_TYPE_F16, AXF_TYPE_Q5_0, AXF_TYPE_Q8_0, AxfError, call
from oracle import oracle as O

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def close(gpu, ref):
    err = np.abs(gpu.astype(np.float64) - ref) - (ATOL + RTOL * np.abs(ref))
    return bool(np.all(err <= 0)), float(np.max(np.abs(gpu - ref)))


def blocks(qtype, rows, cols, seed):
    """Random rows of valid blocks: fp16 scales ~1e-2, random integer codes."""
    rng = np.random.default_rng(seed)
    nb = cols // 32
    d = (rng.uniform(0.002, 0.02, (rows, nb)) * rng.choice([-1, 1], (rows, nb))).astype(np.float16)
    if qtype == AXF_TYPE_Q8_0:
        q = rng.integers(-128, 128, (rows, nb, 32)).astype(np.int8)
        return np.concatenate([d.view(np.uint8).reshape(rows, nb, 2), q.view(np.uint8)],
                              axis=2).reshape(-1)
    q = rng.integers(0, 256, (rows, nb, 20)).astype(np.uint8)  # qh (4 B) + qs (16 B)
    return np.concatenate([d.view(np.uint8).reshape(rows, nb, 2), q], axis=2).reshape(-1)


SHAPES = [(1000, 896), (4096, 4096), (77, 2048), (5, 32), (300, 160)]


@pytest.mark.parametrize("rows,cols", SHAPES)
def test_gemv_q8_0w_q8(ctx, rows, cols):
    W = blocks(AXF_TYPE_Q8_0, rows, cols, rows + cols)
    x = np.random.default_rng(cols).standard_normal(cols).astype(np.float32)
    xq = O.quantize_q8_0(x)
    want = O.gemv_q8_0w_q8(W, xq, rows, cols)
    dW, dx, dy = ctx.upload(W), ctx.upload(xq), ctx.upload(np.full(rows, np.nan, np.float32))
    call("axf_hip_gemv_q8_0w_q8", ctx.handle, dy.ptr, dW.ptr, dx.ptr, rows, cols, cols // 32 * 34, 0)
    got = ctx.download(dy, np.float32, rows)
    ok, err = close(got, want)
    assert ok, err
    call("axf_hip_gemv_q8_0w_q8", ctx.handle, dy.ptr, dW.ptr, dx.ptr, rows, cols, cols // 32 * 34, 1)
    ok, err = close(ctx.download(dy, np.float32, rows), 2 * want.astype(np.float64))
    assert ok, err


@pytest.mark.parametrize("qtype", [AXF_TYPE_Q8_0, AXF_TYPE_Q5_0, AXF_TYPE_F16])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_gemv_f32_activation(ctx, qtype, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols)
    if qtype == AXF_TYPE_F16:
        W = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float16)
    else:
        W = blocks(qtype, rows, cols, rows * 3 + cols)
    x = rng.standard_normal(cols).astype(np.float32)
    bias = rng.standard_normal(rows).astype(np.float32) if qtype == AXF_TYPE_F16 else None
    want = O.gemv_misc(qtype, W, x, rows, cols, bias)
    dW, dx, dy = ctx.upload(W), ctx.upload(x), ctx.upload(np.full(rows, np.nan, np.float32))
    if qtype == AXF_TYPE_F16:
        db = ctx.upload(bias)
        call("axf_hip_gemv_f16_f32", ctx.handle, dy.ptr, dW.ptr, dx.ptr, db.ptr, rows, cols)
    else:
        name = "axf_hip_gemv_q8_0w_f32" if qtype == AXF_TYPE_Q8_0 else "axf_hip_gemv_q5_0_f32"
        call(name, ctx.handle, dy.ptr, dW.ptr, dx.ptr, rows, cols, O.misc_row_bytes(qtype, cols))
    ok, err = close(ctx.download(dy, np.float32, rows), want)
    assert ok, err


GEMM_SHAPES = [(4864, 896, 512), (896, 896, 37), (130, 4864, 16), (1000, 64, 3), (64, 32, 70)]


@pytest.mark.parametrize("qtype", [AXF_TYPE_Q8_0, AXF_TYPE_Q5_0, AXF_TYPE_F16])
@pytest.mark.parametrize("rows,cols,T", GEMM_SHAPES)
def test_gemm_f32_rows(ctx, qtype, rows, cols, T):
    """axf_hip_gemm_misc_f32 (the prefill's fp32-row GEMM) against the oracle's
    per-token GEMV (gemv_wt on each row, as gemm_wt_q8's fallback runs it):
    the Qwen2.5-0.5B ffn_gate / attn_q shapes, ragged rows and token groups,
    fewer tokens than one group; then accumulate doubles the product."""
    rng = np.random.default_rng(rows + 13 * cols + T)
    if qtype == AXF_TYPE_F16:
        W = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float16)
    else:
        W = blocks(qtype, rows, cols, rows * 5 + cols)
    X = rng.standard_normal((T, cols)).astype(np.float32)
    check_t = range(T) if T <= 40 else sorted({0, 1, 31, 32, T // 2, T - 1})
    want = {t: O.gemv_misc(qtype, W, X[t], rows, cols) for t in check_t}
    rb = O.misc_row_bytes(qtype, cols)
    dW, dX = ctx.upload(W), ctx.upload(X)
    dY = ctx.upload(np.full(T * rows, np.nan, np.float32))
    call("axf_hip_gemm_misc_f32", ctx.handle, qtype, dY.ptr, dW.ptr, dX.ptr, rows, T, cols, rb, 0)
    got = ctx.download(dY, np.float32, T * rows).reshape(T, rows)
    assert not np.isnan(got).any(), "every output written"
    for t in check_t:
        ok, err = close(got[t], want[t])
        assert ok, f"token {t}: {err}"
    call("axf_hip_gemm_misc_f32", ctx.handle, qtype, dY.ptr, dW.ptr, dX.ptr, rows, T, cols, rb, 1)
    got2 = ctx.download(dY, np.float32, T * rows).reshape(T, rows)
    np.testing.assert_array_equal(got2, got + got)  # y + y: the accumulate adds the same sums


@pytest.mark.parametrize("qtype", [AXF_TYPE_Q8_0, AXF_TYPE_Q5_0, AXF_TYPE_F16])
def test_gemm_f32_rows_activation_scales(ctx, qtype):
    """Token rows of very different magnitudes (1e-7 to 1e4, one row with a
    single 3e4 outlier, one all-zero row): the matrix-core form scales each row
    by its own power of two before the fp16 hi/lo split, so every row keeps
    fp32-level relative accuracy (1e-5 of its own largest output)."""
    rows, cols, T = 200, 896, 48
    rng = np.random.default_rng(77 + qtype)
    if qtype == AXF_TYPE_F16:
        W = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float16)
    else:
        W = blocks(qtype, rows, cols, 91 + qtype)
    mags = np.array([10.0 ** (k % 12 - 7) for k in range(T)], np.float32)
    X = (rng.standard_normal((T, cols)) * mags[:, None]).astype(np.float32)
    X[5, 17] = 3e4
    X[9] = 0.0
    rb = O.misc_row_bytes(qtype, cols)
    dW, dX = ctx.upload(W), ctx.upload(X)
    dY = ctx.upload(np.full(T * rows, np.nan, np.float32))
    call("axf_hip_gemm_misc_f32", ctx.handle, qtype, dY.ptr, dW.ptr, dX.ptr, rows, T, cols, rb, 0)
    got = ctx.download(dY, np.float32, T * rows).reshape(T, rows)
    for t in range(T):
        want = O.gemv_misc(qtype, W, X[t], rows, cols).astype(np.float64)
        scale = float(np.max(np.abs(want)))
        err = float(np.max(np.abs(got[t] - want)))
        assert err <= 1e-5 * scale + (0.0 if scale else 0.0), f"token {t}: {err:.3e} of {scale:.3e}"


def test_gemm_misc_rejects_bad_arguments(ctx):
    W, X, Y = ctx.alloc(1 << 16), ctx.alloc(1 << 16), ctx.alloc(1 << 16)
    with pytest.raises(AxfError, match="multiple of 32"):
        call("axf_hip_gemm_misc_f32", ctx.handle, AXF_TYPE_Q5_0, Y.ptr, W.ptr, X.ptr, 4, 2, 48, 44, 0)
    with pytest.raises(AxfError, match="qtype"):
        call("axf_hip_gemm_misc_f32", ctx.handle, 12, Y.ptr, W.ptr, X.ptr, 4, 2, 256, 144, 0)
    with pytest.raises(AxfError, match="16-byte aligned"):
        call("axf_hip_gemm_misc_f32", ctx.handle, AXF_TYPE_F16, Y.ptr, W.ptr + 2, X.ptr, 4, 2, 64, 128, 0)
    with pytest.raises(AxfError, match="row_bytes"):
        call("axf_hip_gemm_misc_f32", ctx.handle, AXF_TYPE_Q8_0, Y.ptr, W.ptr, X.ptr, 4, 2, 64, 66, 0)


@pytest.mark.parametrize("qtype", [AXF_TYPE_Q8_0, AXF_TYPE_Q5_0, AXF_TYPE_F16])
def test_embed_rows_bitexact(ctx, qtype):
    rows, cols = 50, 896
    if qtype == AXF_TYPE_F16:
        W = np.random.default_rng(2).standard_normal((rows, cols)).astype(np.float16).reshape(-1)
    else:
        W = blocks(qtype, rows, cols, 5)
    rb = O.misc_row_bytes(qtype, cols)
    dW, dy = ctx.upload(W), ctx.alloc(cols * 4)
    for tok in (0, 17, rows - 1):
        call("axf_hip_embed", ctx.handle, dy.ptr, qtype, dW.ptr, tok, rows, cols)
        want = O.dequant_row(qtype, W.view(np.uint8)[tok * rb:(tok + 1) * rb], cols)
        np.testing.assert_array_equal(ctx.download(dy, np.float32, cols), want)


def test_misc_rejects_bad_arguments(ctx):
    W = ctx.alloc(4096)
    x = ctx.alloc(4096)
    y = ctx.alloc(4096)
    with pytest.raises(AxfError, match="multiple of 32"):
        call("axf_hip_gemv_q5_0_f32", ctx.handle, y.ptr, W.ptr, x.ptr, 4, 48, 44)
    with pytest.raises(AxfError, match="2-byte aligned"):
        call("axf_hip_gemv_q8_0w_q8", ctx.handle, y.ptr, W.ptr + 1, x.ptr, 4, 32, 34, 0)
    with pytest.raises(AxfError, match="16-byte aligned"):
        call("axf_hip_gemv_f16_f32", ctx.handle, y.ptr, W.ptr + 2, x.ptr, None, 4, 64)
    with pytest.raises(AxfError, match="row_bytes"):
        call("axf_hip_gemv_q8_0w_f32", ctx.handle, y.ptr, W.ptr, x.ptr, 4, 64, 66)


SMALL = dict(n_layer=2, n_embd=512, n_heads=8, n_kv_heads=4, ffn_dim=1024, n_vocab=1000,
             n_ctx=64, rms_eps=1e-5, rope_theta=10000.0)


@pytest.mark.parametrize("embd,head", [(AXF_TYPE_Q8_0, AXF_TYPE_Q8_0), (AXF_TYPE_F16, AXF_TYPE_Q5_0),
                                       (AXF_TYPE_Q5_0, AXF_TYPE_F16), (12, AXF_TYPE_Q8_0)])
def test_decoder_with_other_embedding_and_head(ctx, embd, head):
    """A model whose token_embd / output are Q8_0, Q5_0 or F16 (the layers
    Q4_K / Q6_K), on both the batched prefill and the decode step, against the
    oracle's decoder: within the tolerance, or within twice the reorder noise
    measured on the same input (the oracle's token path and the GPU's decode
    path, each against the oracle's batch)."""
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    hp = Hparams(**SMALL)
    m = SynthLlama(hp, seed=31, norm_std=0.1, embd_type=embd, head_type=head)
    # 6 tokens: the prefill GEMMs stay on the dot4 kernels, whose order is
    # closest to the oracle's (this test is about the embedding and head)
    toks = np.array([1, 42, 7, 999, 500, 3], np.int32)
    om = O.OracleModel(hp, m.tensors)
    om.forward_batch(toks, 0)
    ol = om.logits().astype(np.float64)
    om.reset()
    for t, tok in enumerate(toks):
        om.forward_token(int(tok), t)
    ot = om.logits().astype(np.float64)
    om.close()
    with LlamaHip(ctx, m) as g:
        g.forward_batch(toks, 0)
        gl = g.logits()
        for t, tok in enumerate(toks):
            g.forward_token(int(tok), t)
        gt = g.logits()
    noise = max(float(np.max(np.abs(ot - ol))), float(np.max(np.abs(gt - ol))))
    for got, ref in ((gl, ol), (gt, ot)):
        ok, err = close(got, ref)
        assert ok or err <= 2 * noise + 1e-4, (err, noise)
