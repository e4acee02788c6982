"""Op-by-op parity of the fused kernels the decode step runs.

The decode step's layer is five fused launches (q|k|v GEMVs with the RMSNorm
prologue; attention with bias, RoPE and the K/V store; o with x +=; gate|up
with the RMSNorm prologue and the SwiGLU epilogue; down with the Q8_0 prologue
and x +=).  axf_llama_forward_layer_stages runs them one at a time, and
axf_llama_get_buffer / axf_llama_get_kv read back what each wrote, so each is
compared with the oracle on the device's own inputs (no error carried in
from an earlier op):

  * K/V cache rows and the attention output's Q8_0 blocks: bit-exact;
  * projections, attention, residual updates, SwiGLU output: within the
    north-star tolerance |gpu - ref| <= 1e-4 + 1e-3 |ref| (attention within
    1e-6 + 1e-5 |ref|).

The RMSNorm prologues quantise inside the GEMV; their Q8_0 blocks are taken
from the standalone RMSNorm kernel, which shares the prologue's summation
order, and are checked against the oracle's blocks (equal except where the
oracle's value lies within fp32 noise of a rounding boundary).
Reference: llama_forward_token's layer body, llama_model.cpp:1222-1325.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def within(gpu, ref, rtol=1e-3, atol=1e-4):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    bad = np.abs(gpu - ref) > atol + rtol * np.abs(ref)
    return (not bad.any()), float(np.max(np.abs(gpu - ref))), int(bad.sum())


def check(tag, got, want, rtol=1e-3, atol=1e-4):
    ok, err, nbad = within(got, want, rtol, atol)
    print(f"  {tag}: max |err| {err:.3e}", flush=True)
    assert ok, f"{tag}: {nbad} elements outside tolerance, max |err| {err:.3e}"


def device_norm_q8(ctx, x, w, eps):
    """Q8_0 of RMSNorm(x) * w from the device's RMSNorm kernel, checked
    against the oracle's blocks: a block may differ only by a one-step
    rounding of an element whose oracle value x*id sits within 1e-3 of .5."""
    n = x.size
    dx, dw = ctx.upload(np.ascontiguousarray(x, np.float32)), ctx.upload(w)
    y, yq = ctx.alloc(n * 4), ctx.alloc(n // 32 * 36)
    ctx.rmsnorm(y, yq, dx, dw, n, eps)
    got = ctx.download(yq, np.uint8, n // 32 * 36)
    want = O.quantize_q8_0(O.rmsnorm(x, w, eps))
    if not np.array_equal(got, want):
        from qblocks import unpack_q8

        dg, qg = unpack_q8(got)
        dw_, qw = unpack_q8(want)
        xn = O.rmsnorm(x, w, eps).reshape(-1, 32).astype(np.float64)
        frac = np.abs(xn / np.where(dw_ > 0, dw_, 1)[:, None])
        frac = np.abs(frac - np.floor(frac) - 0.5)
        diff = qg != qw
        assert np.all(np.abs(qg - qw) <= 1) and np.all(frac[diff] < 1e-3)
        assert np.allclose(dg, dw_, rtol=1e-6, atol=0)
    return got


def fused_stage_parity(ctx, cfg, prior, with_bias, seed):
    from llm_core_amd import _ffi, hip
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    cfg = dict(cfg)
    cfg["n_vocab"] = 256
    cfg["n_layer"] = 1
    hp = Hparams(n_ctx=prior + 1, **cfg)
    m = SynthLlama(hp, seed=seed, norm_std=0.1, with_bias=with_bias)
    T = {k: v[1] for k, v in m.tensors.items()}
    E, H, KVH, HD, FD = hp.n_embd, hp.n_heads, hp.n_kv_heads, hp.head_dim, hp.ffn_dim
    qo, kvo, pos = H * HD, KVH * HD, prior
    kc = hip.synth_normal(prior * kvo, 41).reshape(prior, kvo)
    vc = hip.synth_normal(prior * kvo, 42).reshape(prior, kvo)
    x0 = hip.synth_normal(E, 43)
    cos_t, sin_t = O.rope_table(HD, hp.rope_theta, hp.n_ctx)
    zero = np.zeros(kvo, np.float32)

    g = LlamaHip(ctx, m)
    try:
        g.set_kv(0, kc, vc, prior)
        g.set_x(x0)

        # 1. q|k|v GEMVs with the attention RMSNorm in the prologue (before bias)
        g.forward_layer_stages(0, pos, 1, 1)
        qkv = g.buffer(_ffi.AXF_LLAMA_BUF_QKV)
        xq = device_norm_q8(ctx, x0, T["blk.0.attn_norm.weight"], hp.rms_eps)
        check("q", qkv[:qo], O.gemv_q8(O.Q4K, T["blk.0.attn_q.weight"], xq, qo, E))
        check("k", qkv[qo:qo + kvo], O.gemv_q8(O.Q4K, T["blk.0.attn_k.weight"], xq, kvo, E))
        check("v", qkv[qo + kvo:], O.gemv_q8(O.Q6K, T["blk.0.attn_v.weight"], xq, kvo, E))

        # 2. attention: bias + RoPE of q and k, K/V row `pos` stored, output and Q8_0
        g.forward_layer_stages(0, pos, 2, 2)
        q = qkv[:qo] + T.get("blk.0.attn_q.bias", np.zeros(qo, np.float32))
        k = qkv[qo:qo + kvo] + T.get("blk.0.attn_k.bias", zero)
        v = qkv[qo + kvo:] + T.get("blk.0.attn_v.bias", zero)
        kr = O.rope(k, pos, KVH, HD, cos_t, sin_t)
        k_dev, v_dev = g.get_kv(0, 0, pos + 1)
        assert np.array_equal(k_dev[pos], kr), "stored K row differs from RoPE(k + bk)"
        assert np.array_equal(v_dev[pos], v), "stored V row differs from v + bv"
        assert np.array_equal(k_dev[:pos], kc) and np.array_equal(v_dev[:pos], vc)
        att_want = O.attention(O.rope(q, pos, H, HD, cos_t, sin_t), k_dev, v_dev, pos + 1, H,
                               KVH, HD)
        att = g.buffer(_ffi.AXF_LLAMA_BUF_ATTN)
        check("attention", att, att_want, 1e-5, 1e-6)
        aq = g.buffer(_ffi.AXF_LLAMA_BUF_ATTN_Q8)
        assert np.array_equal(aq, O.quantize_q8_0(att)), "attention Q8_0 blocks differ"

        # 3. o projection, x += o
        g.forward_layer_stages(0, pos, 3, 3)
        x1 = g.buffer(_ffi.AXF_LLAMA_BUF_X)
        check("x + o", x1, x0 + O.gemv_q8(O.Q4K, T["blk.0.attn_output.weight"], aq, E, qo))

        # 4. gate|up with the FFN RMSNorm prologue and the SwiGLU epilogue
        g.forward_layer_stages(0, pos, 4, 4)
        h = g.buffer(_ffi.AXF_LLAMA_BUF_H)
        xq2 = device_norm_q8(ctx, x1, T["blk.0.ffn_norm.weight"], hp.rms_eps)
        gate = O.gemv_q8(O.Q4K, T["blk.0.ffn_gate.weight"], xq2, FD, E)
        up = O.gemv_q8(O.Q4K, T["blk.0.ffn_up.weight"], xq2, FD, E)
        check("swiglu(gate, up)", h, O.swiglu(gate, up))

        # 5. down projection of Q8_0(h) (quantised in the prologue), x += down
        g.forward_layer_stages(0, pos, 5, 5)
        x2 = g.buffer(_ffi.AXF_LLAMA_BUF_X)
        check("x + down", x2,
              x1 + O.gemv_q8(O.Q6K, T["blk.0.ffn_down.weight"], O.quantize_q8_0(h), E, FD))

        # the whole layer in one call runs the same kernels: the same bits
        g.set_kv(0, kc, vc, prior)
        g.set_x(x0)
        g.forward_layer(0, pos)
        assert np.array_equal(g.get_x(), x2)
    finally:
        g.close()


def test_fused_stages_qwen25_3b(ctx):
    """Config 3: hidden 2048, GQA 16/2 (one query head per attention
    workgroup, only the first stores the K/V row), FFN 11008, KV 1024, biases."""
    from llm_core_amd.model import QWEN25_3B_LAYER

    fused_stage_parity(ctx, QWEN25_3B_LAYER, 1024, True, 3)


def test_fused_stages_llama7b_shape(ctx):
    """The decode benchmark's layer: hidden 4096, 32/32 heads, FFN 11008, ctx 2048."""
    from llm_core_amd.model import LLAMA2_7B

    fused_stage_parity(ctx, LLAMA2_7B, 2047, False, 4)


def test_fused_stages_hidden3072(ctx):
    """Hidden 3072 (12 super-blocks), GQA 24/8, FFN 8192, biases, context 300."""
    cfg = dict(n_embd=3072, n_heads=24, n_kv_heads=8, ffn_dim=8192, rms_eps=1e-6,
               rope_theta=1e6)
    fused_stage_parity(ctx, cfg, 300, True, 5)


def test_layer_stage_arguments(ctx):
    from llm_core_amd._ffi import AxfError
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    hp = Hparams(n_layer=1, n_embd=256, n_heads=4, n_kv_heads=2, ffn_dim=512, n_vocab=64,
                 n_ctx=8)
    g = LlamaHip(ctx, SynthLlama(hp, seed=1))
    try:
        for bad in ((0, 0, 0, 1), (0, 0, 3, 2), (0, 0, 1, 6), (1, 0, 1, 1), (0, 8, 1, 1)):
            with pytest.raises(AxfError):
                g.forward_layer_stages(*bad)
        with pytest.raises(AxfError):
            g.get_kv(0, 4, 5)
    finally:
        g.close()
