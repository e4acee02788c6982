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

from gpu_helpers import layer_stage_errors

pytestmark = pytest.mark.gpu


def fused_stage_parity(ctx, cfg, prior, with_bias, seed):
    from llm_core_amd import hip
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    cfg = dict(cfg)
    cfg["n_vocab"] = 256
    cfg["n_layer"] = 1
    hp = Hparams(n_ctx=prior + 1, **cfg)
    m = SynthLlama(hp, seed=seed, norm_std=0.1, with_bias=with_bias)
    T = {k: v[1] for k, v in m.tensors.items()}
    E, kvo, pos = hp.n_embd, hp.n_kv_heads * hp.head_dim, prior
    kc = hip.synth_normal(prior * kvo, 41).reshape(prior, kvo)
    vc = hip.synth_normal(prior * kvo, 42).reshape(prior, kvo)
    x0 = hip.synth_normal(E, 43)

    g = LlamaHip(ctx, m)
    try:
        g.set_kv(0, kc, vc, prior)
        g.set_x(x0)
        for tag, err, nbad, rel in layer_stage_errors(ctx, g, T, hp, 0, pos):
            print(f"  {tag}: max |err| {err:.3e}, norm-wise {rel:.2e}", flush=True)
            assert nbad == 0, f"{tag}: {nbad} elements outside tolerance, max |err| {err:.3e}"
        x2 = g.get_x()

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


def test_fused_stages_qk_norm_before_rope(ctx):
    """Per-head q/k RMSNorm before RoPE (qwen3): bias, norm, RoPE of q and of
    the stored K row (bit-exact), then the same attention and FFN stages."""
    cfg = dict(n_embd=2048, n_heads=16, n_kv_heads=8, ffn_dim=6144, rms_eps=1e-6,
               rope_theta=1e6, qk_norm_order=1)
    fused_stage_parity(ctx, cfg, 700, True, 6)


def test_fused_stages_qk_norm_after_rope(ctx):
    """Per-head q/k RMSNorm after RoPE (hunyuan-dense)."""
    cfg = dict(n_embd=1024, n_heads=8, n_kv_heads=2, ffn_dim=3072, rms_eps=1e-5,
               rope_theta=1e4, qk_norm_order=2)
    fused_stage_parity(ctx, cfg, 129, False, 7)


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
