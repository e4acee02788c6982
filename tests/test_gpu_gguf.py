"""GGUF file -> device-resident decoder (axf_llama_from_gguf), against the same
model registered tensor by tensor (axf_llama_set_tensor): the same bytes reach
the same kernels, so logits and greedy tokens must be identical, bit for bit."""
import copy

import numpy as np
import pytest

from llm_core_amd import gguf as G
from llm_core_amd._ffi import AXF_ERR_INVALID_ARG, AXF_ERR_UNSUPPORTED, AxfError
from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

pytestmark = pytest.mark.gpu

SMALL = dict(n_layer=2, n_embd=512, n_heads=8, n_kv_heads=4, ffn_dim=1024, n_vocab=1000,
             n_ctx=64, rms_eps=1e-5, rope_theta=10000.0)


def _same_outputs(ctx, a: LlamaHip, b: LlamaHip, prompt, n_gen=12):
    a.forward_batch(prompt, 0)
    b.forward_batch(prompt, 0)
    la, lb = a.logits(), b.logits()
    assert np.array_equal(la, lb), float(np.max(np.abs(la - lb)))
    ta = a.generate(prompt, n_gen, use_graph=True)
    tb = b.generate(prompt, n_gen, use_graph=True)
    assert np.array_equal(ta, tb), (ta, tb)


@pytest.mark.parametrize("embd,head", [(12, 14), (8, 6), (1, 8)])
def test_llama_file_matches_tensor_api(ctx, tmp_path, embd, head):
    """Q4_K embedding + Q6_K head (Q4_K_M), and the other types the reference's
    embedding and head paths take (Q8_0 / Q5_0 / F16)."""
    hp = Hparams(**SMALL)
    m = SynthLlama(hp, seed=4, norm_std=0.1, embd_type=embd, head_type=head)
    path = G.llama_gguf(m).write(tmp_path / "llama.gguf")
    with LlamaHip.from_gguf(ctx, path) as g, LlamaHip(ctx, m) as ref:
        # context = min(context_length 64, 4096); eps and theta come back as fp32
        assert (g.hp.n_layer, g.hp.n_embd, g.hp.n_heads, g.hp.n_kv_heads, g.hp.ffn_dim,
                g.hp.n_vocab, g.hp.n_ctx) == (2, 512, 8, 4, 1024, 1000, 64)
        assert g.hp.rms_eps == np.float32(1e-5) and g.hp.rope_theta == 10000.0
        assert g.device_bytes() == ref.device_bytes()
        prompt = np.array([1, 17, 400, 9, 999, 3, 250, 42], np.int32)
        _same_outputs(ctx, g, ref, prompt)


def test_qwen2_tied_head_no_vocab_array(ctx, tmp_path):
    """qwen2 metadata with q/k/v biases, no output.weight (the head reuses
    token_embd), no tokenizer array (vocabulary from token_embd's rows), and a
    context capped by max_context_len."""
    hp = Hparams(**SMALL)
    m = SynthLlama(hp, seed=9, norm_std=0.1, with_bias=True)
    path = G.llama_gguf(m, arch="qwen2", tokens=False, tied=True).write(tmp_path / "q.gguf")
    tied = copy.copy(m)
    tied.tensors = {k: v for k, v in m.tensors.items() if k != "output.weight"}
    with LlamaHip.from_gguf(ctx, path, max_context_len=32) as g:
        assert (g.hp.n_vocab, g.hp.n_ctx) == (1000, 32)
        small = copy.copy(tied)
        small.hp = Hparams(**{**SMALL, "n_ctx": 32})
        with LlamaHip(ctx, small) as ref:
            _same_outputs(ctx, g, ref, np.array([1, 5, 6, 7, 8], np.int32), n_gen=8)


@pytest.mark.parametrize("arch,order", [("qwen3", 1), ("hunyuan-dense", 2)])
def test_qk_norm_architectures(ctx, tmp_path, arch, order):
    """qwen3 (per-head q/k norms before RoPE) and hunyuan-dense (after RoPE):
    the order comes from general.architecture (llama_model.cpp:1520-1522), the
    norm weights from blk.N.attn_{q,k}_norm.weight; the file equals the tensor
    API model with that order.  (hunyuan-dense files without
    rope.scaling.alpha keep freq_base unscaled.)"""
    hp = Hparams(**{**SMALL, "qk_norm_order": order})
    m = SynthLlama(hp, seed=12, norm_std=0.2)
    path = G.llama_gguf(m, arch=arch).write(tmp_path / "qk.gguf")
    with LlamaHip.from_gguf(ctx, path) as g, LlamaHip(ctx, m) as ref:
        assert g.hp.qk_norm_order == order
        assert g.device_bytes() == ref.device_bytes()
        _same_outputs(ctx, g, ref, np.array([1, 33, 7, 920, 4, 61], np.int32), n_gen=8)
    # the same weights without the order give other logits (the norms matter)
    plain = copy.copy(m)
    plain.hp = Hparams(**SMALL)
    with LlamaHip(ctx, m) as a, LlamaHip(ctx, plain) as b:
        a.forward_batch(np.array([1, 33, 7], np.int32), 0)
        b.forward_batch(np.array([1, 33, 7], np.int32), 0)
        assert not np.allclose(a.logits(), b.logits(), atol=1e-3)


def _expect_error(ctx, path, code, text):
    with pytest.raises(AxfError) as e:
        LlamaHip.from_gguf(ctx, path)
    assert e.value.code == code and text in str(e.value), str(e.value)


def test_rejected_files(ctx, tmp_path):
    hp = Hparams(**{**SMALL, "n_layer": 1})
    m = SynthLlama(hp, seed=2)
    # a per-head norm weight of the wrong length (qwen3: head_dim floats)
    w = G.llama_gguf(m, arch="qwen3")
    w.add_tensor("blk.0.attn_q_norm.weight", np.ones(32, np.float32), G.GGML_F32, (32,))
    _expect_error(ctx, w.write(tmp_path / "b.gguf"), AXF_ERR_INVALID_ARG, "attn_q_norm")
    # a weight type the decoder does not run (Q4_0 = 2: 18-byte blocks of 32)
    bad = copy.copy(m)
    bad.tensors = dict(m.tensors)
    w = G.llama_gguf(bad)
    w.infos = [i for i in w.infos if b"blk.0.attn_output.weight" not in i]
    w.add_tensor("blk.0.attn_output.weight", np.zeros(512 * 512 // 32 * 18, np.uint8), 2, (512, 512))
    _expect_error(ctx, w.write(tmp_path / "c.gguf"), AXF_ERR_UNSUPPORTED, "GGML type 2")
    # tokenizer vocabulary and token_embd disagree
    w = G.llama_gguf(m, tokens=False)
    w.add_array("tokenizer.ggml.tokens", G.STRING, ["x"] * 999)
    _expect_error(ctx, w.write(tmp_path / "d.gguf"), AXF_ERR_INVALID_ARG, "999 entries")
    # the file ends inside the last tensor's data
    data = G.llama_gguf(m).to_bytes()
    p = tmp_path / "e.gguf"
    p.write_bytes(data[:-100])
    _expect_error(ctx, p, AXF_ERR_INVALID_ARG, "data lies outside the file")
