"""Pins of the oracle's decoder composition for layer matrices of the other
GGUF weight types (Q8_0, Q5_0, F16) and hidden sizes that are not a multiple
of 256, by closed forms.

The reference routes every layer matrix through gemv_wt_q8 in the decode step
(/root/reference/src/models/llama_model.cpp:767-831) and gemm_wt_q8 in the
batched prefill (:837-879):
  * decode: Q4_K / Q6_K / Q8_0 weights take the Q8_0 activation (Q8_0 through
    gemv_q8_0_weight_q8, :825-828); Q5_0 and F16 weights take the fp32
    activation through gemv_wt (:830; q5_0_dot_row :713-724, the F16 GEMV
    :672-680) - the normalised row xb, the attention output, or the SwiGLU
    output;
  * prefill: only Q4_K and Q6_K take Q8_0 activations; Q8_0 weights, like
    Q5_0 and F16, fall back to gemv_wt per token with the fp32 rows
    (q8_0_weight_dot_row, :701-712; the fallback loop :876-879).
Identity matrices of each type make these paths visible: with fp32
activations the GEMV returns its input exactly; with Q8_0 activations it
returns the input's Q8_0 dequantisation.  Each test checks that the other
choice would give a different result, so taking the wrong activation fails.
The oracle's per-type GEMVs are pinned on their own (tests/test_oracle_misc.py:
F16 bit-exact against the compiled reference, Q8_0 / Q5_0 by hand-built blocks).
"""
from dataclasses import dataclass

import numpy as np
import pytest

from oracle import oracle as O
from qblocks import F16W, F32, Q4K, Q5_0W, Q8_0W, dequant_q8, misc_identity, misc_random
from test_oracle_compose import HP, expand_gqa, f32, random_model, rope_tab

TYPES = [Q8_0W, Q5_0W, F16W]


def decode_act(qt: int, xf: np.ndarray) -> np.ndarray:
    """What an identity GEMV of type qt returns in the decode step."""
    return dequant_q8(O.quantize_q8_0(xf)) if qt == Q8_0W else xf


def gemv_any(t: dict, name: str, xq8, xf, rows: int, cols: int) -> np.ndarray:
    """gemv_wt_q8's dispatch on the oracle's pinned GEMVs."""
    qt, w = t[name]
    if qt in (Q4K, 14):
        return O.gemv_q8(qt, w, xq8, rows, cols)
    if qt == Q8_0W:
        return O.gemv_q8_0w_q8(w, xq8, rows, cols)
    return O.gemv_misc(qt, w, xf, rows, cols)


@pytest.mark.parametrize("qt", TYPES)
def test_decode_v_projection_takes_the_reference_activation(qt):
    hp = HP()
    t = random_model(hp, seed=11)
    kvo = hp.n_kv_heads * hp.head_dim
    t["blk.0.attn_v.weight"] = (qt, misc_identity(qt, kvo, hp.n_embd))
    t["blk.0.attn_output.weight"] = (Q4K, np.zeros(hp.n_embd * (hp.n_embd // 256) * 144, np.uint8))
    t["blk.0.ffn_norm.weight"] = (F32, np.zeros(hp.n_embd, np.float32))
    m = O.OracleModel(hp, t)
    try:
        x = f32(np.random.default_rng(12).standard_normal(hp.n_embd))
        m.x_view()[:] = x
        pos = 3
        m.forward_layer(0, pos)
        xn = O.rmsnorm(x, t["blk.0.attn_norm.weight"][1], hp.rms_eps)
        want = decode_act(qt, xn)[:kvo] + t["blk.0.attn_v.bias"][1]
        _, v = m.kv_view()
        assert np.array_equal(v[0, pos], want)
        other = (xn if qt == Q8_0W else dequant_q8(O.quantize_q8_0(xn)))[:kvo] + t["blk.0.attn_v.bias"][1]
        assert not np.array_equal(other, want)
    finally:
        m.close()


@pytest.mark.parametrize("qt", TYPES)
def test_decode_o_projection_takes_the_attention_output(qt):
    hp = HP()
    t = random_model(hp, seed=13)
    t["blk.0.attn_output.weight"] = (qt, misc_identity(qt, hp.n_embd, hp.n_embd))
    t["blk.0.ffn_norm.weight"] = (F32, np.zeros(hp.n_embd, np.float32))
    m = O.OracleModel(hp, t)
    try:
        x = f32(np.random.default_rng(14).standard_normal(hp.n_embd))
        m.x_view()[:] = x
        m.forward_layer(0, 0)  # one position: the attention output is V of each head's kv head
        kvo = hp.n_kv_heads * hp.head_dim
        xq = O.quantize_q8_0(O.rmsnorm(x, t["blk.0.attn_norm.weight"][1], hp.rms_eps))
        v0 = O.gemv_q8(14, t["blk.0.attn_v.weight"][1], xq, kvo, hp.n_embd) + t["blk.0.attn_v.bias"][1]
        att = expand_gqa(v0, hp)
        assert np.array_equal(m.attn_out_view(), att)
        assert np.array_equal(m.x_view(), x + decode_act(qt, att))
        alt = att if qt == Q8_0W else dequant_q8(O.quantize_q8_0(att))
        assert not np.array_equal(x + alt, x + decode_act(qt, att))
    finally:
        m.close()


@pytest.mark.parametrize("qt", TYPES)
def test_decode_down_projection_takes_the_swiglu_output(qt):
    hp = HP()
    t = random_model(hp, seed=15)
    t["blk.0.attn_output.weight"] = (Q4K, np.zeros(hp.n_embd * (hp.n_embd // 256) * 144, np.uint8))
    t["blk.0.ffn_down.weight"] = (qt, misc_identity(qt, hp.n_embd, hp.ffn_dim))
    m = O.OracleModel(hp, t)
    try:
        x = f32(np.random.default_rng(16).standard_normal(hp.n_embd))
        m.x_view()[:] = x
        m.forward_layer(0, 2)
        E, FD = hp.n_embd, hp.ffn_dim
        xq = O.quantize_q8_0(O.rmsnorm(x, t["blk.0.ffn_norm.weight"][1], hp.rms_eps))
        h = O.swiglu(O.gemv_q8(Q4K, t["blk.0.ffn_gate.weight"][1], xq, FD, E),
                     O.gemv_q8(Q4K, t["blk.0.ffn_up.weight"][1], xq, FD, E))
        assert np.array_equal(m.h_view(), h)
        assert np.array_equal(m.x_view(), x + decode_act(qt, h)[:E])
    finally:
        m.close()


@pytest.mark.parametrize("qt", TYPES)
def test_prefill_takes_fp32_rows_for_every_other_type(qt):
    """Batched prefill: Q8_0 weights too take the fp32 rows (gemm_wt_q8 has no
    Q8_0 branch), unlike the decode step."""
    hp = HP()
    t = random_model(hp, seed=17)
    kvo = hp.n_kv_heads * hp.head_dim
    t["blk.0.attn_v.weight"] = (qt, misc_identity(qt, kvo, hp.n_embd))
    m = O.OracleModel(hp, t)
    try:
        toks = [3, 7, 11, 5]
        m.forward_batch(toks, 0)
        _, v = m.kv_view()
        qe, we = t["token_embd.weight"]
        rb = O.row_bytes(qe, hp.n_embd)
        for i, tok in enumerate(toks):
            x = O.dequant(qe, we[tok * rb:(tok + 1) * rb])
            xn = O.rmsnorm(x, t["blk.0.attn_norm.weight"][1], hp.rms_eps)
            assert np.array_equal(v[0, i], xn[:kvo] + t["blk.0.attn_v.bias"][1])
        if qt == Q8_0W:  # the decode step of the same first token takes the Q8_0 row
            v = v.copy()  # (the view dies with the state)
            m.reset()
            m.forward_token(toks[0], 0)
            _, v2 = m.kv_view()
            assert not np.array_equal(v2[0, 0], v[0, 0])
    finally:
        m.close()


@dataclass
class HP96(HP):
    """Hidden 96 (not a multiple of 256): 3 heads of 32, one kv head, FFN 160."""
    n_layer: int = 2
    n_embd: int = 96
    n_heads: int = 3
    n_kv_heads: int = 1
    ffn_dim: int = 160
    n_vocab: int = 40
    n_ctx: int = 8


def model96(hp: HP96, seed: int, types) -> dict:
    rng = np.random.default_rng(seed)
    E, FD, qo, kvo = hp.n_embd, hp.ffn_dim, hp.n_heads * hp.head_dim, hp.n_kv_heads * hp.head_dim
    t = {"token_embd.weight": (Q8_0W, misc_random(rng, Q8_0W, hp.n_vocab, E, 2e-2)),
         "output_norm.weight": (F32, f32(rng.uniform(0.5, 1.5, E)))}
    for layer in range(hp.n_layer):
        b = f"blk.{layer}."
        t[b + "attn_norm.weight"] = (F32, f32(rng.uniform(0.5, 1.5, E)))
        t[b + "ffn_norm.weight"] = (F32, f32(rng.uniform(0.5, 1.5, E)))
        for name, (rows, cols) in {"attn_q": (qo, E), "attn_k": (kvo, E), "attn_v": (kvo, E),
                                   "attn_output": (E, qo), "ffn_gate": (FD, E),
                                   "ffn_up": (FD, E), "ffn_down": (E, FD)}.items():
            qt = types[name]
            t[b + name + ".weight"] = (qt, misc_random(rng, qt, rows, cols))
        t[b + "attn_q.bias"] = (F32, f32(rng.standard_normal(qo) * 0.1))
        t[b + "attn_k.bias"] = (F32, f32(rng.standard_normal(kvo) * 0.1))
        t[b + "attn_v.bias"] = (F32, f32(rng.standard_normal(kvo) * 0.1))
    return t


MIXES = {
    # llama.cpp's Q4_K_M fall-backs for rows of 896-style widths: Q5_0 for the
    # Q4_K matrices, Q8_0 for the Q6_K ones
    "q4km_fallback": {"attn_q": Q5_0W, "attn_k": Q5_0W, "attn_v": Q8_0W, "attn_output": Q5_0W,
                      "ffn_gate": Q5_0W, "ffn_up": Q5_0W, "ffn_down": Q8_0W},
    "f16_q8": {"attn_q": F16W, "attn_k": Q8_0W, "attn_v": F16W, "attn_output": Q8_0W,
               "ffn_gate": Q8_0W, "ffn_up": F16W, "ffn_down": F16W},
}


@pytest.mark.parametrize("mix", sorted(MIXES))
def test_hidden_96_decode_step_composes_the_pinned_pieces(mix):
    """Two decode steps of a 2-layer hidden-96 model against the reference's
    wiring written with the oracle's pinned pieces (RMSNorm, Q8_0, per-type
    GEMVs, RoPE, attention, SwiGLU), bit for bit."""
    hp = HP96()
    t = model96(hp, 21, MIXES[mix])
    m = O.OracleModel(hp, t)
    E, H, KVH, HD, FD = hp.n_embd, hp.n_heads, hp.n_kv_heads, hp.head_dim, hp.ffn_dim
    kvo = KVH * HD
    c, s = rope_tab(hp)
    kc = np.zeros((hp.n_layer, hp.n_ctx, kvo), np.float32)
    vc = np.zeros_like(kc)
    try:
        for pos, tok in enumerate((5, 17)):
            m.forward_token(tok, pos)
            qe, we = t["token_embd.weight"]
            rb = O.misc_row_bytes(qe, E)
            x = O.dequant_row(qe, we[tok * rb:(tok + 1) * rb], E)
            for layer in range(hp.n_layer):
                b = f"blk.{layer}."
                xn = O.rmsnorm(x, t[b + "attn_norm.weight"][1], hp.rms_eps)
                xq = O.quantize_q8_0(xn)
                q = gemv_any(t, b + "attn_q.weight", xq, xn, H * HD, E) + t[b + "attn_q.bias"][1]
                k = gemv_any(t, b + "attn_k.weight", xq, xn, kvo, E) + t[b + "attn_k.bias"][1]
                v = gemv_any(t, b + "attn_v.weight", xq, xn, kvo, E) + t[b + "attn_v.bias"][1]
                q = O.rope(q, pos, H, HD, c, s)
                kc[layer, pos] = O.rope(k, pos, KVH, HD, c, s)
                vc[layer, pos] = v
                att = O.attention(q, kc[layer], vc[layer], pos + 1, H, KVH, HD)
                x = x + gemv_any(t, b + "attn_output.weight", O.quantize_q8_0(att), att, E, E)
                xn = O.rmsnorm(x, t[b + "ffn_norm.weight"][1], hp.rms_eps)
                xq = O.quantize_q8_0(xn)
                h = O.swiglu(gemv_any(t, b + "ffn_gate.weight", xq, xn, FD, E),
                             gemv_any(t, b + "ffn_up.weight", xq, xn, FD, E))
                x = x + gemv_any(t, b + "ffn_down.weight", O.quantize_q8_0(h), h, E, FD)
            xn = O.rmsnorm(x, t["output_norm.weight"][1], hp.rms_eps)
            logits = gemv_any(t, "token_embd.weight", O.quantize_q8_0(xn), xn, hp.n_vocab, E)
            k_o, v_o = m.kv_view()
            assert np.array_equal(k_o[:, pos], kc[:, pos])
            assert np.array_equal(v_o[:, pos], vc[:, pos])
            assert np.array_equal(m.logits(), logits)
    finally:
        m.close()


@pytest.mark.parametrize("mix", sorted(MIXES))
def test_hidden_96_prefill_agrees_with_decode_where_the_paths_match(mix):
    """The batched prefill of the same model: identical cache rows to the
    decode path for every matrix type whose prefill activation is the decode
    one (all but Q8_0), and the greedy generation runs to the context end."""
    hp = HP96()
    t = model96(hp, 23, MIXES[mix])
    m = O.OracleModel(hp, t)
    try:
        toks = [1, 9, 30, 4]
        m.forward_batch(toks, 0)
        kb, vb = (a.copy() for a in m.kv_view())
        lb = m.logits().copy()
        m.reset()
        for pos, tok in enumerate(toks):
            m.forward_token(tok, pos)
        kt, vt = m.kv_view()
        same = all(qt != Q8_0W for qt in MIXES[mix].values())
        if same:
            assert np.array_equal(kb[:, :4], kt[:, :4]) and np.array_equal(vb[:, :4], vt[:, :4])
            assert np.array_equal(lb, m.logits())
        else:  # Q8_0 matrices read fp32 rows in the prefill, Q8_0 rows in decode
            assert not np.array_equal(vb[:, :4], vt[:, :4])
            assert np.max(np.abs(lb - m.logits())) < 0.05 * max(1.0, float(np.max(np.abs(lb))))
        toks_out, _ = m.generate([1, 2, 3], 10)
        assert len(toks_out) == hp.n_ctx - 3  # stops at the context end
    finally:
        m.close()
