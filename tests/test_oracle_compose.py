"""Pins of the oracle's decoder composition (orc_forward_layer / _token /
_batch, orc_generate_greedy in oracle/axf_oracle.c) by closed forms.

Each test switches parts of a layer off or gives them identity weights, so
the expected result follows from the reference's wiring and from oracle
functions that are pinned on their own (dequant, Q8_0, the GEMVs: bit-exact
against the compiled reference kernels; RMSNorm, RoPE, SwiGLU: closed forms).
The wiring under test is the body of llama_forward_token
(/root/reference/src/models/llama_model.cpp:1207-1333), llama_forward_batch
(:1339-1462) and the loop of llama_generate_cpu_impl (:1561-1624):

  x_n = RMSNorm(x) * attn_norm -> Q8_0 -> q, k, v GEMVs; + bias; RoPE(q),
  RoPE(k) stored in the cache row `pos`, v stored unrotated;
  attention over rows 0..pos (head h reads kv head h / (H/KVH));
  Q8_0(attn) -> o GEMV; x += o;
  RMSNorm(x) * ffn_norm -> Q8_0 -> gate, up GEMVs; h = silu(gate) * up;
  Q8_0(h) -> down GEMV; x += down;
  after the last layer: RMSNorm(x) * output_norm -> Q8_0 -> head GEMV.

Identity weights are Q4_K (d = 1, dmin = 0, scales 1): every output of such a
GEMV is one product d_x * q_x, so it returns the Q8_0-dequantised activation
exactly.  Weights that are switched off are all-zero blocks, or a zero norm
weight (RMSNorm(x) * 0 = 0 quantises to zero blocks and every GEMV of it is 0).
Every test also checks that a plausible wiring slip would change the result.
"""
from dataclasses import dataclass

import numpy as np

from oracle import oracle as O
from qblocks import (F32, Q4K, Q6K, dequant_q8, q4k_identity, q4k_random, q4k_zero,
                     q6k_random, unpack_q8)


@dataclass
class HP:
    n_layer: int = 1
    n_embd: int = 256
    n_heads: int = 4
    n_kv_heads: int = 2
    ffn_dim: int = 512
    n_vocab: int = 96
    n_ctx: int = 16
    rms_eps: float = 1e-5
    rope_theta: float = 10000.0

    @property
    def head_dim(self):
        return self.n_embd // self.n_heads


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def random_model(hp: HP, seed: int, biases: bool = True) -> dict:
    """Q4_K_M mix of random blocks (Q6_K for v, down and the head)."""
    rng = np.random.default_rng(seed)
    E, FD, qo, kvo = hp.n_embd, hp.ffn_dim, hp.n_heads * hp.head_dim, hp.n_kv_heads * hp.head_dim
    t = {
        "token_embd.weight": (Q4K, q4k_random(rng, hp.n_vocab, E, 4e-3)),
        "output_norm.weight": (F32, f32(rng.uniform(0.5, 1.5, E))),
        "output.weight": (Q6K, q6k_random(rng, hp.n_vocab, E)),
    }
    for layer in range(hp.n_layer):
        b = f"blk.{layer}."
        t[b + "attn_norm.weight"] = (F32, f32(rng.uniform(0.5, 1.5, E)))
        t[b + "ffn_norm.weight"] = (F32, f32(rng.uniform(0.5, 1.5, E)))
        t[b + "attn_q.weight"] = (Q4K, q4k_random(rng, qo, E))
        t[b + "attn_k.weight"] = (Q4K, q4k_random(rng, kvo, E))
        t[b + "attn_v.weight"] = (Q6K, q6k_random(rng, kvo, E))
        t[b + "attn_output.weight"] = (Q4K, q4k_random(rng, E, qo))
        t[b + "ffn_gate.weight"] = (Q4K, q4k_random(rng, FD, E))
        t[b + "ffn_up.weight"] = (Q4K, q4k_random(rng, FD, E))
        t[b + "ffn_down.weight"] = (Q6K, q6k_random(rng, E, FD))
        if biases:
            t[b + "attn_q.bias"] = (F32, f32(rng.standard_normal(qo) * 0.5))
            t[b + "attn_k.bias"] = (F32, f32(rng.standard_normal(kvo) * 0.5))
            t[b + "attn_v.bias"] = (F32, f32(rng.standard_normal(kvo) * 0.5))
    return t


def gemv(t: dict, name: str, xq8, rows: int, cols: int) -> np.ndarray:
    qt, w = t[name]
    return O.gemv_q8(qt, w, xq8, rows, cols)


def rope_tab(hp: HP):
    return O.rope_table(hp.head_dim, hp.rope_theta, hp.n_ctx)


def embed_row(t: dict, tok: int, E: int) -> np.ndarray:
    qt, w = t["token_embd.weight"]
    rb = O.row_bytes(qt, E)
    return O.dequant(qt, w[tok * rb:(tok + 1) * rb])


def head_logits(t: dict, hp: HP, x: np.ndarray) -> np.ndarray:
    """RMSNorm(x) * output_norm -> Q8_0 -> head (output.weight, else token_embd)."""
    xn = O.rmsnorm(x, t["output_norm.weight"][1], hp.rms_eps)
    name = "output.weight" if "output.weight" in t else "token_embd.weight"
    return gemv(t, name, O.quantize_q8_0(xn), hp.n_vocab, hp.n_embd)


def expand_gqa(v_row: np.ndarray, hp: HP) -> np.ndarray:
    """Query head h reads kv head h // (H / KVH)."""
    hd, g = hp.head_dim, hp.n_heads // hp.n_kv_heads
    return np.concatenate([v_row[(h // g) * hd:(h // g + 1) * hd] for h in range(hp.n_heads)])


def switch_off(t: dict, hp: HP, layer: int = 0, attn: bool = True, ffn: bool = True):
    """attn: o projection all zero blocks; ffn: ffn_norm = 0."""
    b = f"blk.{layer}."
    if attn:
        t[b + "attn_output.weight"] = (Q4K, q4k_zero(hp.n_embd, hp.n_heads * hp.head_dim))
    if ffn:
        t[b + "ffn_norm.weight"] = (F32, np.zeros(hp.n_embd, np.float32))


# ---------------------------------------------------------------------------
# (ii) attention and FFN switched off: x passes unchanged; the cache rows
# ---------------------------------------------------------------------------

def test_layer_off_keeps_x_and_writes_rotated_k_and_plain_v():
    hp = HP()
    t = random_model(hp, seed=1)
    switch_off(t, hp)
    m = O.OracleModel(hp, t)
    try:
        rng = np.random.default_rng(2)
        pos = 5
        k, v = m.kv_view()
        k[0, :pos] = rng.standard_normal(k[0, :pos].shape)
        v[0, :pos] = rng.standard_normal(v[0, :pos].shape)
        k_before, v_before = k.copy(), v.copy()
        x = f32(rng.standard_normal(hp.n_embd))
        m.x_view()[:] = x
        m.forward_layer(0, pos)
        assert np.array_equal(m.x_view(), x)            # both residual branches add exact zeros

        E, H, KVH, HD = hp.n_embd, hp.n_heads, hp.n_kv_heads, hp.head_dim
        kvo = KVH * HD
        xq = O.quantize_q8_0(O.rmsnorm(x, t["blk.0.attn_norm.weight"][1], hp.rms_eps))
        c, s = rope_tab(hp)
        kp = gemv(t, "blk.0.attn_k.weight", xq, kvo, E) + t["blk.0.attn_k.bias"][1]
        vp = gemv(t, "blk.0.attn_v.weight", xq, kvo, E) + t["blk.0.attn_v.bias"][1]
        qp = gemv(t, "blk.0.attn_q.weight", xq, H * HD, E) + t["blk.0.attn_q.bias"][1]
        want_k = O.rope(kp, pos, KVH, HD, c, s)
        assert np.array_equal(k[0, pos], want_k)        # K stored after bias, then RoPE
        assert np.array_equal(v[0, pos], vp)            # V stored with bias, unrotated
        assert np.array_equal(m.q_view(), O.rope(qp, pos, H, HD, c, s))
        # no other cache row moved
        assert np.array_equal(k[0, :pos], k_before[0, :pos])
        assert np.array_equal(k[0, pos + 1:], k_before[0, pos + 1:])
        assert np.array_equal(v[0, :pos], v_before[0, :pos])

        # the slips this pins would give other rows
        bk = t["blk.0.attn_k.bias"][1]
        assert not np.allclose(want_k, O.rope(kp - bk, pos, KVH, HD, c, s) + bk, atol=1e-3)
        assert not np.allclose(want_k, kp, atol=1e-3)                    # K unrotated
        xq_ffn = O.quantize_q8_0(O.rmsnorm(x, t["blk.0.ffn_norm.weight"][1], hp.rms_eps))
        assert not np.array_equal(xq_ffn, xq)                            # other norm weight
    finally:
        m.close()


# ---------------------------------------------------------------------------
# seq = 1 attention returns V: head h takes kv head h // G, o adds Q8_0 of it
# ---------------------------------------------------------------------------

def test_first_position_attention_is_v_through_identity_o():
    hp = HP()
    t = random_model(hp, seed=3)
    t["blk.0.attn_output.weight"] = (Q4K, q4k_identity(hp.n_embd, hp.n_embd))
    switch_off(t, hp, attn=False)
    m = O.OracleModel(hp, t)
    try:
        x = f32(np.random.default_rng(4).standard_normal(hp.n_embd))
        m.x_view()[:] = x
        m.forward_layer(0, 0)
        kvo = hp.n_kv_heads * hp.head_dim
        xq = O.quantize_q8_0(O.rmsnorm(x, t["blk.0.attn_norm.weight"][1], hp.rms_eps))
        v0 = gemv(t, "blk.0.attn_v.weight", xq, kvo, hp.n_embd) + t["blk.0.attn_v.bias"][1]
        att = expand_gqa(v0, hp)
        assert np.array_equal(m.attn_out_view(), att)
        assert np.array_equal(m.x_view(), x + dequant_q8(O.quantize_q8_0(att)))
        # a head mapping h % KVH instead of h // G would read other rows
        g = hp.n_heads // hp.n_kv_heads
        alt = np.concatenate([v0[(h % hp.n_kv_heads) * hp.head_dim:][:hp.head_dim]
                              for h in range(hp.n_heads)])
        assert g > 1 and not np.array_equal(alt, att)
    finally:
        m.close()


# ---------------------------------------------------------------------------
# (iii) q = 0: uniform attention = mean of V rows 0..pos; x += Wo Q8_0(mean)
# ---------------------------------------------------------------------------

def test_zero_query_gives_mean_of_v_rows():
    hp = HP()
    t = random_model(hp, seed=5)
    E, kvo = hp.n_embd, hp.n_kv_heads * hp.head_dim
    t["blk.0.attn_q.weight"] = (Q4K, q4k_zero(hp.n_heads * hp.head_dim, E))
    del t["blk.0.attn_q.bias"]
    t["blk.0.attn_v.weight"] = (Q4K, q4k_identity(kvo, E))
    t["blk.0.attn_output.weight"] = (Q4K, q4k_identity(E, E))
    switch_off(t, hp, attn=False)
    m = O.OracleModel(hp, t)
    try:
        rng = np.random.default_rng(6)
        pos = 7
        k, v = m.kv_view()
        k[0, :pos] = rng.standard_normal(k[0, :pos].shape) * 3
        v[0, :pos] = rng.standard_normal(v[0, :pos].shape)
        x = f32(rng.standard_normal(E))
        m.x_view()[:] = x
        m.forward_layer(0, pos)
        xn = O.rmsnorm(x, t["blk.0.attn_norm.weight"][1], hp.rms_eps)
        v_new = dequant_q8(O.quantize_q8_0(xn))[:kvo] + t["blk.0.attn_v.bias"][1]
        assert np.array_equal(v[0, pos], v_new)
        mean = v[0, :pos + 1].astype(np.float64).mean(axis=0)
        att = m.attn_out_view()
        want = expand_gqa(mean, hp)
        assert np.max(np.abs(att - want)) <= 2e-6 * np.max(np.abs(want))
        # the residual adds Wo * Q8_0(attention) = its Q8_0 dequantisation
        assert np.array_equal(m.x_view(), x + dequant_q8(O.quantize_q8_0(att)))
        # and that is the float64 mean within half a Q8_0 step per block
        step = np.repeat(np.abs(want).reshape(-1, 32).max(axis=1) / 127, 32)
        assert np.all(np.abs(m.x_view() - x - want) <= 0.5 * step * (1 + 1e-3) + 1e-6)
        # attending to rows 0..pos-1 only (an off-by-one seq) gives another mean
        assert not np.allclose(expand_gqa(v[0, :pos].mean(axis=0), hp), want, atol=1e-3)
    finally:
        m.close()


# ---------------------------------------------------------------------------
# FFN wiring: ffn_norm feeds gate and up, h = silu(gate) * up feeds down
# ---------------------------------------------------------------------------

def test_ffn_identity_weights():
    hp = HP()
    t = random_model(hp, seed=7)
    E, FD = hp.n_embd, hp.ffn_dim
    switch_off(t, hp, ffn=False)
    t["blk.0.ffn_gate.weight"] = (Q4K, q4k_identity(FD, E, 1))
    t["blk.0.ffn_up.weight"] = (Q4K, q4k_identity(FD, E, 3))
    t["blk.0.ffn_down.weight"] = (Q4K, q4k_identity(E, FD, 1))
    m = O.OracleModel(hp, t)
    try:
        x = f32(np.random.default_rng(8).standard_normal(E))
        m.x_view()[:] = x
        m.forward_layer(0, 3)
        d, q = unpack_q8(
            O.quantize_q8_0(O.rmsnorm(x, t["blk.0.ffn_norm.weight"][1], hp.rms_eps)))
        g = np.zeros(FD, np.float32)
        u = np.zeros(FD, np.float32)
        g[:E] = (d[:, None] * q.astype(np.float32)).reshape(-1)
        u[:E] = (d[:, None] * (3 * q).astype(np.float32)).reshape(-1)
        h = O.swiglu(g, u)
        assert np.array_equal(m.h_view(), h)
        assert np.array_equal(m.x_view(), x + dequant_q8(O.quantize_q8_0(h))[:E])
        # gate and up swapped, or attn_norm in place of ffn_norm, give another h
        assert not np.allclose(O.swiglu(u, g), h, atol=1e-4)
        xa = O.rmsnorm(x, t["blk.0.attn_norm.weight"][1], hp.rms_eps)
        assert not np.allclose(dequant_q8(O.quantize_q8_0(xa)), g[:E], atol=1e-3)
    finally:
        m.close()


# ---------------------------------------------------------------------------
# (i) no layers: logits = head(Q8_0(RMSNorm(embed(tok)) * output_norm))
# ---------------------------------------------------------------------------

def test_zero_layer_model_is_embedding_then_final_norm_and_head():
    hp = HP(n_layer=0)
    t = random_model(hp, seed=9)
    for tied in (False, True):
        tt = dict(t)
        if tied:
            del tt["output.weight"]                     # falls back to token_embd
        m = O.OracleModel(hp, tt)
        try:
            for tok in (0, 17, hp.n_vocab - 1):
                m.forward_token(tok, 2)
                e = embed_row(tt, tok, hp.n_embd)
                assert np.array_equal(m.logits(), head_logits(tt, hp, e))
                # reference leaves x normalised in place (rms_norm_avx2, :1328)
                assert np.array_equal(m.x_view(),
                                      O.rmsnorm(e, tt["output_norm.weight"][1], hp.rms_eps))
        finally:
            m.close()
    # doubling output_norm doubles every logit exactly (Q8_0 is scale-exact
    # under powers of two): the final norm is applied before the head
    t2 = dict(t)
    t2["output_norm.weight"] = (F32, f32(2 * t["output_norm.weight"][1]))
    m1, m2 = O.OracleModel(hp, t), O.OracleModel(hp, t2)
    try:
        m1.forward_token(5, 0)
        m2.forward_token(5, 0)
        assert np.array_equal(m2.logits(), 2 * m1.logits())
    finally:
        m1.close()
        m2.close()


# ---------------------------------------------------------------------------
# (iv) relative positions: scores q_m . k_n depend on m - n only
# ---------------------------------------------------------------------------

def test_attention_scores_depend_on_relative_position():
    hp = HP(n_ctx=64)
    t = random_model(hp, seed=11)
    rng = np.random.default_rng(12)
    xa = f32(rng.standard_normal(hp.n_embd))
    xb = f32(rng.standard_normal(hp.n_embd))
    H, KVH, HD = hp.n_heads, hp.n_kv_heads, hp.head_dim
    g = H // KVH

    def scores(p):
        m = O.OracleModel(hp, t)
        try:
            m.x_view()[:] = xa
            m.forward_layer(0, p)
            m.x_view()[:] = xb
            m.forward_layer(0, p + 1)
            q = m.q_view().reshape(H, HD).copy()
            k, _ = m.kv_view()
            rows = k[0, [p, p + 1]].reshape(2, KVH, HD)
            return np.array([[q[h] @ rows[j, h // g] for j in range(2)] for h in range(H)])
        finally:
            m.close()

    base = scores(1)
    scale = np.max(np.abs(base))
    for p in (4, 17, 40):
        assert np.max(np.abs(scores(p) - base)) <= 1e-5 * scale
    # with K stored unrotated the scores would move with the position
    c, s = rope_tab(hp)
    q1 = O.rope(np.ones(H * HD, np.float32), 2, H, HD, c, s)
    q2 = O.rope(np.ones(H * HD, np.float32), 30, H, HD, c, s)
    assert abs(float(q1[:HD] @ np.ones(HD)) - float(q2[:HD] @ np.ones(HD))) > 1e-2


# ---------------------------------------------------------------------------
# (v) the generation loop: token chain and the n_past >= n_ctx stop
# ---------------------------------------------------------------------------

def test_greedy_loop_chain_and_context_stop():
    hp = HP(n_ctx=8)
    t = random_model(hp, seed=13)
    switch_off(t, hp)          # the layer passes x through: next token = f(previous)

    def f(tok):
        return O.argmax(head_logits(t, hp, embed_row(t, tok, hp.n_embd)))

    prompt = [3, 9, 1, 4, 7]
    chain = [f(prompt[-1])]
    for _ in range(10):
        chain.append(f(chain[-1]))
    m = O.OracleModel(hp, t)
    try:
        for batched in (True, False):
            toks, margins = m.generate(prompt, 10, batched_prefill=batched)
            # n_past starts at 5; tokens are emitted while n_past < 8
            assert list(toks) == chain[:3]
            lg = head_logits(t, hp, embed_row(t, prompt[-1], hp.n_embd))
            assert margins[0] == O.top2_margin(lg)
            toks, _ = m.generate(prompt, 2, batched_prefill=batched)
            assert list(toks) == chain[:2]
            toks, _ = m.generate(prompt + [2, 5, 6], 4, batched_prefill=batched)
            assert len(toks) == 0                       # prompt fills the context
            toks, _ = m.generate([5], 3, batched_prefill=batched)
            assert list(toks) == [f(5), f(f(5)), f(f(f(5)))]
    finally:
        m.close()


# ---------------------------------------------------------------------------
# batched prefill: per-row positions, causal rows, final norm of the last row
# ---------------------------------------------------------------------------

def test_batch_rows_positions_and_causal_mean():
    hp = HP()
    t = random_model(hp, seed=15)
    E, H, KVH, HD = hp.n_embd, hp.n_heads, hp.n_kv_heads, hp.head_dim
    kvo = KVH * HD
    t["blk.0.attn_q.weight"] = (Q4K, q4k_zero(H * HD, E))
    del t["blk.0.attn_q.bias"]
    t["blk.0.attn_v.weight"] = (Q4K, q4k_identity(kvo, E))
    t["blk.0.attn_output.weight"] = (Q4K, q4k_identity(E, E))
    switch_off(t, hp, attn=False)
    m = O.OracleModel(hp, t)
    try:
        rng = np.random.default_rng(16)
        pos0, toks = 3, [11, 40, 2, 77]
        k, v = m.kv_view()
        k[0, :pos0] = rng.standard_normal(k[0, :pos0].shape)
        v[0, :pos0] = rng.standard_normal(v[0, :pos0].shape)
        v_old = v[0, :pos0].copy()
        m.forward_batch(toks, pos0)
        c, s = rope_tab(hp)
        an = t["blk.0.attn_norm.weight"][1]
        vrows = [r for r in v_old]
        xqs = [O.quantize_q8_0(O.rmsnorm(embed_row(t, tok, E), an, hp.rms_eps)) for tok in toks]
        # Q4_K projections of a batch run the GEMM kernel (gemm_wt_q8, :837-879)
        K = O.gemm_q4k_q8(t["blk.0.attn_k.weight"][1], np.concatenate(xqs), kvo, len(toks), E)
        for i, xq in enumerate(xqs):
            kp = K[i] + t["blk.0.attn_k.bias"][1]
            assert np.array_equal(k[0, pos0 + i], O.rope(kp, pos0 + i, KVH, HD, c, s))
            vr = dequant_q8(xq)[:kvo] + t["blk.0.attn_v.bias"][1]
            assert np.array_equal(v[0, pos0 + i], vr)
            vrows.append(vr)
        # the last row attends to rows 0..pos0+T-1 (uniformly, q = 0)
        mean = np.mean(np.array(vrows, np.float64), axis=0)
        x_last = embed_row(t, toks[-1], E) + expand_gqa(mean, hp)
        want = O.rmsnorm(f32(x_last), t["output_norm.weight"][1], hp.rms_eps)
        got = m.x_view()
        # x_last differs from the device-free float64 value by the Q8_0
        # step of the attention output (<= 1/254 of the block maximum)
        assert np.max(np.abs(got - want)) <= 0.01 * np.max(np.abs(want))
        assert np.array_equal(m.logits(),
                              gemv(t, "output.weight", O.quantize_q8_0(got), hp.n_vocab, E))
        # the batch equals the same tokens run one by one
        m2 = O.OracleModel(hp, t)
        try:
            k2, v2 = m2.kv_view()
            k2[0, :pos0] = k[0, :pos0]
            v2[0, :pos0] = v_old
            for i, tok in enumerate(toks):
                m2.forward_token(tok, pos0 + i)
            assert np.max(np.abs(m2.logits() - m.logits())) <= 1e-5 * np.max(np.abs(m.logits()))
            # (the GEMM and the GEMV sum in different orders: fp32 rounding apart)
            assert np.max(np.abs(k2[0, :pos0 + 4] - k[0, :pos0 + 4])) <= 1e-5 * np.max(np.abs(k))
        finally:
            m2.close()
    finally:
        m.close()


# ---------------------------------------------------------------------------
# per-head q/k RMSNorm (qwen3: before RoPE; hunyuan-dense: after RoPE;
# llama_model.cpp:1236-1248, batch :1388-1403; rms_norm_heads_inplace :421-429)
# ---------------------------------------------------------------------------

def test_rmsnorm_heads_closed_forms():
    hd, heads, eps = 128, 3, 1e-6
    rng = np.random.default_rng(21)
    w = f32(rng.uniform(0.5, 2.0, hd))
    x = f32(np.concatenate([np.full(hd, 3.0), rng.standard_normal(hd), np.full(hd, -0.25)]))
    y = O.rmsnorm_heads(x, w, heads, hd, eps)
    # a constant head c: w * c / sqrt(c^2 + eps), to fp32 rounding
    for h, c in ((0, 3.0), (2, -0.25)):
        want = w * (c / np.sqrt(c * c + eps))
        np.testing.assert_allclose(y[h * hd:(h + 1) * hd], want, rtol=3e-7, atol=0)
    # each head on its own, with the same weight vector: head 1 equals the
    # whole-vector RMSNorm of that head alone, bit for bit
    assert np.array_equal(y[hd:2 * hd], O.rmsnorm(x[hd:2 * hd], w, eps))
    # scaling one head leaves the others' bits unchanged
    x2 = x.copy()
    x2[hd:2 * hd] *= 10.0
    y2 = O.rmsnorm_heads(x2, w, heads, hd, eps)
    assert np.array_equal(y2[:hd], y[:hd]) and np.array_equal(y2[2 * hd:], y[2 * hd:])
    # a slip that normalises over all heads at once gives other values
    assert not np.allclose(O.rmsnorm(x, np.tile(w, heads), eps), y, atol=1e-3)


def qk_norm_case(order: int, seed: int):
    """A switched-off layer with per-head q/k norm weights at position 6: the
    cache K row and q after the layer, and their closed forms."""
    hp = HP(n_ctx=16)
    hp.qk_norm_order = order
    t = random_model(hp, seed=seed)
    switch_off(t, hp)
    rng = np.random.default_rng(seed + 1)
    HD, H, KVH, E = hp.head_dim, hp.n_heads, hp.n_kv_heads, hp.n_embd
    qn, kn = f32(rng.uniform(0.3, 3.0, HD)), f32(rng.uniform(0.3, 3.0, HD))
    t["blk.0.attn_q_norm.weight"] = (F32, qn)
    t["blk.0.attn_k_norm.weight"] = (F32, kn)
    m = O.OracleModel(hp, t)
    try:
        pos = 6
        x = f32(rng.standard_normal(E))
        m.x_view()[:] = x
        m.forward_layer(0, pos)
        k, v = m.kv_view()
        got_k, got_v, got_q = k[0, pos].copy(), v[0, pos].copy(), m.q_view().copy()
    finally:
        m.close()
    xq = O.quantize_q8_0(O.rmsnorm(x, t["blk.0.attn_norm.weight"][1], hp.rms_eps))
    qp = gemv(t, "blk.0.attn_q.weight", xq, H * HD, E) + t["blk.0.attn_q.bias"][1]
    kp = gemv(t, "blk.0.attn_k.weight", xq, KVH * HD, E) + t["blk.0.attn_k.bias"][1]
    vp = gemv(t, "blk.0.attn_v.weight", xq, KVH * HD, E) + t["blk.0.attn_v.bias"][1]
    c, s = rope_tab(hp)
    eps = hp.rms_eps
    before = (O.rope(O.rmsnorm_heads(qp, qn, H, HD, eps), pos, H, HD, c, s),
              O.rope(O.rmsnorm_heads(kp, kn, KVH, HD, eps), pos, KVH, HD, c, s))
    after = (O.rmsnorm_heads(O.rope(qp, pos, H, HD, c, s), qn, H, HD, eps),
             O.rmsnorm_heads(O.rope(kp, pos, KVH, HD, c, s), kn, KVH, HD, eps))
    plain = (O.rope(qp, pos, H, HD, c, s), O.rope(kp, pos, KVH, HD, c, s))
    return (got_q, got_k, got_v), vp, before, after, plain


def test_qk_norm_before_rope():
    (q, k, v), vp, before, after, plain = qk_norm_case(1, seed=31)
    assert np.array_equal(q, before[0]) and np.array_equal(k, before[1])
    assert np.array_equal(v, vp)  # V: bias only, no norm
    # the orders differ once RoPE rotates (position 6) and the weights vary
    assert not np.allclose(before[1], after[1], atol=1e-3)
    assert not np.allclose(before[1], plain[1], atol=1e-3)


def test_qk_norm_after_rope():
    (q, k, v), vp, before, after, plain = qk_norm_case(2, seed=33)
    assert np.array_equal(q, after[0]) and np.array_equal(k, after[1])
    assert np.array_equal(v, vp)
    assert not np.allclose(after[0], before[0], atol=1e-3)


def test_qk_norm_weights_ignored_without_order():
    (q, k, v), vp, before, after, plain = qk_norm_case(0, seed=35)
    assert np.array_equal(q, plain[0]) and np.array_equal(k, plain[1])


def test_qk_norm_batch_rows():
    """llama_forward_batch's order (:1388-1403) on a switched-off layer: every
    new cache row is the closed form of its own GEMM row, for both orders."""
    for order in (1, 2):
        hp = HP(n_ctx=16)
        hp.qk_norm_order = order
        t = random_model(hp, seed=41 + order)
        switch_off(t, hp)
        rng = np.random.default_rng(50 + order)
        HD, KVH, E = hp.head_dim, hp.n_kv_heads, hp.n_embd
        kn = f32(rng.uniform(0.3, 3.0, HD))
        t["blk.0.attn_q_norm.weight"] = (F32, f32(rng.uniform(0.3, 3.0, HD)))
        t["blk.0.attn_k_norm.weight"] = (F32, kn)
        m = O.OracleModel(hp, t)
        try:
            pos0, toks = 2, [5, 60, 33]
            m.forward_batch(toks, pos0)
            k, _ = m.kv_view()
            an = t["blk.0.attn_norm.weight"][1]
            xqs = [O.quantize_q8_0(O.rmsnorm(embed_row(t, tok, E), an, hp.rms_eps)) for tok in toks]
            K = O.gemm_q4k_q8(t["blk.0.attn_k.weight"][1], np.concatenate(xqs), KVH * HD,
                              len(toks), E)
            c, s = rope_tab(hp)
            for i in range(len(toks)):
                kp = K[i] + t["blk.0.attn_k.bias"][1]
                p = pos0 + i
                if order == 1:
                    want = O.rope(O.rmsnorm_heads(kp, kn, KVH, HD, hp.rms_eps), p, KVH, HD, c, s)
                else:
                    want = O.rmsnorm_heads(O.rope(kp, p, KVH, HD, c, s), kn, KVH, HD, hp.rms_eps)
                assert np.array_equal(k[0, p], want), (order, i)
        finally:
            m.close()
