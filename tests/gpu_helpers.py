"""Helpers shared by the GPU parity tests (not a test module)."""
import numpy as np

from oracle import oracle as O


def within(gpu, ref, rtol=1e-3, atol=1e-4):
    """The north-star bound |gpu - ref| <= atol + rtol |ref| elementwise:
    (ok, max |err|, number of elements outside)."""
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    bad = np.abs(gpu - ref) > atol + rtol * np.abs(ref)
    return (not bad.any()), float(np.max(np.abs(gpu - ref))), int(bad.sum())


def check(tag, got, want, rtol=1e-3, atol=1e-4):
    ok, err, nbad = within(got, want, rtol, atol)
    print(f"  {tag}: max |err| {err:.3e}", flush=True)
    assert ok, f"{tag}: {nbad} elements outside tolerance, max |err| {err:.3e}"


def device_norm_q8(ctx, x, w, eps):
    return device_norm(ctx, x, w, eps)[0]


def gemv_typed(qt, W, xq8, xf, rows, cols):
    """The oracle's GEMV for a layer matrix of type qt in the decode step
    (gemv_wt_q8, llama_model.cpp:767-831): Q4_K / Q6_K / Q8_0 on the Q8_0
    activation xq8, Q5_0 / F16 on the fp32 activation xf."""
    if qt in (O.Q4K, O.Q6K):
        return O.gemv_q8(qt, W, xq8, rows, cols)
    if qt == 8:
        return O.gemv_q8_0w_q8(W, xq8, rows, cols)
    return O.gemv_misc(qt, W, xf, rows, cols)


def device_norm(ctx, x, w, eps):
    """Q8_0 of RMSNorm(x) * w from the device's RMSNorm kernel (the fused GEMV
    prologues share its summation order).  Checked two ways: the device's
    fp32 RMSNorm is within fp32 summation noise of the oracle's (1e-5
    relative, norm-wise), and the device's blocks are bit for bit the Q8_0
    quantisation of that fp32 output.  So where the two differ from the
    oracle's own blocks, the device's RMSNorm value lies across a rounding
    boundary from the oracle's."""
    n = x.size
    dx, dw = ctx.upload(np.ascontiguousarray(x, np.float32)), ctx.upload(w)
    y, yq = ctx.alloc(n * 4), ctx.alloc(n // 32 * 36)
    ctx.rmsnorm(y, yq, dx, dw, n, eps)
    got = ctx.download(yq, np.uint8, n // 32 * 36)
    yd = ctx.download(y, np.float32, n)
    for b in (dx, dw, y, yq):
        b.free()
    yo = O.rmsnorm(x, w, eps).astype(np.float64)
    rel = np.linalg.norm(yd - yo) / np.linalg.norm(yo)
    assert rel < 1e-5, f"device RMSNorm differs from the oracle's by {rel:.2e} (norm-wise)"
    assert np.array_equal(got, O.quantize_q8_0(yd)), "device Q8_0 differs from Q8_0(device RMSNorm)"
    return got, yd


def layer_stage_errors(ctx, g, T, hp, layer, pos, types=None):
    """Run the five fused stages of `layer` at `pos` on the device (from the
    device's current x and cache rows 0..pos-1) and compare each with the
    oracle on that stage's device inputs.  Returns a list of
    (stage, max |err|, elements outside the north-star bound, norm-wise
    relative error); the K/V rows and the attention Q8_0 blocks must be
    bit-exact (asserted).  T maps tensor names to host arrays; types maps
    the layer's matrix names (attn_q, ...) to their GGUF types (default: the
    Q4_K_M mix, Q6_K for attn_v and ffn_down)."""
    from llm_core_amd import _ffi

    E, H, KVH, HD, FD = hp.n_embd, hp.n_heads, hp.n_kv_heads, hp.head_dim, hp.ffn_dim
    qo, kvo = H * HD, KVH * HD
    b = f"blk.{layer}."
    cos_t, sin_t = O.rope_table(HD, hp.rope_theta, hp.n_ctx)
    res = []

    def rec(tag, got, want, rtol=1e-3, atol=1e-4):
        ok, err, nbad = within(got, want, rtol, atol)
        w = np.asarray(want, np.float64)
        rel = float(np.linalg.norm(np.asarray(got, np.float64) - w) / max(np.linalg.norm(w), 1e-30))
        res.append((tag, err, nbad, rel))

    qt = {n: O.Q4K for n in ("attn_q", "attn_k", "attn_output", "ffn_gate", "ffn_up")}
    qt.update({"attn_v": O.Q6K, "ffn_down": O.Q6K})
    qt.update(types or {})
    x0 = g.buffer(_ffi.AXF_LLAMA_BUF_X)
    g.forward_layer_stages(layer, pos, 1, 1)
    qkv = g.buffer(_ffi.AXF_LLAMA_BUF_QKV)
    xq, xf = device_norm(ctx, x0, T[b + "attn_norm.weight"], hp.rms_eps)
    rec("q", qkv[:qo], gemv_typed(qt["attn_q"], T[b + "attn_q.weight"], xq, xf, qo, E))
    rec("k", qkv[qo:qo + kvo], gemv_typed(qt["attn_k"], T[b + "attn_k.weight"], xq, xf, kvo, E))
    rec("v", qkv[qo + kvo:], gemv_typed(qt["attn_v"], T[b + "attn_v.weight"], xq, xf, kvo, E))

    g.forward_layer_stages(layer, pos, 2, 2)
    zero = np.zeros(kvo, np.float32)
    q = qkv[:qo] + T.get(b + "attn_q.bias", np.zeros(qo, np.float32))
    k = qkv[qo:qo + kvo] + T.get(b + "attn_k.bias", zero)
    v = qkv[qo + kvo:] + T.get(b + "attn_v.bias", zero)
    # per-head q/k norms (llama_model.cpp:1236-1248): before RoPE (1) or after it (2)
    order = getattr(hp, "qk_norm_order", 0)

    def finish(x, w, nh):
        if order == 1 and w is not None:
            x = O.rmsnorm_heads(x, w, nh, HD, hp.rms_eps)
        x = O.rope(x, pos, nh, HD, cos_t, sin_t)
        if order == 2 and w is not None:
            x = O.rmsnorm_heads(x, w, nh, HD, hp.rms_eps)
        return x

    k_dev, v_dev = g.get_kv(layer, 0, pos + 1)
    assert np.array_equal(k_dev[pos], finish(k, T.get(b + "attn_k_norm.weight"), KVH)), "stored K row"
    assert np.array_equal(v_dev[pos], v), "stored V row"
    att = g.buffer(_ffi.AXF_LLAMA_BUF_ATTN)
    rec("attention", att, O.attention(finish(q, T.get(b + "attn_q_norm.weight"), H), k_dev, v_dev,
                                      pos + 1, H, KVH, HD), 1e-5, 1e-6)
    aq = g.buffer(_ffi.AXF_LLAMA_BUF_ATTN_Q8)
    assert np.array_equal(aq, O.quantize_q8_0(att)), "attention Q8_0 blocks"

    g.forward_layer_stages(layer, pos, 3, 3)
    x1 = g.buffer(_ffi.AXF_LLAMA_BUF_X)
    rec("x + o", x1, x0 + gemv_typed(qt["attn_output"], T[b + "attn_output.weight"], aq, att, E, qo))

    g.forward_layer_stages(layer, pos, 4, 4)
    h = g.buffer(_ffi.AXF_LLAMA_BUF_H)
    xq2, xf2 = device_norm(ctx, x1, T[b + "ffn_norm.weight"], hp.rms_eps)
    gate = gemv_typed(qt["ffn_gate"], T[b + "ffn_gate.weight"], xq2, xf2, FD, E)
    up = gemv_typed(qt["ffn_up"], T[b + "ffn_up.weight"], xq2, xf2, FD, E)
    rec("swiglu(gate, up)", h, O.swiglu(gate, up))

    g.forward_layer_stages(layer, pos, 5, 5)
    x2 = g.buffer(_ffi.AXF_LLAMA_BUF_X)
    rec("x + down", x2, x1 + gemv_typed(qt["ffn_down"], T[b + "ffn_down.weight"], O.quantize_q8_0(h),
                                        h, E, FD))
    return res
