"""GPU decoder parity against the oracle's llama_forward_token restatement.

  * config 3: one Qwen2.5-3B-like layer (hidden 2048, 16/2 heads, head_dim
    128, FFN 11008, eps 1e-6, theta 1e6) over a KV cache holding 1024 prior
    positions of N(0, 1), with q/k/v biases and non-unit norm weights;
  * config 2: the Q6_K 151936 x 2048 output head and greedy argmax, full size;
  * greedy generation on a small synthetic LLaMA: identical token ids between
    HIP-graph replay, eager launches and the oracle (token-by-token prefill and
    the reference's batched prefill) for 32 tokens on models without near-ties;
    elsewhere a divergence is accepted only at an oracle near-tie.
"""
import numpy as np
import pytest

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def within(gpu, ref, rtol=1e-3, atol=1e-4):
    gpu = np.asarray(gpu, np.float64)
    ref = np.asarray(ref, np.float64)
    bad = np.abs(gpu - ref) > atol + rtol * np.abs(ref)
    return (not bad.any()), float(np.max(np.abs(gpu - ref)))


def _layer_parity(ctx, cfg, prior, with_bias, seed, max_abs=2e-3):
    from llm_core_amd import hip
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    cfg = dict(cfg)
    cfg["n_vocab"] = 256  # the head is not exercised by a single layer
    cfg["n_layer"] = 1
    hp = Hparams(n_ctx=prior + 1, **cfg)
    m = SynthLlama(hp, seed=seed, norm_std=0.1, with_bias=with_bias)
    kve = hp.n_kv_heads * hp.head_dim
    kv_k = hip.synth_normal(prior * kve, 31).reshape(prior, kve)
    kv_v = hip.synth_normal(prior * kve, 32).reshape(prior, kve)
    x0 = hip.synth_normal(hp.n_embd, 33)

    om = O.OracleModel(hp, m.tensors)
    ok_, ov_ = om.kv_view()
    ok_[0, :prior] = kv_k
    ov_[0, :prior] = kv_v
    om.x_view()[:] = x0
    om.forward_layer(0, prior)
    want_x = om.x_view().copy()
    want_k, want_v = ok_[0, prior].copy(), ov_[0, prior].copy()
    om.close()

    g = LlamaHip(ctx, m)
    g.set_kv(0, kv_k, kv_v, prior)
    g.set_x(x0)
    g.forward_layer(0, prior)
    got_x = g.get_x()
    got_k, got_v = g.get_kv(0, prior, 1)
    g.close()
    # the K row (bias, RoPE) and V row (bias) the fused attention kernel stored
    for tag, got, want in (("K row", got_k[0], want_k), ("V row", got_v[0], want_v)):
        ok, err = within(got, want)
        assert ok, f"{tag} at position {prior}: max |err| {err:.3e}"
    # The layer re-quantizes four activations to Q8_0; fp32 reduction order
    # (GPU vs x86) can flip an element sitting within an ulp of a rounding
    # boundary by one q8 step, which moves the layer update by up to ~1e-3
    # (see test_layer_stepwise_qwen25_3b for the per-op bounds on identical
    # inputs).  The update x_out - x0 is therefore compared norm-wise.
    d_gpu, d_orc = got_x.astype(np.float64) - x0, want_x.astype(np.float64) - x0
    rel = np.linalg.norm(d_gpu - d_orc) / np.linalg.norm(d_orc)
    assert rel < 1e-3, f"layer update relative error {rel}"
    assert np.max(np.abs(got_x - want_x)) < max_abs
    # the layer added a non-trivial update to the residual
    assert np.max(np.abs(want_x - x0)) > 1e-2


def test_layer_parity_qwen25_3b(ctx):
    """Config 3: hidden 2048 (32-lane rows), GQA 16/2, FFN 11008, KV 1024, biases."""
    from llm_core_amd.model import QWEN25_3B_LAYER

    _layer_parity(ctx, QWEN25_3B_LAYER, 1024, True, 3)


def test_layer_parity_llama7b_shape(ctx):
    """One LLaMA-2-7B-shaped layer (hidden 4096: 64-lane rows, 32/32 heads,
    FFN 11008) at context 2048: the shapes of the decode benchmark."""
    from llm_core_amd.model import LLAMA2_7B

    _layer_parity(ctx, LLAMA2_7B, 2047, False, 4)


def test_layer_parity_hidden3072(ctx):
    """Hidden 3072 (12 super-blocks: half-block units on 24 of the 32 lanes of
    a row), GQA 24/8, FFN 8192, biases, context 300.  One element of this
    layer's update differs by 2.5e-3 after a one-step Q8_0 rounding flip (the
    norm-wise error stays below 1e-3), hence the wider elementwise bound."""
    cfg = dict(n_embd=3072, n_heads=24, n_kv_heads=8, ffn_dim=8192, rms_eps=1e-6,
               rope_theta=1e6)
    _layer_parity(ctx, cfg, 300, True, 5, max_abs=4e-3)


def test_layer_stepwise_qwen25_3b(ctx):
    """Each GPU op of the config-3 layer on exactly the oracle's inputs:
    integer/byte ops and RoPE bit-exact, GEMVs and attention within the
    north-star tolerance, RMSNorm within 2e-6 relative."""
    from llm_core_amd import hip
    from llm_core_amd.model import QWEN25_3B_LAYER, Hparams, SynthLlama

    cfg = dict(QWEN25_3B_LAYER)
    cfg["n_vocab"] = 256
    hp = Hparams(n_ctx=1025, **cfg)
    m = SynthLlama(hp, seed=3, norm_std=0.1, with_bias=True)
    E, H, KVH, HD, FD = hp.n_embd, hp.n_heads, hp.n_kv_heads, hp.head_dim, hp.ffn_dim
    kve, pos = KVH * HD, 1024
    T = {k: v[1] for k, v in m.tensors.items()}
    kc = np.zeros((hp.n_ctx, kve), np.float32)
    vc = np.zeros((hp.n_ctx, kve), np.float32)
    kc[:pos] = hip.synth_normal(pos * kve, 31).reshape(pos, kve)
    vc[:pos] = hip.synth_normal(pos * kve, 32).reshape(pos, kve)
    x0 = hip.synth_normal(E, 33)
    cos_t, sin_t = O.rope_table(HD, hp.rope_theta, hp.n_ctx)

    def dev(a):
        return ctx.upload(np.ascontiguousarray(a))

    def gpu_gemv(qt, name, xq, rows, cols):
        y = ctx.alloc(rows * 4)
        ctx.gemv_q8(qt, y, dev(T[name]), dev(xq), rows, cols, O.row_bytes(qt, cols))
        return ctx.download(y, np.float32, rows)

    def check(tag, got, want, rtol=1e-3, atol=1e-4):
        ok, err = within(got, want, rtol, atol)
        assert ok, f"{tag}: max abs err {err}"

    # attention block
    xb = O.rmsnorm(x0, T["blk.0.attn_norm.weight"], hp.rms_eps)
    y = ctx.alloc(E * 4)
    ctx.rmsnorm(y, None, dev(x0), dev(T["blk.0.attn_norm.weight"]), E, hp.rms_eps)
    check("attn rmsnorm", ctx.download(y, np.float32, E), xb, 2e-6, 1e-7)
    xq = O.quantize_q8_0(xb)
    q = O.gemv_q8(O.Q4K, T["blk.0.attn_q.weight"], xq, E, E) + T["blk.0.attn_q.bias"]
    k = O.gemv_q8(O.Q4K, T["blk.0.attn_k.weight"], xq, kve, E) + T["blk.0.attn_k.bias"]
    v = O.gemv_q8(O.Q6K, T["blk.0.attn_v.weight"], xq, kve, E) + T["blk.0.attn_v.bias"]
    check("q", gpu_gemv(O.Q4K, "blk.0.attn_q.weight", xq, E, E) + T["blk.0.attn_q.bias"], q)
    check("k", gpu_gemv(O.Q4K, "blk.0.attn_k.weight", xq, kve, E) + T["blk.0.attn_k.bias"], k)
    check("v", gpu_gemv(O.Q6K, "blk.0.attn_v.weight", xq, kve, E) + T["blk.0.attn_v.bias"], v)
    qr = O.rope(q, pos, H, HD, cos_t, sin_t)
    kr = O.rope(k, pos, KVH, HD, cos_t, sin_t)
    dq = ctx.alloc(q.nbytes)
    ctx.rope(dq, dev(q), pos, H, HD, dev(cos_t), dev(sin_t))
    assert np.array_equal(ctx.download(dq, np.float32, q.size), qr)
    kc[pos], vc[pos] = kr, v
    ao = O.attention(qr, kc[:pos + 1], vc[:pos + 1], pos + 1, H, KVH, HD)
    da = ctx.alloc(ao.nbytes)
    ctx.attn_decode(da, None, dev(qr), dev(kc[:pos + 1]), dev(vc[:pos + 1]), pos + 1, H, KVH, HD)
    check("attention", ctx.download(da, np.float32, ao.size), ao, 1e-5, 1e-6)
    aq = O.quantize_q8_0(ao)
    o = O.gemv_q8(O.Q4K, T["blk.0.attn_output.weight"], aq, E, E)
    check("o", gpu_gemv(O.Q4K, "blk.0.attn_output.weight", aq, E, E), o)
    x1 = x0 + o
    # FFN block
    xb2 = O.rmsnorm(x1, T["blk.0.ffn_norm.weight"], hp.rms_eps)
    xq2 = O.quantize_q8_0(xb2)
    gate = O.gemv_q8(O.Q4K, T["blk.0.ffn_gate.weight"], xq2, FD, E)
    up = O.gemv_q8(O.Q4K, T["blk.0.ffn_up.weight"], xq2, FD, E)
    check("gate", gpu_gemv(O.Q4K, "blk.0.ffn_gate.weight", xq2, FD, E), gate)
    check("up", gpu_gemv(O.Q4K, "blk.0.ffn_up.weight", xq2, FD, E), up)
    sw = O.swiglu(gate, up)
    ds = ctx.alloc(sw.nbytes)
    ctx.swiglu(ds, None, dev(gate), dev(up), FD)
    assert np.array_equal(ctx.download(ds, np.float32, FD), sw)
    sq = O.quantize_q8_0(sw)
    down = O.gemv_q8(O.Q6K, T["blk.0.ffn_down.weight"], sq, E, FD)
    check("down", gpu_gemv(O.Q6K, "blk.0.ffn_down.weight", sq, E, FD), down)
    x2 = x1 + down
    # the composed oracle ops reproduce the oracle's own layer bit for bit
    om = O.OracleModel(hp, m.tensors)
    ok_, ov_ = om.kv_view()
    ok_[0, :pos] = kc[:pos]
    ov_[0, :pos] = vc[:pos]
    om.x_view()[:] = x0
    om.forward_layer(0, pos)
    assert np.array_equal(om.x_view(), x2)
    om.close()


def test_output_head_c2_full(ctx):
    from llm_core_amd import hip

    rows, cols = 151936, 2048
    W = hip.synth_weight(hip.AXF_TYPE_Q6_K, rows, cols, 2)
    x = hip.synth_normal(cols, 22)
    xq = O.quantize_q8_0(x)
    want = O.gemv_q8(O.Q6K, W, xq, rows, cols)
    dW, dx, dy, di = ctx.upload(W), ctx.upload(x), ctx.alloc(rows * 4), ctx.alloc(4)
    dq = ctx.alloc(cols // 32 * 36)
    ctx.quantize_q8_0(dq, dx, cols)
    assert np.array_equal(ctx.download(dq, np.uint8, cols // 32 * 36), xq)
    ctx.gemv_q8(hip.AXF_TYPE_Q6_K, dy, dW, dq, rows, cols, hip.row_bytes(hip.AXF_TYPE_Q6_K, cols))
    ctx.argmax(di, dy, rows)
    got = ctx.download(dy, np.float32, rows)
    ok, err = within(got, want)
    assert ok, err
    idx = int(ctx.download(di, np.int32, 1)[0])
    assert idx == int(np.argmax(got))
    if idx != O.argmax(want):
        assert O.top2_margin(want) < 1e-4, "argmax differs without a near tie"
    dW.free()


SMALL = dict(n_layer=2, n_embd=512, n_heads=8, n_kv_heads=4, ffn_dim=1024, n_vocab=1000,
             n_ctx=64, rms_eps=1e-5, rope_theta=10000.0)


# A single Q8_0 rounding flip of one activation (fp32 summation order decides
# ties that land within an ulp of .5) moves a logit by about |w|*d_x, ~1e-3 on
# these models; the exact-sequence test uses models whose oracle margins stay
# above this bound for all 32 tokens.
NEAR_TIE = 5e-3


def _run(ctx, seed, n_gen=32):
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    hp = Hparams(**SMALL)
    m = SynthLlama(hp, seed=seed, norm_std=0.1)
    rng = np.random.default_rng(seed)
    prompt = np.concatenate([[1], rng.integers(0, hp.n_vocab, 7)]).astype(np.int32)

    g = LlamaHip(ctx, m)
    graph = g.generate(prompt, n_gen, use_graph=True)  # batched prefill
    eager = g.generate(prompt, n_gen, use_graph=False)
    graph2 = g.generate(prompt, n_gen, use_graph=True)  # replays are repeatable
    tbt = g.generate(prompt, n_gen, use_graph=True, batched_prefill=False)
    g.forward_token(int(prompt[0]), 0)
    gl = g.logits()
    g.close()
    assert np.array_equal(graph, eager), "graph replay and eager launches disagree"
    assert np.array_equal(graph, graph2), "second graph generation differs"
    assert np.array_equal(graph, tbt), "batched and token-by-token prefill disagree"

    om = O.OracleModel(hp, m.tensors)
    seq = om.generate(prompt, n_gen, batched_prefill=False)
    bat = om.generate(prompt, n_gen, batched_prefill=True)
    om.reset()
    om.forward_token(int(prompt[0]), 0)
    ol = om.logits()
    om.close()
    ok, err = within(gl, ol)
    assert ok, f"logits max abs err {err}"
    return graph, seq, bat


@pytest.mark.parametrize("seed", [7, 12, 33])
def test_greedy_32_tokens_identical(ctx, seed):
    """Models whose oracle margins over the 32 tokens all exceed NEAR_TIE: the
    GPU's greedy ids equal the oracle's under both prefill schemes."""
    graph, (tseq, mseq), (tbat, mbat) = _run(ctx, seed)
    assert min(mseq.min(), mbat.min()) >= NEAR_TIE and np.array_equal(tseq, tbat)
    assert np.array_equal(graph, tseq), (graph, tseq)


# Per-step logit bounds with identical history (KV re-synced to the oracle's):
# without a Q8_0 flip the step agrees to fp32 noise; a single one-step flip of
# a layer-0 activation moves the logits of these small-residual models by up
# to ~2e-2 (measured by flipping the activation nearest a rounding boundary in
# the oracle itself), and such flips are rare.
STEP_NOISE = 1e-5
ONE_FLIP = 3e-2


@pytest.mark.parametrize("seed", [5, 23])
def test_teacher_forced_step_logits(ctx, seed):
    """Both sides decode the oracle's greedy sequence; before every step the
    GPU's KV cache is set to the oracle's so each step starts from identical
    history.  Per step: logits within STEP_NOISE, or within ONE_FLIP at a few
    positions; the greedy pick agrees wherever the oracle's top-1/top-2 margin
    exceeds twice the step's logit difference."""
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    hp = Hparams(**SMALL)
    m = SynthLlama(hp, seed=seed, norm_std=0.1)
    rng = np.random.default_rng(seed)
    prompt = np.concatenate([[1], rng.integers(0, hp.n_vocab, 7)]).astype(np.int32)
    om = O.OracleModel(hp, m.tensors)
    gen, _ = om.generate(prompt, 32, batched_prefill=False)
    seq = np.concatenate([prompt, gen[:-1]])
    om.reset()
    g = LlamaHip(ctx, m)
    flips = 0
    for pos, tok in enumerate(seq):
        if pos:
            kk, vv = om.kv_view()
            for layer in range(hp.n_layer):
                g.set_kv(layer, kk[layer, :pos], vv[layer, :pos], pos)
        om.forward_token(int(tok), pos)
        g.forward_token(int(tok), pos)
        ol, gl = om.logits(), g.logits()
        diff = float(np.max(np.abs(gl.astype(np.float64) - ol)))
        assert diff < ONE_FLIP, f"pos {pos}: logits differ by {diff}"
        flips += diff > STEP_NOISE
        if O.top2_margin(ol) > 2 * diff:
            assert int(np.argmax(gl)) == O.argmax(ol), f"pos {pos}: greedy pick differs"
    g.close()
    om.close()
    assert flips <= len(seq) // 5, f"{flips} of {len(seq)} steps beyond fp32 noise"
    print(f"seed {seed}: {flips} of {len(seq)} steps with a Q8_0 flip")


def test_generate_rejects_bad_input(ctx):
    from llm_core_amd._ffi import AxfError
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    hp = Hparams(**SMALL)
    synth = SynthLlama(hp, seed=9)
    g = LlamaHip(ctx, synth)
    with pytest.raises(AxfError):
        g.generate(np.array([1, 5000], np.int32), 4)  # token id beyond the vocabulary
    with pytest.raises(AxfError):
        g.generate(np.arange(60, dtype=np.int32), 10)  # exceeds n_ctx
    # the context stop of llama_generate_cpu_impl (:1613): with 60 prompt
    # tokens and n_ctx 64 the reference emits 4 tokens; the oracle's loop
    # (pinned on the CPU) agrees, and the device takes 4 but refuses 5
    prompt = np.arange(1, 61, dtype=np.int32)
    om = O.OracleModel(hp, synth.tensors)
    try:
        want, _ = om.generate(prompt, 5)
    finally:
        om.close()
    assert len(want) == hp.n_ctx - len(prompt)
    assert len(g.generate(prompt, len(want))) == len(want)
    with pytest.raises(AxfError):
        g.generate(prompt, len(want) + 1)
    g.close()


# ---------------------------------------------------------------------------
# batched prefill (llama_forward_batch)
# ---------------------------------------------------------------------------

def _prefill_case(ctx, hp_kwargs, seed, T, splits=(), with_bias=False, layer_types=None):
    """Last-row logits and residual after a batched prefill of T tokens (run as
    the given chunk boundaries on the GPU), against the oracle's single batch."""
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    hp = Hparams(**hp_kwargs)
    m = SynthLlama(hp, seed=seed, norm_std=0.1, with_bias=with_bias, layer_types=layer_types)
    rng = np.random.default_rng(seed)
    toks = np.concatenate([[1], rng.integers(0, hp.n_vocab, T - 1)]).astype(np.int32)
    om = O.OracleModel(hp, m.tensors)
    om.forward_batch(toks, 0)
    ol, ox = om.logits(), om.x_view().copy()
    # the oracle's own token-by-token path: its distance to the batch measures
    # how far fp32 reordering moves these logits on this input (a Q8_0 rounding
    # flip of one activation moves them by ~1e-2 on the small models; about one
    # input in three has such a near-tie somewhere)
    om.reset()
    for t, tok in enumerate(toks):
        om.forward_token(int(tok), t)
    noise = float(np.max(np.abs(om.logits().astype(np.float64) - ol)))
    om.close()
    g = LlamaHip(ctx, m)
    bounds = [0, *splits, T]
    for a, b in zip(bounds[:-1], bounds[1:]):
        g.forward_batch(toks[a:b], a)
    gl, gx = g.logits(), g.get_x()
    # the GPU's decode path over the same tokens (the per-token GEMVs, checked
    # against the oracle by the decode tests) sums in a third order: its
    # distance to the oracle's batch is another sample of the same noise (each
    # step rewrites cache row t before attending to rows 0..t)
    for t, tok in enumerate(toks):
        g.forward_token(int(tok), t)
    noise = max(noise, float(np.max(np.abs(g.logits().astype(np.float64) - ol))))
    g.close()
    return gl, ol, gx, ox, noise


def _check_prefill(gl, ol, noise):
    """Logits within the tolerance, or within twice the oracle's own reorder
    noise on this input; the greedy pick agrees wherever the oracle's
    top-1/top-2 margin exceeds the observed difference."""
    err = float(np.max(np.abs(gl.astype(np.float64) - ol)))
    ok, _ = within(gl, ol)
    assert ok or err <= 2 * noise + 1e-4, f"logits max abs err {err}, oracle noise {noise}"
    if O.top2_margin(ol) > 2 * err:
        assert int(np.argmax(gl)) == O.argmax(ol)


@pytest.mark.parametrize("seed,T", [(3, 24), (8, 9), (21, 64)])
def test_forward_batch_small(ctx, seed, T):
    gl, ol, gx, ox, noise = _prefill_case(ctx, SMALL, seed, T)
    _check_prefill(gl, ol, noise)
    rel = np.linalg.norm(gx.astype(np.float64) - ox) / np.linalg.norm(ox)
    assert rel < 1e-3 or noise > 1e-3, f"final-norm row relative error {rel}"


def test_forward_batch_in_chunks(ctx):
    """Prefill as three calls (positions 0, 5, 30) equals the single batch."""
    gl, ol, gx, ox, noise = _prefill_case(ctx, SMALL, 11, 40, splits=(5, 30))
    _check_prefill(gl, ol, noise)


def test_forward_batch_qwen25_3b_layer(ctx):
    """One Qwen2.5-3B-like layer (hidden 2048, 16/2 heads, FFN 11008, q/k/v
    biases) prefilling 48 tokens: last-row logits and residual."""
    cfg = dict(n_layer=1, n_embd=2048, n_heads=16, n_kv_heads=2, ffn_dim=11008, n_vocab=512,
               n_ctx=64, rms_eps=1e-6, rope_theta=1e6)
    gl, ol, gx, ox, noise = _prefill_case(ctx, cfg, 4, 48, with_bias=True)
    # four Q8_0 re-quantisations per layer: the final-norm row norm-wise as in
    # the decode layer test, the logits against the oracle's own reorder noise
    rel = np.linalg.norm(gx.astype(np.float64) - ox) / np.linalg.norm(ox)
    assert rel < 1e-3, f"final-norm row relative error {rel}"
    _check_prefill(gl, ol, max(noise, 1e-3))


@pytest.mark.parametrize("down", ["q6_k", "q4_k", "q8_0"])
def test_forward_batch_swiglu_epilogue(ctx, down):
    """Hidden 2304 (9 super-blocks per row: ffn_gate|ffn_up interleaved by
    8-row blocks) prefilling 80 tokens: the fp16 gate|up GEMM writes SwiGLU's
    Q8_0 blocks in its epilogue, with their fp16 re-layout, which a Q4_K down
    projection reads (the fp16 Q6_K kernel would, at 256 tiles and more), and
    for a Q8_0 down projection, which takes the fp32 rows, those too; last-row
    logits and residual against the oracle's batch."""
    from llm_core_amd.model import AXF_TYPE_Q4_K, AXF_TYPE_Q8_0, Q4K_M_TYPES

    cfg = dict(n_layer=1, n_embd=2304, n_heads=18, n_kv_heads=6, ffn_dim=1024, n_vocab=512,
               n_ctx=96, rms_eps=1e-5, rope_theta=10000.0)
    types = {"q6_k": None, "q4_k": dict(Q4K_M_TYPES, ffn_down=AXF_TYPE_Q4_K),
             "q8_0": dict(Q4K_M_TYPES, ffn_down=AXF_TYPE_Q8_0)}[down]
    gl, ol, gx, ox, noise = _prefill_case(ctx, cfg, 5, 80, layer_types=types)
    _check_prefill(gl, ol, noise)
    rel = np.linalg.norm(gx.astype(np.float64) - ox) / np.linalg.norm(ox)
    assert rel < 1e-3 or noise > 1e-3, f"final-norm row relative error {rel}"


def test_forward_batch_swiglu_epilogue_in_chunks(ctx):
    """The same model prefilling 160 tokens as two 80-token calls (the second at
    position 80: the re-layouts of a chunk that attends to the cache rows of
    the first) against the oracle's single batch."""
    cfg = dict(n_layer=1, n_embd=2304, n_heads=18, n_kv_heads=6, ffn_dim=1024, n_vocab=512,
               n_ctx=192, rms_eps=1e-5, rope_theta=10000.0)
    gl, ol, gx, ox, noise = _prefill_case(ctx, cfg, 6, 160, splits=(80,))
    _check_prefill(gl, ol, noise)
    rel = np.linalg.norm(gx.astype(np.float64) - ox) / np.linalg.norm(ox)
    assert rel < 1e-3 or noise > 1e-3, f"final-norm row relative error {rel}"


@pytest.mark.parametrize("order", [1, 2])
def test_forward_batch_qk_norm(ctx, order):
    """Per-head q/k RMSNorm before RoPE (qwen3) or after it (hunyuan-dense),
    q/k/v biases, 2 layers, a prefill of 40 tokens in two calls: last-row
    logits and residual against the oracle's batch (the decode step's kernels
    are checked stage by stage in test_gpu_fused)."""
    cfg = {**SMALL, "qk_norm_order": order}
    gl, ol, gx, ox, noise = _prefill_case(ctx, cfg, 30 + order, 40, splits=(17,),
                                          with_bias=True)
    _check_prefill(gl, ol, noise)
    rel = np.linalg.norm(gx.astype(np.float64) - ox) / np.linalg.norm(ox)
    assert rel < 1e-3 or noise > 1e-3, f"final-norm row relative error {rel}"


def test_forward_batch_rejects_bad_input(ctx):
    from llm_core_amd._ffi import AxfError
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    hp = Hparams(**SMALL)
    g = LlamaHip(ctx, SynthLlama(hp, seed=1))
    with pytest.raises(AxfError):
        g.forward_batch(np.array([1, hp.n_vocab], np.int32))  # token out of range
    with pytest.raises(AxfError):
        g.forward_batch(np.ones(hp.n_ctx, np.int32), 1)  # past the context
    g.close()
