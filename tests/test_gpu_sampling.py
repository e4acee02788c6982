"""The device sampler against the oracle's restatement of sample() and
apply_rep_penalty (llama_model.cpp:1466-1498, :1595-1605), and the sampled
generation loop (axf_llama_generate_sampled) against a teacher-forced oracle."""
import numpy as np
import pytest

from llm_core_amd import hip
from oracle import oracle as O

pytestmark = pytest.mark.gpu

# a decision within this distance of flipping may go either way: expf on the
# device and in glibc may differ by an ulp, which moves a cumulative
# probability by ~k ulps
EXP_SLACK = 1e-5


def slack(k, n_vocab):
    kk = k if 0 < k < n_vocab else n_vocab
    return EXP_SLACK + 2 * kk * 2.0 ** -23

PARAMS = [  # temperature, top_k, top_p, rep_penalty, last_n
    (1.0, 40, 1.0, 1.0, 64),
    (0.7, 40, 0.9, 1.1, 64),
    (1.3, 200, 0.95, 1.3, 16),
    (0.5, 1, 1.0, 1.0, 64),
    (0.0, 40, 1.0, 1.2, 8),     # greedy after the penalty
    (0.9, 0, 1.0, 1.0, 64),     # whole vocabulary (beyond 16384: the in-place global sort)
    (1.0, 5000, 0.95, 1.0, 64),  # k above a chunk (4096): every entry is a candidate
]


@pytest.mark.parametrize("n_vocab", [1000, 16000, 32000, 151936])
def test_sample_matches_oracle(ctx, n_vocab):
    rng = np.random.default_rng(n_vocab)
    compared = skipped = 0
    for (T, k, p, pen, last_n) in PARAMS:
        for trial in range(6):
            x = (rng.standard_normal(n_vocab) * 2.5).astype(np.float32)
            hist = rng.integers(0, n_vocab, 40).astype(np.int32)
            hist[5] = hist[9] = hist[20]  # a repeated id is penalised twice
            r = float(hip.sampling_uniforms(trial + 7 * k, 1)[0])
            d = ctx.upload(x)
            tok = ctx.sample(d, n_vocab, T, k, p, pen, last_n, hist, r)
            pen_x = O.rep_penalty(x, hist, last_n, pen)
            # the penalty is applied in place, as on state.logits, and exactly
            np.testing.assert_array_equal(ctx.download(d, np.float32, n_vocab), pen_x)
            want, margin = O.sample(pen_x, k, p, T, r)
            if tok != want:
                assert margin < slack(k, n_vocab), (T, k, p, pen, trial, tok, want, margin)
                skipped += 1
            compared += 1
            d.free()
    assert skipped <= compared // 20


def test_greedy_first_index_of_maximum(ctx):
    x = np.random.default_rng(1).standard_normal(151936).astype(np.float32)
    x[77777] = x[4242] = x.max() + 1.0
    d = ctx.upload(x)
    assert ctx.sample(d, x.size, temperature=0.0) == 4242
    assert ctx.sample(d, x.size, temperature=0.5, top_k=1) == 4242  # tie: lower index first


def test_sample_any_k_at_large_vocabulary(ctx):
    """Either side of the 16384-candidate LDS sort (38 chunks x 431 fits, x 432
    does not) and far beyond it, against the oracle."""
    n = 151936
    rng = np.random.default_rng(5)
    for k in (431, 432, 20000, 0):
        x = (rng.standard_normal(n) * 3.0).astype(np.float32)
        r = float(hip.sampling_uniforms(k + 1, 1)[0])
        d = ctx.upload(x)
        tok = ctx.sample(d, n, temperature=0.8, top_k=k, top_p=0.9, r=r)
        want, margin = O.sample(x, k, 0.9, 0.8, r)
        assert tok == want or margin < slack(k, n), (k, tok, want, margin)
        d.free()


SMALL = dict(n_layer=2, n_embd=512, n_heads=8, n_kv_heads=4, ffn_dim=1024, n_vocab=1000,
             n_ctx=64, rms_eps=1e-5, rope_theta=10000.0)


@pytest.mark.parametrize("cfg", [
    dict(temperature=0.8, top_k=40, top_p=0.95, rep_penalty=1.1, rep_penalty_last_n=16),
    dict(temperature=1.0, top_k=40),
    dict(temperature=0.0, rep_penalty=1.3, rep_penalty_last_n=8),
])
def test_generate_sampled_teacher_forced(ctx, cfg):
    """The device loop equals an eager step-by-step GPU replay (same kernels,
    so the same tokens), and every step's choice equals the oracle's on its own
    logits after the same history, unless the oracle's decision lies within the
    logit difference's reach (2 * max|dlogit| / T of the cumulative sums)."""
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    hp = Hparams(**SMALL)
    m = SynthLlama(hp, seed=13, norm_std=0.1)
    prompt = np.array([1, 55, 320, 7, 999, 12, 600], np.int32)
    n_new = 24
    with LlamaHip(ctx, m) as g:
        toks = g.generate_sampled(prompt, n_new, use_graph=True, **cfg)
        assert toks.size == n_new
        assert np.array_equal(toks, g.generate_sampled(prompt, n_new, use_graph=False, **cfg))
        r = hip.sampling_uniforms(42, n_new)
        T = cfg.get("temperature", 1.0)
        k, p = cfg.get("top_k", 40), cfg.get("top_p", 1.0)
        pen, last_n = cfg.get("rep_penalty", 1.0), cfg.get("rep_penalty_last_n", 64)
        om = O.OracleModel(hp, m.tensors)
        om.forward_batch(prompt, 0)
        g.forward_batch(prompt, 0)
        hist = list(prompt)
        flips = []
        for i in range(n_new):
            if i > 0:
                om.forward_token(int(toks[i - 1]), len(prompt) + i - 1)
                g.forward_token(int(toks[i - 1]), len(prompt) + i - 1)
            gl = g.logits()
            d = ctx.upload(gl)
            assert ctx.sample(d, hp.n_vocab, T, k, p, pen, last_n, np.array(hist, np.int32),
                              float(r[i])) == toks[i], i
            d.free()
            ol = om.logits()
            want, margin = O.sample(O.rep_penalty(ol, hist, last_n, pen), k, p, T, float(r[i]))
            if want != toks[i]:
                dl = float(np.max(np.abs(gl.astype(np.float64) - ol)))
                reach = (2 * dl / T if T > 0 else 2 * dl) + EXP_SLACK
                assert margin <= reach, (i, toks[i], want, margin, dl)
                flips.append((i, margin, dl))
            hist.append(int(toks[i]))
        om.close()
        # a Q8_0 rounding flip in the cached history moves every later step's
        # logits by ~1e-2, which puts many decisions within reach; most must still agree
        assert len(flips) <= n_new // 4, flips


def test_generate_sampled_stops_at_eos_and_context(ctx):
    from llm_core_amd.model import Hparams, LlamaHip, SynthLlama

    hp = Hparams(**{**SMALL, "n_ctx": 16})
    m = SynthLlama(hp, seed=3, norm_std=0.1)
    prompt = np.array([1, 2, 3, 4, 5], np.int32)
    with LlamaHip(ctx, m) as g:
        full = g.generate_sampled(prompt, 40, temperature=0.9, top_k=40)
        assert full.size == 16 - 5  # tokens are emitted while n_past < n_ctx
        eos = int(full[4])
        first = int(np.argmax(full == eos))
        cut = g.generate_sampled(prompt, 40, temperature=0.9, top_k=40, eos_id=eos)
        assert np.array_equal(cut, full[:first])  # EOS itself is not emitted
        assert g.generate_sampled(prompt, 3, temperature=0.9, top_k=40).size == 3
