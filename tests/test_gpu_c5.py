"""Config 5 at full size: the LLaMA-2-7B-architecture Q4_K_M model (32 layers,
hidden 4096, 32 heads, FFN 11008, vocab 32000, theta 1e4; Q6_K for v, down
and the head), a 512-token uniform-random prompt, greedy decode, context 2048
(llama_generate_cpu_impl, llama_model.cpp:1502-1631).

  * property checks at full size: the 32 greedy ids are identical between
    HIP-graph replay and eager launches, and repeatable; the token-by-token
    prefill gives the same ids wherever the device's own teacher-forced top-2
    margin exceeds the logit difference between the two prefill paths;
  * with the cache rows 0..510 of the device's batched prefill, the last
    prompt row (position 511) and three teacher-forced decode steps run stage
    by stage through all 32 layers: each fused stage (q|k|v, attention with
    the K/V store, o, gate|up with SwiGLU, down) is compared with the oracle on
    that stage's device inputs at the north-star tolerance (K/V rows and the
    attention's Q8_0 bit-exact); then the whole step in one call must give the
    same bits, and its logits must match the oracle's head on the device's
    final row.  Whole-model comparisons would test the random model's
    sensitivity instead: a Q8_0 requantisation that lands on the other side of
    a rounding boundary (device and oracle sum RMSNorm in different orders)
    moves that layer's update by up to a few 1e-3, and such differences grow
    through the later layers.  The test prints that growth (the batched
    prefill's row 511 against the decode path's row over the same cache, per
    layer) and requires layer 0, where nothing has grown yet, to agree to fp32
    rounding;
  * against the reference itself: tests/golden/c5_greedy.json holds the 32
    greedy ids of the same model on the reference's compiled x86 kernels
    (tests/golden/make_c5_greedy.py; a 512-token prompt starting with BOS) and
    the reference's top-2 margin at each; the device's ids must equal them up
    to the first step whose reference margin is within the device's measured
    prefill-path noise (where fp32 summation order can decide the token).
"""
import json
from pathlib import Path

import numpy as np
import pytest

from gpu_helpers import device_norm_q8, layer_stage_errors, within
from oracle import oracle as O

FIXTURE = Path(__file__).resolve().parent / "golden" / "c5_greedy.json"

pytestmark = [pytest.mark.gpu, pytest.mark.slow]

N_PROMPT, N_GEN = 512, 32


def rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / np.linalg.norm(want)), float(np.max(np.abs(got - want)))


@pytest.mark.timeout(900)
def test_config5_full_size(ctx):
    from llm_core_amd.model import LLAMA2_7B, Hparams, LlamaHip, SynthLlama

    hp = Hparams(n_ctx=2048, **LLAMA2_7B)
    model = SynthLlama(hp, seed=5)
    prompt = np.random.default_rng(5).integers(0, hp.n_vocab, N_PROMPT).astype(np.int32)
    g = LlamaHip(ctx, model)
    try:
        graph = g.generate(prompt, N_GEN, use_graph=True)
        eager = g.generate(prompt, N_GEN, use_graph=False)
        again = g.generate(prompt, N_GEN, use_graph=True)
        print(f"\n  greedy ids (graph): {list(graph[:12])} ...", flush=True)
        assert np.array_equal(graph, eager), "graph replay and eager launches differ"
        assert np.array_equal(graph, again), "graph replays are not repeatable"

        # teacher-forced device logits along the batched-prefill run
        g.forward_batch(prompt, 0)
        dev_logits = [g.logits()]
        k511, v511 = zip(*(g.get_kv(layer, N_PROMPT - 1, 1) for layer in range(hp.n_layer)))
        kv_dev = [g.get_kv(layer, 0, N_PROMPT - 1) for layer in range(hp.n_layer)]
        for i in range(N_GEN - 1):
            g.forward_token(int(graph[i]), N_PROMPT + i)
            dev_logits.append(g.logits())
        for i in range(N_GEN):
            assert int(np.argmax(dev_logits[i])) == int(graph[i])
        margins = np.array([O.top2_margin(lg) for lg in dev_logits])

        # the token-by-token prefill (the llama_forward_token path over the prompt)
        tbt = g.generate(prompt, N_GEN, use_graph=True, batched_prefill=False)
        for t in range(N_PROMPT):
            g.forward_token(int(prompt[t]), t)
        tbt0 = g.logits()
        _, d0 = rel_err(tbt0, dev_logits[0])
        print(f"  prefill paths: last-row logits max |diff| {d0:.2e}; "
              f"margins min {margins.min():.3e}", flush=True)
        same = int(np.argmax(graph != tbt)) if np.any(graph != tbt) else N_GEN
        print(f"  token-by-token prefill: first {same} of {N_GEN} ids equal the batched run's",
              flush=True)
        for i in range(N_GEN):
            if graph[i] != tbt[i]:
                # the first divergence must sit at a step the paths' difference can flip
                assert margins[i] <= 2 * max(d0, 1e-3), (
                    f"step {i}: batched {graph[i]} vs token-by-token {tbt[i]}, "
                    f"margin {margins[i]:.3e}")
                break
    finally:
        g.close()

    # oracle, stage by stage at every layer: the cache rows 0..510 of the
    # device's batched prefill, then the last prompt row (position 511) and
    # three teacher-forced decode steps.  Each fused stage of each layer is
    # compared with the oracle on that stage's device inputs.
    g = LlamaHip(ctx, model)
    try:
        for layer, (kk, vv) in enumerate(kv_dev):
            g.set_kv(layer, kk, vv, N_PROMPT - 1)
        T = {k: v[1] for k, v in model.tensors.items()}
        qt, emb = model.tensors["token_embd.weight"]
        rb = O.row_bytes(qt, hp.n_embd)
        out_qt, out_w = model.tensors["output.weight"]
        growth = []
        for tok, pos in ([(int(prompt[-1]), N_PROMPT - 1)] +
                         [(int(graph[i]), N_PROMPT + i) for i in range(3)]):
            g.set_x(O.dequant(qt, emb[tok * rb:(tok + 1) * rb]))
            worst = {}
            for layer in range(hp.n_layer):
                for tag, err, nbad, rel in layer_stage_errors(ctx, g, T, hp, layer, pos):
                    assert nbad == 0, (f"pos {pos} layer {layer} {tag}: {nbad} elements outside "
                                       f"tolerance, max |err| {err:.3e}")
                    worst[tag] = max(worst.get(tag, 0.0), rel)
                if pos == N_PROMPT - 1:
                    # the batched prefill's row 511 vs the decode path's, same rows 0..510
                    growth.append(rel_err(k511[layer][0], g.get_kv(layer, pos, 1)[0][0])[0])
            xf = g.get_x()
            g.forward_token(tok, pos)                  # the same kernels in one call + head
            assert np.array_equal(g.get_x(), xf)
            got = g.logits()
            # the head on the device's Q8_0 of the final norm (oracle-checked inside)
            xq = device_norm_q8(ctx, xf, model.tensors["output_norm.weight"][1], hp.rms_eps)
            want = O.gemv_q8(out_qt, out_w, xq, hp.n_vocab, hp.n_embd)
            r, mx = rel_err(got, want)
            m = O.top2_margin(want)
            print(f"  pos {pos}: worst stage errors (norm-wise) "
                  + ", ".join(f"{k} {v:.1e}" for k, v in worst.items())
                  + f"; logits max |diff| {mx:.2e}, margin {m:.3e}, argmax gpu "
                  f"{int(np.argmax(got))} oracle {O.argmax(want)}", flush=True)
            ok, err, _ = within(got, want)
            assert ok, f"pos {pos}: logits max |err| {err:.3e}"
            if m > 2 * mx:
                assert int(np.argmax(got)) == O.argmax(want), f"position {pos}: argmax differs"
        print("  batched-prefill K row 511 vs the decode path on the same cache, per layer: "
              + " ".join(f"{v:.1e}" for v in growth), flush=True)
        assert growth[0] < 1e-5, "layer 0 K rows of the two paths differ beyond fp32 rounding"
    finally:
        g.close()


@pytest.mark.timeout(900)
def test_config5_against_the_reference(ctx):
    """The device against the reference's own generation on the same config-5
    model and prompt, teacher-forced: the device prefills the prompt (batched)
    and then decodes the reference's ids one by one, so that
    both sides hold the same history at every step.  Per step, the device's
    logits at the reference's 8 largest are compared with the reference's
    values.  The bound for that difference is twice the largest logit
    difference between the device's own two prefill paths on this prompt
    (batched, and token by token through the decode kernels): both are fp32
    summation-order effects (a Q8_0 requantisation that lands across a
    rounding boundary moves a layer's update, and such moves grow through 32
    random layers).  The device's argmax must be the reference's id at every
    step where the reference's top-2 margin exceeds twice that step's
    measured difference.  Free-running greedy ids are reported, not asserted:
    the reference's third step is a near-tie (margin 1e-3), which any other
    summation order may decide the other way."""
    from llm_core_amd.model import LLAMA2_7B, Hparams, LlamaHip, SynthLlama

    fx = json.loads(FIXTURE.read_text())
    hp = Hparams(n_ctx=fx["model"]["n_ctx"], **LLAMA2_7B)
    prompt = np.array(fx["prompt"], np.int32)
    rule = np.concatenate([[1], np.random.default_rng(5).integers(0, hp.n_vocab, prompt.size - 1)])
    assert np.array_equal(prompt, rule), "fixture prompt does not follow its rule"
    ref_ids, ref_m = np.array(fx["ids"]), np.array(fx["margins"])
    top_ids, top_v = np.array(fx["top_ids"]), np.array(fx["top_logits"], np.float64)
    assert np.array_equal(top_ids[:, 0], ref_ids)
    n = ref_ids.size
    model = SynthLlama(hp, seed=5)
    with LlamaHip(ctx, model) as g:
        free = g.generate(prompt, n, use_graph=True)
        g.forward_batch(prompt, 0)
        lb = g.logits().astype(np.float64)
        err, agree = np.zeros(n), np.zeros(n, bool)
        dev_m = np.zeros(n)
        for t in range(n):
            lg = g.logits().astype(np.float64) if t else lb
            err[t] = np.max(np.abs(lg[top_ids[t]] - top_v[t]))
            agree[t] = int(np.argmax(lg)) == ref_ids[t]
            s2 = np.sort(lg)[-2:]
            dev_m[t] = s2[1] - s2[0]
            g.forward_token(int(ref_ids[t]), prompt.size + t)
        for t, tok in enumerate(prompt):
            g.forward_token(int(tok), t)
        noise = float(np.max(np.abs(g.logits().astype(np.float64) - lb)))
    lead = int(np.argmax(free != ref_ids)) if np.any(free != ref_ids) else n
    scale = float(np.mean(np.abs(top_v[:, 0])))
    print(f"\n  free-running: {lead} of {n} leading ids equal the reference's (its step-{lead} margin "
          f"{ref_m[min(lead, n - 1)]:.3e})\n  teacher-forced: device argmax = reference id at {int(agree.sum())} "
          f"of {n} steps; top-8 logit |diff| max {err.max():.3e}, median {np.median(err):.3e} "
          f"(top logit ~{scale:.2f}); device two-path prefill noise {noise:.3e}", flush=True)
    for t in np.nonzero(~agree)[0]:
        print(f"    step {t}: reference margin {ref_m[t]:.3e}, device margin {dev_m[t]:.3e}, "
              f"step |diff| {err[t]:.3e}", flush=True)
    assert err.max() <= 2 * noise, f"top-8 logits differ by {err.max():.3e} > 2 x path noise {noise:.3e}"
    bad = [int(t) for t in np.nonzero(~agree & (ref_m > 2 * err))[0]]
    assert not bad, f"argmax differs at steps {bad} where the reference's margin exceeds twice the step's difference"
