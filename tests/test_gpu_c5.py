"""Config 5 at full size: the LLaMA-2-7B-architecture Q4_K_M model (32 layers,
hidden 4096, 32 heads, FFN 11008, vocab 32000, theta 1e4; Q6_K for v, down
and the head), a 512-token uniform-random prompt, greedy decode, context 2048
(llama_generate_cpu_impl, llama_model.cpp:1502-1631).

  * property checks at full size: the 32 greedy ids are identical between
    HIP-graph replay and eager launches, and repeatable; the token-by-token
    prefill gives the same ids wherever the device's own teacher-forced top-2
    margin exceeds the logit difference between the two prefill paths;
  * the oracle, with its KV cache rows 0..510 copied from the device's
    batched prefill, recomputes the last prompt row and three teacher-forced
    decode steps (positions 511..514).  Its K/V rows at 511 and its logits
    are compared with the device's, and the device's greedy choice must equal
    the oracle's wherever the oracle's top-2 margin exceeds twice the logit
    difference.  The bound on the logits is norm-wise (a Q8_0 requantisation
    of an activation that sits within fp32 noise of a rounding boundary moves
    single logits by up to ~1e-3 after 32 layers; see DESIGN.md's parity
    section for the measurement).
"""
import numpy as np
import pytest

from oracle import oracle as O

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
        for i in range(N_GEN):
            if graph[i] != tbt[i]:
                # the first divergence must sit at a step the paths' difference can flip
                assert margins[i] <= 2 * max(d0, 1e-3), (
                    f"step {i}: batched {graph[i]} vs token-by-token {tbt[i]}, "
                    f"margin {margins[i]:.3e}")
                break
    finally:
        g.close()

    # oracle: KV rows 0..510 from the device's batched prefill, then the last
    # prompt row (position 511) and three teacher-forced decode steps
    om = O.OracleModel(hp, model.tensors)
    try:
        ok_, ov_ = om.kv_view()
        for layer, (kk, vv) in enumerate(kv_dev):
            ok_[layer, :N_PROMPT - 1] = kk
            ov_[layer, :N_PROMPT - 1] = vv
        om.forward_token(int(prompt[-1]), N_PROMPT - 1)
        for layer in range(hp.n_layer):
            for tag, got, want in (("K", k511[layer][0], ok_[layer, N_PROMPT - 1]),
                                   ("V", v511[layer][0], ov_[layer, N_PROMPT - 1])):
                r, _ = rel_err(got, want)
                assert r < 1e-3, f"layer {layer} {tag} row {N_PROMPT - 1}: relative error {r:.2e}"
        steps = [(N_PROMPT - 1, om.logits(), dev_logits[0])]
        for i in range(3):
            om.forward_token(int(graph[i]), N_PROMPT + i)
            steps.append((N_PROMPT + i, om.logits(), dev_logits[i + 1]))
        for pos, want, got in steps:
            r, mx = rel_err(got, want)
            m = O.top2_margin(want)
            print(f"  pos {pos}: logits relative error {r:.2e}, max |diff| {mx:.2e}, "
                  f"oracle margin {m:.3e}, argmax gpu {int(np.argmax(got))} "
                  f"oracle {O.argmax(want)}", flush=True)
            assert r < 1e-3, f"position {pos}: logits relative error {r:.2e}"
            if m > 2 * mx:
                assert int(np.argmax(got)) == O.argmax(want), f"position {pos}: argmax differs"
    finally:
        om.close()
