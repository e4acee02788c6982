"""Sampling on the host side: the reference's random stream (std::mt19937 and
libstdc++'s uniform_real_distribution<float>, llama_model.cpp:1556 / :1494)
and the oracle's restatement of sample() / apply_rep_penalty
(llama_model.cpp:1466-1498, :1595-1605), pinned by what the mathematics fixes.
No GPU needed."""
import json
from pathlib import Path

import numpy as np
import pytest

from llm_core_amd import hip
from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "sampling_uniforms.json"


def test_mt19937_standard_value():
    """C++ [rand.predef]: the 10000th output of a default-seeded (5489) mt19937
    is 4123659995."""
    assert int(hip.mt19937(5489, 10000)[-1]) == 4123659995


@pytest.mark.parametrize("seed", [42, 1, 5489, 2**32 - 1])
def test_mt19937_matches_numpy(seed):
    """numpy's MT19937 with the legacy integer seeding (init_genrand) is an
    independent implementation of the same generator."""
    bg = np.random.MT19937()
    bg._legacy_seeding(seed)
    np.testing.assert_array_equal(hip.mt19937(seed, 2000), bg.random_raw(2000).astype(np.uint32))


def test_stream_matches_libstdcxx_golden():
    """Raw outputs and float draws against g++/libstdc++ itself
    (tests/golden/make_sampling_golden.py)."""
    g = json.loads(GOLDEN.read_text())
    for seed, d in g["seeds"].items():
        np.testing.assert_array_equal(hip.mt19937(int(seed), g["n"]), np.array(d["mt19937"], np.uint32))
        bits = hip.sampling_uniforms(int(seed), g["n"]).view(np.uint32)
        np.testing.assert_array_equal(bits, np.array(d["uniform_f32_bits"], np.uint32))


def test_uniform_draw_is_u_over_2_32():
    """generate_canonical<float, 24> with one 32-bit output: float(u) / 2^32, in
    [0, 1) (a value that rounds to 1 becomes the largest float below 1)."""
    u = hip.mt19937(7, 5000)
    x = hip.sampling_uniforms(7, 5000)
    want = u.astype(np.float32) / np.float32(2.0**32)
    want[want >= 1] = np.nextafter(np.float32(1), np.float32(0))
    np.testing.assert_array_equal(x, want)
    assert x.min() >= 0 and x.max() < 1


def test_rep_penalty_closed_form():
    x = np.array([2.0, -1.0, 0.5, 3.0, -4.0, 0.0], np.float32)
    # window of 4 over history [3, 0, 1, 1, 2]: ids 0, 1, 1, 2 (id 1 twice)
    y = O.rep_penalty(x, [3, 0, 1, 1, 2], 4, 2.0)
    np.testing.assert_array_equal(y, np.array([1.0, -4.0, 0.25, 3.0, -4.0, 0.0], np.float32))
    np.testing.assert_array_equal(O.rep_penalty(x, [5, 9999, -1], 64, 3.0), x)  # 0 * 3; out of range
    np.testing.assert_array_equal(O.rep_penalty(x, [0, 1], 64, 1.0), x)


def test_sample_greedy_and_top1():
    x = np.random.default_rng(0).standard_normal(5000).astype(np.float32)
    best = int(np.argmax(x))
    for r in (0.0, 0.5, 0.999):
        assert O.sample(x, 40, 1.0, 0.0, r)[0] == best          # greedy
        assert O.sample(x, 1, 1.0, 0.7, r)[0] == best           # top_k = 1
        assert O.sample(x, 40, 1e-9, 1.3, r)[0] == best         # nucleus of one


def test_sample_two_tokens_closed_form():
    """Two tokens: p0 = 1 / (1 + exp((b - a) / T)); the draw r picks 0 iff r < p0."""
    a, b, T = 0.3, -0.9, 0.7
    p0 = 1.0 / (1.0 + np.exp((b - a) / T))
    x = np.array([a, b], np.float32)
    for r in np.linspace(0, 0.999, 101, dtype=np.float32):
        tok, m = O.sample(x, 0, 1.0, T, float(r))
        if abs(r - p0) > 1e-6:
            assert tok == (0 if r < p0 else 1), (r, p0)


def test_sample_inverts_the_distribution():
    """Over a fine grid of draws, the chosen tokens' frequencies are the
    softmax probabilities of the top-k (renormalised after the top-p cut)."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(300).astype(np.float32) * 2
    T, k, top_p = 0.8, 25, 0.9
    s = np.sort(x / T)[::-1][:k].astype(np.float64)
    p = np.exp(s - s[0])
    p /= p.sum()
    cut = int(np.searchsorted(np.cumsum(p), top_p) + 1)
    p = p[:cut] / p[:cut].sum()
    order = np.argsort(-(x / T), kind="stable")[:cut]
    grid = (np.arange(20000) + 0.5) / 20000
    counts = np.zeros(x.size)
    for r in grid:
        counts[O.sample(x, k, top_p, T, float(r))[0]] += 1
    np.testing.assert_allclose(counts[order] / grid.size, p, atol=2e-4)
    assert counts.sum() == counts[order].sum()  # nothing outside the nucleus


def test_temperature_is_a_logit_scale():
    """T = 2 on x equals T = 1 on x / 2 (division by 2 is exact)."""
    x = np.random.default_rng(4).standard_normal(1000).astype(np.float32)
    for r in np.linspace(0.01, 0.99, 25):
        assert O.sample(x, 50, 0.95, 2.0, float(r))[0] == O.sample(x / 2, 50, 0.95, 1.0, float(r))[0]
