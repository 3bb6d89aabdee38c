"""The sampler oracle (oracle/wick_sampler.c) pinned on the CPU.

What pins it:
  - the reference's own unit tests of the sampler (src/sampler.rs:150-171);
  - published known answers of its generators: splitmix64 from seed 0, and
    xoshiro256** from the state {1, 2, 3, 4} (the first ten outputs);
  - the distribution drawn against the closed-form softmax in float64 (a
    chi-square test), with and without the top-k / top-p / min-p cuts, whose
    kept sets follow from the probabilities by hand;
  - the repetition penalty against its definition applied once per distinct id;
  - the candidate order against f32::total_cmp on values whose order is known.
"""
import math

import numpy as np
import pytest

import oracle_lib as ol
from wick_amd.sampler import SamplerConfig


def test_splitmix64_known_answer():
    """Rng::new(0) holds the first four splitmix64 outputs for seed 0."""
    assert ol.OracleRng(0).state() == (0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F,
                                       0xF88BB8A8724C81EC)


def test_xoshiro256starstar_known_answer():
    r = ol.OracleRng(state=(1, 2, 3, 4))
    want = [11520, 0, 1509978240, 1215971899390074240, 1216172134540287360, 607988272756665600,
            16172922978634559625, 8476171486693032832, 10595114339597558777, 2904607092377533576]
    assert [r.next_u64() for _ in range(10)] == want


def test_next_f32_is_the_top_24_bits():
    a, b = ol.OracleRng(123), ol.OracleRng(123)
    for _ in range(1000):
        u = a.next_u64()
        f = b.next_f32()
        assert f == (u >> 40) / 16777216.0 and 0.0 <= f < 1.0


def test_reference_greedy_and_filters():
    """src/sampler.rs:150-161."""
    logits = np.array([0.0, 3.0, 1.0, 2.9], np.float32)
    assert ol.OracleSampler(SamplerConfig.greedy()).sample(logits.copy(), []) == 1
    s = ol.OracleSampler(SamplerConfig(temperature=0.0, repetition_penalty=1.5))
    assert s.sample(logits, [1]) == 3
    s = ol.OracleSampler(SamplerConfig(temperature=1.0, top_k=1))
    for _ in range(50):
        assert s.sample(np.array([0.0, 3.0, 1.0, 2.9], np.float32), []) == 1


def test_reference_sampling_follows_the_distribution():
    """src/sampler.rs:163-171: probabilities 1/4 and 3/4."""
    s = ol.OracleSampler(SamplerConfig(temperature=1.0, top_k=0, top_p=1.0))
    logits = np.array([0.0, math.log(3.0)], np.float32)
    n = 20000
    ones = sum(s.sample(logits.copy(), []) == 1 for _ in range(n))
    assert abs(ones / n - 0.75) < 0.02


def chi2(counts, probs):
    n = counts.sum()
    exp = n * np.asarray(probs, np.float64)
    return float(((counts - exp) ** 2 / exp).sum())


# chi-square 0.999 quantiles by degrees of freedom
CHI2_999 = {1: 10.83, 2: 13.82, 3: 16.27, 7: 24.32}


def draw_counts(cfg, logits, n, history=()):
    s = ol.OracleSampler(cfg)
    counts = np.zeros(logits.size, np.int64)
    for _ in range(n):
        counts[s.sample(logits.copy(), history)] += 1
    return counts


def test_distribution_is_the_tempered_softmax():
    rng = np.random.default_rng(0)
    logits = rng.normal(0, 1.5, 8).astype(np.float32)
    t = 0.8
    p = np.exp((logits.astype(np.float64) - logits.max()) / t)
    p /= p.sum()
    counts = draw_counts(SamplerConfig(temperature=t, top_k=0, top_p=1.0, seed=1), logits, 40000)
    assert chi2(counts, p) < CHI2_999[7]


# probabilities 0.5, 0.3, 0.15, 0.05 at temperature 1, on shuffled ids
PROBS = np.array([0.5, 0.3, 0.15, 0.05])
PERM = np.array([2, 0, 3, 1])  # PROBS[j] belongs to id PERM[j]


def cut_logits():
    logits = np.empty(4, np.float32)
    logits[PERM] = np.log(PROBS).astype(np.float32)
    return logits


@pytest.mark.parametrize("cfg,kept", [
    (SamplerConfig(temperature=1.0, top_k=2, top_p=1.0), 2),   # top-k
    (SamplerConfig(temperature=1.0, top_k=0, top_p=0.7), 2),   # 0.5 < 0.7 <= 0.8
    (SamplerConfig(temperature=1.0, top_k=0, top_p=0.9), 3),   # 0.8 < 0.9 <= 0.95
    (SamplerConfig(temperature=1.0, top_k=0, top_p=1.0, min_p=0.2), 3),  # 0.05 < 0.5 * 0.2
    (SamplerConfig(temperature=1.0, top_k=0, top_p=1.0, min_p=0.7), 1),  # 0.3 < 0.35
    (SamplerConfig(temperature=1.0, top_k=0, top_p=0.01), 1),
])
def test_cuts_keep_the_right_prefix_and_renormalise(cfg, kept):
    logits = cut_logits()
    tok, ids, probs, keep = ol.OracleSampler(cfg).sample_detail(logits.copy())
    assert keep == kept
    assert list(ids[:kept]) == list(PERM[:kept])
    assert np.allclose(probs[:kept] / probs[:kept].sum(), PROBS[:kept] / PROBS[:kept].sum(), rtol=1e-5)
    counts = draw_counts(cfg, logits, 20000)
    assert counts[PERM[kept:]].sum() == 0
    if kept > 1:
        want = PROBS[:kept] / PROBS[:kept].sum()
        assert chi2(counts[PERM[:kept]], want) < CHI2_999[kept - 1]


def test_repetition_penalty_once_per_distinct_id():
    rng = np.random.default_rng(2)
    logits = rng.normal(0, 2, 64).astype(np.float32)
    history = [3, 7, 3, 3, 70, 63, 0, 7, 1000]  # duplicates and ids outside the vocabulary
    want = logits.copy()
    for t in sorted({t for t in history if t < 64}):
        want[t] = want[t] / np.float32(1.3) if want[t] > 0 else want[t] * np.float32(1.3)
    got = logits.copy()
    tok = ol.OracleSampler(SamplerConfig(temperature=0.0, repetition_penalty=1.3)).sample(got, history)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert tok == int(np.argmax(want))
    same = logits.copy()
    ol.OracleSampler(SamplerConfig(temperature=0.0)).sample(same, history)
    assert np.array_equal(same, logits)


def test_candidates_in_total_order_with_ties_by_id():
    logits = np.array([1.0, 3.0, 3.0, -0.0, 3.0, 0.0, -np.inf, 2.0], np.float32)
    _, ids, _, _ = ol.OracleSampler(SamplerConfig(temperature=1.0, top_k=0, top_p=1.0)).sample_detail(logits)
    # 3.0 (ids 1, 2, 4), 2.0, 1.0, +0.0 above -0.0, then -inf
    assert list(ids) == [1, 2, 4, 7, 0, 5, 3, 6]
    _, ids, _, _ = ol.OracleSampler(SamplerConfig(temperature=1.0, top_k=2, top_p=1.0)).sample_detail(logits)
    assert list(ids) == [1, 2]


def test_greedy_draw_leaves_the_generator():
    s = ol.OracleSampler(SamplerConfig.greedy())
    before = s.rng.state()
    s.sample(np.array([0.5, 0.25], np.float32))
    assert s.rng.state() == before
