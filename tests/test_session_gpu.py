"""DeviceSession on the GPU: prefix reuse gives the logits a fresh prefill gives
(the reference's chunked-vs-batch bound, tests/tiny_models.rs:89: 1e-4) and the
CPU oracle's, and greedy continuations agree."""
import json
import os

import numpy as np
import pytest

import oracle_lib as ol
from wick_amd.device_model import DeviceModel
from wick_amd.model import Config, load_weights
from wick_amd.session import DeviceSession, greedy

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny")


def fixture(name):
    d = os.path.join(GOLDEN, name)
    cfg = Config.load(d)
    with open(os.path.join(d, "expected.json")) as f:
        exp = json.load(f)
    return cfg, load_weights(d, cfg), exp


@pytest.mark.parametrize("name", ["qwen2-bias-bf16", "qwen3-qknorm-f32"])
def test_prefix_reuse_matches_fresh_prefill(name):
    cfg, w, exp = fixture(name)
    rng = np.random.default_rng(3)
    a = [int(x) for x in rng.integers(0, cfg.vocab, 40)]
    b = a[:30] + [int(x) for x in rng.integers(0, cfg.vocab, 10)]
    om = ol.OracleModel(cfg, w)
    want = om.forward(om.new_state(64), b)[0]
    with DeviceModel(cfg, w) as m, DeviceSession(m, 64) as s, DeviceSession(m, 64) as fresh:
        greedy(s, a, 3)
        logits, keep = s.prefill(b)
        assert keep == 30
        ref, keep0 = fresh.prefill(b)
        assert keep0 == 0
        assert np.abs(logits[0] - ref[0]).max() < 1e-4
        assert np.abs(logits[0] - want).max() < 1e-4
        # the same prompt again recomputes only its last token
        again, keep2 = s.prefill(b)
        assert keep2 == 39 and np.abs(again[0] - logits[0]).max() < 1e-4
        assert greedy(s, b, 5)[0] == greedy(fresh, b, 5)[0]


def test_long_prompt_in_chunks_matches_cpu():
    cfg, w, exp = fixture("llama3-scaled-f32")
    rng = np.random.default_rng(5)
    prompt = [int(x) for x in rng.integers(0, cfg.vocab, 300)]
    om = ol.OracleModel(cfg, w)
    want = om.forward(om.new_state(320), prompt)[0]
    with DeviceModel(cfg, w) as m, DeviceSession(m, 320) as s:
        logits, keep = s.prefill(prompt)
    assert keep == 0 and np.abs(logits[0] - want).max() < 1e-4
