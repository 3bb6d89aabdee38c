"""The device sampler (include/wick_hip_sampler.h) and the generate loop
(wick_hip_model_generate) against the CPU oracle of src/sampler.rs.

Bar: the drawn ids, the penalised logits, the candidate ids in order, the
candidate probabilities (bit for bit: the device's exp has the bits of the C
library's expf, which wick's f32::exp calls -- tests/test_exp_f32.py), the kept
count and the generator state are identical to the oracle's.  Vocabularies: a tiny one, 1000, and
the two the benchmarks use (SmolLM2 49152, Qwen 151936), so both the LDS path
(candidate sets up to 4096) and the global radix sort run.
"""
import numpy as np
import pytest

import oracle_lib as ol
from wick_amd.sampler import DeviceSampler, SamplerConfig

pytestmark = pytest.mark.gpu

CONFIGS = {
    "default": SamplerConfig(seed=11),
    "greedy": SamplerConfig.greedy(),
    "greedy_penalty": SamplerConfig(temperature=0.0, repetition_penalty=1.3),
    "top1": SamplerConfig(temperature=1.0, top_k=1, seed=5),
    "whole_vocab": SamplerConfig(temperature=1.0, top_k=0, top_p=1.0, seed=6),
    "whole_vocab_top_p": SamplerConfig(temperature=0.8, top_k=0, top_p=0.95, seed=7),
    "k4096": SamplerConfig(temperature=1.1, top_k=4096, top_p=0.5, seed=8),
    "k5000": SamplerConfig(temperature=1.2, top_k=5000, top_p=1.0, seed=9),
    "min_p": SamplerConfig(temperature=1.0, top_k=0, top_p=1.0, min_p=0.05, seed=10),
    "penalty": SamplerConfig(repetition_penalty=1.2, seed=12),
    "hot": SamplerConfig(temperature=2.0, top_k=100, top_p=0.99, min_p=0.01, seed=13),
}
VOCABS = [7, 1000, 49152, 151936]


def logits_of(kind, n, rng):
    if kind == "normal":
        x = rng.normal(0, 3, n)
    elif kind == "flat":  # most values share their top exponent/mantissa bits
        x = rng.normal(0, 0.02, n)
    elif kind == "ties":
        x = np.round(rng.normal(0, 2, n) * 2) / 2
    elif kind == "lm":  # a peaked head over a long tail
        x = rng.normal(-5, 2, n)
        x[rng.integers(0, n, max(1, n // 1000))] += 12
    elif kind == "const":  # every slice is one run of ties: the split top-k falls back to the full path
        x = np.full(n, 0.5)
        x[rng.integers(0, n, 3)] = 1.5
    elif kind == "nan":
        x = rng.normal(0, 3, n)
        x[rng.integers(0, n)] = np.nan
    else:
        raise ValueError(kind)
    return x.astype(np.float32)


def ulp_diff(a, b):
    a = a.view(np.int32).astype(np.int64)
    b = b.view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7FFFFFFF), a)
    b = np.where(b < 0, -(b & 0x7FFFFFFF), b)
    return np.abs(a - b)


def check_draw(ds, os_, logits, history, name):
    got_l, want_l = logits.copy(), logits.copy()
    got = ds.sample(got_l, history)
    want, ids, probs, keep = os_.sample_detail(want_l, history)
    assert np.array_equal(got_l.view(np.uint32), want_l.view(np.uint32)), f"{name}: penalised logits differ"
    gids, gprobs, gkeep = ds.last_candidates()
    assert np.array_equal(gids, ids), f"{name}: candidate order differs"
    assert gkeep == keep, f"{name}: keep {gkeep} != {keep}"
    nan = np.isnan(probs)
    assert np.array_equal(np.isnan(gprobs), nan)
    if (~nan).any():
        d = int(ulp_diff(gprobs[~nan], probs[~nan]).max())
        assert d == 0, f"{name}: probabilities differ by {d} ulp"
    assert got == want, f"{name}: drew {got}, oracle {want}"


@pytest.mark.parametrize("vocab", VOCABS)
@pytest.mark.parametrize("name", list(CONFIGS))
def test_sampler_matches_oracle(vocab, name):
    cfg = CONFIGS[name]
    rng = np.random.default_rng(vocab + len(name))
    kinds = ["normal", "flat", "ties", "lm"] + (["nan", "const"] if name in ("default", "whole_vocab", "top1") else [])
    draws = 2 if vocab > 50000 else 4
    with DeviceSampler(cfg, vocab) as ds:
        os_ = ol.OracleSampler(cfg)
        for kind in kinds:
            for d in range(draws):
                logits = logits_of(kind, vocab, rng)
                history = rng.integers(0, vocab + 16, 300).astype(np.uint32)
                print(f"vocab {vocab} {name} {kind} draw {d}", flush=True)
                check_draw(ds, os_, logits, history, f"{vocab}/{name}/{kind}/{d}")
        assert ds.rng_state() == os_.rng.state()


def test_reference_unit_cases_on_device():
    """src/sampler.rs:150-171 through the device sampler."""
    logits = np.array([0.0, 3.0, 1.0, 2.9], np.float32)
    with DeviceSampler(SamplerConfig.greedy(), 4) as ds:
        assert ds.sample(logits.copy(), []) == 1
    with DeviceSampler(SamplerConfig(temperature=0.0, repetition_penalty=1.5), 4) as ds:
        assert ds.sample(logits, [1]) == 3
    with DeviceSampler(SamplerConfig(temperature=1.0, top_k=1), 4) as ds:
        for _ in range(50):
            assert ds.sample(np.array([0.0, 3.0, 1.0, 2.9], np.float32), []) == 1
    with DeviceSampler(SamplerConfig(temperature=1.0, top_k=0, top_p=1.0), 2) as ds:
        n = 4000
        ones = sum(ds.sample(np.array([0.0, np.log(3.0)], np.float32), []) == 1 for _ in range(n))
        assert abs(ones / n - 0.75) < 0.03


def test_device_pointer_entry_point():
    import torch
    vocab = 49152
    cfg = SamplerConfig(repetition_penalty=1.1, seed=99)
    rng = np.random.default_rng(3)
    s = torch.cuda.Stream()
    with DeviceSampler(cfg, vocab, stream=s.cuda_stream) as ds:
        os_ = ol.OracleSampler(cfg)
        out = torch.zeros(1, dtype=torch.int32, device="cuda")
        for _ in range(5):
            host = logits_of("lm", vocab, rng)
            hist = rng.integers(0, vocab, 50).astype(np.int32)
            x = torch.from_numpy(host.copy()).cuda()
            h = torch.from_numpy(hist).cuda()
            torch.cuda.synchronize()
            ds.sample_device(x.data_ptr(), h.data_ptr(), h.numel(), out.data_ptr())
            s.synchronize()
            want_l = host.copy()
            want = os_.sample(want_l, hist.astype(np.uint32))
            assert int(out.item()) == want
            assert np.array_equal(x.cpu().numpy().view(np.uint32), want_l.view(np.uint32))


# ---------------------------------------------------------------- generate

def oracle_generate(cfg, w, tokens, max_tokens, scfg, capacity, stops=()):
    """Session::generate's loop (src/engine.rs:164-204) on the CPU oracle."""
    om = ol.OracleModel(cfg, w)
    st = om.new_state(capacity)
    logits = om.forward(st, tokens)[0]
    s = ol.OracleSampler(scfg)
    hist = list(tokens)
    out = []
    max_tokens = min(max_tokens, capacity - len(tokens))
    while len(out) < max_tokens:
        tok = s.sample(logits.copy(), hist if scfg.repetition_penalty != 1.0 else [])
        if tok in stops:
            break
        out.append(tok)
        if len(out) < max_tokens:
            hist.append(tok)
            logits = om.forward(st, [tok])[0]
    return out, st["len"]


def tiny(name):
    import json
    import os
    from wick_amd.model import Config, load_weights
    d = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny", name)
    cfg = Config.load(d)
    return cfg, load_weights(d, cfg)


GEN_CASES = {
    "default": SamplerConfig(seed=21),
    "penalty_min_p": SamplerConfig(temperature=0.9, top_k=0, top_p=0.95, min_p=0.02, repetition_penalty=1.3,
                                   seed=22),
}


@pytest.mark.parametrize("model", ["llama3-scaled-f32", "qwen2-bias-bf16", "qwen3-qknorm-f32"])
@pytest.mark.parametrize("case", list(GEN_CASES))
def test_generate_matches_oracle(model, case):
    from wick_amd.device_model import DeviceModel
    cfg, w = tiny(model)
    scfg = GEN_CASES[case]
    rng = np.random.default_rng(5)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab, 37)]
    want, want_len = oracle_generate(cfg, w, prompt, 40, scfg, 128)
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(128)
        with m.new_sampler(scfg) as s:
            got = m.generate(cache, s, prompt, 40)
        assert cache.len == want_len == len(prompt) + 39
    assert got == want


@pytest.mark.parametrize("stops", [False, True])
def test_generate_across_plan_changes(stops):
    """A long sampled loop: from 150 to 230 positions the decode plan changes at
    193 (one chunk per kv head -> split-K, with its merge pass) in the middle of
    the loop.  The ids equal the oracle's Session::generate, with and without a
    stop list that never matches."""
    from wick_amd.device_model import DeviceModel
    from wick_amd.model import Config
    from wick_amd.synthetic import random_weights
    cfg = Config("llama", 128, 256, 2, 6, 2, 64, 500, rms_eps=1e-5, rope_theta=10000.0)
    w = random_weights(cfg, seed=51, std=0.08)
    scfg = SamplerConfig(temperature=0.8, top_k=20, top_p=0.95, repetition_penalty=1.1, seed=9)
    rng = np.random.default_rng(52)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab, 150)]
    want, want_len = oracle_generate(cfg, w, prompt, 80, scfg, 256)
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(256)
        with m.new_sampler(scfg) as s:
            got = m.generate(cache, s, prompt, 80, stops=(cfg.vocab + 7,) if stops else ())
        assert cache.len == want_len
    assert got == want


def test_generate_stops_and_room():
    from wick_amd.device_model import DeviceModel
    cfg, w = tiny("qwen3-qknorm-f32")
    scfg = SamplerConfig(temperature=1.0, top_k=0, top_p=1.0, seed=3)
    rng = np.random.default_rng(6)
    prompt = [int(t) for t in rng.integers(0, cfg.vocab, 20)]
    chain, _ = oracle_generate(cfg, w, prompt, 30, scfg, 128)
    j = next(i for i in range(5, 30) if chain[i] not in chain[:i])
    stop = chain[j]
    want, want_len = oracle_generate(cfg, w, prompt, 30, scfg, 128, stops=(stop,))
    assert want == chain[:j] and want_len == len(prompt) + j
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(128)
        with m.new_sampler(scfg) as s:
            got = m.generate(cache, s, prompt, 30, stops=(stop, cfg.vocab + 5))
        assert got == want and cache.len == want_len
        # room: a 24-position cache leaves 4 tokens after a 20-token prompt
        small = m.new_cache(24)
        with m.new_sampler(scfg) as s:
            got = m.generate(small, s, prompt, 30)
        assert got == chain[:4] and small.len == 23
        with m.new_sampler(scfg) as s:
            assert m.generate(m.new_cache(20), s, prompt, 30) == []


def test_session_generate_reuses_the_prefix():
    from wick_amd.device_model import DeviceModel
    from wick_amd.session import DeviceSession
    cfg, w = tiny("llama3-scaled-f32")
    scfg = SamplerConfig(seed=4)
    rng = np.random.default_rng(8)
    turn1 = [int(t) for t in rng.integers(0, cfg.vocab, 30)]
    with DeviceModel(cfg, w) as m, DeviceSession(m, 160) as sess:
        r1 = sess.generate(turn1, max_tokens=12, sampler=scfg)
        assert r1.reused_tokens == 0 and r1.finish == "length" and len(r1.tokens) == 12
        assert r1.tokens == oracle_generate(cfg, w, turn1, 12, scfg, 160)[0]
        turn2 = turn1 + r1.tokens + [int(t) for t in rng.integers(0, cfg.vocab, 9)]
        r2 = sess.generate(turn2, max_tokens=10, sampler=scfg)
        assert r2.reused_tokens == len(turn1) + 11  # the last drawn id was never fed
        assert r2.tokens == oracle_generate(cfg, w, turn2, 10, scfg, 160)[0]
        assert len(sess) == len(turn2) + 9


def test_generate_errors():
    from wick_amd import _native
    from wick_amd.device_model import DeviceModel
    cfg, w = tiny("llama3-scaled-f32")
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(32)
        with m.new_sampler(SamplerConfig()) as s:
            cache.len = 3
            with pytest.raises(_native.WickHipError, match="start"):
                m.generate(cache, s, [1, 2, 3], 4)
            cache.len = 0
            with pytest.raises(_native.WickHipError, match="vocabulary"):
                m.generate(cache, s, [cfg.vocab], 4)
        with DeviceSampler(SamplerConfig(), cfg.vocab) as other:
            with pytest.raises(_native.WickHipError, match="stream"):
                m.generate(cache, other, [1, 2], 4)
        with DeviceSampler(SamplerConfig(), cfg.vocab + 1, stream=None) as other:
            with pytest.raises(_native.WickHipError):
                m.generate(cache, other, [1, 2], 4)
