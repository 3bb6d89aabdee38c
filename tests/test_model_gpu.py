"""The device-resident forward (include/wick_hip_model.h) against the CPU oracle
and the reference's transformers-scored tiny fixtures.

Thresholds are the reference's own (tests/tiny_models.rs): logits within 1e-3
of transformers (:68), a reordered computation of the same forward within
1e-4 (:89, chunked vs batch; here GPU vs CPU accumulation order), and greedy
ids identical (:111).
"""
import json
import os

import numpy as np
import pytest

import oracle_lib as ol
from wick_amd import _native
from wick_amd.device_model import DeviceModel
from wick_amd.model import Config, load_weights
from wick_amd.synthetic import random_prompt, random_weights, smollm2_135m

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny")
MODELS = ["llama3-scaled-f32", "qwen2-bias-bf16", "qwen3-qknorm-f32"]


def fixture(name):
    d = os.path.join(GOLDEN, name)
    cfg = Config.load(d)
    with open(os.path.join(d, "expected.json")) as f:
        exp = json.load(f)
    return cfg, load_weights(d, cfg), exp


@pytest.mark.parametrize("name", MODELS)
def test_tiny_logits_match_transformers_and_cpu(name):
    cfg, w, exp = fixture(name)
    with DeviceModel(cfg, w) as m:
        got = m.forward(m.new_cache(256), exp["tokens"], all_logits=True)
    worst = np.abs(got - np.array(exp["logits"], np.float32)).max()
    assert worst < 1e-3, f"{name}: logits differ from transformers by {worst}"
    om = ol.OracleModel(cfg, w)
    want = om.forward(om.new_state(256), exp["tokens"], all_logits=True)
    d = np.abs(got - want).max()
    print(f"{name}: max |gpu - cpu| over {got.size} logits = {d:.2e}")
    assert d < 1e-4


@pytest.mark.parametrize("name", MODELS)
def test_tiny_incremental_matches_batch(name):
    cfg, w, exp = fixture(name)
    with DeviceModel(cfg, w) as m:
        batch = m.forward(m.new_cache(256), exp["tokens"], all_logits=True)
        cache = m.new_cache(256)
        pos = 0
        for size in [1, 5, 2, 7, 1, 1, 13, 3, 15]:
            rows = m.forward(cache, exp["tokens"][pos:pos + size], all_logits=True)
            d = np.abs(rows - batch[pos:pos + size]).max()
            assert d < 1e-4, f"{name}: position {pos} differs by {d}"
            pos += size


@pytest.mark.parametrize("name", MODELS)
def test_tiny_greedy_on_device(name):
    cfg, w, exp = fixture(name)
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(256)
        first = m.prefill(cache, exp["greedy_prompt"])
        ids = [first] + m.decode(cache, first, len(exp["greedy"]) - 1)
    assert ids == exp["greedy"]


@pytest.mark.parametrize("case", ["tie", "nan0", "nan_other", "odd_pairs"])
def test_device_argmax_edge_cases(case):
    """The device argmax reduces the LM head's per-4-row (value, index) pairs;
    sampler::argmax (src/sampler.rs:129-137) keeps the first index of the
    maximum, never picks a NaN, and never leaves index 0 when its logit is NaN.
    Rows of the LM head are copied or poisoned so the logits hold exact ties
    and NaNs; prefill's and decode's ids must equal the oracle's argmax of the
    logits forward() returns for the same tokens."""
    import dataclasses
    cfg, w, exp = fixture("llama3-scaled-f32")
    w = dict(w)
    prompt = exp["greedy_prompt"]
    if case == "odd_pairs":  # 90 rows: 23 pairs, the last of 2 rows
        cfg = dataclasses.replace(cfg, vocab=90)
        w["embed"] = np.ascontiguousarray(w["embed"][:90])
        w["lm_head"] = np.ascontiguousarray(w["lm_head"][:90])
        prompt = [t % 90 for t in prompt]
    with DeviceModel(cfg, w) as m:
        logits = m.forward(m.new_cache(64), prompt)[-1]
    best = int(np.argmax(logits))
    head = w["lm_head"].copy()
    if case == "tie":  # the best row copied to a smaller and a larger index
        lo = 1 if best != 1 else 2
        head[lo] = head[best]
        head[(best + 37) % cfg.vocab] = head[best]
    elif case == "nan0":
        head[0, 5] = np.nan
    elif case == "nan_other":
        head[best, 5] = np.nan
    elif case == "odd_pairs":  # the maximum in the last, 2-row pair
        head[89] = head[best] * (1.5 if logits[best] > 0 else 0.5)
    w["lm_head"] = head
    with DeviceModel(cfg, w) as m:
        want = m.forward(m.new_cache(64), prompt)[-1]
        tok = ol.argmax(want)
        cache = m.new_cache(64)
        first = m.prefill(cache, prompt)
        nxt = m.decode(cache, first, 2)
        want2 = m.forward(m.new_cache(64), list(prompt) + [first])[-1]
    assert first == tok
    assert nxt[0] == ol.argmax(want2)
    if case == "tie":
        assert tok == min(lo, best) and want[lo] == want[best]
    elif case == "nan0":
        assert np.isnan(want[0]) and tok == 0
    elif case == "nan_other":
        assert np.isnan(want[best]) and (tok != best) == (best != 0)
    elif case == "odd_pairs":
        assert tok == 89


def oracle_greedy(cfg, w, prompt, n_gen, capacity):
    om = ol.OracleModel(cfg, w)
    st = om.new_state(capacity)
    logits = om.forward(st, prompt)
    first_logits = logits[0].copy()
    ids = []
    for _ in range(n_gen):
        tok = ol.argmax(logits[0])
        ids.append(tok)
        logits = om.forward(st, [tok])
    return ids, first_logits


def test_smollm2_135m_greedy_ids_match_cpu():
    """random-init SmolLM2-135M, 128-token prompt, 64 greedy tokens, all on the device."""
    cfg = smollm2_135m()
    w = random_weights(cfg, seed=0)
    prompt = random_prompt(1, 128, cfg.vocab)
    want, want_logits = oracle_greedy(cfg, w, prompt, 64, 128 + 64 + 8)
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(128 + 64 + 8)
        logits = m.forward(cache, prompt)
        d = np.abs(logits[0] - want_logits).max()
        print(f"prefill logits: max |gpu - cpu| = {d:.2e}")
        assert d < 1e-4
        cache.len = 0
        first = m.prefill(cache, prompt)
        got = [first] + m.decode(cache, first, 63)
    assert got == want


def test_decode_matches_step_by_step_forward():
    """decode() keeps ids on the device and replays runs of steps that share a decode plan
    from a captured HIP graph; forward() + host argmax, launched step by step, must give
    the same chain and the same cache bits.  40 -> 240 positions: one-chunk plans of 64,
    128 and 192 keys, then split-K with the merge pass (runs of 24, 64, 64 and 48 steps)."""
    cfg = smollm2_135m()
    cfg.layers = 4
    w = random_weights(cfg, seed=3)
    prompt = random_prompt(4, 40, cfg.vocab)
    n = 200
    with DeviceModel(cfg, w) as m:
        c1 = m.new_cache(256)
        first = m.prefill(c1, prompt)
        chain = m.decode(c1, first, n)
        c2 = m.new_cache(256)
        logits = m.forward(c2, prompt)
        assert int(np.argmax(logits[0])) == first
        tok, steps = first, []
        for _ in range(n):
            logits = m.forward(c2, [tok])
            tok = ol.argmax(logits[0])
            steps.append(tok)
        k1, v1 = c1.read(3, 0, 40 + n)
        k2, v2 = c2.read(3, 0, 40 + n)
        c1.len = 40  # prefix reuse: back to the prompt, one step launched directly
        again = m.decode(c1, first, 1)
    assert chain == steps
    assert np.array_equal(k1, k2) and np.array_equal(v1, v2)
    assert again == chain[:1]


def _bias_and_norms(cfg, w, seed):
    """Give every layer q/k/v biases and QK-norm weights (Qwen2's and Qwen3's extra tensors)."""
    rng = np.random.default_rng(seed)
    r = lambda n, s=0.1, c=0.0: (c + s * rng.standard_normal(n)).astype(np.float32)  # noqa: E731
    for lw in w["layers"]:
        lw.update(bq=r(cfg.q_dim), bk=r(cfg.kv_dim), bv=r(cfg.kv_dim), q_norm=r(cfg.head_dim, 0.1, 1.0),
                  k_norm=r(cfg.head_dim, 0.1, 1.0))
    return w


def _replay_case(name):
    if name in MODELS:
        cfg, w, _ = fixture(name)
        return cfg, w
    if name == "group18-d64-bias-qknorm":
        cfg = Config("qwen3", 128, 256, 2, 36, 2, 64, 512, rms_eps=1e-6, rope_theta=1e6, attn_bias=True, qk_norm=True)
        return cfg, _bias_and_norms(cfg, random_weights(cfg, seed=21, std=0.05), 22)
    cfg = Config("llama", 256, 512, 2, 8, 2, 128, 512, rms_eps=1e-5, rope_theta=500000.0)
    return cfg, random_weights(cfg, seed=23, std=0.05)


@pytest.mark.parametrize("name", ["qwen2-bias-bf16", "qwen3-qknorm-f32", "llama3-scaled-f32",
                                  "group18-d64-bias-qknorm", "d128-group4"])
def test_decode_replay_matches_step_by_step(name):
    """64 decode steps at 65..128 positions share one decode plan, so decode() launches the
    first and replays the other 63 from a captured HIP graph: head_dim 16 with biases, 32 with
    QK-norm, a group of 18 (two 16-head slices writing the same k/v rows) with both, and
    head_dim 128.  The ids and every layer's cache bits must equal forward() + host argmax
    launched step by step."""
    cfg, w = _replay_case(name)
    prompt = random_prompt(9, 64, cfg.vocab)
    n = 64
    with DeviceModel(cfg, w) as m:
        c1 = m.new_cache(160)
        first = m.prefill(c1, prompt)
        chain = m.decode(c1, first, n)
        c2 = m.new_cache(160)
        logits = m.forward(c2, prompt)
        assert int(np.argmax(logits[0])) == first
        tok, steps = first, []
        for _ in range(n):
            logits = m.forward(c2, [tok])
            tok = ol.argmax(logits[0])
            steps.append(tok)
        for layer in range(cfg.layers):
            k1, v1 = c1.read(layer, 0, 64 + n)
            k2, v2 = c2.read(layer, 0, 64 + n)
            assert np.array_equal(k1, k2) and np.array_equal(v1, v2), f"{name}: layer {layer} cache differs"
    assert chain == steps


@pytest.mark.parametrize("shape", ["d64-g1-kv4", "d64-g2-kv3", "d64-g4-kv2", "d128-g2-kv2", "d64-g3-kv4-bias-qknorm"])
def test_fused_projection_and_valu_core_shapes(shape):
    """One-token forwards take the fused attention + output projection (partial
    products per unit, summed by the gate/up prologue) and, at head_dim 64 with
    groups of at most 4, the VALU attention core.  Shapes around their limits:
    groups 1, 2, 3, 4, up to 4 kv heads (the most partial vectors), head_dim
    128, biases and QK-norm.  20-token prompt, then 30 greedy steps across the
    32- and 64-key tile boundaries: logits within 1e-4 of the CPU oracle and
    the same ids at every step."""
    d, g, kvh = {"d64-g1-kv4": (64, 1, 4), "d64-g2-kv3": (64, 2, 3), "d64-g4-kv2": (64, 4, 2),
                 "d128-g2-kv2": (128, 2, 2), "d64-g3-kv4-bias-qknorm": (64, 3, 4)}[shape]
    heads = g * kvh
    extra = shape.endswith("bias-qknorm")
    cfg = Config("qwen3" if extra else "llama", 192, 256, 2, heads, kvh, d, 300, rms_eps=1e-5, rope_theta=10000.0,
                 attn_bias=extra, qk_norm=extra)
    w = random_weights(cfg, seed=31, std=0.08)
    if extra:
        w = _bias_and_norms(cfg, w, 32)
    prompt = [int(x) for x in random_prompt(33, 20, cfg.vocab)]
    om = ol.OracleModel(cfg, w)
    ost = om.new_state(64)
    want = om.forward(ost, prompt)
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(64)
        got = m.forward(cache, prompt)
        for step in range(30):
            diff = np.abs(got[0] - want[0]).max()
            assert diff < 1e-4, f"{shape}: step {step} logits differ by {diff}"
            tok = ol.argmax(want[0])
            assert int(np.argmax(got[0])) == tok, f"{shape}: step {step}"
            got = m.forward(cache, [tok])
            want = om.forward(ost, [tok])


@pytest.mark.parametrize("chunk", [320, 512])
def test_fixed_decode_chunk_past_the_fused_limit(chunk):
    """A decode chunk option above the fused attention + output projection's 256
    keys, at contexts that fit one chunk: every one-token forward must take the
    separate attention and o_proj launches (the fused launcher refuses such a
    plan).  SmolLM2's shape over 20..60 positions: logits within 1e-4 of the CPU
    oracle and the same greedy ids, through forward() and decode()."""
    cfg = smollm2_135m()
    cfg.layers = 2
    w = random_weights(cfg, seed=51)
    prompt = [int(x) for x in random_prompt(52, 20, cfg.vocab)]
    om = ol.OracleModel(cfg, w)
    ost = om.new_state(64)
    want = om.forward(ost, prompt)
    ids = []
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(64)
        cache.set_option(_native.OPT_DECODE_CHUNK, chunk)
        got = m.forward(cache, prompt)
        for step in range(40):
            diff = np.abs(got[0] - want[0]).max()
            assert diff < 1e-4, f"chunk {chunk}: step {step} logits differ by {diff}"
            tok = ol.argmax(want[0])
            assert int(np.argmax(got[0])) == tok, f"chunk {chunk}: step {step}"
            ids.append(tok)
            got = m.forward(cache, [tok])
            want = om.forward(ost, [tok])
        c2 = m.new_cache(64)
        c2.set_option(_native.OPT_DECODE_CHUNK, chunk)
        first = m.prefill(c2, prompt)
        assert first == ids[0]
        assert m.decode(c2, first, 39) == ids[1:]


def test_decode_loop_on_interleaved_splits():
    """One-token forwards over 1200..1240 positions at head_dim 128 (group 4) with
    512-key decode chunks (8 rounds of the 4 waves' 16-key groups): 3 workgroups
    per kv head, so the split deals the groups round-robin and the new key's k/v
    rows are appended by whichever chunk holds them.  Logits
    within 1e-4 of the CPU oracle and the same greedy ids through forward() and
    through decode(), which replays captured steps reading the length on the
    device."""
    cfg = Config("qwen3", 256, 384, 2, 8, 2, 128, 300, rms_eps=1e-6, rope_theta=1e6, attn_bias=True, qk_norm=True)
    w = _bias_and_norms(cfg, random_weights(cfg, seed=61, std=0.05), 62)
    prompt = [int(x) for x in random_prompt(64, 1200, cfg.vocab)]
    om = ol.OracleModel(cfg, w)
    ost = om.new_state(1280)
    want = om.forward(ost, prompt)
    ids = []
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(1280)
        cache.set_option(_native.OPT_DECODE_CHUNK, 512)
        got = m.forward(cache, prompt)
        for step in range(40):
            diff = np.abs(got[-1] - want[-1]).max()
            assert diff < 1e-4, f"step {step}: logits differ by {diff}"
            tok = ol.argmax(want[-1])
            assert int(np.argmax(got[-1])) == tok, f"step {step}"
            ids.append(tok)
            got = m.forward(cache, [tok])
            want = om.forward(ost, [tok])
        c2 = m.new_cache(1280)
        c2.set_option(_native.OPT_DECODE_CHUNK, 512)
        first = m.prefill(c2, prompt)
        assert first == ids[0]
        assert m.decode(c2, first, 39) == ids[1:]


@pytest.mark.parametrize("shape", ["kv8-d32", "hidden2304-d64", "kv6-d128-bias-qknorm"])
def test_unfused_single_token_paths(shape):
    """One-token forwards whose attention cannot carry the output projection --
    more than 4 (kv head, head slice) units, or a hidden size above the gate/up
    prologue's 2048 -- run attention and the o_proj product as two launches.
    Logits within 1e-4 of the CPU oracle and the same greedy ids over 40 steps,
    through forward() and through decode() (which replays a captured step)."""
    hidden, heads, kvh, d, extra = {"kv8-d32": (256, 8, 8, 32, False), "hidden2304-d64": (2304, 4, 2, 64, False),
                                    "kv6-d128-bias-qknorm": (192, 12, 6, 128, True)}[shape]
    cfg = Config("qwen3" if extra else "llama", hidden, 384, 2, heads, kvh, d, 300, rms_eps=1e-5,
                 rope_theta=10000.0, attn_bias=extra, qk_norm=extra)
    w = random_weights(cfg, seed=41, std=0.05)
    if extra:
        w = _bias_and_norms(cfg, w, 42)
    prompt = [int(x) for x in random_prompt(43, 20, cfg.vocab)]
    om = ol.OracleModel(cfg, w)
    ost = om.new_state(64)
    want = om.forward(ost, prompt)
    ids = []
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(64)
        got = m.forward(cache, prompt)
        for step in range(40):
            diff = np.abs(got[0] - want[0]).max()
            assert diff < 1e-4, f"{shape}: step {step} logits differ by {diff}"
            tok = ol.argmax(want[0])
            assert int(np.argmax(got[0])) == tok, f"{shape}: step {step}"
            ids.append(tok)
            got = m.forward(cache, [tok])
            want = om.forward(ost, [tok])
        c2 = m.new_cache(64)
        first = m.prefill(c2, prompt)
        assert first == ids[0]
        assert m.decode(c2, first, 39) == ids[1:]


def test_prefill_chunks_of_256():
    """A 300-token prompt runs as chunks of 256 + 44 (src/engine.rs:107, :134)."""
    cfg, w, exp = fixture("qwen3-qknorm-f32")
    rng = np.random.default_rng(7)
    prompt = [int(x) for x in rng.integers(0, cfg.vocab, 300)]
    om = ol.OracleModel(cfg, w)
    want = om.forward(om.new_state(320), prompt)[0]
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(320)
        nxt = m.prefill(cache, prompt)
        assert cache.len == 300
        rows = m.forward(m.new_cache(320), prompt, all_logits=True)
    assert np.abs(rows[-1] - want).max() < 1e-4
    assert nxt == ol.argmax(want)


@pytest.mark.parametrize("name", MODELS)
def test_decode_across_the_split_threshold(name):
    """Decode steps at 180..210 positions: single-chunk decode, then split-K + merge, both
    with the preparation in the decode kernel's prologue; logits and ids against the CPU."""
    cfg, w, exp = fixture(name)
    rng = np.random.default_rng(11)
    prompt = [int(x) for x in rng.integers(0, cfg.vocab, 180)]
    om = ol.OracleModel(cfg, w)
    ost = om.new_state(256)
    want = om.forward(ost, prompt)
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(256)
        got = m.forward(cache, prompt)
        for step in range(30):
            assert np.abs(got[0] - want[0]).max() < 1e-4, f"{name}: step {step}"
            tok = ol.argmax(want[0])
            assert int(np.argmax(got[0])) == tok
            got = m.forward(cache, [tok])
            want = om.forward(ost, [tok])
        k_gpu, v_gpu = cache.read(cfg.layers - 1, 0, 210)
    k_cpu = ost["k"][cfg.layers - 1, :210]
    assert np.abs(k_gpu - k_cpu).max() < 1e-4


def test_model_errors():
    cfg, w, exp = fixture("llama3-scaled-f32")
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(8)
        with pytest.raises(_native.WickHipError, match="vocabulary"):
            m.forward(cache, [cfg.vocab])
        with pytest.raises(_native.WickHipError, match="context length"):
            m.forward(cache, list(range(9)))
        with pytest.raises(_native.WickHipError, match="steps"):
            m.decode(cache, 1, 0)
        from wick_amd import DeviceKvCache
        with DeviceKvCache(cfg.layers, 8, cfg.kv_heads, cfg.head_dim) as other:
            with pytest.raises(_native.WickHipError, match="stream"):
                m.forward(other, [1])
        cache.len = 0
        assert m.forward(cache, [1, 2, 3]).shape == (1, cfg.vocab)


@pytest.mark.parametrize("case", range(8))
def test_random_config_sweep(case):
    """Seeded random architectures through the device-resident forward: hidden
    size, heads, kv heads, head_dim, FFN width, vocabulary, layer count, tied or
    separate LM head, Qwen2 biases / Qwen3 QK-norm.  Prompt logits within 1e-4
    of the CPU oracle, then greedy decode() (graph-replayed runs included) equal
    to the oracle's ids."""
    rng = np.random.default_rng(700 + case)
    d = int(rng.choice([16, 32, 64, 128]))
    kvh = int(rng.integers(1, 5))
    g = int(rng.choice([1, 2, 3, 4, 6, 8]))
    heads = kvh * g
    hidden = int(rng.choice([64, 128, 192, 256, 384]))
    arch = str(rng.choice(["llama", "qwen2", "qwen3"]))
    cfg = Config(arch, hidden, int(rng.choice([128, 256, 320])), int(rng.integers(1, 4)), heads, kvh, d,
                 int(rng.integers(300, 1200)), rms_eps=1e-5, rope_theta=float(rng.choice([1e4, 1e6])),
                 tie_embeddings=bool(rng.random() < 0.5), attn_bias=arch == "qwen2", qk_norm=arch == "qwen3")
    w = random_weights(cfg, seed=710 + case, std=0.06)
    if cfg.attn_bias or cfg.qk_norm:
        w = _bias_and_norms(cfg, w, 720 + case)
        for lw in w["layers"]:
            if not cfg.attn_bias:
                lw.update(bq=None, bk=None, bv=None)
            if not cfg.qk_norm:
                lw.update(q_norm=None, k_norm=None)
    if not cfg.tie_embeddings:
        w["lm_head"] = (0.06 * np.random.default_rng(730 + case).standard_normal((cfg.vocab, hidden))).astype(np.float32)
    n_prompt, n_gen = int(rng.integers(5, 70)), 30
    prompt = [int(x) for x in random_prompt(740 + case, n_prompt, cfg.vocab)]
    print(f"case {case}: {arch} hidden={hidden} layers={cfg.layers} Hq={heads} Hkv={kvh} d={d} "
          f"vocab={cfg.vocab} tied={cfg.tie_embeddings} prompt={n_prompt}", flush=True)
    cap = n_prompt + n_gen + 4
    want, want_logits = oracle_greedy(cfg, w, prompt, n_gen, cap)
    with DeviceModel(cfg, w) as m:
        cache = m.new_cache(cap)
        logits = m.forward(cache, prompt)
        diff = np.abs(logits[0] - want_logits).max()
        assert diff < 1e-4, f"prompt logits differ by {diff}"
        cache.len = 0
        first = m.prefill(cache, prompt)
        got = [first] + m.decode(cache, first, n_gen - 1)
    assert got == want
