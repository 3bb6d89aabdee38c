"""Pin the CPU oracle before it checks anything.

- transformers-scored golden fixtures held by the reference
  (/root/reference/tests/fixtures/tiny, copied to tests/golden/tiny), with the
  reference's own thresholds (tests/tiny_models.rs:68, :89, :111);
- closed forms and special cases of attention / softmax / RoPE;
- an independent float64 brute force of attention.
"""
import json
import os

import numpy as np
import pytest

import oracle_lib as ol
from wick_amd.model import Config, load_weights

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tiny")
MODELS = ["llama3-scaled-f32", "qwen2-bias-bf16", "qwen3-qknorm-f32"]


def expected(name):
    with open(os.path.join(GOLDEN, name, "expected.json")) as f:
        return json.load(f)


def oracle_model(name):
    d = os.path.join(GOLDEN, name)
    cfg = Config.load(d)
    return ol.OracleModel(cfg, load_weights(d, cfg))


# ------------------------------------------------------------ golden vectors

@pytest.mark.parametrize("name", MODELS)
@pytest.mark.parametrize("order", [ol.AVX2, ol.SCALAR])
def test_matches_transformers(name, order):
    """tests/tiny_models.rs:58-71: every position's logits within 1e-3."""
    exp = expected(name)
    m = oracle_model(name)
    st = m.new_state(256)
    got = m.forward(st, exp["tokens"], all_logits=True, order=order, threads=4)
    want = np.array(exp["logits"], np.float32)
    assert got.shape == want.shape
    worst = np.abs(got - want).max()
    assert worst < 1e-3, f"{name}: logits differ by {worst}"


@pytest.mark.parametrize("name", MODELS)
def test_incremental_matches_batch(name):
    """tests/tiny_models.rs:73-95: uneven chunks give the batch logits within 1e-4."""
    exp = expected(name)
    m = oracle_model(name)
    batch = m.forward(m.new_state(256), exp["tokens"], all_logits=True, threads=3)
    st = m.new_state(256)
    pos = 0
    for size in [1, 5, 2, 7, 1, 1, 13, 3, 15]:
        rows = m.forward(st, exp["tokens"][pos:pos + size], all_logits=True, threads=3)
        d = np.abs(rows - batch[pos:pos + size]).max()
        assert d < 1e-4, f"{name}: chunk at {pos} differs by {d}"
        pos += size
    assert pos == len(exp["tokens"])


@pytest.mark.parametrize("name", MODELS)
def test_greedy_continuation(name):
    """tests/tiny_models.rs:97-113: 16 greedy ids after an 8-token prompt, identical."""
    exp = expected(name)
    m = oracle_model(name)
    st = m.new_state(256)
    logits = m.forward(st, exp["greedy_prompt"], threads=2)
    out = []
    for _ in range(len(exp["greedy"])):
        tok = ol.argmax(logits[0])
        out.append(tok)
        logits = m.forward(st, [tok], threads=2)
    assert out == exp["greedy"]


# ------------------------------------------------------------ primitives

def xorshift_data(n, seed):
    """The generator of src/kernels.rs:385-395 (u32 xorshift)."""
    s = (seed * 2654435761 + 1) & 0xFFFFFFFF
    out = np.empty(n, np.float32)
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = np.float32(s % 2000) / np.float32(1000.0) - np.float32(1.0)
    return out


@pytest.mark.parametrize("n", [8, 64, 96, 1000, 4104])
def test_dot_simd_matches_scalar(n):
    """src/kernels.rs:397-410: SIMD and scalar orders within 1e-3*(1+|want|)."""
    w = xorshift_data(n, 1)
    for k in range(4):
        x = xorshift_data(n, 10 + k)
        want = ol.dot(w, x, ol.SCALAR)
        got = ol.dot(w, x, ol.AVX2)
        assert abs(got - want) < 1e-3 * (1 + abs(want))
        assert abs(want - float(np.dot(w.astype(np.float64), x.astype(np.float64)))) < 1e-3 * (1 + abs(want))


def test_dot_exact_on_small_integers():
    # every partial sum is an exact small integer, so both orders give the exact product
    rng = np.random.default_rng(7)
    for n in (8, 16, 64, 128, 13):
        w = rng.integers(-8, 9, n).astype(np.float32)
        x = rng.integers(-8, 9, n).astype(np.float32)
        exact = float(np.dot(w.astype(np.int64), x.astype(np.int64)))
        assert ol.dot(w, x, ol.AVX2) == exact
        assert ol.dot(w, x, ol.SCALAR) == exact


def test_dot_avx2_order_is_wick_hsum():
    # lane sums that cancel only in wick's hsum order: ((a0+a4)+(a2+a6))+((a1+a5)+(a3+a7))
    big = np.float32(2.0 ** 25)
    w = np.array([big, 1, 1, 1, -big, 0, 0, 0], np.float32)
    x = np.ones(8, np.float32)
    # hsum: (big + -big) + (1 + 0) + ... = 3 exactly; a sequential sum would lose the 1s
    assert ol.dot(w, x, ol.AVX2) == 3.0
    seq = np.float32(-0.0)
    for v in w:
        seq = np.float32(seq + v)
    assert ol.dot(w, x, ol.SCALAR) == float(seq)


def test_softmax_closed_forms():
    assert ol.softmax(np.array([3.5], np.float32))[0] == 1.0
    p = ol.softmax(np.full(8, -2.25, np.float32))
    assert np.all(p == np.float32(0.125))
    a, b = 0.7, -1.9
    p = ol.softmax(np.array([a, b], np.float32))
    assert abs(p[0] - 1 / (1 + np.exp(b - a))) < 1e-7
    assert abs(p.sum() - 1) < 1e-6


def test_rmsnorm_closed_form():
    x = np.full(64, 3.0, np.float32)
    w = np.full(64, 2.0, np.float32)
    out = ol.rmsnorm(x, w, 0.0)
    assert np.allclose(out, 2.0, atol=1e-6)


def test_rope_preserves_pair_norm_and_is_identity_at_zero():
    rng = np.random.default_rng(1)
    inv = ol.rope_inv_freq(10000.0, 64)
    v = rng.standard_normal(128).astype(np.float32)
    assert np.array_equal(ol.rope(v, 64, 0, inv), v)  # sin 0 = 0, cos 0 = 1 exactly
    r = ol.rope(v, 64, 77, inv)
    for h in range(2):
        a, b = v[h * 64:h * 64 + 32], v[h * 64 + 32:(h + 1) * 64]
        ra, rb = r[h * 64:h * 64 + 32], r[h * 64 + 32:(h + 1) * 64]
        assert np.allclose(a * a + b * b, ra * ra + rb * rb, rtol=1e-5, atol=1e-6)


def test_prep_composition_order_and_special_cases():
    """ol.prep = bias, then per-head QK-norm, then RoPE (src/model.rs:470-480); v gets the bias only."""
    rng = np.random.default_rng(4)
    heads, kv_heads, d = 4, 2, 32
    inv = ol.rope_inv_freq(10000.0, d)
    q = rng.standard_normal((3, heads * d)).astype(np.float32)
    k = rng.standard_normal((3, kv_heads * d)).astype(np.float32)
    v = rng.standard_normal((3, kv_heads * d)).astype(np.float32)
    bias = (rng.standard_normal(heads * d).astype(np.float32), rng.standard_normal(kv_heads * d).astype(np.float32),
            rng.standard_normal(kv_heads * d).astype(np.float32))
    norms = (rng.uniform(0.5, 1.5, d).astype(np.float32), rng.uniform(0.5, 1.5, d).astype(np.float32))
    # position 0 without constants: identity, bit for bit
    pq, pk, pv = ol.prep(q[:1], k[:1], v[:1], heads, kv_heads, d, 0, inv)
    assert np.array_equal(pq, q[:1]) and np.array_equal(pk, k[:1]) and np.array_equal(pv, v[:1])
    # position 0 with bias and norm: RoPE is the identity, so q = rmsnorm(q + bq) per head
    pq, pk, pv = ol.prep(q[:1], k[:1], v[:1], heads, kv_heads, d, 0, inv, bias=bias, norms=norms, eps=1e-6)
    assert np.array_equal(pv[0], v[0] + bias[2])
    for h in range(heads):
        want = ol.rmsnorm(q[0, h * d:(h + 1) * d] + bias[0][h * d:(h + 1) * d], norms[0], 1e-6)
        assert np.array_equal(pq[0, h * d:(h + 1) * d], want)
    # rmsnorm_inplace and rmsnorm are the same arithmetic
    assert np.array_equal(ol.rmsnorm_inplace(q[0, :d], norms[0], 1e-6), ol.rmsnorm(q[0, :d], norms[0], 1e-6))
    # later positions: an f64 restatement agrees to f32 rounding, and v is not rotated
    pq, pk, pv = ol.prep(q, k, v, heads, kv_heads, d, 50, inv, bias=bias, norms=norms, eps=1e-6)
    assert np.array_equal(pv, v + np.stack([bias[2]] * 3))
    x = (q.astype(np.float64) + bias[0]).reshape(3, heads, d)
    x = x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) * norms[0]
    ang = (np.arange(50, 53)[:, None] * inv[None, :].astype(np.float64))[:, None, :]
    a, b = x[..., :d // 2], x[..., d // 2:]
    want = np.concatenate([a * np.cos(ang) - b * np.sin(ang), b * np.cos(ang) + a * np.sin(ang)], -1)
    assert np.allclose(pq.reshape(3, heads, d), want, atol=2e-6, rtol=1e-5)


def test_inv_freq_closed_forms_and_host_agreement():
    for theta, d in ((10000.0, 64), (1e6, 128), (500000.0, 128), (50000.0, 16)):
        inv = ol.rope_inv_freq(theta, d)
        assert inv[0] == 1.0
        assert abs(inv[d // 4] - theta ** -0.5) <= 1e-7 * theta ** -0.5 * 4
        cfg = Config("llama", 1, 1, 1, 1, 1, d, 1, rope_theta=theta)
        assert np.array_equal(inv, cfg.rope_inv_freq())
    cfg = Config.load(os.path.join(GOLDEN, "llama3-scaled-f32"))
    assert cfg.rope_scaling is not None
    assert np.array_equal(ol.rope_inv_freq(cfg.rope_theta, cfg.head_dim, cfg.rope_scaling), cfg.rope_inv_freq())


# ------------------------------------------------------------ attention

def attention_f64(q, k, v, t, start, heads, kv_heads, d):
    g = heads // kv_heads
    q = q.reshape(t, heads, d).astype(np.float64)
    k = k.reshape(-1, kv_heads, d).astype(np.float64)
    v = v.reshape(-1, kv_heads, d).astype(np.float64)
    out = np.zeros((t, heads, d))
    scale = 1.0 / np.sqrt(d)
    for i in range(t):
        L = start + i + 1
        for h in range(heads):
            s = k[:L, h // g] @ q[i, h] * scale
            p = np.exp(s - s.max())
            p /= p.sum()
            out[i, h] = p @ v[:L, h // g]
    return out.reshape(t, heads * d)


@pytest.mark.parametrize("t,start,heads,kv_heads,d", [
    (1, 0, 4, 2, 16), (1, 200, 14, 2, 64), (7, 30, 9, 3, 64), (16, 0, 16, 8, 128), (5, 11, 32, 4, 64),
    (3, 2, 4, 4, 32), (2, 40, 6, 1, 24)])
@pytest.mark.parametrize("order", [ol.AVX2, ol.SCALAR])
def test_attention_matches_f64_bruteforce(t, start, heads, kv_heads, d, order):
    rng = np.random.default_rng(t * 1000 + start)
    L = start + t
    q = rng.standard_normal((t, heads * d)).astype(np.float32)
    k = rng.standard_normal((L, kv_heads * d)).astype(np.float32)
    v = rng.standard_normal((L, kv_heads * d)).astype(np.float32)
    got = ol.attention(q, k, v, t, start, heads, kv_heads, d, order=order)
    want = attention_f64(q, k, v, t, start, heads, kv_heads, d)
    assert np.abs(got - want).max() < 2e-6


def test_attention_special_cases():
    rng = np.random.default_rng(3)
    heads, kvh, d = 8, 2, 64
    # len = 1: softmax of one score is exactly 1, output is V[0] bit for bit
    q = rng.standard_normal((1, heads * d)).astype(np.float32)
    k = rng.standard_normal((1, kvh * d)).astype(np.float32)
    v = rng.standard_normal((1, kvh * d)).astype(np.float32)
    att = ol.attention(q, k, v, 1, 0, heads, kvh, d).reshape(heads, d)
    for h in range(heads):
        assert np.array_equal(att[h], v[0].reshape(kvh, d)[h // 4])
    # constant keys: uniform weights, output is the mean of V
    L = 50
    k = np.tile(rng.standard_normal((1, kvh * d)).astype(np.float32), (L, 1))
    v = rng.standard_normal((L, kvh * d)).astype(np.float32)
    att = ol.attention(q, k, v, 1, L - 1, heads, kvh, d).reshape(heads, d)
    mean = v.reshape(L, kvh, d).astype(np.float64).mean(0)
    for h in range(heads):
        assert np.abs(att[h] - mean[h // 4]).max() < 1e-6
    # one dominant score selects that row
    q = np.zeros((1, heads * d), np.float32)
    q[0, :] = 1.0
    k = np.zeros((L, kvh * d), np.float32)
    k[17, :] = 100.0
    att = ol.attention(q, k, v, 1, L - 1, heads, kvh, d).reshape(heads, d)
    for h in range(heads):
        assert np.array_equal(att[h], v[17].reshape(kvh, d)[h // 4])


def test_attention_is_causal_and_shares_gqa_groups():
    rng = np.random.default_rng(5)
    t, start, heads, kvh, d = 6, 9, 8, 2, 32
    L = start + t
    q = rng.standard_normal((t, heads * d)).astype(np.float32)
    q4 = q.reshape(t, heads, d)
    q4[:, 1] = q4[:, 0]  # heads 0 and 1 share kv head 0
    k = rng.standard_normal((L, kvh * d)).astype(np.float32)
    v = rng.standard_normal((L, kvh * d)).astype(np.float32)
    a = ol.attention(q, k, v, t, start, heads, kvh, d).reshape(t, heads, d)
    assert np.array_equal(a[:, 0], a[:, 1])
    k2, v2 = k.copy(), v.copy()
    k2[start + 3:] = 9.0
    v2[start + 3:] = -9.0
    b = ol.attention(q, k2, v2, t, start, heads, kvh, d).reshape(t, heads, d)
    assert np.array_equal(a[:3], b[:3])  # tokens 0..2 cannot see positions >= start+3
    assert not np.array_equal(a[3:], b[3:])


def test_attention_thread_count_independent():
    rng = np.random.default_rng(9)
    t, start, heads, kvh, d = 9, 13, 14, 2, 64
    L = start + t
    q = rng.standard_normal((t, heads * d)).astype(np.float32)
    k = rng.standard_normal((L, kvh * d)).astype(np.float32)
    v = rng.standard_normal((L, kvh * d)).astype(np.float32)
    a1 = ol.attention(q, k, v, t, start, heads, kvh, d, threads=1)
    a8 = ol.attention(q, k, v, t, start, heads, kvh, d, threads=8)
    assert np.array_equal(a1, a8)
