"""Seeded sweep over the planner's choices: random shapes through the C ABI
against the CPU oracle.

Each case draws a head_dim, kv heads, GQA group, cache length and chunk length
(decode t = 1, short chunks, long chunks), and sometimes a forced decode chunk
size (16-key steps, not always whole tile groups), so the cases fall on the one-chunk and split decode paths (MFMA and VALU
cores, 4- and 8-wave workgroups, every merge slot count), the prefill kernels
and the preparation paths (bias, QK-norm, RoPE) without naming them.  Outputs
within 2e-5 abs / 1e-4 rel of the oracle; appended cache rows bit-exact.
"""
import numpy as np
import pytest

import oracle_lib as ol
from util import within_tol
from wick_amd import DeviceKvCache, _native

pytestmark = pytest.mark.gpu

N_CASES = 48


def draw(rng):
    d = int(rng.choice([16, 32, 64, 128]))
    kv_heads = int(rng.integers(1, 9))
    group = int(rng.choice([1, 2, 3, 4, 5, 7, 8, 16, 17]))
    kind = rng.random()
    if kind < 0.6:
        t = 1
    elif kind < 0.85:
        t = int(rng.integers(2, 40))
    else:
        t = int(rng.integers(40, 300))
    start = int(rng.integers(0, 6000 if t == 1 else 1500))
    chunk = int(rng.choice([0, 0, 0, 64, 80, 128, 208, 336, 512])) if t == 1 else 0
    return d, kv_heads, group, t, start, chunk


@pytest.mark.parametrize("case", range(N_CASES))
def test_attention_sweep(case):
    rng = np.random.default_rng(1000 + case)
    d, kv_heads, group, t, start, chunk = draw(rng)
    heads = kv_heads * group
    L = start + t
    q = rng.standard_normal((t, heads * d), dtype=np.float32)
    k = rng.standard_normal((L, kv_heads * d), dtype=np.float32)
    v = rng.standard_normal((L, kv_heads * d), dtype=np.float32)
    print(f"case {case}: d={d} Hkv={kv_heads} group={group} t={t} start={start} chunk={chunk}", flush=True)
    with DeviceKvCache(1, L + int(rng.integers(0, 50)), kv_heads, d) as kv:
        if chunk:
            kv.set_option(_native.OPT_DECODE_CHUNK, chunk)
        kv.append(0, 0, k, v)
        got = kv.attention(0, heads, q, start)
    want = ol.attention(q, k, v, t, start, heads, kv_heads, d)
    ok, mabs, mrel = within_tol(got, want)
    assert ok, f"max abs {mabs:.3e}, max rel {mrel:.3e}"


@pytest.mark.parametrize("case", range(N_CASES // 2))
def test_attend_sweep(case):
    """The same draws through wick_hip_attend (raw q/k/v: preparation, append,
    attention) for a prefix chunk and then two single-token steps."""
    rng = np.random.default_rng(5000 + case)
    d, kv_heads, group, t, start, _ = draw(rng)
    heads = kv_heads * group
    start = min(start, 1200)
    bias, norm = bool(rng.random() < 0.5), bool(rng.random() < 0.5)
    theta = float(rng.choice([1e4, 1e6]))
    inv = ol.rope_inv_freq(theta, d)
    b = n = None
    if bias:
        b = (rng.standard_normal(heads * d, dtype=np.float32) * 0.5,
             rng.standard_normal(kv_heads * d, dtype=np.float32) * 0.5,
             rng.standard_normal(kv_heads * d, dtype=np.float32) * 0.5)
    if norm:
        n = (rng.uniform(0.5, 1.5, d).astype(np.float32), rng.uniform(0.5, 1.5, d).astype(np.float32))
    chunks = [max(start, 1), 1, 1]
    cap = sum(chunks) + 3
    cpu_k = np.zeros((cap, kv_heads * d), np.float32)
    cpu_v = np.zeros((cap, kv_heads * d), np.float32)
    print(f"case {case}: d={d} Hkv={kv_heads} group={group} chunks={chunks} bias={bias} norm={norm}", flush=True)
    with DeviceKvCache(1, cap, kv_heads, d) as kv:
        kv.set_rope(inv)
        kw = {}
        if b is not None:
            kw.update(bq=b[0], bk=b[1], bv=b[2])
        if n is not None:
            kw.update(q_norm=n[0], k_norm=n[1])
        kv.set_prep(0, heads, eps=1e-6, **kw)
        pos = 0
        for tc in chunks:
            q = rng.standard_normal((tc, heads * d), dtype=np.float32)
            kr = rng.standard_normal((tc, kv_heads * d), dtype=np.float32)
            vr = rng.standard_normal((tc, kv_heads * d), dtype=np.float32)
            att = kv.attend(0, heads, q, kr, vr, pos)
            pq, pk, pv = ol.prep(q, kr, vr, heads, kv_heads, d, pos, inv, bias=b, norms=n, eps=1e-6)
            cpu_k[pos:pos + tc] = pk
            cpu_v[pos:pos + tc] = pv
            gk, gv = kv.read(0, 0, pos + tc)
            assert np.array_equal(gk.view(np.uint32), cpu_k[:pos + tc].view(np.uint32)), "K cache not bit-exact"
            assert np.array_equal(gv.view(np.uint32), cpu_v[:pos + tc].view(np.uint32)), "V cache not bit-exact"
            want = ol.attention(pq, cpu_k, cpu_v, tc, pos, heads, kv_heads, d)
            ok, mabs, mrel = within_tol(att, want)
            assert ok, f"chunk at {pos}: max abs {mabs:.3e}, max rel {mrel:.3e}"
            pos += tc
