"""Parity of the device input preparation with the CPU oracle.

wick_hip_attend / wick_hip_attend_device take the raw q, k, v projections of a
chunk of tokens, apply bias, QK-norm and RoPE (src/model.rs:464-480), append k
and v to the cache (:481-483) and run attention (:485).  The prepared q and the
appended cache rows must be bit-identical to the oracle's CPU arithmetic; the
attention output must be within |gpu - cpu| <= 2e-5 + 1e-4*|cpu|.
"""
import numpy as np
import pytest

import oracle_lib as ol
from util import within_tol
from wick_amd import DeviceKvCache, _native

pytestmark = pytest.mark.gpu


def raw_inputs(seed, t, heads, kv_heads, d, bias=False, norm=False):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((t, heads * d), dtype=np.float32)
    k = rng.standard_normal((t, kv_heads * d), dtype=np.float32)
    v = rng.standard_normal((t, kv_heads * d), dtype=np.float32)
    b = None
    if bias:
        b = (rng.standard_normal(heads * d, dtype=np.float32) * 0.5,
             rng.standard_normal(kv_heads * d, dtype=np.float32) * 0.5,
             rng.standard_normal(kv_heads * d, dtype=np.float32) * 0.5)
    n = None
    if norm:  # weights away from 1.0 so a dropped multiply shows
        n = (rng.uniform(0.5, 1.5, d).astype(np.float32), rng.uniform(0.5, 1.5, d).astype(np.float32))
    return q, k, v, b, n


def register(kv, layer, heads, b, n, eps):
    kwargs = {}
    if b is not None:
        kwargs.update(bq=b[0], bk=b[1], bv=b[2])
    if n is not None:
        kwargs.update(q_norm=n[0], k_norm=n[1])
    kv.set_prep(layer, heads, eps=eps, **kwargs)


def run_chunks(heads, kv_heads, d, chunks, theta, bias, norm, eps=1e-6, seed=0, capacity=None):
    """Feed `chunks` (token counts) through attend(); compare cache, q and att per chunk."""
    inv = ol.rope_inv_freq(theta, d)
    total = sum(chunks)
    cap = capacity or total
    cpu_k = np.zeros((cap, kv_heads * d), np.float32)
    cpu_v = np.zeros((cap, kv_heads * d), np.float32)
    with DeviceKvCache(2, cap, kv_heads, d) as kv:
        kv.set_rope(inv)
        start = 0
        for ci, t in enumerate(chunks):
            q, k, v, b, n = raw_inputs(seed + ci, t, heads, kv_heads, d, bias, norm)
            if ci == 0:
                register(kv, 1, heads, b, n, eps)
                consts = (b, n)
            b, n = consts
            att = kv.attend(1, heads, q, k, v, start)
            pq, pk, pv = ol.prep(q, k, v, heads, kv_heads, d, start, inv, bias=b, norms=n, eps=eps)
            cpu_k[start:start + t] = pk
            cpu_v[start:start + t] = pv
            gk, gv = kv.read(1, 0, start + t)
            assert np.array_equal(gk.view(np.uint32), cpu_k[:start + t].view(np.uint32)), "K cache not bit-exact"
            assert np.array_equal(gv.view(np.uint32), cpu_v[:start + t].view(np.uint32)), "V cache not bit-exact"
            want = ol.attention(pq, cpu_k, cpu_v, t, start, heads, kv_heads, d)
            ok, mabs, mrel = within_tol(att, want)
            print(f"chunk {ci}: t={t} start={start} Hq={heads} Hkv={kv_heads} d={d}: max abs {mabs:.2e} rel {mrel:.2e}")
            assert ok, f"max abs {mabs:.3e}, max rel {mrel:.3e}"
            # layer 0 was never written
            k0, v0 = kv.read(0, 0, start + t)
            assert not k0.any() and not v0.any()
            start += t


def test_qwen3_shape_qk_norm_prefill_then_decode():
    # config 3's preparation: QK-norm then RoPE theta 1e6, head_dim 128; the
    # single-token steps run the preparation inside the decode kernel
    run_chunks(16, 8, 128, [300, 1, 1], 1e6, bias=False, norm=True)


def test_decode_prep_with_split_chunks():
    # len > 192: the decode splits into contiguous chunks; only the last chunk's workgroups append
    run_chunks(14, 2, 64, [700, 1, 1], 1e6, bias=True, norm=True)


@pytest.mark.parametrize("heads,kv_heads,d,chunk,base", [(32, 8, 128, 512, 1918), (14, 2, 64, 1024, 2900),
                                                        (40, 2, 64, 1024, 2900)])
def test_decode_prep_interleaved_new_key_not_in_last_chunk(heads, kv_heads, d, chunk, base):
    """Single-token steps with the preparation in the decode kernel's prologue,
    on plans that interleave key groups across a kv head's workgroups: the new
    position's k and v rows are prepared and appended by the workgroups whose
    groups hold it, which here are not the last chunk's (with 40 heads per 2 kv
    heads, by both 16-head slices of the kv head, which write the same bits)."""
    gk = 16 if d == 128 else 32
    inv = ol.rope_inv_freq(1e6, d)
    rng = np.random.default_rng(base)
    steps, eps = 4, 1e-6
    cap = base + steps
    cpu_k = np.zeros((cap, kv_heads * d), np.float32)
    cpu_v = np.zeros((cap, kv_heads * d), np.float32)
    cpu_k[:base] = rng.standard_normal((base, kv_heads * d), dtype=np.float32)
    cpu_v[:base] = rng.standard_normal((base, kv_heads * d), dtype=np.float32)
    n = (rng.uniform(0.5, 1.5, d).astype(np.float32), rng.uniform(0.5, 1.5, d).astype(np.float32))
    not_last = []
    with DeviceKvCache(1, cap, kv_heads, d) as kv:
        kv.set_rope(inv)
        kv.set_option(_native.OPT_DECODE_CHUNK, chunk)
        kv.set_prep(0, heads, q_norm=n[0], k_norm=n[1], eps=eps)
        kv.append(0, 0, cpu_k[:base], cpu_v[:base])
        for s in range(steps):
            start = base + s
            L = start + 1
            nchunks = -(-L // chunk)
            assert chunk >= 4 * 4 * gk and nchunks > 1, "plan does not interleave"
            not_last.append((L - 1) // (4 * gk) % nchunks != nchunks - 1)
            q, k, v, _, _ = raw_inputs(base + 100 + s, 1, heads, kv_heads, d)
            att = kv.attend(0, heads, q, k, v, start)
            pq, pk, pv = ol.prep(q, k, v, heads, kv_heads, d, start, inv, norms=n, eps=eps)
            cpu_k[start] = pk[0]
            cpu_v[start] = pv[0]
            gk_rows, gv_rows = kv.read(0, 0, L)
            assert np.array_equal(gk_rows.view(np.uint32), cpu_k[:L].view(np.uint32)), "K cache not bit-exact"
            assert np.array_equal(gv_rows.view(np.uint32), cpu_v[:L].view(np.uint32)), "V cache not bit-exact"
            want = ol.attention(pq, cpu_k[:L], cpu_v[:L], 1, start, heads, kv_heads, d)
            ok, mabs, mrel = within_tol(att, want)
            print(f"step {s}: L={L} {kv.last_grid()} workgroups, max abs {mabs:.2e} rel {mrel:.2e}")
            assert ok, (s, mabs, mrel)
    assert all(not_last)


def test_decode_prep_with_head_slices():
    # group 20 > 16: two head slices per kv head both prepare (identical) k and v
    run_chunks(40, 2, 64, [50, 1, 1], 1e4, bias=True, norm=True)
    run_chunks(40, 2, 64, [300, 1], 1e4, bias=True, norm=True)


@pytest.mark.parametrize("heads,kv_heads", [(40, 2), (9, 3), (14, 2)])
def test_decode_prep_one_wide_chunk(heads, kv_heads):
    # 141..142 positions at head_dim 64: one chunk per unit on an 8-wave
    # workgroup (group 20 also splits into two head slices per kv head)
    run_chunks(heads, kv_heads, 64, [140, 1, 1], 1e4, bias=True, norm=True)


@pytest.mark.parametrize("heads,kv_heads", [(3, 3), (6, 3), (9, 3)])
def test_decode_wave_local_prep_steps(heads, kv_heads):
    """Groups of 1-3 at head_dim 64 prepare wave-locally in the VALU core: 40
    single-token steps after 700 positions (split chunks; the new key crosses
    32-key group boundaries at 704 and 736, so the wave that holds it changes),
    then a run across the one-chunk / split boundary at 192 positions."""
    run_chunks(heads, kv_heads, 64, [700] + [1] * 40, 1e4, bias=True, norm=True)
    run_chunks(heads, kv_heads, 64, [180] + [1] * 20, 1e4, bias=False, norm=False, seed=5)


def test_qwen2_shape_bias_chunked_then_decode():
    run_chunks(14, 2, 64, [37, 100, 1, 1], 1e6, bias=True, norm=False)


def test_smollm2_shape_plain_prefill_then_decode():
    run_chunks(9, 3, 64, [128, 1, 1, 1], 1e4, bias=False, norm=False)


@pytest.mark.parametrize("d", [16, 32])
def test_small_head_dims_bias_and_norm(d):
    run_chunks(4, 2, d, [20, 5, 1], 1e4, bias=True, norm=True)


def test_high_positions_use_their_table_rows():
    # positions near the end of a 40000-slot cache (RoPE theta 5e5, d 128)
    inv = ol.rope_inv_freq(500000.0, 128)
    cap, start, t, heads, kv_heads, d = 40000, 39990, 10, 4, 2, 128
    q, k, v, _, _ = raw_inputs(9, t, heads, kv_heads, d)
    with DeviceKvCache(1, cap, kv_heads, d) as kv:
        kv.set_rope(inv)
        kv.set_prep(0, heads)
        kv.attend(0, heads, q, k, v, start)
        gk, gv = kv.read(0, start, t)
    pq, pk, pv = ol.prep(q, k, v, heads, kv_heads, d, start, inv)
    assert np.array_equal(gk.view(np.uint32), pk.view(np.uint32))
    assert np.array_equal(gv.view(np.uint32), pv.view(np.uint32))


def test_long_decode_steps_attend_llama3_8b_shape():
    """configs[4] as the model's decode loop (Session::step -> Model::forward,
    /root/reference/src/engine.rs:142-145, src/model.rs:464-485): the cache
    holds 65472 positions, then 64 steps hand every layer the token's raw q, k
    and v; single-token attend prepares q in the decode kernel's prologue and
    appends the RoPE'd k and v at the next position there.  The appended rows
    are bit-exact against the oracle's preparation, the first and the last
    step's outputs (65473 and 65536 positions) match the oracle.  Two layers of
    the config's per-layer shape (Hq 32 / Hkv 8, d 128) keep the host copy
    small."""
    heads, kvh, d, L, nsteps, layers = 32, 8, 128, 65536, 64, 2
    base = L - nsteps
    inv = ol.rope_inv_freq(500000.0, d)
    rng = np.random.default_rng(7)
    ks = [rng.standard_normal((L, kvh * d), dtype=np.float32) for _ in range(layers)]
    vs = [rng.standard_normal((L, kvh * d), dtype=np.float32) for _ in range(layers)]
    raw = [[raw_inputs(1000 * layer + s, 1, heads, kvh, d)[:3] for s in range(nsteps)] for layer in range(layers)]
    outs = {}
    with DeviceKvCache(layers, L, kvh, d) as kv:
        kv.set_rope(inv)
        for layer in range(layers):
            kv.set_prep(layer, heads, eps=1e-5)
            kv.append(layer, 0, ks[layer][:base], vs[layer][:base])
        for s in range(nsteps):
            for layer in range(layers):
                q, k, v = raw[layer][s]
                att = kv.attend(layer, heads, q, k, v, base + s)
                if s in (0, nsteps - 1):
                    outs[(layer, s)] = att
        got = [kv.read(layer, base, nsteps) for layer in range(layers)]
    pq = {}
    for layer in range(layers):
        for s in range(nsteps):
            q, k, v = raw[layer][s]
            pq[(layer, s)], pk, pv = ol.prep(q, k, v, heads, kvh, d, base + s, inv, eps=1e-5)
            ks[layer][base + s], vs[layer][base + s] = pk[0], pv[0]
        gk, gv = got[layer]
        assert np.array_equal(gk.view(np.uint32), ks[layer][base:].view(np.uint32)), f"layer {layer}: K rows"
        assert np.array_equal(gv.view(np.uint32), vs[layer][base:].view(np.uint32)), f"layer {layer}: V rows"
    for (layer, s), att in outs.items():
        n = base + s + 1
        want = ol.attention(pq[(layer, s)], ks[layer][:n], vs[layer][:n], 1, base + s, heads, kvh, d)
        ok, mabs, mrel = within_tol(att, want)
        print(f"layer {layer} step {s} ({n} positions): max abs {mabs:.2e} max rel {mrel:.2e}")
        assert ok, (layer, s, mabs, mrel)


def test_attend_device_rewrites_q_in_place():
    torch = pytest.importorskip("torch")
    heads, kv_heads, d, t, start = 16, 8, 128, 64, 0
    inv = ol.rope_inv_freq(1e6, d)
    q, k, v, b, n = raw_inputs(11, t, heads, kv_heads, d, bias=True, norm=True)
    with DeviceKvCache(1, 256, kv_heads, d) as kv:
        kv.set_rope(inv)
        register(kv, 0, heads, b, n, 1e-6)
        stream = torch.cuda.Stream()
        kv.set_stream(stream.cuda_stream)
        qd, kd, vd = (torch.from_numpy(a).cuda() for a in (q, k, v))
        att = torch.empty_like(qd)
        torch.cuda.synchronize()
        kv.attend_device(0, heads, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), t, start, att.data_ptr())
        kv.synchronize()
        gq, gatt = qd.cpu().numpy(), att.cpu().numpy()
        gk, gv = kv.read(0, 0, t)
    pq, pk, pv = ol.prep(q, k, v, heads, kv_heads, d, start, inv, bias=b, norms=n, eps=1e-6)
    assert np.array_equal(gq.view(np.uint32), pq.view(np.uint32)), "prepared q not bit-exact"
    assert np.array_equal(gk.view(np.uint32), pk.view(np.uint32))
    assert np.array_equal(gv.view(np.uint32), pv.view(np.uint32))
    ok, mabs, mrel = within_tol(gatt, ol.attention(pq, pk, pv, t, start, heads, kv_heads, d))
    assert ok, f"max abs {mabs:.3e}, max rel {mrel:.3e}"


def test_attend_device_single_token_leaves_q():
    """t = 1 prepares q inside the decode kernel: q_dev keeps the raw projection."""
    torch = pytest.importorskip("torch")
    heads, kv_heads, d = 16, 8, 128
    inv = ol.rope_inv_freq(1e6, d)
    q, k, v, b, n = raw_inputs(12, 5, heads, kv_heads, d, bias=True, norm=True)
    with DeviceKvCache(1, 256, kv_heads, d) as kv:
        kv.set_rope(inv)
        register(kv, 0, heads, b, n, 1e-6)
        kv.attend(0, heads, q[:4], k[:4], v[:4], 0)
        qd, kd, vd = (torch.from_numpy(np.ascontiguousarray(a[4:])).cuda() for a in (q, k, v))
        att = torch.empty_like(qd)
        torch.cuda.synchronize()
        kv.attend_device(0, heads, qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), 1, 4, att.data_ptr())
        kv.synchronize()
        gq, gatt = qd.cpu().numpy(), att.cpu().numpy()
        gk, gv = kv.read(0, 0, 5)
    assert np.array_equal(gq.view(np.uint32), q[4:].view(np.uint32)), "q_dev changed"
    pq, pk, pv = ol.prep(q, k, v, heads, kv_heads, d, 0, inv, bias=b, norms=n, eps=1e-6)
    assert np.array_equal(gk.view(np.uint32), pk.view(np.uint32))
    assert np.array_equal(gv.view(np.uint32), pv.view(np.uint32))
    ok, mabs, mrel = within_tol(gatt, ol.attention(pq[4:], pk, pv, 1, 4, heads, kv_heads, d))
    assert ok, f"max abs {mabs:.3e}, max rel {mrel:.3e}"


def test_prep_errors():
    inv = ol.rope_inv_freq(1e4, 64)
    q, k, v, _, _ = raw_inputs(1, 2, 4, 2, 64)
    with DeviceKvCache(2, 16, 2, 64) as kv:
        with pytest.raises(_native.WickHipError, match="RoPE"):
            kv.attend(0, 4, q, k, v, 0)
        kv.set_rope(inv)
        with pytest.raises(_native.WickHipError, match="preparation constants"):
            kv.attend(0, 4, q, k, v, 0)
        kv.set_prep(0, 4)
        with pytest.raises(_native.WickHipError, match="heads"):
            kv.attend(0, 2, q[:, :128], k, v, 0)
        with pytest.raises(_native.WickHipError, match="all three"):
            kv.set_prep(1, 4, bq=np.zeros(256, np.float32))
        with pytest.raises(_native.WickHipError, match="both"):
            kv.set_prep(1, 4, q_norm=np.ones(64, np.float32))
        with pytest.raises(_native.WickHipError, match="capacity"):
            kv.attend(0, 4, q, k, v, 15)
        # nothing was appended by the failed calls
        gk, gv = kv.read(0, 0, 16)
        assert not gk.any() and not gv.any()
