"""Parity of the HIP attention path (through the C ABI) with the CPU oracle.

Shapes follow the benchmark configurations; sizes are those the oracle
finishes in seconds.  Tolerance: |gpu - cpu| <= 2e-5 + 1e-4*|cpu| per element.
Integer/byte work (the KV append) must be bit-exact.
"""
import numpy as np
import pytest

import oracle_lib as ol
from util import inv_freq, rmsnorm_heads_np, rope_np, within_tol
from wick_amd import DeviceKvCache, _native

pytestmark = pytest.mark.gpu


def make_inputs(seed, t, start, heads, kv_heads, d, theta=None, qk_norm=False):
    rng = np.random.default_rng(seed)
    L = start + t
    q = rng.standard_normal((t, heads * d), dtype=np.float32)
    k = rng.standard_normal((L, kv_heads * d), dtype=np.float32)
    v = rng.standard_normal((L, kv_heads * d), dtype=np.float32)
    if qk_norm:
        q = rmsnorm_heads_np(q, heads, d, 1e-6)
        k = rmsnorm_heads_np(k, kv_heads, d, 1e-6)
    if theta is not None:
        inv = inv_freq(theta, d)
        q = rope_np(q, heads, d, np.arange(start, L), inv)
        k = rope_np(k, kv_heads, d, np.arange(L), inv)
    return q, k, v


def run_gpu(q, k, v, t, start, heads, kv_heads, d, capacity=None, options=()):
    L = start + t
    with DeviceKvCache(1, capacity or L, kv_heads, d) as kv:
        for opt, val in options:
            kv.set_option(opt, val)
        kv.append(0, 0, k[:L], v[:L])
        return kv.attention(0, heads, q, start)


def check(q, k, v, t, start, heads, kv_heads, d, **kw):
    got = run_gpu(q, k, v, t, start, heads, kv_heads, d, **kw)
    want = ol.attention(q, k, v, t, start, heads, kv_heads, d)
    ok, mabs, mrel = within_tol(got, want)
    print(f"t={t} start={start} Hq={heads} Hkv={kv_heads} d={d}: max abs {mabs:.2e} max rel {mrel:.2e}")
    assert ok, f"max abs {mabs:.3e}, max rel {mrel:.3e}"
    return got


# ---- decode (t = 1): config 2 (Qwen2.5 shape), config 5 (Llama-3-8B shape), config 1 (SmolLM2 shape)

@pytest.mark.parametrize("L", [512, 4096, 32768])
def test_decode_qwen25_shape(L):
    q, k, v = make_inputs(2, 1, L - 1, 14, 2, 64, theta=1e6)
    check(q, k, v, 1, L - 1, 14, 2, 64)


def test_decode_llama3_8b_shape_65536():
    q, k, v = make_inputs(5, 1, 65535, 32, 8, 128, theta=500000.0)
    check(q, k, v, 1, 65535, 32, 8, 128)


def test_decode_llama3_8b_shape_32768():
    """The Llama-3-8B shape at the headline's 32K context.  The automatic plan
    sizes chunks in 16-key steps to fill one resident round (94 chunks of 352
    keys on a 256-CU MI355X), so most chunks are not a whole number of the
    kernel's 64-key rounds of tile groups."""
    L = 32768
    q, k, v = make_inputs(55, 1, L - 1, 32, 8, 128, theta=500000.0)
    with DeviceKvCache(1, L, 8, 128) as kv:
        kv.append(0, 0, k, v)
        got = kv.attention(0, 32, q, L - 1)
        grid = kv.last_grid()
    want = ol.attention(q, k, v, 1, L - 1, 32, 8, 128)
    ok, mabs, mrel = within_tol(got, want)
    print(f"L={L}: {grid} workgroups, max abs {mabs:.2e} max rel {mrel:.2e}")
    assert ok, (mabs, mrel)
    assert grid % 8 == 0


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("chunk", [80, 208, 336, 688])
def test_decode_chunks_in_16_key_steps(chunk, d):
    """Chunks that are multiples of 16 keys but not of the 32-key tile groups
    (head_dim 64) or of a workgroup's 4 groups: the last group of a wave's range,
    and whole waves, fall past the chunk's end.  The context leaves the last chunk
    ragged."""
    L = 37 * chunk - 5
    q, k, v = make_inputs(chunk + d, 1, L - 1, 14, 2, d)
    check(q, k, v, 1, L - 1, 14, 2, d, options=[(_native.OPT_DECODE_CHUNK, chunk)])


def test_decode_chunk_option_values():
    with DeviceKvCache(1, 64, 2, 64) as kv:
        for bad in (-16, 16, 48, 100, 72):
            with pytest.raises(_native.WickHipError):
                kv.set_option(_native.OPT_DECODE_CHUNK, bad)
        for good in (0, 64, 80, 4096):
            kv.set_option(_native.OPT_DECODE_CHUNK, good)
        for bad in (-1, 2, 3):
            with pytest.raises(_native.WickHipError):
                kv.set_option(_native.OPT_DECODE_ORDER, bad)
        for good in (0, 1):
            kv.set_option(_native.OPT_DECODE_ORDER, good)


# The automatic key order interleaves a split on the MFMA core (head_dim 128, or
# 64 with more than 4 heads per kv head) whose chunks hold at least 4 rounds of
# the 4 waves' key groups (16 keys at head_dim 128, 32 at 64).
def interleaves(d, chunk):
    gk = 16 if d == 128 else 32
    return chunk >= 4 * 4 * gk


@pytest.mark.parametrize("d,heads,kv_heads,chunk,L", [
    (128, 32, 8, 512, 5000),     # 10 chunks, 313 groups: 7 full rounds + a partial one
    (128, 32, 8, 256, 4096),     # 16 chunks, 256 groups: exactly 4 full rounds, no partial one
    (128, 8, 2, 1024, 9001),     # ragged last group
    (64, 14, 2, 1024, 6000),     # double-buffered core, 32-key groups
    (64, 40, 2, 1024, 4500),     # two 16-head slices per kv head (4 units); a partial round of one group
])
def test_decode_key_orders(d, heads, kv_heads, chunk, L):
    """Both split-K key orders against the oracle, on plans where the automatic
    order interleaves key groups across a kv head's workgroups (every unit
    starting its rounds at a different one), and bit-stable from call to call."""
    assert interleaves(d, chunk) and L > chunk
    q, k, v = make_inputs(L + d, 1, L - 1, heads, kv_heads, d)
    want = ol.attention(q, k, v, 1, L - 1, heads, kv_heads, d)
    outs = {}
    with DeviceKvCache(1, L, kv_heads, d) as kv:
        kv.append(0, 0, k, v)
        kv.set_option(_native.OPT_DECODE_CHUNK, chunk)
        for order in (0, 1):
            kv.set_option(_native.OPT_DECODE_ORDER, order)
            outs[order] = kv.attention(0, heads, q, L - 1)
            again = kv.attention(0, heads, q, L - 1)
            assert np.array_equal(outs[order].view(np.uint32), again.view(np.uint32)), "not bit-stable"
            ok, mabs, mrel = within_tol(outs[order], want)
            print(f"order {order}: {kv.last_grid()} workgroups, max abs {mabs:.2e} max rel {mrel:.2e}")
            assert ok, (order, mabs, mrel)
    # a different summation order: equal within rounding, not bit-identical
    assert np.abs(outs[0] - outs[1]).max() < 1e-5


def test_long_decode_steps_append_llama3_8b_shape():
    """configs[4] as a decode loop (Session::step -> Model::forward,
    /root/reference/src/engine.rs:142-145, src/model.rs:481-485): the cache holds
    65472 positions, then 64 steps each append the token's k/v row at the next
    position of every layer and attend over the grown cache, up to 65536.  The
    appended rows read back bit-exact; the first and the last step's outputs
    (65473 and 65536 positions) match the oracle.  Two layers of the config's
    per-layer shape (Hq 32 / Hkv 8, d 128, 512 MiB of K+V each) keep the host
    copy small."""
    heads, kvh, d, L, nsteps, layers = 32, 8, 128, 65536, 64, 2
    base = L - nsteps
    inv = inv_freq(500000.0, d)
    rng = np.random.default_rng(5)
    ks, vs, qs = [], [], []
    for layer in range(layers):
        k = rope_np(rng.standard_normal((L, kvh * d), dtype=np.float32), kvh, d, np.arange(L), inv)
        ks.append(k)
        vs.append(rng.standard_normal((L, kvh * d), dtype=np.float32))
        qs.append(rope_np(rng.standard_normal((nsteps, heads * d), dtype=np.float32), heads, d,
                          np.arange(base, L), inv))
    outs = {}
    with DeviceKvCache(layers, L, kvh, d) as kv:
        for layer in range(layers):
            kv.append(layer, 0, ks[layer][:base], vs[layer][:base])
        grids = []
        for s in range(nsteps):
            for layer in range(layers):
                kv.append(layer, base + s, ks[layer][base + s:base + s + 1], vs[layer][base + s:base + s + 1])
                att = kv.attention(layer, heads, qs[layer][s:s + 1], base + s)
                if s in (0, nsteps - 1):
                    outs[(layer, s)] = att
            grids.append(kv.last_grid())
        for layer in range(layers):
            kr, vr = kv.read(layer, base, nsteps)
            assert np.array_equal(kr, ks[layer][base:]) and np.array_equal(vr, vs[layer][base:]), layer
    print(f"decode grids over the 64 steps: {sorted(set(grids))}")
    for (layer, s), got in outs.items():
        n = base + s + 1
        want = ol.attention(qs[layer][s:s + 1], ks[layer][:n], vs[layer][:n], 1, base + s, heads, kvh, d)
        ok, mabs, mrel = within_tol(got, want)
        print(f"layer {layer} step {s} ({n} positions): max abs {mabs:.2e} max rel {mrel:.2e}")
        assert ok, (layer, s, mabs, mrel)


def test_cache_past_the_32_bit_byte_offsets():
    """Maximum sizes: a head_dim-128 cache of 4,195,328 positions per kv head
    (2.15 GB per kv head and tensor, past what the lean prefill's 32-bit buffer
    ranges address, so prefill takes its global-load kernel, and kv head 1's rows
    start past 2^31 bytes).  A 200-token prefill at the start, then one decode
    token over 4,195,321 positions (the cache filled with a tiled block of 65,537
    random rows).  The prefill is checked against the oracle.  Over 4.2 million
    positions wick's own sequential f32 sums drift past the 2e-5 bar, so the
    decode is checked against f64 arithmetic instead, which the tiling makes
    cheap: each of the 65,537 distinct rows enters with its multiplicity."""
    heads, kvh, d = 4, 2, 128
    cap = 4195328
    L = cap - 7
    rng = np.random.default_rng(17)
    base_k = rng.standard_normal((65537, kvh * d), dtype=np.float32)
    base_v = rng.standard_normal((65537, kvh * d), dtype=np.float32)
    with DeviceKvCache(1, cap, kvh, d) as kv:
        qp, kp, vp = make_inputs(18, 200, 0, heads, kvh, d)
        kv.append(0, 0, kp, vp)
        got = kv.attention(0, heads, qp, 0)
        ok, mabs, mrel = within_tol(got, ol.attention(qp, kp, vp, 200, 0, heads, kvh, d))
        print(f"prefill t=200 at capacity {cap}: max abs {mabs:.2e} max rel {mrel:.2e}", flush=True)
        assert ok, (mabs, mrel)
        k = np.resize(base_k, (L, kvh * d))
        v = np.resize(base_v, (L, kvh * d))
        for c0 in range(0, L, 1 << 20):
            kv.append(0, c0, k[c0:c0 + (1 << 20)], v[c0:c0 + (1 << 20)])
        print(f"cache filled to {L} positions", flush=True)
        q = rng.standard_normal((1, heads * d), dtype=np.float32)
        got = kv.attention(0, heads, q, L - 1)
        kr, vr = kv.read(0, L - 3, 3)
        assert np.array_equal(kr, k[L - 3:]) and np.array_equal(vr, v[L - 3:])
    # f64 attention over the tiled cache: row r of the block appears mult[r] times
    P = base_k.shape[0]
    full, rem = divmod(L, P)
    mult = np.full(P, float(full))
    mult[:rem] += 1.0
    want = np.zeros((1, heads * d))
    for h in range(heads):
        j = h // (heads // kvh)
        kb = base_k[:, j * d:(j + 1) * d].astype(np.float64)
        vb = base_v[:, j * d:(j + 1) * d].astype(np.float64)
        sc = kb @ q[0, h * d:(h + 1) * d].astype(np.float64) * float(np.float32(1.0) / np.sqrt(np.float32(d)))
        w = mult * np.exp(sc - sc.max())
        want[0, h * d:(h + 1) * d] = (w @ vb) / w.sum()
    ok, mabs, mrel = within_tol(got, want)
    print(f"decode over {L} positions against f64: max abs {mabs:.2e} max rel {mrel:.2e}")
    ref = ol.attention(q, k, v, 1, L - 1, heads, kvh, d)
    print(f"  (the oracle's f32 sums against f64: max abs {np.abs(ref - want).max():.2e})")
    assert ok, (mabs, mrel)


@pytest.mark.parametrize("L", [1, 2, 15, 16, 17, 63, 64, 65, 129, 1000, 4097])
@pytest.mark.parametrize("d", [16, 32, 64, 128])
def test_decode_lengths_and_head_dims(L, d):
    q, k, v = make_inputs(L * 7 + d, 1, L - 1, 9, 3, d)
    check(q, k, v, 1, L - 1, 9, 3, d)


@pytest.mark.parametrize("L", [129, 160, 192])
@pytest.mark.parametrize("heads,kv_heads", [(40, 2), (9, 3), (14, 2)])
def test_decode_one_wide_chunk(L, heads, kv_heads):
    """129..192 positions at head_dim 64 run as one chunk per unit on an 8-wave
    workgroup (no merge pass)."""
    q, k, v = make_inputs(L + heads, 1, L - 1, heads, kv_heads, 64)
    check(q, k, v, 1, L - 1, heads, kv_heads, 64)


@pytest.mark.parametrize("chunk", [64, 128, 192, 256, 1024, 4096, 8192])
def test_decode_chunk_sizes(chunk):
    # chunk counts from 1 (no merge pass) up to 128
    L = 8191
    q, k, v = make_inputs(11, 1, L - 1, 14, 2, 64)
    check(q, k, v, 1, L - 1, 14, 2, 64, options=[(_native.OPT_DECODE_CHUNK, chunk)])


@pytest.mark.parametrize("d", [16, 32, 64, 128])
def test_decode_many_chunks_all_head_dims(d):
    # 256 chunks (the most one call uses) through the merge pass at every head_dim
    L = 16384
    q, k, v = make_inputs(d + 100, 1, L - 1, 12, 3, d)
    check(q, k, v, 1, L - 1, 12, 3, d, options=[(_native.OPT_DECODE_CHUNK, 64)])


@pytest.mark.parametrize("d", [64, 128])
def test_decode_merge_slot_counts(d):
    """The merge pass loads 16 x NB child slots (NB = 1, 2, 4, 8, 16: the fewest
    that cover the chunks).  Chunk counts at every edge of those sizes, largest
    first on one handle, so the workspace slots past each call's chunks hold
    the previous call's states: they must not leak into the result."""
    L_max = 64 * 256
    with DeviceKvCache(1, L_max, 2, d) as kv:
        kv.set_option(_native.OPT_DECODE_CHUNK, 64)
        q, k, v = make_inputs(300 + d, 1, L_max - 1, 14, 2, d)
        kv.append(0, 0, k, v)
        for n in (256, 255, 129, 128, 65, 64, 33, 32, 17, 16, 2):
            L = 64 * (n - 1) + 1 + (n % 7)  # n chunks, the last one ragged
            assert -(-L // 64) == n
            kk, vv = k[:L], v[:L]
            got = kv.attention(0, 14, q, L - 1)
            want = ol.attention(q, kk, vv, 1, L - 1, 14, 2, d)
            ok, mabs, mrel = within_tol(got, want)
            print(f"d={d} chunks={n} L={L}: max abs {mabs:.2e} max rel {mrel:.2e}")
            assert ok, (n, mabs, mrel)


def test_decode_repeated_launches_reuse_workspace():
    # the split-K workspace is shared by every call on a handle: many launches
    # in a row, alternating layers, must all be right
    L = 6000
    with DeviceKvCache(2, L, 2, 64) as kv:
        kv.set_option(_native.OPT_DECODE_CHUNK, 64)
        data = []
        for layer in range(2):
            q, k, v = make_inputs(40 + layer, 1, L - 1, 14, 2, 64)
            kv.append(layer, 0, k, v)
            data.append((q, ol.attention(q, k, v, 1, L - 1, 14, 2, 64)))
        first = [kv.attention(layer, 14, data[layer][0], L - 1) for layer in range(2)]
        for it in range(20):
            layer = it % 2
            got = kv.attention(layer, 14, data[layer][0], L - 1)
            assert np.array_equal(got, first[layer])
        for layer in range(2):
            assert within_tol(first[layer], data[layer][1])[0]


@pytest.mark.parametrize("heads,kv_heads", [(40, 2), (16, 1), (8, 8), (7, 7), (33, 1)])
def test_decode_group_sizes(heads, kv_heads):
    # group > 16 needs several 16-head slices per kv head
    L = 3000
    q, k, v = make_inputs(heads, 1, L - 1, heads, kv_heads, 64)
    check(q, k, v, 1, L - 1, heads, kv_heads, 64)


def test_decode_len1_is_v0_exactly():
    q, k, v = make_inputs(1, 1, 0, 14, 2, 64)
    got = run_gpu(q, k, v, 1, 0, 14, 2, 64).reshape(14, 64)
    for h in range(14):
        assert np.array_equal(got[h], v[0].reshape(2, 64)[h // 7])


def test_decode_bit_stable_and_capacity_larger_than_len():
    L = 20000
    q, k, v = make_inputs(4, 1, L - 1, 14, 2, 64)
    a = run_gpu(q, k, v, 1, L - 1, 14, 2, 64, capacity=L + 333)
    with DeviceKvCache(1, L + 333, 2, 64) as kv:
        kv.append(0, 0, k, v)
        outs = [kv.attention(0, 14, q, L - 1) for _ in range(3)]
    for o in outs:
        assert np.array_equal(o, a)
    want = ol.attention(q, k, v, 1, L - 1, 14, 2, 64)
    assert within_tol(a, want)[0]


# ---- prefill: config 3 (Qwen3 shape with QK-norm), config 4 (TinyLlama chunked), config 1 (SmolLM2)

@pytest.mark.parametrize("T", [512, 2048])
def test_prefill_qwen3_shape(T):
    q, k, v = make_inputs(3, T, 0, 16, 8, 128, theta=1e6, qk_norm=True)
    check(q, k, v, T, 0, 16, 8, 128)


def test_chunked_prefill_tinyllama_shape():
    """1536 cached positions, 512 appended: appended cache bit-exact, output within tolerance."""
    heads, kvh, d, S, t = 32, 4, 64, 1536, 512
    q, k, v = make_inputs(4, t, S, heads, kvh, d, theta=10000.0)
    with DeviceKvCache(2, S + t, kvh, d) as kv:
        kv.append(1, 0, k[:S], v[:S])
        kv.append(1, S, k[S:], v[S:])
        kr, vr = kv.read(1, 0, S + t)
        assert np.array_equal(kr, k) and np.array_equal(vr, v)
        got = kv.attention(1, heads, q, S)
    want = ol.attention(q, k, v, t, S, heads, kvh, d)
    ok, mabs, mrel = within_tol(got, want)
    assert ok, (mabs, mrel)


def test_prefill_smollm2_shape():
    q, k, v = make_inputs(1, 128, 0, 9, 3, 64, theta=10000.0)
    check(q, k, v, 128, 0, 9, 3, 64)


@pytest.mark.parametrize("t,start", [(2, 0), (3, 5), (5, 1), (7, 3), (13, 15), (15, 33), (17, 0), (33, 100), (100, 7)])
@pytest.mark.parametrize("d", [16, 32, 64, 128])
def test_prefill_ragged(t, start, d):
    q, k, v = make_inputs(t * 31 + start + d, t, start, 4, 2, d)
    check(q, k, v, t, start, 4, 2, d)


@pytest.mark.parametrize("heads,kv_heads", [(9, 3), (14, 2), (32, 4), (6, 6)])
def test_prefill_groups(heads, kv_heads):
    t, start = 300, 20
    q, k, v = make_inputs(heads + 1, t, start, heads, kv_heads, 64)
    check(q, k, v, t, start, heads, kv_heads, 64)


@pytest.mark.parametrize("d", [16, 32, 64, 128])
def test_prefill_on_a_prefix_all_head_dims(d):
    t, start = 77, 200
    q, k, v = make_inputs(d * 3 + 1, t, start, 8, 2, d)
    check(q, k, v, t, start, 8, 2, d)


@pytest.mark.parametrize("t,start,heads,kv_heads,d", [(1032, 37, 16, 8, 128), (516, 0, 32, 8, 128),
                                                      (777, 300, 24, 8, 128), (600, 200, 32, 4, 64),
                                                      (2050, 0, 9, 3, 64)])
def test_prefill_two_blocks_per_workgroup(t, start, heads, kv_heads, d):
    # Grids that still give each of the 256 CUs two workgroups with two 16-row blocks
    # per workgroup take that kernel (odd block counts leave the last pair half empty;
    # the head_dim-64 shapes are also resident at once, so heavy and light pairs mix).
    q, k, v = make_inputs(t + start + heads, t, start, heads, kv_heads, d)
    L = start + t
    with DeviceKvCache(1, L, kv_heads, d) as kv:
        kv.append(0, 0, k, v)
        got = kv.attention(0, heads, q, start)
        nblocks = (t * (heads // kv_heads) + 15) // 16
        assert kv.last_grid() == kv_heads * ((nblocks + 1) // 2), "two blocks per workgroup expected"
        again = kv.attention(0, heads, q, start)
    assert np.array_equal(got, again)
    want = ol.attention(q, k, v, t, start, heads, kv_heads, d)
    ok, mabs, mrel = within_tol(got, want)
    print(f"t={t} start={start} Hq={heads} Hkv={kv_heads}: max abs {mabs:.2e} max rel {mrel:.2e}")
    assert ok, f"max abs {mabs:.3e}, max rel {mrel:.3e}"


@pytest.mark.parametrize("T", [300, 700])
def test_prefill_bit_stable(T):
    # T=300: the whole grid resident at once (heavy and light blocks paired); T=700: not
    q, k, v = make_inputs(8, T, 0, 16, 8, 128)
    a = run_gpu(q, k, v, T, 0, 16, 8, 128)
    b = run_gpu(q, k, v, T, 0, 16, 8, 128)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("d", [64, 128])
def test_prefill_beyond_lean_range_takes_split_kernel(d):
    """A cache whose kv-head rows span more than a signed 32-bit byte range
    (capacity > (2^31 - 1) / (4 d), ~2.1 GB of K per kv head) is past the lean
    prefill kernel's buffer offsets; the launcher falls back to the split
    kernel, which must agree with the oracle as well."""
    cap = 0x7FFFFFFF // (4 * d) + 64
    t, start = 48, 16
    q, k, v = make_inputs(900 + d, t, start, 4, 1, d)
    check(q, k, v, t, start, 4, 1, d, capacity=cap)


def test_incremental_chunks_match_one_batch():
    """The tests/tiny_models.rs:73-95 property on the device cache: chunks vs one batch."""
    heads, kvh, d = 4, 2, 32
    sizes = [1, 5, 2, 7, 1, 1, 13, 3, 15]
    T = sum(sizes)
    q, k, v = make_inputs(12, T, 0, heads, kvh, d, theta=1e6)
    batch = run_gpu(q, k, v, T, 0, heads, kvh, d)
    with DeviceKvCache(1, 256, kvh, d) as kv:
        pos = 0
        for s in sizes:
            kv.append(0, pos, k[pos:pos + s], v[pos:pos + s])
            rows = kv.attention(0, heads, q[pos:pos + s], pos)
            assert np.abs(rows - batch[pos:pos + s]).max() < 1e-5
            pos += s


# ---- errors: checked on the host, nothing launched

def test_errors_are_reported():
    with DeviceKvCache(2, 64, 2, 64) as kv:
        with pytest.raises(_native.WickHipError) as e:
            kv.attention(0, 5, np.zeros((1, 5 * 64), np.float32), 0)
        assert e.value.code == _native.EINVAL and "multiple" in str(e.value)
        with pytest.raises(_native.WickHipError):
            kv.attention(0, 4, np.zeros((4, 4 * 64), np.float32), 61)
        with pytest.raises(_native.WickHipError):
            kv.attention(2, 4, np.zeros((1, 4 * 64), np.float32), 0)
        with pytest.raises(_native.WickHipError):
            kv.append(0, 60, np.zeros((5, 128), np.float32), np.zeros((5, 128), np.float32))
        with pytest.raises(_native.WickHipError):
            kv.set_option(_native.OPT_DECODE_CHUNK, 100)
        # device arrays move as float4: a pointer off a 16-byte boundary is refused
        import torch
        qd = torch.zeros(4 * 64 + 4, dtype=torch.float32, device="cuda")
        att = torch.zeros(4 * 64 + 4, dtype=torch.float32, device="cuda")
        with pytest.raises(_native.WickHipError) as e:
            kv.attention_device(0, 4, qd.data_ptr() + 4, 1, 0, att.data_ptr())
        assert e.value.code == _native.EINVAL and "aligned" in str(e.value)
        with pytest.raises(_native.WickHipError):
            kv.attention_device(0, 4, qd.data_ptr(), 1, 0, att.data_ptr() + 8)


def test_decode_hip_graph_replays_match_eager():
    """bench.py replays decode calls captured in a HIP graph: every replay, with
    eager work and synchronisations in between, must give the eager result bit
    for bit (the graph holds no memset nodes)."""
    import torch
    L, heads, kvh, d, layers = 9000, 14, 2, 64, 3
    dev = torch.device("cuda:0")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s), DeviceKvCache(layers, L, kvh, d) as kv:
        kv.set_stream(s.cuda_stream)
        qs = []
        for layer in range(layers):
            q, k, v = make_inputs(70 + layer, 1, L - 1, heads, kvh, d)
            kv.append(layer, 0, k, v)
            qs.append(q)
        qd = torch.tensor(np.concatenate(qs), device=dev)
        att = torch.zeros_like(qd)
        hd = heads * d

        def step():
            for layer in range(layers):
                kv.attention_device(layer, heads, qd.data_ptr() + 4 * hd * layer, 1, L - 1,
                                    att.data_ptr() + 4 * hd * layer)
        step()
        s.synchronize()
        eager = att.cpu().numpy().copy()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step()
        for it in range(4):
            att.zero_()
            g.replay()
            s.synchronize()
            assert np.array_equal(att.cpu().numpy(), eager), f"replay {it}"
            kv.attention(it % layers, heads, qs[it % layers], L - 1)  # eager work between replays
