"""wick_hip_attention_device_noalloc, the entry point that allocates nothing.

Its decode keeps the split-K partial states in a static per-GPU device array
instead of the handle's workspace; everything else is wick_hip_attention_device.
Each case calls both entry points through the C ABI on the same device inputs
and requires bit-identical outputs (the same kernels run), and checks the
result against the CPU oracle (2e-5 + 1e-4*|ref|).  Calls come in a row, the
later ones smaller, so that states a previous call left in the shared array
would show up if a merge read them.
"""
import numpy as np
import pytest

import oracle_lib as ol
from util import inv_freq, rope_np, within_tol
from wick_amd import DeviceKvCache, _native

pytestmark = pytest.mark.gpu


def _inputs(seed, t, L, heads, kv_heads, d, theta):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((t, heads * d), dtype=np.float32)
    k = rng.standard_normal((L, kv_heads * d), dtype=np.float32)
    v = rng.standard_normal((L, kv_heads * d), dtype=np.float32)
    inv = inv_freq(theta, d)
    return rope_np(q, heads, d, np.arange(L - t, L), inv), rope_np(k, kv_heads, d, np.arange(L), inv), v


def _both(kv, heads, q, t, start):
    """(wick_hip_attention_device, wick_hip_attention_device_noalloc) outputs for q."""
    import torch
    qd = torch.from_numpy(q).cuda()
    a = torch.full_like(qd, float("nan"))
    b = torch.full_like(qd, float("nan"))
    torch.cuda.synchronize()
    kv.attention_device(0, heads, qd.data_ptr(), t, start, a.data_ptr())
    kv.attention_device_noalloc(0, heads, qd.data_ptr(), t, start, b.data_ptr())
    kv.synchronize()
    return a.cpu().numpy(), b.cpu().numpy()


def _check(name, kv, q, k, v, t, L, heads, kv_heads, d):
    start = L - t
    got_ref, got = _both(kv, heads, q, t, start)
    assert np.array_equal(got.view(np.uint32), got_ref.view(np.uint32)), f"{name}: outputs differ in bits"
    want = ol.attention(q, k[:L], v[:L], t, start, heads, kv_heads, d)
    ok, mabs, mrel = within_tol(got, want)
    print(f"{name}: t={t} L={L} Hq={heads} Hkv={kv_heads} d={d} grid={kv.last_grid()} "
          f"max abs {mabs:.2e} max rel {mrel:.2e}", flush=True)
    assert ok, f"{name}: max abs {mabs:.3e}, max rel {mrel:.3e}"


def test_noalloc_matches_the_allocating_entry_point_on_calls_in_a_row():
    # 1) Llama-3-8B shape (8 kv heads, d 128): 8 units, the largest footprint here
    heads, kv_heads, d, L = 32, 8, 128, 8192
    q, k, v = _inputs(5, 1, L, heads, kv_heads, d, 500000.0)
    with DeviceKvCache(1, L, kv_heads, d) as kv:
        kv.append(0, 0, k, v)
        _check("llama3-8b 8192", kv, q, k, v, 1, L, heads, kv_heads, d)
    # 2) Qwen2.5 shape at 32K (256 chunks per unit), then the same handle at
    #    shorter contexts: fewer chunks and fewer units' worth of states read
    heads, kv_heads, d, L = 14, 2, 64, 32768
    q, k, v = _inputs(2, 1, L, heads, kv_heads, d, 1e6)
    with DeviceKvCache(1, L, kv_heads, d) as kv:
        kv.append(0, 0, k, v)
        _check("qwen2.5 32768", kv, q, k, v, 1, L, heads, kv_heads, d)
        for Ls in (4096, 1000, 100):
            qs = _inputs(Ls, 1, Ls, heads, kv_heads, d, 1e6)[0]
            _check(f"qwen2.5 {Ls}", kv, qs, k, v, 1, Ls, heads, kv_heads, d)


def test_noalloc_first_on_a_fresh_handle_allocates_nothing():
    """The no-allocation entry point called first on a fresh handle, its inputs
    appended from device arrays (no staging): the handle's staging and workspace
    stay empty and the GPU's free memory unchanged over decode calls at 32K, 4096
    and 100 positions and a 100-token chunk.  The allocating entry point on the
    same handle afterwards grows its workspace and gives the same bits."""
    import torch
    heads, kv_heads, d, L = 14, 2, 64, 32768
    q, k, v = _inputs(12, 1, L, heads, kv_heads, d, 1e6)
    qc = _inputs(13, 100, 300, heads, kv_heads, d, 1e6)[0]
    kd, vd = torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda()
    qd, qcd = torch.from_numpy(q).cuda(), torch.from_numpy(qc).cuda()
    att = torch.full_like(qd, float("nan"))
    attc = torch.full_like(qcd, float("nan"))
    # one stream for everything, first used by another handle running the same
    # kernels, so the runtime's lazily created per-stream and per-kernel state
    # exists before the free memory is read
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with DeviceKvCache(1, L, kv_heads, d) as warm:
        warm.set_stream(stream.cuda_stream)
        warm.append_device(0, 0, L, kd.data_ptr(), vd.data_ptr())
        for Ls in (L, 4096, 100):
            warm.attention_device_noalloc(0, heads, qd.data_ptr(), 1, Ls - 1, att.data_ptr())
        warm.attention_device_noalloc(0, heads, qcd.data_ptr(), 100, 200, attc.data_ptr())
        warm.synchronize()
    with DeviceKvCache(1, L, kv_heads, d) as kv:
        kv.set_stream(stream.cuda_stream)
        kv.append_device(0, 0, L, kd.data_ptr(), vd.data_ptr())
        kv.synchronize()
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        assert kv.scratch_bytes() == 0
        outs = {}
        for Ls in (L, 4096, 100):
            kv.attention_device_noalloc(0, heads, qd.data_ptr(), 1, Ls - 1, att.data_ptr())
            kv.synchronize()
            outs[Ls] = att.cpu().numpy()
        kv.attention_device_noalloc(0, heads, qcd.data_ptr(), 100, 200, attc.data_ptr())
        kv.synchronize()
        outc = attc.cpu().numpy()
        assert kv.scratch_bytes() == 0, "the no-allocation entry point grew the handle's buffers"
        assert torch.cuda.mem_get_info()[0] == free0, "device memory was allocated"
        for Ls, got in outs.items():
            want = ol.attention(q, k[:Ls], v[:Ls], 1, Ls - 1, heads, kv_heads, d)
            ok, mabs, mrel = within_tol(got, want)
            print(f"fresh handle, no-alloc first: L={Ls} max abs {mabs:.2e} max rel {mrel:.2e}", flush=True)
            assert ok, (Ls, mabs, mrel)
        wantc = ol.attention(qc, k[:300], v[:300], 100, 200, heads, kv_heads, d)
        assert within_tol(outc, wantc)[0]
        ref = torch.full_like(qd, float("nan"))
        kv.attention_device(0, heads, qd.data_ptr(), 1, L - 1, ref.data_ptr())
        kv.synchronize()
        assert kv.scratch_bytes() > 0
        assert np.array_equal(ref.cpu().numpy().view(np.uint32), outs[L].view(np.uint32))


def test_noalloc_prefill_uses_no_workspace_and_matches():
    heads, kv_heads, d, t, L = 32, 4, 64, 100, 300
    q, k, v = _inputs(4, t, L, heads, kv_heads, d, 10000.0)
    with DeviceKvCache(1, L, kv_heads, d) as kv:
        kv.append(0, 0, k, v)
        _check("tinyllama chunk", kv, q, k, v, t, L, heads, kv_heads, d)


def test_noalloc_rejects_a_shape_beyond_the_static_workspace():
    import torch
    heads, kv_heads, d, L = 64, 64, 128, 64  # 64 units x 16 x 256 x 130 floats > 8 Mi
    with DeviceKvCache(1, L, kv_heads, d) as kv:
        q = torch.zeros(heads * d, device="cuda")
        att = torch.zeros_like(q)
        torch.cuda.synchronize()
        with pytest.raises(_native.WickHipError, match="static workspace"):
            kv.attention_device_noalloc(0, heads, q.data_ptr(), 1, L - 1, att.data_ptr())
        # the allocating entry point still serves the shape
        kv.attention_device(0, heads, q.data_ptr(), 1, L - 1, att.data_ptr())
        kv.synchronize()
