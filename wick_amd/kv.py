"""Host-side handle of the device-resident KV cache and the attention entry points.

Mirrors, over the C ABI, what wick's Rust code holds and calls:
  KvCache       /root/reference/src/model.rs:251-275 (now [layer][kv_head][pos][head_dim] in HBM)
  cache append  /root/reference/src/model.rs:481-483
  attention     /root/reference/src/model.rs:518-553 (called per layer at :485)
  input prep    /root/reference/src/model.rs:464-484 (bias, QK-norm, RoPE, append) via attend()
"""
import ctypes

import numpy as np

from . import _native


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class DeviceKvCache:
    """K and V for `layers` layers of `capacity` positions on the current GPU."""

    def __init__(self, layers, capacity, kv_heads, head_dim):
        lib = _native.load()
        h = ctypes.c_void_p()
        _native.check(lib.wick_hip_kv_create(layers, capacity, kv_heads, head_dim, ctypes.byref(h)))
        self._lib = lib
        self.handle = h
        self.layers, self.capacity, self.kv_heads, self.head_dim = layers, capacity, kv_heads, head_dim
        self.kv_dim = kv_heads * head_dim
        # wick's KvCache::len: positions already processed (src/model.rs:256)
        self.len = 0

    @classmethod
    def adopt(cls, handle, layers, capacity, kv_heads, head_dim):
        """Wrap a handle made by the library (e.g. wick_hip_model_new_cache); destroyed on close."""
        self = cls.__new__(cls)
        self._lib = _native.load()
        self.handle = handle
        self.layers, self.capacity, self.kv_heads, self.head_dim = layers, capacity, kv_heads, head_dim
        self.kv_dim = kv_heads * head_dim
        self.len = 0
        return self

    def close(self):
        if self.handle:
            self._lib.wick_hip_kv_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # ---- host-array entry points (synchronous)
    def append(self, layer, start, k, v):
        """Write rows k, v ([t][kv_heads*head_dim]) at positions start.. of `layer`."""
        k, v = _f32(k).reshape(-1, self.kv_dim), _f32(v).reshape(-1, self.kv_dim)
        assert k.shape == v.shape
        _native.check(self._lib.wick_hip_kv_append(self.handle, layer, start, k.shape[0], _ptr(k), _ptr(v)))

    def read(self, layer, pos0, n):
        """Positions pos0..pos0+n of `layer` in wick's layout [n][kv_heads*head_dim]."""
        k = np.empty((n, self.kv_dim), np.float32)
        v = np.empty((n, self.kv_dim), np.float32)
        _native.check(self._lib.wick_hip_kv_read(self.handle, layer, pos0, n, _ptr(k), _ptr(v)))
        return k, v

    def attention(self, layer, heads, q, start):
        """Model::attention for the t rows of q ([t][heads*head_dim]) at positions start..start+t."""
        q = _f32(q).reshape(-1, heads * self.head_dim)
        att = np.empty_like(q)
        _native.check(self._lib.wick_hip_attention(self.handle, layer, heads, _ptr(q), q.shape[0], start, _ptr(att)))
        return att

    def set_rope(self, inv_freq):
        """RoPE table for attend(): inv_freq [head_dim/2] as Config::rope_inv_freq gives it."""
        f = _f32(inv_freq).reshape(-1)
        assert f.size == self.head_dim // 2
        _native.check(self._lib.wick_hip_kv_set_rope(self.handle, _ptr(f)))

    def set_prep(self, layer, heads, bq=None, bk=None, bv=None, q_norm=None, k_norm=None, eps=1e-6):
        """Per-layer bias / QK-norm constants for attend() (None = absent)."""
        arrs = [None if a is None else _f32(a).reshape(-1) for a in (bq, bk, bv, q_norm, k_norm)]
        ptrs = [None if a is None else _ptr(a) for a in arrs]
        _native.check(self._lib.wick_hip_kv_set_prep(self.handle, layer, heads, *ptrs, ctypes.c_float(eps)))

    def attend(self, layer, heads, q, k, v, start):
        """src/model.rs:464-485 for one layer: raw projections q, k, v of t tokens in,
        attention output out; k and v are prepared and appended at start.."""
        q = _f32(q).reshape(-1, heads * self.head_dim)
        k, v = _f32(k).reshape(-1, self.kv_dim), _f32(v).reshape(-1, self.kv_dim)
        assert k.shape[0] == q.shape[0] and v.shape == k.shape
        att = np.empty_like(q)
        _native.check(self._lib.wick_hip_attend(self.handle, layer, heads, _ptr(q), _ptr(k), _ptr(v), q.shape[0],
                                                start, _ptr(att)))
        return att

    # ---- device-pointer entry points (asynchronous on the handle's stream)
    def attend_device(self, layer, heads, q_ptr, k_ptr, v_ptr, t, start, att_ptr):
        _native.check(self._lib.wick_hip_attend_device(self.handle, layer, heads, ctypes.c_void_p(q_ptr),
                                                       ctypes.c_void_p(k_ptr), ctypes.c_void_p(v_ptr), t, start,
                                                       ctypes.c_void_p(att_ptr)))

    def append_device(self, layer, start, t, k_ptr, v_ptr):
        _native.check(self._lib.wick_hip_kv_append_device(self.handle, layer, start, t, ctypes.c_void_p(k_ptr),
                                                          ctypes.c_void_p(v_ptr)))

    def attention_device(self, layer, heads, q_ptr, t, start, att_ptr):
        _native.check(self._lib.wick_hip_attention_device(self.handle, layer, heads, ctypes.c_void_p(q_ptr), t, start,
                                                          ctypes.c_void_p(att_ptr)))

    def attention_device_noalloc(self, layer, heads, q_ptr, t, start, att_ptr):
        """attention_device through the entry point that allocates nothing (its
        decode workspace is a static per-GPU array shared by every such call)."""
        _native.check(self._lib.wick_hip_attention_device_noalloc(self.handle, layer, heads, ctypes.c_void_p(q_ptr), t,
                                                                  start, ctypes.c_void_p(att_ptr)))

    def set_stream(self, stream_ptr):
        _native.check(self._lib.wick_hip_kv_set_stream(self.handle, ctypes.c_void_p(stream_ptr)))

    def synchronize(self):
        _native.check(self._lib.wick_hip_kv_synchronize(self.handle))

    def set_option(self, option, value):
        _native.check(self._lib.wick_hip_kv_set_option(self.handle, option, value))

    def last_grid(self):
        return self._lib.wick_hip_kv_last_grid(self.handle)

    def scratch_bytes(self):
        """Staging and decode workspace bytes the handle has allocated so far."""
        return int(self._lib.wick_hip_kv_scratch_bytes(self.handle))
