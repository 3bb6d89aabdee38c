"""ctypes wrapper of include/wick_hip_model.h: wick's Model::forward resident on the GPU.

DeviceModel mirrors wick's Model (/root/reference/src/model.rs:152-249) for f32
weights; new_cache() is State::new (:300-302); forward() is Model::forward
(:420-516); prefill() / decode() are Session::prefill (src/engine.rs:120-139)
and the greedy loop of cmd_bench (src/main.rs:223-258) with sampler::argmax
(src/sampler.rs:129-137) on the device; new_sampler() / generate() are
Sampler::new (src/sampler.rs:67-71) and the token loop of Session::generate
(src/engine.rs:164-204) with the sampler on the device.
"""
import ctypes

import numpy as np

from . import _native
from .kv import DeviceKvCache
from .model import LAYER_TENSORS
from .sampler import DeviceSampler, c_config


class ModelConfig(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("intermediate", ctypes.c_int), ("layers", ctypes.c_int),
                ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("vocab", ctypes.c_int), ("rms_eps", ctypes.c_float)]


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


class DeviceModel:
    """Weights copied to HBM once; every forward runs on the model's stream."""

    def __init__(self, cfg, weights):
        lib = _native.load()
        self._lib = lib
        self.cfg = cfg
        keep = []

        def ptr(a):
            a = _f32(a)
            if a is None:
                return None
            keep.append(a)
            return a.ctypes.data

        tensors = (ctypes.c_void_p * (cfg.layers * len(LAYER_TENSORS)))()
        for i, lw in enumerate(weights["layers"]):
            for j, name in enumerate(LAYER_TENSORS):
                tensors[i * len(LAYER_TENSORS) + j] = ptr(lw[name])
        mc = ModelConfig(cfg.hidden, cfg.intermediate, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.vocab,
                         cfg.rms_eps)
        h = ctypes.c_void_p()
        _native.check(lib.wick_hip_model_create(ctypes.byref(mc), ptr(cfg.rope_inv_freq()), ptr(weights["embed"]),
                                                ptr(weights.get("lm_head")), ptr(weights["norm"]), tensors,
                                                ctypes.byref(h)))
        self.handle = h  # the host copies in `keep` may go: the library copied them

    def close(self):
        if getattr(self, "handle", None):
            self._lib.wick_hip_model_destroy(self.handle)
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

    def new_cache(self, capacity):
        """State::new: a device KV cache for this model (len tracks KvCache::len)."""
        h = ctypes.c_void_p()
        _native.check(self._lib.wick_hip_model_new_cache(self.handle, capacity, ctypes.byref(h)))
        c = self.cfg
        return DeviceKvCache.adopt(h, c.layers, capacity, c.kv_heads, c.head_dim)

    def forward(self, cache, tokens, all_logits=False):
        """Model::forward: tokens at positions cache.len..; returns logits [1 or t][vocab]."""
        toks = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        t = toks.size
        out = np.empty((t if all_logits else 1, self.cfg.vocab), np.float32)
        _native.check(self._lib.wick_hip_model_forward(self.handle, cache.handle, toks.ctypes.data, t, cache.len,
                                                       1 if all_logits else 0, out.ctypes.data))
        cache.len += t
        return out

    def prefill(self, cache, prompt):
        """The prompt in 256-token chunks at cache.len..; returns the greedy next id."""
        toks = np.ascontiguousarray(prompt, dtype=np.uint32).reshape(-1)
        nxt = ctypes.c_uint32()
        _native.check(self._lib.wick_hip_model_prefill(self.handle, cache.handle, toks.ctypes.data, toks.size,
                                                       cache.len, ctypes.byref(nxt)))
        cache.len += toks.size
        return int(nxt.value)

    def decode(self, cache, first, steps):
        """`steps` greedy single-token forwards from token `first`; returns the ids [steps]."""
        out = np.empty(steps, np.uint32)
        _native.check(self._lib.wick_hip_model_decode(self.handle, cache.handle, int(first), cache.len, steps,
                                                      out.ctypes.data))
        cache.len += steps
        return [int(i) for i in out]

    def new_sampler(self, cfg):
        """Sampler::new for this model's vocabulary, on the model's stream."""
        h = ctypes.c_void_p()
        c = c_config(cfg)
        _native.check(self._lib.wick_hip_model_new_sampler(self.handle, ctypes.byref(c), ctypes.byref(h)))
        return DeviceSampler(cfg, self.cfg.vocab, handle=h)

    def generate(self, cache, sampler, tokens, max_tokens, stops=()):
        """Session::generate's token loop: tokens is the session's whole token list, of
        which the cache holds the first cache.len; returns the drawn ids (a stop id
        ends the list and is not included).  cache.len is updated to what the cache
        holds afterwards."""
        toks = np.ascontiguousarray(tokens, dtype=np.uint32).reshape(-1)
        st = np.ascontiguousarray(list(stops), dtype=np.uint32).reshape(-1)
        out = np.empty(max(int(max_tokens), 1), np.uint32)
        n_out, clen = ctypes.c_int(), ctypes.c_int()
        _native.check(self._lib.wick_hip_model_generate(self.handle, cache.handle, sampler.handle, toks.ctypes.data,
                                                        toks.size, cache.len, int(max_tokens), st.ctypes.data, st.size,
                                                        out.ctypes.data, ctypes.byref(n_out), ctypes.byref(clen)))
        cache.len = clen.value
        return [int(i) for i in out[:n_out.value]]
