"""ctypes binding of the C++ host mirror (wick_amd/host/wick_host.h).

HostModel mirrors wick's Model (/root/reference/src/model.rs:152-249) for f32
weights and HostState its State (:294-302); forward() is Model::forward
(:420-516) with the KV cache and attention on the GPU through the C ABI.
"""
import ctypes
import os

import numpy as np

from . import _native
from .model import LAYER_TENSORS

_HERE = os.path.dirname(os.path.abspath(__file__))
HOST_LIB = os.path.join(_HERE, "libwick_host.so")
_lib = None


class HostConfig(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("intermediate", ctypes.c_int), ("layers", ctypes.c_int),
                ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("vocab", ctypes.c_int), ("rms_eps", ctypes.c_float)]


def load():
    global _lib
    if _lib is None:
        _native.load()  # libwick_hip.so first: libwick_host.so links it
        if not os.path.exists(HOST_LIB):
            raise RuntimeError(f"{HOST_LIB} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
        lib = ctypes.CDLL(HOST_LIB)
        P, I = ctypes.c_void_p, ctypes.c_int
        lib.wick_host_model_create.restype = P
        lib.wick_host_model_create.argtypes = [ctypes.POINTER(HostConfig), P, P, P, P, ctypes.POINTER(P), I]
        lib.wick_host_model_destroy.argtypes = [P]
        lib.wick_host_state_create.restype = P
        lib.wick_host_state_create.argtypes = [P, I]
        lib.wick_host_state_destroy.argtypes = [P]
        lib.wick_host_state_len.restype = I
        lib.wick_host_state_len.argtypes = [P]
        lib.wick_host_state_set_len.restype = I
        lib.wick_host_state_set_len.argtypes = [P, I]
        lib.wick_host_state_kv.restype = P
        lib.wick_host_state_kv.argtypes = [P]
        lib.wick_host_forward.restype = I
        lib.wick_host_forward.argtypes = [P, P, P, I, I, P, P]
        lib.wick_host_last_error.restype = ctypes.c_char_p
        _lib = lib
    return _lib


def _err(what):
    raise RuntimeError(f"{what}: {load().wick_host_last_error().decode(errors='replace')}")


class HostModel:
    def __init__(self, cfg, weights, threads=None):
        lib = load()
        self.cfg = cfg
        self._keep = []

        def ptr(a):
            if a is None:
                return None
            a = np.ascontiguousarray(a, dtype=np.float32)
            self._keep.append(a)
            return a.ctypes.data

        inv = ptr(cfg.rope_inv_freq())
        tensors = (ctypes.c_void_p * (cfg.layers * len(LAYER_TENSORS)))()
        for i, lw in enumerate(weights["layers"]):
            for j, name in enumerate(LAYER_TENSORS):
                tensors[i * len(LAYER_TENSORS) + j] = ptr(lw[name])
        hc = HostConfig(cfg.hidden, cfg.intermediate, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.vocab,
                        cfg.rms_eps)
        threads = threads or min(os.cpu_count() or 1, 64)
        h = lib.wick_host_model_create(ctypes.byref(hc), inv, ptr(weights["embed"]), ptr(weights.get("lm_head")),
                                       ptr(weights["norm"]), tensors, threads)
        if not h:
            _err("wick_host_model_create")
        self.handle = h

    def close(self):
        if getattr(self, "handle", None):
            load().wick_host_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def new_state(self, capacity):
        return HostState(self, capacity)

    def forward(self, state, tokens, all_logits=False, trace=False):
        c = self.cfg
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        t = toks.size
        logits = np.empty((t if all_logits else 1, c.vocab), np.float32)
        at = np.empty((c.layers, t, c.q_dim), np.float32) if trace else None
        rc = load().wick_host_forward(self.handle, state.handle, toks.ctypes.data, t, 1 if all_logits else 0,
                                      logits.ctypes.data, at.ctypes.data if trace else None)
        if rc != 0:
            _err("wick_host_forward")
        return (logits, at) if trace else logits


class HostState:
    def __init__(self, model, capacity):
        h = load().wick_host_state_create(model.handle, capacity)
        if not h:
            _err("wick_host_state_create")
        self.handle = h
        self.capacity = capacity

    @property
    def len(self):
        return load().wick_host_state_len(self.handle)

    @len.setter
    def len(self, n):
        if load().wick_host_state_set_len(self.handle, n) != 0:
            raise ValueError(f"bad cache length {n}")

    def close(self):
        if getattr(self, "handle", None):
            load().wick_host_state_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
