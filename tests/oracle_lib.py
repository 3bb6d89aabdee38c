"""ctypes wrapper of oracle/liboracle.so -- the CPU checker (test infrastructure).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this.
"""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "oracle", "liboracle.so")
AVX2, SCALAR = 0, 1

_lib = None
_FP = ctypes.POINTER(ctypes.c_float)


class WoLayer(ctypes.Structure):
    _fields_ = [(n, _FP) for n in ("attn_norm", "wq", "wk", "wv", "wo", "bq", "bk", "bv", "q_norm", "k_norm",
                                    "ffn_norm", "w_gate", "w_up", "w_down")]


class WoModel(ctypes.Structure):
    _fields_ = [("hidden", ctypes.c_int), ("intermediate", ctypes.c_int), ("layers", ctypes.c_int),
                ("heads", ctypes.c_int), ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int),
                ("vocab", ctypes.c_int), ("rms_eps", ctypes.c_float), ("inv_freq", _FP), ("embed", _FP),
                ("lm_head", _FP), ("norm", _FP), ("layer", ctypes.POINTER(WoLayer))]


class WoSamplerConfig(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32), ("top_p", ctypes.c_float),
                ("min_p", ctypes.c_float), ("repetition_penalty", ctypes.c_float), ("seed", ctypes.c_uint64)]


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            import subprocess
            subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)
        lib = ctypes.CDLL(LIB)
        P = ctypes.c_void_p
        I = ctypes.c_int
        lib.wo_dot.restype = ctypes.c_float
        lib.wo_dot.argtypes = [P, P, I, I]
        lib.wo_softmax.argtypes = [P, I]
        lib.wo_rmsnorm.argtypes = [P, P, ctypes.c_float, P, I]
        lib.wo_rmsnorm_inplace.argtypes = [P, P, ctypes.c_float, I]
        lib.wo_rope.argtypes = [P, I, I, I, P]
        lib.wo_rope_inv_freq.argtypes = [ctypes.c_float, I, ctypes.c_float, ctypes.c_float, ctypes.c_float, I, P]
        lib.wo_attention.argtypes = [P, P, P, P, I, I, I, I, I, I, I]
        lib.wo_forward.restype = I
        lib.wo_forward.argtypes = [ctypes.POINTER(WoModel), P, P, I, ctypes.POINTER(I), P, I, I, P, I, I, P, P]
        lib.wo_argmax.restype = ctypes.c_uint32
        lib.wo_argmax.argtypes = [P, I]
        lib.wo_rng_seed.argtypes = [ctypes.c_uint64, P]
        lib.wo_rng_next_u64.restype = ctypes.c_uint64
        lib.wo_rng_next_u64.argtypes = [P]
        lib.wo_rng_next_f32.restype = ctypes.c_float
        lib.wo_rng_next_f32.argtypes = [P]
        lib.wo_sample.restype = ctypes.c_uint32
        lib.wo_sample.argtypes = [ctypes.POINTER(WoSamplerConfig), P, P, I, P, I, P, P, ctypes.POINTER(I),
                                  ctypes.POINTER(I)]
        _lib = lib
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def _c(a, dt=np.float32):
    return np.ascontiguousarray(a, dtype=dt)


def threads_default():
    return max(1, min(os.cpu_count() or 1, 16))


def dot(w, x, order=AVX2):
    w, x = _c(w), _c(x)
    return load().wo_dot(_p(w), _p(x), w.size, order)


def softmax(x):
    x = _c(x).copy()
    load().wo_softmax(_p(x), x.size)
    return x


def rmsnorm(x, w, eps):
    x, w = _c(x), _c(w)
    out = np.empty_like(x)
    load().wo_rmsnorm(_p(x), _p(w), eps, _p(out), x.size)
    return out


def rmsnorm_inplace(x, w, eps):
    """wo_rmsnorm_inplace (src/kernels.rs:351-357) on a copy of x."""
    x, w = _c(x).copy(), _c(w)
    load().wo_rmsnorm_inplace(_p(x), _p(w), eps, x.size)
    return x


def prep(q, k, v, heads, kv_heads, head_dim, start, inv_freq, bias=None, norms=None, eps=1e-6):
    """The per-token preparation of Model::forward (src/model.rs:464-480) on the CPU:
    bias add, per-head QK-norm, RoPE at positions start.. .  Returns new arrays."""
    q, k, v = _c(q).copy(), _c(k).copy(), _c(v).copy()
    d = head_dim
    for i in range(q.shape[0]):
        if bias is not None:
            q[i] += bias[0]
            k[i] += bias[1]
            v[i] += bias[2]
        if norms is not None:
            for h in range(heads):
                q[i, h * d:(h + 1) * d] = rmsnorm_inplace(q[i, h * d:(h + 1) * d], norms[0], eps)
            for h in range(kv_heads):
                k[i, h * d:(h + 1) * d] = rmsnorm_inplace(k[i, h * d:(h + 1) * d], norms[1], eps)
        q[i] = rope(q[i], d, start + i, inv_freq)
        k[i] = rope(k[i], d, start + i, inv_freq)
    return q, k, v


def rope(v, head_dim, pos, inv_freq):
    v = _c(v).copy()
    inv = _c(inv_freq)
    load().wo_rope(_p(v), v.size, head_dim, pos, _p(inv))
    return v


def rope_inv_freq(theta, head_dim, scaling=None):
    out = np.empty(head_dim // 2, np.float32)
    if scaling is None:
        load().wo_rope_inv_freq(theta, head_dim, 0.0, 0.0, 0.0, 0, _p(out))
    else:
        load().wo_rope_inv_freq(theta, head_dim, scaling.factor, scaling.low_freq_factor, scaling.high_freq_factor,
                                scaling.original_max_position, _p(out))
    return out


def attention(q, keys, values, t, start, heads, kv_heads, head_dim, order=AVX2, threads=None):
    """Model::attention restated: q [t][heads*d], keys/values [>=start+t][kv_heads*d] -> att."""
    q, keys, values = _c(q), _c(keys), _c(values)
    assert q.size == t * heads * head_dim
    assert keys.size >= (start + t) * kv_heads * head_dim and values.size == keys.size
    att = np.empty((t, heads * head_dim), np.float32)
    load().wo_attention(_p(q), _p(keys), _p(values), _p(att), t, start, heads, kv_heads, head_dim, order,
                        threads or threads_default())
    return att


def argmax(x):
    x = _c(x)
    return int(load().wo_argmax(_p(x), x.size))


class OracleModel:
    """f32 Model::forward restated (src/model.rs:420-516) over a host KvCache."""

    def __init__(self, cfg, weights, inv_freq=None):
        self.cfg = cfg
        self._keep = []
        inv = _c(inv_freq if inv_freq is not None else rope_inv_freq(cfg.rope_theta, cfg.head_dim, cfg.rope_scaling))
        self._keep.append(inv)

        def fp(a):
            if a is None:
                return None
            a = _c(a)
            self._keep.append(a)
            return a.ctypes.data_as(_FP)

        layers = (WoLayer * cfg.layers)()
        for i, lw in enumerate(weights["layers"]):
            for name, _ in WoLayer._fields_:
                setattr(layers[i], name, fp(lw[name]))
        self._layers = layers
        self.m = WoModel(cfg.hidden, cfg.intermediate, cfg.layers, cfg.heads, cfg.kv_heads, cfg.head_dim, cfg.vocab,
                         cfg.rms_eps, inv.ctypes.data_as(_FP), fp(weights["embed"]), fp(weights.get("lm_head")),
                         fp(weights["norm"]), layers)

    def new_state(self, capacity):
        c = self.cfg
        return {"k": np.zeros((c.layers, capacity, c.kv_dim), np.float32),
                "v": np.zeros((c.layers, capacity, c.kv_dim), np.float32), "len": 0, "capacity": capacity}

    def forward(self, state, tokens, all_logits=False, order=AVX2, threads=None, trace=False):
        c = self.cfg
        toks = _c(tokens, np.uint32)
        t = toks.size
        n = t if all_logits else 1
        logits = np.empty((n, c.vocab), np.float32)
        clen = ctypes.c_int(state["len"])
        qt = np.empty((c.layers, t, c.q_dim), np.float32) if trace else None
        at = np.empty((c.layers, t, c.q_dim), np.float32) if trace else None
        rc = load().wo_forward(ctypes.byref(self.m), _p(state["k"]), _p(state["v"]), state["capacity"],
                               ctypes.byref(clen), _p(toks), t, 1 if all_logits else 0, _p(logits), order,
                               threads or threads_default(), _p(qt), _p(at))
        if rc != 0:
            raise ValueError("context length exceeded")
        state["len"] = clen.value
        if trace:
            return logits, qt, at
        return logits


class OracleRng:
    """Rng (src/sampler.rs:29-60) restated."""

    def __init__(self, seed=None, state=None):
        self.s = (ctypes.c_uint64 * 4)()
        if state is not None:
            for i in range(4):
                self.s[i] = state[i]
        else:
            load().wo_rng_seed(seed, self.s)

    def state(self):
        return tuple(int(v) for v in self.s)

    def next_u64(self):
        return int(load().wo_rng_next_u64(self.s))

    def next_f32(self):
        return float(load().wo_rng_next_f32(self.s))


class OracleSampler:
    """Sampler::new + Sampler::sample (src/sampler.rs:62-127) restated; cfg is any
    object with SamplerConfig's fields."""

    def __init__(self, cfg):
        self.cfg = WoSamplerConfig(cfg.temperature, cfg.top_k, cfg.top_p, cfg.min_p, cfg.repetition_penalty,
                                   cfg.seed)
        self.rng = OracleRng(cfg.seed)

    def sample(self, logits, history=()):
        """logits: float32 array, penalised in place as wick's &mut [f32]."""
        return self.sample_detail(logits, history)[0]

    def sample_detail(self, logits, history=()):
        """(id, candidate ids [k], their probabilities [k], keep)."""
        assert logits.dtype == np.float32 and logits.flags.c_contiguous
        n = logits.size
        hist = _c(history, np.uint32)
        ids = np.empty(n, np.uint32)
        probs = np.empty(n, np.float32)
        k, keep = ctypes.c_int(), ctypes.c_int()
        tok = load().wo_sample(ctypes.byref(self.cfg), self.rng.s, _p(logits), n, _p(hist), hist.size, _p(ids),
                               _p(probs), ctypes.byref(k), ctypes.byref(keep))
        return int(tok), ids[:k.value].copy(), probs[:k.value].copy(), keep.value
