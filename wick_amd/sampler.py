"""ctypes wrapper of include/wick_hip_sampler.h: wick's sampler on the GPU.

SamplerConfig mirrors wick's (/root/reference/src/sampler.rs:3-27) with its
defaults; DeviceSampler is Sampler (:62-127) with the generator state and the
candidate scratch in device memory.
"""
import ctypes
from dataclasses import dataclass

import numpy as np

from . import _native


@dataclass
class SamplerConfig:
    """SamplerConfig (src/sampler.rs:3-20): temperature <= 0 is greedy, top_k 0 is
    the whole vocabulary, top_p >= 1 and min_p <= 0 are off."""
    temperature: float = 0.7
    top_k: int = 40
    top_p: float = 0.9
    min_p: float = 0.0
    repetition_penalty: float = 1.0
    seed: int = 0x5EED

    @classmethod
    def greedy(cls):
        """SamplerConfig::greedy (:23-26)."""
        return cls(temperature=0.0)


class _Config(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32), ("top_p", ctypes.c_float),
                ("min_p", ctypes.c_float), ("repetition_penalty", ctypes.c_float), ("seed", ctypes.c_uint64)]


def c_config(cfg):
    if cfg.top_k < 0:
        raise ValueError("top_k must be >= 0")
    return _Config(cfg.temperature, cfg.top_k, cfg.top_p, cfg.min_p, cfg.repetition_penalty, cfg.seed)


class DeviceSampler:
    """Sampler::new for logits of `vocab` entries; launches on `stream` (a
    hipStream_t as an int; None = the default stream), or adopt a handle made
    by wick_hip_model_new_sampler."""

    def __init__(self, cfg, vocab, stream=None, handle=None):
        self._lib = _native.load()
        self.cfg = cfg
        self.vocab = vocab
        if handle is None:
            h = ctypes.c_void_p()
            c = c_config(cfg)
            _native.check(self._lib.wick_hip_sampler_create(ctypes.byref(c), vocab, stream, ctypes.byref(h)))
            handle = h
        self.handle = handle

    def close(self):
        if getattr(self, "handle", None):
            self._lib.wick_hip_sampler_destroy(self.handle)
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

    def sample(self, logits, history=()):
        """Sampler::sample on a host float32 array [vocab], penalised in place like
        wick's &mut [f32]; returns the drawn id."""
        if not (isinstance(logits, np.ndarray) and logits.dtype == np.float32 and logits.flags.c_contiguous
                and logits.flags.writeable):
            raise TypeError("logits must be a writeable C-contiguous float32 array")
        if logits.size != self.vocab:
            raise ValueError(f"logits has {logits.size} entries, the sampler {self.vocab}")
        hist = np.ascontiguousarray(history, dtype=np.uint32).reshape(-1)
        out = ctypes.c_uint32()
        _native.check(self._lib.wick_hip_sampler_sample(self.handle, logits.ctypes.data, hist.ctypes.data, hist.size,
                                                        ctypes.byref(out)))
        return int(out.value)

    def sample_device(self, logits_ptr, history_ptr, n_history, out_ptr):
        """The same on device pointers, asynchronous on the sampler's stream."""
        _native.check(self._lib.wick_hip_sampler_sample_device(self.handle, logits_ptr, history_ptr, n_history,
                                                               out_ptr))

    def rng_state(self):
        st = (ctypes.c_uint64 * 4)()
        _native.check(self._lib.wick_hip_sampler_rng_state(self.handle, st))
        return tuple(int(v) for v in st)

    def last_candidates(self):
        """(candidate ids [k], probabilities [k], keep) of the last sampling draw."""
        k, keep = ctypes.c_int(), ctypes.c_int()
        _native.check(self._lib.wick_hip_sampler_last_candidates(self.handle, ctypes.byref(k), ctypes.byref(keep),
                                                                 None, None, 0))
        ids = np.empty(k.value, np.uint32)
        probs = np.empty(k.value, np.float32)
        _native.check(self._lib.wick_hip_sampler_last_candidates(self.handle, ctypes.byref(k), ctypes.byref(keep),
                                                                 ids.ctypes.data, probs.ctypes.data, ids.size))
        return ids, probs, keep.value
