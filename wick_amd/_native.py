"""ctypes bindings of the C ABI in include/wick_hip.h, wick_hip_model.h and wick_hip_sampler.h.

This is the binding a host program writes for the library (the Rust side would
declare the same symbols in an `extern "C"` block).  There is no fallback: if
the shared library is missing, loading fails loudly.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
HIP_LIB = os.path.join(_HERE, "libwick_hip.so")

OK = 0
EINVAL = -1
EHIP = -2
ENOMEM = -3
EDEVICE = -4

OPT_DECODE_CHUNK = 1
OPT_DECODE_ORDER = 2

# Every symbol include/*.h declares, with its ctypes signature.
_P = ctypes.c_void_p
_I = ctypes.c_int
_FP = ctypes.POINTER(ctypes.c_float)
SIGNATURES = {
    "wick_hip_kv_create": (_I, [_I, _I, _I, _I, ctypes.POINTER(_P)]),
    "wick_hip_kv_destroy": (None, [_P]),
    "wick_hip_kv_append": (_I, [_P, _I, _I, _I, _P, _P]),
    "wick_hip_kv_read": (_I, [_P, _I, _I, _I, _P, _P]),
    "wick_hip_attention": (_I, [_P, _I, _I, _P, _I, _I, _P]),
    "wick_hip_last_error": (ctypes.c_char_p, []),
    "wick_hip_kv_append_device": (_I, [_P, _I, _I, _I, _P, _P]),
    "wick_hip_attention_device": (_I, [_P, _I, _I, _P, _I, _I, _P]),
    "wick_hip_attention_device_noalloc": (_I, [_P, _I, _I, _P, _I, _I, _P]),
    "wick_hip_kv_set_stream": (_I, [_P, _P]),
    "wick_hip_kv_synchronize": (_I, [_P]),
    "wick_hip_kv_set_option": (_I, [_P, _I, _I]),
    "wick_hip_kv_last_grid": (_I, [_P]),
    "wick_hip_kv_scratch_bytes": (ctypes.c_longlong, [_P]),
    "wick_hip_kv_set_rope": (_I, [_P, _P]),
    "wick_hip_kv_set_prep": (_I, [_P, _I, _I, _P, _P, _P, _P, _P, ctypes.c_float]),
    "wick_hip_attend": (_I, [_P, _I, _I, _P, _P, _P, _I, _I, _P]),
    "wick_hip_attend_device": (_I, [_P, _I, _I, _P, _P, _P, _I, _I, _P]),
    # wick_hip_model.h
    "wick_hip_model_create": (_I, [_P, _P, _P, _P, _P, _P, ctypes.POINTER(_P)]),
    "wick_hip_model_destroy": (None, [_P]),
    "wick_hip_model_new_cache": (_I, [_P, _I, ctypes.POINTER(_P)]),
    "wick_hip_model_forward": (_I, [_P, _P, _P, _I, _I, _I, _P]),
    "wick_hip_model_prefill": (_I, [_P, _P, _P, _I, _I, _P]),
    "wick_hip_model_decode": (_I, [_P, _P, ctypes.c_uint32, _I, _I, _P]),
    "wick_hip_model_new_sampler": (_I, [_P, _P, ctypes.POINTER(_P)]),
    "wick_hip_model_generate": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _I, _P, _P, _P]),
    # wick_hip_sampler.h
    "wick_hip_sampler_create": (_I, [_P, _I, _P, ctypes.POINTER(_P)]),
    "wick_hip_sampler_destroy": (None, [_P]),
    "wick_hip_sampler_sample_device": (_I, [_P, _P, _P, _I, _P]),
    "wick_hip_sampler_sample": (_I, [_P, _P, _P, _I, _P]),
    "wick_hip_sampler_rng_state": (_I, [_P, _P]),
    "wick_hip_sampler_last_candidates": (_I, [_P, _P, _P, _P, _P, _I]),
}

_lib = None


class WickHipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"wick_hip error {code}: {msg}")
        self.code = code


def load():
    """Load libwick_hip.so (built in-tree by __graft_entry__.build())."""
    global _lib
    if _lib is None:
        if not os.path.exists(HIP_LIB):
            raise RuntimeError(f"{HIP_LIB} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
        lib = ctypes.CDLL(HIP_LIB)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def check(rc):
    if rc != OK:
        msg = load().wick_hip_last_error().decode(errors="replace")
        raise WickHipError(rc, msg)
    return rc
