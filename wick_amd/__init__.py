"""MI355X-native attention hot path for wick (causal GQA over a device KV cache).

The product is the C ABI in include/wick_hip.h, implemented by HIP kernels for
gfx950 in wick_amd/csrc and built into wick_amd/libwick_hip.so.  This package
holds the ctypes binding of that ABI and the build step.
"""
from . import _native  # noqa: F401
from .kv import DeviceKvCache  # noqa: F401
