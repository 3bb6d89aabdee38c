"""libwick_probe.so's wick_synth_normal (bench.py's inputs) against a Python
restatement: row r of tensor t is Rng::new(seed) advanced by t long jumps and r
jumps, turned into normals by Box-Muller in double (u1 = ((a >> 11) + 1) / 2^53,
u2 = (b >> 11) / 2^53, x0 = sqrt(-2 ln u1) cos(2 pi u2), x1 = ... sin(...)),
times the scale, rounded to f32.  The device's double log / cos / sin may
differ from the host's in the last bit, so values agree to 1 f32 ulp."""
import ctypes
import math
import os

import numpy as np
import pytest

from test_synth import constants, poly_jump
from wick_amd.synthetic import WickRng

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def reference_row(seed, tensor, row, n, scale):
    c = constants()
    rng = WickRng(seed)
    s = rng.s
    for _ in range(tensor):
        s = poly_jump(s, c["kLongJump"])
    for _ in range(row):
        s = poly_jump(s, c["kJump"])
    rng.s = s
    out = np.empty(n, np.float32)
    for i in range(0, n, 2):
        a, b = rng.next_u64(), rng.next_u64()
        u1, u2 = ((a >> 11) + 1) * 2.0 ** -53, (b >> 11) * 2.0 ** -53
        rad, th = math.sqrt(-2.0 * math.log(u1)), 6.283185307179586 * u2
        out[i] = np.float32(rad * math.cos(th) * float(np.float32(scale)))
        out[i + 1] = np.float32(rad * math.sin(th) * float(np.float32(scale)))
    return out


def test_device_rows_match_the_python_restatement():
    torch = pytest.importorskip("torch")
    lib = ctypes.CDLL(os.path.join(ROOT, "wick_amd", "libwick_probe.so"))
    lib.wick_synth_normal.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_int,
                                      ctypes.c_ulonglong, ctypes.c_float, ctypes.c_void_p]
    for seed, tensor, rows, cols, scale in [(2, 0, 3, 128, 1.0), (5, 3, 300, 1024, 1.0), (0, 1, 2, 576, 0.02)]:
        x = torch.empty(rows, cols, device="cuda")
        assert lib.wick_synth_normal(x.data_ptr(), tensor, rows, cols, seed, scale,
                                     torch.cuda.current_stream().cuda_stream) == 0
        got = x.cpu().numpy()
        for r in sorted({0, 1, rows - 1}):
            want = reference_row(seed, tensor, r, cols, scale)
            d = np.abs(got[r].view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64)).max()
            assert d <= 1, (seed, tensor, r, int(d))
        print(f"seed {seed} tensor {tensor} {rows}x{cols}: mean {got.mean():+.4f} std {got.std():.4f}")
        assert abs(got.std() / scale - 1.0) < 0.05

