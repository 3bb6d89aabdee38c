"""Synthetic models and inputs for the benchmark configurations (no checkpoints are available offline).

smollm2_135m() is the SmolLM2-135M architecture of the e2e benchmark: Llama, 30 layers,
hidden 576, 9 query / 3 KV heads, head_dim 64, FFN 1536 SiLU-gated, RMSNorm eps
1e-5, RoPE theta 10000, vocab 49152, tied embeddings.  Matrices are f32
N(0, std) in a fixed order -- drawn with numpy's PCG64 from the given seed, or by
a caller-supplied generator (`normal` below); norm weights are 1.0 (the Hugging
Face initialisation).  wick_generator_weights() draws them with wick's own
generator on the device (DeviceNormals, the benchmark's inputs), and
wick_prompt() draws token ids with it on the host.
"""
import ctypes
import os

import numpy as np

from .model import Config

PROBE_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libwick_probe.so")

_M64 = (1 << 64) - 1


class WickRng:
    """wick's generator (/root/reference/src/sampler.rs:28-55): xoshiro256** seeded
    through splitmix64, in Python integers."""

    def __init__(self, seed):
        z, s = seed & _M64, []
        for _ in range(4):
            z = (z + 0x9E3779B97F4A7C15) & _M64
            x = z
            x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & _M64
            x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & _M64
            s.append(x ^ (x >> 31))
        self.s = s

    def next_u64(self):
        s = self.s
        out = (((s[1] * 5) & _M64) << 7 | ((s[1] * 5) & _M64) >> 57) & _M64
        out = (out * 9) & _M64
        t = (s[1] << 17) & _M64
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = ((s[3] << 45) | (s[3] >> 19)) & _M64
        return out


def wick_prompt(seed, n, vocab):
    """n token ids from wick's generator seeded with `seed`: next_u64() % vocab, in order."""
    rng = WickRng(seed)
    return np.array([rng.next_u64() % vocab for _ in range(n)], dtype=np.uint32)


def smollm2_135m():
    return Config(arch="llama", hidden=576, intermediate=1536, layers=30, heads=9, kv_heads=3, head_dim=64,
                  vocab=49152, max_position=8192, rms_eps=float(np.float32(1e-5)), rope_theta=10000.0,
                  tie_embeddings=True)


def random_weights(cfg, seed=0, std=0.02, normal=None):
    """Weights of cfg's architecture.  normal(rows, cols, std), when given, supplies
    each matrix (called once per matrix in the order below); otherwise numpy's PCG64
    seeded with `seed` draws them."""
    rng = np.random.default_rng(seed)

    def mat(rows, cols):
        if normal is not None:
            return np.ascontiguousarray(normal(rows, cols, std), dtype=np.float32)
        a = rng.standard_normal((rows, cols), dtype=np.float32)
        a *= np.float32(std)
        return a

    h, q, kv, ff = cfg.hidden, cfg.q_dim, cfg.kv_dim, cfg.intermediate
    w = {"embed": mat(cfg.vocab, h), "norm": np.ones(h, np.float32), "lm_head": None, "layers": []}
    for _ in range(cfg.layers):
        w["layers"].append({
            "attn_norm": np.ones(h, np.float32), "wq": mat(q, h), "wk": mat(kv, h), "wv": mat(kv, h), "wo": mat(h, q),
            "bq": None, "bk": None, "bv": None, "q_norm": None, "k_norm": None,
            "ffn_norm": np.ones(h, np.float32), "w_gate": mat(ff, h), "w_up": mat(ff, h), "w_down": mat(h, ff)})
    return w


def random_prompt(seed, n, vocab):
    return np.random.default_rng(seed).integers(0, vocab, n).astype(np.uint32)


class DeviceNormals:
    """A configuration's N(0, 1) inputs from wick's generator, made on the GPU:
    xoshiro256** seeded through splitmix64 with the configuration's seed
    (/root/reference/src/sampler.rs:28-55), Box-Muller in double, times a scale,
    by libwick_probe.so's wick_synth_normal.  The i-th tensor asked for reads
    substream i of the seed's stream (i long jumps), its rows successive jumps,
    so any tensor's rows are known without drawing the ones before them."""

    def __init__(self, torch, device, seed):
        self.torch, self.device, self.seed, self.count = torch, device, seed, 0
        self.lib = ctypes.CDLL(PROBE_LIB)
        self.lib.wick_synth_normal.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_int,
                                               ctypes.c_ulonglong, ctypes.c_float, ctypes.c_void_p]

    def normal(self, rows, cols, scale=1.0):
        """The next tensor, [rows][cols] f32 on the device (synchronous on torch's current stream)."""
        x = self.torch.empty(rows, cols, device=self.device)
        rc = self.lib.wick_synth_normal(x.data_ptr(), self.count, rows, cols, self.seed, scale,
                                        self.torch.cuda.current_stream().cuda_stream)
        if rc:
            raise RuntimeError(f"wick_synth_normal: HIP error {rc}")
        self.count += 1
        return x


def wick_generator_weights(torch, cfg, seed=0, std=0.02, device="cuda"):
    """random_weights(cfg) with every matrix drawn by wick's generator (seed `seed`,
    N(0, std)) on the GPU and copied to host memory: the e2e configuration's weights."""
    syn = DeviceNormals(torch, device, seed)
    return random_weights(cfg, normal=lambda rows, cols, s: syn.normal(rows, cols, s).cpu().numpy())
