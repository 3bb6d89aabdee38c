"""Synthetic models and inputs for the benchmark configurations (no checkpoints are available offline).

smollm2_135m() is the SmolLM2-135M architecture of the e2e benchmark: Llama, 30 layers,
hidden 576, 9 query / 3 KV heads, head_dim 64, FFN 1536 SiLU-gated, RMSNorm eps
1e-5, RoPE theta 10000, vocab 49152, tied embeddings.  Matrices are f32
N(0, 0.02) drawn with numpy's PCG64 from the given seed, in a fixed order;
norm weights are 1.0 (the Hugging Face initialisation).
"""
import numpy as np

from .model import Config


def smollm2_135m():
    return Config(arch="llama", hidden=576, intermediate=1536, layers=30, heads=9, kv_heads=3, head_dim=64,
                  vocab=49152, max_position=8192, rms_eps=float(np.float32(1e-5)), rope_theta=10000.0,
                  tie_embeddings=True)


def random_weights(cfg, seed=0, std=0.02):
    rng = np.random.default_rng(seed)

    def mat(rows, cols):
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
