"""Shared helpers for the parity tests."""
import numpy as np

ATOL, RTOL = 2e-5, 1e-4  # the north star's tolerance on f32 outputs


def within_tol(got, want, atol=ATOL, rtol=RTOL):
    """Per-element |got - want| <= atol + rtol*|want|; returns (ok, max_abs, max_rel over |want| >= 1e-3)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    ok = bool(np.all(err <= atol + rtol * np.abs(want))) and bool(np.all(np.isfinite(got)))
    big = np.abs(want) >= 1e-3
    max_rel = float((err[big] / np.abs(want[big])).max()) if big.any() else 0.0
    return ok, float(err.max()), max_rel


def rope_np(x, heads, head_dim, positions, inv_freq):
    """Rotate-half RoPE (src/model.rs:404-414) on rows x [n][heads*head_dim] at `positions`, f32 math."""
    x = x.reshape(len(positions), heads, head_dim).copy()
    half = head_dim // 2
    ang = np.asarray(positions, np.float32)[:, None] * inv_freq[None, :].astype(np.float32)
    s, c = np.sin(ang).astype(np.float32)[:, None, :], np.cos(ang).astype(np.float32)[:, None, :]
    a, b = x[..., :half].copy(), x[..., half:].copy()
    x[..., :half] = a * c - b * s
    x[..., half:] = b * c + a * s
    return x.reshape(len(positions), heads * head_dim)


def rmsnorm_heads_np(x, heads, head_dim, eps):
    """Per-head rmsnorm with weight 1.0 (the QK-norm of src/model.rs:475-478)."""
    x = x.reshape(-1, heads, head_dim).astype(np.float32)
    ss = (x * x).sum(-1, keepdims=True, dtype=np.float32) / np.float32(head_dim)
    return (x * (np.float32(1.0) / np.sqrt(ss + np.float32(eps)))).reshape(-1, heads * head_dim).astype(np.float32)


def inv_freq(theta, head_dim):
    return np.array([np.float32(1.0 / theta ** (2.0 * i / head_dim)) for i in range(head_dim // 2)], np.float32)
