"""Textbook float64 formulas for the attention path -- TEST INFRASTRUCTURE ONLY.

These pin the strict-f32 restatement in flock_oracle.c from outside: they are
written from the mathematics (not from the reference's loop structure) and share
no code with it. A plausible mistake in the restatement -- a wrong GQA map, an
off-by-one causal bound, the wrong RoPE partner, a dropped scale -- moves its
output by O(1) against these, while honest f32 rounding moves it by ~1e-6.
"""
from __future__ import annotations

import numpy as np


def rmsnorm(x, g, n: int, n_vecs: int, eps: float) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps) * g per n-wide vector, in float64."""
    x = np.asarray(x, np.float64).reshape(n_vecs, n)
    g = np.asarray(g, np.float64)
    return (x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * g).ravel()


def inv_freq(head_dim: int, base: float) -> np.ndarray:
    """1 / base^(2j/d), j < d/2, in float64."""
    j = np.arange(head_dim // 2, dtype=np.float64)
    return 1.0 / np.power(np.float64(base), 2.0 * j / head_dim)


def rope(x, n_tokens: int, n_heads: int, head_dim: int, pos0: int, inv_f,
         pairing: str = "neox") -> np.ndarray:
    """Rotate pair (a, b) by theta = pos * inv_f[j] as a complex multiply."""
    x = np.asarray(x, np.float64).reshape(n_tokens, n_heads, head_dim)
    half = head_dim // 2
    if pairing == "neox":
        a, b = x[..., :half], x[..., half:]
    else:
        a, b = x[..., 0::2], x[..., 1::2]
    pos = (pos0 + np.arange(n_tokens, dtype=np.float64))[:, None, None]
    theta = pos * np.asarray(inv_f, np.float64)[None, None, :]
    z = (a + 1j * b) * np.exp(1j * theta)
    out = np.empty_like(x)
    if pairing == "neox":
        out[..., :half], out[..., half:] = z.real, z.imag
    else:
        out[..., 0::2], out[..., 1::2] = z.real, z.imag
    return out.ravel()


def attention(q, k, v, n_heads: int, n_kv_heads: int, head_dim: int, n_queries: int,
              pos0: int) -> np.ndarray:
    """softmax(q k^T / sqrt(d)) v with query i seeing keys 0 .. pos0+i.

    q: [n_queries][H][d]; k, v: [>= pos0+n_queries][Hkv][d]. Query head h reads
    kv head h // (H / Hkv). Decode is n_queries = 1, pos0 = n_keys - 1.
    """
    H, Hkv, d = n_heads, n_kv_heads, head_dim
    n_keys = pos0 + n_queries
    q = np.asarray(q, np.float64).reshape(n_queries, H, d)
    k = np.asarray(k, np.float64).reshape(-1, Hkv, d)[:n_keys]
    v = np.asarray(v, np.float64).reshape(-1, Hkv, d)[:n_keys]
    kvh = np.arange(H) // (H // Hkv)
    kh = k[:, kvh, :].transpose(1, 0, 2)            # [H][keys][d]
    vh = v[:, kvh, :].transpose(1, 0, 2)
    s = np.matmul(q.transpose(1, 0, 2), kh.transpose(0, 2, 1)) / np.sqrt(d)  # [H][q][keys]
    mask = np.arange(n_keys)[None, :] > (pos0 + np.arange(n_queries))[:, None]
    s[:, mask] = -np.inf
    s -= s.max(axis=2, keepdims=True)
    np.exp(s, out=s)
    s /= s.sum(axis=2, keepdims=True)
    o = np.matmul(s, vh)  # [H][q][d]
    return o.transpose(1, 0, 2).ravel()
