"""Seeded synthetic KV caches with the value distribution of the benchmark
configs: per-channel log-normal key scales with a few outlier channels per
head, Gaussian values.

Draws: splitmix64 -> two 53-bit uniforms -> Box-Muller in f64 -> f32.  The
same generator feeds the GPU path, the CPU baseline and the tests.
"""
from __future__ import annotations

import numpy as np

_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)
_GOLD = np.uint64(0x9E3779B97F4A7C15)


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + n + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * _GOLD
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def normals(seed: int, n: int, stream: int = 0) -> np.ndarray:
    """n f32 N(0,1) draws; `stream` separates independent sequences."""
    m = (n + 1) // 2
    base = stream * (1 << 40)
    a = splitmix64(seed, m, base)
    b = splitmix64(seed, m, base + m)
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) * (1.0 / 9007199254740992.0)   # (0, 1]
    u2 = (b >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    r = np.sqrt(-2.0 * np.log(u1))
    t = 2.0 * np.pi * u2
    out = np.empty(2 * m, dtype=np.float64)
    out[0::2] = r * np.cos(t)
    out[1::2] = r * np.sin(t)
    return out[:n].astype(np.float32)


def kv_cache(seed: int, layers: int, heads: int, tokens: int, dim: int, k_sigma: float = 0.5,
             outliers: int = 2, outlier_mult: float = 8.0, v_scale: float = 0.5):
    """K, V as float32 arrays [layers, heads, tokens, dim]."""
    zk = normals(seed, layers * heads * tokens * dim, stream=1).reshape(layers, heads, tokens, dim)
    zv = normals(seed, layers * heads * tokens * dim, stream=2).reshape(layers, heads, tokens, dim)
    zs = normals(seed, layers * heads * dim, stream=3).reshape(layers, heads, 1, dim).astype(np.float64)
    scale = np.exp(k_sigma * zs)
    # outlier channels per (layer, head) from a seeded shuffle
    keys = splitmix64(seed, layers * heads * dim, 5 * (1 << 40)).reshape(layers, heads, dim)
    order = np.argsort(keys, axis=-1, kind="stable")[..., :outliers]
    mult = np.ones((layers, heads, dim))
    np.put_along_axis(mult, order, outlier_mult, axis=-1)
    K = (zk.astype(np.float64) * (scale * mult[:, :, None, :])).astype(np.float32)
    V = (zv.astype(np.float64) * v_scale).astype(np.float32)
    return K, V


def corpus_tokens(seed: int, layers: int, heads: int, tokens: int, dim: int, **kw) -> np.ndarray:
    """proveKV corpus layout: one vector per token, [tokens, layers, heads, K|V, dim]
    (proveKV/src/pool.rs:246-257 reads K at l*H*2D + h*2D and V right after)."""
    K, V = kv_cache(seed, layers, heads, tokens, dim, **kw)
    out = np.empty((tokens, layers, heads, 2, dim), dtype=np.float32)
    out[:, :, :, 0, :] = K.transpose(2, 0, 1, 3)
    out[:, :, :, 1, :] = V.transpose(2, 0, 1, 3)
    return out
