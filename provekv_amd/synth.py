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


_CHUNK = 1 << 16   # elements per pass: the temporaries stay in cache


def _splitmix64_into(out: np.ndarray, seed: int, start: int) -> None:
    """out[i] = splitmix64 output number start + i + 1 of `seed`."""
    s30, s27, s31 = np.uint64(30), np.uint64(27), np.uint64(31)
    with np.errstate(over="ignore"):
        z = np.arange(start + 1, start + out.size + 1, dtype=np.uint64)
        z *= _GOLD
        z += np.uint64(seed)
        z ^= z >> s30
        z *= _M1
        z ^= z >> s27
        z *= _M2
        z ^= z >> s31
    out[...] = z


def splitmix64(seed: int, n: int, start: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint64)
    for c0 in range(0, n, _CHUNK):
        _splitmix64_into(out[c0:c0 + _CHUNK], seed, start + c0)
    return out


def normals(seed: int, n: int, stream: int = 0) -> np.ndarray:
    """n f32 N(0,1) draws; `stream` separates independent sequences.  Pair j
    takes uniforms u1 (0, 1] and u2 [0, 1) from splitmix64 outputs j and m + j
    (m = ceil(n / 2)) and yields r cos(2 pi u2), r sin(2 pi u2), r =
    sqrt(-2 ln u1), in f64, rounded to f32."""
    m = (n + 1) // 2
    base = stream * (1 << 40)
    out = np.empty(2 * m, dtype=np.float32)
    a = np.empty(_CHUNK, dtype=np.uint64)
    b = np.empty(_CHUNK, dtype=np.uint64)
    inv53 = 1.0 / 9007199254740992.0
    for c0 in range(0, m, _CHUNK):
        k = min(_CHUNK, m - c0)
        _splitmix64_into(a[:k], seed, base + c0)
        _splitmix64_into(b[:k], seed, base + m + c0)
        u1 = ((a[:k] >> np.uint64(11)).astype(np.float64) + 1.0) * inv53
        u2 = (b[:k] >> np.uint64(11)).astype(np.float64) * inv53
        r = np.sqrt(-2.0 * np.log(u1))
        t = 2.0 * np.pi * u2
        out[2 * c0:2 * (c0 + k):2] = r * np.cos(t)
        out[2 * c0 + 1:2 * (c0 + k):2] = r * np.sin(t)
    return out[:n]


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


def device_kv_bf16(seed: int, layers: int, heads: int, tokens: int, dim: int, k_sigma: float = 0.7,
                   outliers: int = 4, outlier_mult: float = 10.0, v_scale: float = 1.0, device="cuda"):
    """The same value distribution generated on the GPU (for shapes too large
    to generate on the host, e.g. the Llama-3-8B KV of 4.3 GB): K[l, h, t, c]
    = s[l, h, c] z with s = exp(k_sigma z') and `outliers` channels per head
    (a seeded permutation) scaled by `outlier_mult`, V = v_scale z; computed in
    f32, then rounded to bf16 (nearest even).  Returns one bf16 tensor
    [layers, 2 (K|V), heads, tokens, dim].  Seeded by torch's Philox generator
    on `device`: reproducible for a given torch build, not equal to the host
    generator's draws."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    out = torch.empty((layers, 2, heads, tokens, dim), dtype=torch.bfloat16, device=device)
    zs = torch.randn((layers, heads, 1, dim), generator=g, device=device, dtype=torch.float32)
    mult = torch.ones((layers, heads, 1, dim), device=device, dtype=torch.float32)
    for li in range(layers):
        for h in range(heads):
            perm = torch.randperm(dim, generator=g, device=device)[:outliers]
            mult[li, h, 0, perm] = outlier_mult
    scale = torch.exp(k_sigma * zs) * mult
    for li in range(layers):   # one layer at a time: bounded f32 scratch
        z = torch.randn((2, heads, tokens, dim), generator=g, device=device, dtype=torch.float32)
        out[li, 0] = (z[0] * scale[li]).to(torch.bfloat16)
        out[li, 1] = (z[1] * v_scale).to(torch.bfloat16)
    return out


def corpus_tokens(seed: int, layers: int, heads: int, tokens: int, dim: int, **kw) -> np.ndarray:
    """proveKV corpus layout: one vector per token, [tokens, layers, heads, K|V, dim]
    (proveKV/src/pool.rs:246-257 reads K at l*H*2D + h*2D and V right after)."""
    K, V = kv_cache(seed, layers, heads, tokens, dim, **kw)
    out = np.empty((tokens, layers, heads, 2, dim), dtype=np.float32)
    out[:, :, :, 0, :] = K.transpose(2, 0, 1, 3)
    out[:, :, :, 1, :] = V.transpose(2, 0, 1, 3)
    return out
