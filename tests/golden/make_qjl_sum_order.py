"""Writes qjl_sum_order.npz: inputs whose QJL sketch dot for some projection
is so close to zero that its sign depends on the summation order.

The reference computes each sketch dot as ONE sequential f32 sum over the
dimensions in order (turbo-quant/src/qjl.rs:203-220: `iter().zip().map(|(g, r)|
g * r).sum()`).  A kernel that splits the vector over lanes must hand the
partial sums on in exactly that order; any other order (a half or quarter
summed first, a partial sum taken from the wrong lane) flips the sign of these
dots.  Built with the CPU oracle only: start from a seeded random vector,
move one coordinate until the exact dot of a projection changes sign, and keep
the f32 inputs next to the sign change where the reference order and a
rotated order of the lane groups (d = 64: halves; d = 128: quarters) disagree.

Run from the repository root: python tests/golden/make_qjl_sum_order.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

SEED = 42


def residual(x, signs, G):
    blob = O.turbo_encode_batch(x[None], SEED, signs=signs, G=G)
    rec = O.turbo_decode_batch(blob, x.size, SEED, signs=signs)[0]
    return (x - rec).astype(np.float32)


def seq_sum(p):
    acc = np.float32(0.0)
    for v in p:
        acc = np.float32(acc + v)
    return acc


def orders_disagree(x, j, signs, G, groups):
    """sign of the reference's sequential dot vs the dot summed with the lane
    groups in rotated order (group 1 first, ..., group 0 last)."""
    r = residual(x, signs, G)
    p = (G[j] * r).astype(np.float32)
    ref = seq_sum(p)
    w = p.size // groups
    alt = seq_sum(np.concatenate([p[w:], p[:w]]))
    return (ref >= 0) != (alt >= 0), float(ref)


def search(dim, want, rng):
    signs, G = O.turbo_constants(dim, 32, SEED)
    groups = 2 if dim == 64 else 4
    found = []
    while len(found) < want:
        x = rng.standard_normal(dim).astype(np.float32)
        j = int(rng.integers(32))
        k = int(rng.integers(dim))
        def exact(xv):
            r = residual(xv, signs, G).astype(np.float64)
            return float(np.dot(G[j].astype(np.float64), r))
        lo, hi = np.float32(x[k] - 4.0), np.float32(x[k] + 4.0)
        xl, xh = x.copy(), x.copy()
        xl[k], xh[k] = lo, hi
        fl, fh = exact(xl), exact(xh)
        if (fl >= 0) == (fh >= 0):
            continue
        for _ in range(80):   # bisection on the f32 value of x[k]
            mid = np.float32((np.float64(lo) + np.float64(hi)) / 2)
            if mid in (lo, hi):
                break
            xm = x.copy()
            xm[k] = mid
            fm = exact(xm)
            if (fm >= 0) == (fl >= 0):
                lo, fl = mid, fm
            else:
                hi, fh = mid, fm
        for v in (lo, hi):
            xv = x.copy()
            xv[k] = v
            dis, ref = orders_disagree(xv, j, signs, G, groups)
            if dis:
                found.append((xv, j, ref))
                break
    return found


def main():
    rng = np.random.default_rng(20251202)
    out = {}
    for dim, want in ((64, 12), (128, 12)):
        f = search(dim, want, rng)
        out[f"x{dim}"] = np.stack([v for v, _, _ in f])
        out[f"proj{dim}"] = np.array([j for _, j, _ in f], np.int32)
        out[f"refdot{dim}"] = np.array([r for _, _, r in f], np.float32)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "qjl_sum_order.npz")
    np.savez(path, **out)
    print(path, {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
