"""BlockLogU8 radii (turbo-quant/src/radius.rs:58-77) on the GPU.

The encode kernels take mn / mx from the exact logf of the smallest and
largest radius and each code from a hardware log, kept only where the
measured error bound cannot move it across a rounding boundary.  These
cases aim at the exits of that shortcut -- equal radii (span at its 2^-23
floor: every code takes the exact chain), radii across most of the f32
range (the widest bounds short of an overflowing a^2 + b^2), zero radii
(clamped to FLT_MIN), codes placed on rounding boundaries -- and require the
TQB1-L bytes of the oracle, bit for bit, at head_dim 64 and 128.
"""
import numpy as np
import pytest
import scipy.linalg

from oracle import oracle as O
from provekv_amd.codec import RadiiCompression, TurboQuantAdapter

pytestmark = pytest.mark.gpu
SEED = 42


def from_rotated(y):
    """Input x whose normalized FWHT rotation (signs, then H / sqrt(dim):
    rotation.rs:143-222) is y, computed in f64 and rounded to f32."""
    n, dim = y.shape
    signs, _ = O.turbo_constants(dim, 32, SEED)
    h = scipy.linalg.hadamard(dim).astype(np.float64)
    x = (y.astype(np.float64) @ h.T) / np.sqrt(dim) * signs.astype(np.float64)
    return np.ascontiguousarray(x.astype(np.float32))


def pairs(radii, rng):
    """Rotated vectors whose pairs (2i, 2i + 1) have the given radii."""
    th = rng.uniform(-np.pi, np.pi, radii.shape)
    y = np.empty((radii.shape[0], 2 * radii.shape[1]))
    y[:, 0::2] = radii * np.cos(th)
    y[:, 1::2] = radii * np.sin(th)
    return from_rotated(y)


def cases(dim):
    rng = np.random.RandomState(dim)
    m, n = dim // 2, 48
    out = {}
    for s in (1e-30, 1.0, 3.7e15):   # a^2 + b^2 must stay finite (1.8e19 squared overflows)
        out[f"equal_{s:g}"] = pairs(np.full((n, m), s), rng)
    out["full_range"] = pairs(np.exp(rng.uniform(-85.0, 43.0, (n, m))), rng)
    lo = np.exp(rng.uniform(-3, 0, (n, 1)))
    span = rng.uniform(0.5, 40.0, (n, 1))
    k = rng.randint(0, 255, (n, m)) + 0.5
    r = lo * np.exp(k / 255.0 * span)
    r[:, 0] = lo[:, 0]
    r[:, 1] = (lo * np.exp(span))[:, 0]
    out["half_codes"] = pairs(r, rng)
    z = pairs(np.exp(rng.uniform(-2, 2, (n, m))), rng)
    z[::3] = 0.0
    z[1::3, : dim // 2] = 0.0
    out["zeros"] = z
    out["tiny"] = pairs(np.exp(rng.uniform(-95.0, -80.0, (n, m))), rng)
    return out


@pytest.mark.parametrize("dim", [64, 128])
def test_block_log_u8_edge_radii_bit_exact(ctx, dim):
    ad = TurboQuantAdapter(dim, 4, 32, RadiiCompression.Lossy)
    for name, x in cases(dim).items():
        assert np.all(np.isfinite(x)), name
        blob = ad.encode_batch_compact(x, SEED)
        ref = O.turbo_encode_batch(x, SEED, radii_codec=1)
        assert blob == ref, name
        dec = ad.decode_batch_compact(blob, SEED)
        assert np.array_equal(dec.view(np.uint32), O.turbo_decode_batch(ref, dim, SEED).view(np.uint32)), name


def test_radii_log_bound_table(ctx):
    """The bound table measured at context creation: finite, non-decreasing
    in the exponent, and small enough over the radii real KV produces
    (|logf| < 64) for the shortcut to decide almost every code."""
    t = ctx.radii_log_bound()
    print("bound by biased exponent of |logf|:",
          {e: float(t[e]) for e in range(96, 134, 4)})
    assert np.all(np.isfinite(t))
    assert np.all(np.diff(t.astype(np.float64)) >= 0)
    assert t[127 + 5] <= 1e-4


def test_device_checks_ran_at_context_creation(ctx):
    """The first context on the device measured the log bound table and
    checked that the f16 matrix cores keep subnormal operands (the QJL
    acceptance bound counts on it): creation fails otherwise, so a usable
    context with a measured table is the evidence."""
    t = ctx.radii_log_bound()
    assert t[127] > 0.0 and np.isfinite(t[127])
