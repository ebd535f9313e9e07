"""CPU tests of libpkv_hip.so's host half: the C ABI loads and exports every
declared symbol, the profile constants equal the oracle's bit for bit, and
the scalar routines the kernels share (angle bins, logf, expf) equal the
host glibc (the reference's transcendental source) on sampled inputs."""
import ctypes
import os
import re

import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd import device as D

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIBM = ctypes.CDLL("libm.so.6")
LIBM.logf.argtypes = [ctypes.c_float]
LIBM.logf.restype = ctypes.c_float
LIBM.expf.argtypes = [ctypes.c_float]
LIBM.expf.restype = ctypes.c_float


def test_abi_exports_every_declared_symbol():
    header = open(os.path.join(ROOT, "include", "pkv_codec.h")).read()
    declared = set(re.findall(r"\b(pkv_[a-z0-9_]+)\s*\(", header))
    lib = L.lib()
    for name in sorted(declared):
        assert hasattr(lib, name), name
    assert declared == set(L.EXPORTS)


def test_status_strings():
    assert L.status_string(0) == "ok"
    assert "corrupt" in L.status_string(L.ERR_CORRUPT_PAYLOAD)


@pytest.mark.parametrize("dim,proj,seed", [(64, 32, 42), (128, 32, 42), (64, 64, 7), (64, 32, 2 ** 64 - 5)])
def test_turbo_constants_match_oracle(dim, proj, seed):
    s1, g1 = D.turbo_constants(dim, proj, seed)
    s2, g2 = O.turbo_constants(dim, proj, seed)
    assert np.array_equal(s1, s2)
    assert np.array_equal(g1.view(np.uint32), g2.view(np.uint32))


@pytest.mark.parametrize("seed", [42, 0, 123456789])
def test_fib_constants_match_oracle(seed):
    cb, rot, im, tm = D.fib_constants(seed=seed)
    cb2, im2, tm2 = O.fib_codebook(seed=seed)
    rot2, _ = O.stored_rotation(64, seed)
    assert np.array_equal(cb.view(np.uint32), cb2.view(np.uint32))
    assert np.array_equal(rot.view(np.uint64), rot2.view(np.uint64))
    assert tm <= im


def test_fib_profile_constants_fixture():
    """The committed seed-42 constants (tests/golden) equal what the host
    generator produces today.  The fixture is the library's own output: a
    regression pin on the generators, not a parity pin against the reference."""
    cb, rot, _, _ = D.fib_constants(seed=42)
    signs, G = D.turbo_constants(64, 32, 42)
    g = np.load(os.path.join(ROOT, "tests", "golden", "profile_constants_seed42.npz"))
    assert np.array_equal(g["fib_codebook"], cb)
    assert np.array_equal(g["fib_rotation"], rot)
    assert np.array_equal(g["turbo_signs_d64"], signs)
    assert np.array_equal(g["turbo_qjl_32x64"], G)


def _host_logf(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    L.lib().pkv_host_logf(x.ctypes.data, x.size, out.ctypes.data)
    return out


def _host_expf(x):
    x = np.ascontiguousarray(x, np.float32)
    out = np.zeros_like(x)
    L.lib().pkv_host_expf(x.ctypes.data, x.size, out.ctypes.data)
    return out


def _bins(a, b, pbits=3):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.zeros(a.size, np.uint32)
    L.lib().pkv_host_angle_bins(a.ctypes.data, b.ctypes.data, a.size, pbits, out.ctypes.data)
    return out


def test_logf_matches_glibc():
    rng = np.random.RandomState(0)
    bits = rng.randint(0x00800000, 0x7f800000, size=200_000, dtype=np.int64).astype(np.uint32)
    x = bits.view(np.float32)
    x = np.concatenate([x, np.float32([1.0, 1.1754944e-38, 3.4028235e38, 0.5, 2.0])])
    got = _host_logf(x)
    ref = np.array([LIBM.logf(float(v)) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_logf_exhaustive_equal_to_glibc_and_monotone():
    """On every normal positive float (the radii codec clamps to FLT_MIN,
    radius.rs:61) the restated logf equals the host glibc logf bit for bit,
    and it never decreases -- the BlockLogU8 encode takes mn / mx as the logs
    of the smallest / largest radius on that property."""
    from concurrent.futures import ThreadPoolExecutor
    lo, hi, chunk = 0x00800000, 0x7f800000, 1 << 24
    ora = O.lib()

    def run(u0):
        n = min(chunk + 1, hi - u0)   # one overlap element joins the chunks
        x = np.arange(u0, u0 + n, dtype=np.uint32).view(np.float32)
        got = _host_logf(x)
        want = np.empty(n, np.float32)
        ora.ora_logf_bits(u0, n, want.ctypes.data)
        return (np.array_equal(got.view(np.uint32), want.view(np.uint32)),
                bool(np.all(np.diff(got) >= 0)))

    with ThreadPoolExecutor(8) as ex:
        res = list(ex.map(run, range(lo, hi, chunk)))
    assert all(r[0] for r in res)
    assert all(r[1] for r in res)


def test_expf_matches_glibc_in_radius_range():
    rng = np.random.RandomState(1)
    x = rng.uniform(-87.0, 30.0, size=200_000).astype(np.float32)
    got = _host_expf(x)
    ref = np.array([LIBM.expf(float(v)) for v in x], np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_angle_bins_match_glibc_atan2f_formula():
    """Fast octant path + exact fallback vs the oracle (glibc atan2f) on
    random pairs and on pairs placed on / next to every octant line."""
    rng = np.random.RandomState(2)
    a = rng.randn(100_000).astype(np.float32)
    b = rng.randn(100_000).astype(np.float32)
    t = rng.randn(20_000).astype(np.float32)
    eps = np.float32(1e-7)
    extra_a = np.concatenate([t, t, t, -t, t * 0, t, t * 1e-6, t + eps * t, t, np.float32([0, -0.0, 0, -0.0])])
    extra_b = np.concatenate([t * 0, -t * 0, t, t, t, t * 1e-6, t, t, t + eps * t, np.float32([0, 0, -0.0, -0.0])])
    a = np.concatenate([a, extra_a]).astype(np.float32)
    b = np.concatenate([b, extra_b]).astype(np.float32)
    got = _bins(a, b)
    # exact reference: glibc atan2f through ctypes and the f32 bin formula
    LIBM.atan2f.argtypes = [ctypes.c_float, ctypes.c_float]
    LIBM.atan2f.restype = ctypes.c_float
    PI = np.float32(np.pi)
    want = np.empty(a.size, np.uint32)
    for i in range(a.size):
        th = np.float32(LIBM.atan2f(float(b[i]), float(a[i])))
        u = np.float32(np.float32(th + PI) / np.float32(np.float32(2.0) * PI))
        f = np.floor(np.float32(u * np.float32(8.0)))
        want[i] = (int(f) if f > 0 else 0) % 8
    assert np.array_equal(got, want)


def test_octant_fast_path_safe_pairs_keep_the_exact_bin():
    """The encode kernels' octant path (sign bits + the float safety test of
    octant_bin_f, and a finite fl(a^2) + fl(b^2)): every pair it marks safe
    has the bin of the pinned angle_bin path (glibc atan2f formula, test
    above); pairs on and next to the octant lines, outside the covered range
    (2^-47 .. 2^64), zeros, subnormals, infinities and NaN are marked
    unsafe."""
    rng = np.random.RandomState(7)
    n = 300_000
    mag = np.exp(rng.uniform(-30, 42, n))   # one scale per pair, across the covered range
    a = (rng.randn(n) * mag).astype(np.float32)
    b = (rng.randn(n) * mag).astype(np.float32)
    t = rng.randn(50_000).astype(np.float32)
    up = np.nextafter(t, np.float32(np.inf)).astype(np.float32)
    sub = np.float32([1e-40, -1e-40, 1e-45, 0.0, -0.0, 1e-30, 1.0000001e-30, 1e30, 9.999999e29])
    big = np.float32([np.inf, -np.inf, np.nan, 3.4e38, -3.4e38])
    ea = np.concatenate([t, t, -t, up, t, np.repeat(sub, len(sub)), np.repeat(big, 3), np.ones(len(big) * 3, np.float32)])
    eb = np.concatenate([t, up, t, t, t * 0, np.tile(sub, len(sub)), np.tile(np.float32([1, -1, 0]), len(big)),
                         np.repeat(big, 3)])
    a = np.concatenate([a, ea]).astype(np.float32)
    b = np.concatenate([b, eb]).astype(np.float32)
    bins = np.zeros(a.size, np.uint32)
    safe = np.zeros(a.size, np.uint8)
    L.lib().pkv_host_octant_bins(a.ctypes.data, b.ctypes.data, a.size, bins.ctypes.data, safe.ctypes.data)
    want = _bins(a, b)
    ok = safe.astype(bool)
    assert ok[:n].mean() > 0.9   # random pairs: nearly all take the fast path
    assert np.array_equal(bins[ok], want[ok])
    # never safe: on a line (|a| == |b|, a or b zero), out of range, non-finite
    on_line = (np.abs(a) == np.abs(b)) | (a == 0) | (b == 0)
    mx = np.maximum(np.abs(a), np.abs(b))
    out = ~((mx > np.float32(2.0 ** -47)) & (mx < np.float32(2.0 ** 64))) | ~np.isfinite(a) | ~np.isfinite(b)
    assert not np.any(ok & (on_line | out))
    # and inside the range octant_bin_m2 (the integer form) covers
    assert np.all(mx[ok] > np.float32(1e-30)) and np.all(mx[ok] < np.float32(1e30))


def test_profile_constant_service_builds_each_profile_once():
    """One build per distinct profile per process (the reference rebuilds on
    every adapter call, proveKV/src/codec.rs:471-499): a second request is a
    cache hit with identical constants; another seed is a new build."""
    import time
    lib = L.lib()
    lib.pkv_constants_cache_clear()
    cb1, cb2 = np.zeros(128, np.float32), np.zeros(128, np.float32)
    rot1, rot2 = np.zeros(64 * 64), np.zeros(64 * 64)
    t0 = time.perf_counter()
    L.check(lib.pkv_fib_constants(64, 4, 32, 42, 2048, 4, 8, cb1.ctypes.data, rot1.ctypes.data, None, None), "fib")
    t1 = time.perf_counter()
    L.check(lib.pkv_fib_constants(64, 4, 32, 42, 2048, 4, 8, cb2.ctypes.data, rot2.ctypes.data, None, None), "fib")
    t2 = time.perf_counter()
    assert np.array_equal(cb1, cb2) and np.array_equal(rot1, rot2)
    h, m, e = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    lib.pkv_constants_cache_stats(ctypes.byref(h), ctypes.byref(m), ctypes.byref(e))
    assert (h.value, m.value, e.value) == (2, 2, 2)        # codebook + rotation, built once each
    assert t2 - t1 < (t1 - t0) / 5
    cb3 = np.zeros(128, np.float32)
    L.check(lib.pkv_fib_constants(64, 4, 32, 43, 2048, 4, 8, cb3.ctypes.data, None, None, None), "fib")
    assert not np.array_equal(cb3, cb1)
    s1, g1 = np.zeros(64, np.float32), np.zeros(32 * 64, np.float32)
    s2, g2 = np.zeros(64, np.float32), np.zeros(32 * 64, np.float32)
    L.check(lib.pkv_turbo_constants(64, 32, 42, s1.ctypes.data, g1.ctypes.data), "turbo")
    L.check(lib.pkv_turbo_constants(64, 32, 42, s2.ctypes.data, g2.ctypes.data), "turbo")
    assert np.array_equal(s1, s2) and np.array_equal(g1, g2)
    lib.pkv_constants_cache_stats(ctypes.byref(h), ctypes.byref(m), ctypes.byref(e))
    assert (h.value, m.value, e.value) == (3, 4, 4)
    # the cached constants are the oracle's
    ocb, _, _ = O.fib_codebook()
    assert np.array_equal(cb1.reshape(32, 4), ocb)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU: --gpus N > 1 prints a JSON error line and
    exits with status 2 before touching any device."""
    import json
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=root)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert line["n_gpus"] == 2 and "one GPU" in line["error"]


def test_read_fb2_n_blocks():
    """read_fb2_n_blocks (proveKV/src/pool.rs:108-116): a structural read of
    bytes 10..14, None below 14 bytes or without the FB2 magic."""
    from provekv_amd.pool import read_fb2_n_blocks
    hdr = bytearray(b"FB2\x01\x05\x00") + (16).to_bytes(4, "little") + (0x01020304).to_bytes(4, "little")
    assert read_fb2_n_blocks(bytes(hdr)) == 0x01020304
    assert read_fb2_n_blocks(bytes(hdr) + b"\x00" * 5) == 0x01020304   # rest of the header unchecked
    assert read_fb2_n_blocks(bytes(hdr[:13])) is None
    assert read_fb2_n_blocks(b"") is None
    assert read_fb2_n_blocks(b"TQB1" + bytes(hdr[4:])) is None
    assert read_fb2_n_blocks(b"FB2\x07" + bytes(hdr[4:])) == 0x01020304   # version not checked either


def _stable_rel50(v):
    v = np.ascontiguousarray(v, np.float64)
    out = np.zeros(v.size, np.uint8)
    L.lib().pkv_host_f32_stable_rel50(v.ctypes.data, v.size, out.ctypes.data)
    return out.astype(bool)


def test_redo_xhat_stability_test_is_sufficient():
    """The fib encode redo keeps f32(q) for q = x * fl64(1 / |x|) only when
    the bit test says no f32 rounding boundary (midpoint of two adjacent f32
    values, ties included) lies within |q| 2^-50 of q; here every value it
    accepts is checked exactly, in rationals, against its two neighbouring
    midpoints -- on values placed 0..40 f64 ulps either side of midpoints,
    of f32 values themselves, of binade edges and of 2^-126 (below which it
    must refuse), signs mixed.  It must also accept almost every random q,
    or the redo would divide far more often than it needs to."""
    from fractions import Fraction
    rng = np.random.RandomState(5)
    base = []
    ys = rng.randint(0x00800000, 0x3f800001, size=3000).astype(np.uint32).view(np.float32).astype(np.float64)
    yn = np.nextafter(ys.astype(np.float32), np.float32(np.inf)).astype(np.float64)
    base.append((ys + yn) / 2)                                    # midpoints (exact in f64)
    base.append(ys)                                               # f32 values
    base.append(np.ldexp(1.0, np.arange(-130, 2)).astype(np.float64))   # binade edges, 2^-126 among them
    base = np.concatenate(base)
    k = np.concatenate([np.arange(-40, 41), [-(1 << 20), 1 << 20]]).astype(np.int64)
    bits = (base.view(np.int64)[:, None] + k[None, :]).reshape(-1)
    v = bits.view(np.float64)
    v = v[np.isfinite(v) & (v > 0)]
    v = np.concatenate([v, -v[::7], [0.0, -0.0, 5e-324]])
    ok = _stable_rel50(v)
    assert not ok[np.abs(v) < 2.0 ** -126].any()
    acc = v[ok]
    assert acc.size > 0.5 * v.size
    for q in acc:
        a = abs(float(q))
        y = np.float32(a)
        lo = float(np.nextafter(y, np.float32(0)))
        hi = float(np.nextafter(y, np.float32(np.inf)))
        fa, fy = Fraction(a), Fraction(float(y))
        err = fa * Fraction(1, 1 << 50)
        m_lo, m_hi = (fy + Fraction(lo)) / 2, (fy + Fraction(hi)) / 2
        assert m_hi - fa > err and fa - m_lo > err, q
    # random rotated components: refused about 17 times in 2^29
    r = rng.standard_normal(200_000) / 8.0
    assert _stable_rel50(r).mean() > 0.9999
