"""GPU test of the profile-constant service through the C ABI: every distinct
profile's constants (fib codebook + rotation, turbo signs + QJL matrix) are
built once per process and shared by every context and profile handle, where
the reference rebuilds them on each adapter call (FibQuantAdapter::
build_quantizer, proveKV/src/codec.rs:471-499; TurboQuantizer::new,
codec.rs:249, 296).  The constants a device profile holds are the oracle's,
bit for bit, and profiles built from the cache encode identical bytes."""
import ctypes as C
import time

import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd.device import Context

pytestmark = pytest.mark.gpu
SEED = 42


def _stats(lib):
    h, m, e = C.c_uint64(), C.c_uint64(), C.c_uint64()
    lib.pkv_constants_cache_stats(C.byref(h), C.byref(m), C.byref(e))
    return h.value, m.value, e.value


def _fib_profile(lib, ctx, seed):
    p = C.c_void_p()
    L.check(lib.pkv_fib_profile_create(ctx.ptr, 64, 4, 32, seed, 2048, 4, 8, C.byref(p)), "pkv_fib_profile_create")
    return p


def _turbo_profile(lib, ctx, dim, seed):
    p = C.c_void_p()
    L.check(lib.pkv_turbo_profile_create(ctx.ptr, dim, 4, 32, seed, L.TURBO_POLAR_WITH_QJL, C.byref(p)),
            "pkv_turbo_profile_create")
    return p


def _encode(lib, ctx, prof, x):
    n = x.shape[0]
    cap = int(lib.pkv_blob_len(prof, L.RADII_F32, n))
    out = np.zeros(cap, np.uint8)
    olen = C.c_uint64()
    err = L.Error()
    L.check(lib.pkv_encode_batch_compact(ctx.ptr, prof, L.RADII_F32, x.ctypes.data, n, out.ctypes.data, cap,
                                         C.byref(olen), C.byref(err)), "encode")
    return out[:olen.value].tobytes()


def test_constant_service_shares_constants_across_contexts(ctx):
    lib = L.lib()
    lib.pkv_constants_cache_clear()
    assert _stats(lib) == (0, 0, 0)
    ctx2 = Context(0)
    try:
        t0 = time.perf_counter()
        fa = _fib_profile(lib, ctx, SEED)          # builds codebook (Lloyd) + rotation
        t1 = time.perf_counter()
        fb = _fib_profile(lib, ctx2, SEED)         # another context: served from the cache
        t2 = time.perf_counter()
        assert _stats(lib) == (2, 2, 2)
        assert t2 - t1 < (t1 - t0) / 3
        ta = _turbo_profile(lib, ctx, 64, SEED)
        tb = _turbo_profile(lib, ctx2, 64, SEED)
        tc = _turbo_profile(lib, ctx, 128, SEED)
        assert _stats(lib) == (3, 4, 4)            # signs + QJL per (dim, seed), one build each
        # device profiles hold the oracle's constants, bit for bit
        cb, rot = O.fib_constants(SEED)
        for p in (fa, fb):
            a, b = np.zeros(128, np.float32), np.zeros(64 * 64, np.float64)
            L.check(lib.pkv_profile_constants(p, a.ctypes.data, a.nbytes, b.ctypes.data, b.nbytes), "constants")
            assert np.array_equal(a.view(np.uint32), cb.reshape(-1).view(np.uint32))
            assert np.array_equal(b.view(np.uint64), rot.reshape(-1).view(np.uint64))
        for p, dim in ((ta, 64), (tb, 64), (tc, 128)):
            signs, G = O.turbo_constants(dim, 32, SEED)
            a, b = np.zeros(dim, np.float32), np.zeros(32 * dim, np.float32)
            L.check(lib.pkv_profile_constants(p, a.ctypes.data, a.nbytes, b.ctypes.data, b.nbytes), "constants")
            assert np.array_equal(a, signs) and np.array_equal(b.view(np.uint32), G.reshape(-1).view(np.uint32))
        # profiles from the cache encode the same bytes as the oracle on its own constants
        x = np.random.RandomState(5).randn(300, 64).astype(np.float32)
        want = O.fib_encode_batch(x, cb, rot)
        assert _encode(lib, ctx, fa, x) == want and _encode(lib, ctx2, fb, x) == want
        tw = O.turbo_encode_batch(x, SEED)
        assert _encode(lib, ctx, ta, x) == tw and _encode(lib, ctx2, tb, x) == tw
        # a different seed is a different profile: one more build of each constant
        fd = _fib_profile(lib, ctx2, SEED + 1)
        assert _stats(lib) == (3, 6, 6)
        for p in (fa, fb, ta, tb, tc, fd):
            lib.pkv_profile_destroy(p)
    finally:
        ctx2.close()
