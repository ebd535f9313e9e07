"""Lloyd-Max refinement on the device (pkv_lloyd_refine, and the codebook
build of pkv_fib_profile_create that uses it) against the oracle's
refine_codebook restatement: refined codebooks, per-restart MSEs and the
initial MSE bit-identical (f64), empty-cell repairs included.

* the reference's own repair case (fib-quant/src/lloyd.rs:364-402: cell 2
  empty, donor 0 split along its farthest sample) with its assertions;
* random training sets at the fib_k4_n32 shape (2048 samples, 4 restarts,
  8 iterations) and a starved one (40 samples for 32 cells: repairs every
  iteration);
* a set whose only donor has a zero residual: EmptyCellRepairFailed on both;
* whole profile builds after the constant cache is cleared, so the device
  trainer runs: the codebook the profile holds equals the oracle's.
"""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L

pytestmark = pytest.mark.gpu


def device_refine(ctx, samples, starts, iterations):
    s = np.ascontiguousarray(samples, dtype=np.float64)
    st = np.ascontiguousarray(starts, dtype=np.float64)
    ns, k = s.shape
    r, n, _ = st.shape
    out = np.zeros_like(st)
    mse = np.zeros(r)
    init = np.zeros(1)
    rc = L.lib().pkv_lloyd_refine(ctx.ptr, s.ctypes.data, ns, k, n, st.ctypes.data, r, iterations,
                                  out.ctypes.data, mse.ctypes.data, init.ctypes.data)
    return rc, out, mse, float(init[0])


def assert_same(ctx, samples, starts, iterations):
    rc, out, mse, init = device_refine(ctx, samples, starts, iterations)
    assert rc == 0, L.status_string(rc)
    w_out, w_mse, w_init = O.lloyd_refine(samples, starts, iterations)
    assert np.array_equal(out.view(np.uint64), w_out.view(np.uint64))
    assert np.array_equal(mse.view(np.uint64), w_mse.view(np.uint64))
    assert np.float64(init).view(np.uint64) == np.float64(w_init).view(np.uint64)
    return out, mse, init


def test_reference_repair_case(ctx):
    samples = np.array([[0.0, 0.0], [1.0, 0.0], [2.0, 0.0], [10.0, 0.0], [10.1, 0.0]])
    start = np.array([[[0.0, 0.0], [10.0, 0.0], [20.0, 0.0]]])
    out, _, _ = assert_same(ctx, samples, start, 1)
    cb = out[0].reshape(-1)
    assert cb[0] < 1.0 and cb[4] > 1.0        # lloyd.rs:399-400
    assert cb[0] == 1.0 - 1.0e-6 and cb[4] == 1.0 + 1.0e-6   # donor 0 split along +x


@pytest.mark.parametrize("seed,ns", [(0, 2048), (1, 2048), (2, 8192)])
def test_random_sets_match_oracle(ctx, seed, ns):
    """2048 samples run with the training set in LDS, 8192 from global memory."""
    rng = np.random.default_rng(seed)
    samples = rng.normal(size=(ns, 4)) * rng.uniform(0.1, 1.0, size=(ns, 1))
    starts = rng.normal(size=(4, 32, 4)) * 0.5
    assert_same(ctx, samples, starts, 8)


def test_starved_set_repairs_match_oracle(ctx):
    rng = np.random.default_rng(5)
    samples = rng.normal(size=(40, 4))
    starts = rng.normal(size=(3, 32, 4))
    assert_same(ctx, samples, starts, 8)


def test_zero_residual_donor_fails_like_the_oracle(ctx):
    samples = np.ones((6, 4))
    starts = np.array([[[1.0, 1.0, 1.0, 1.0], [5.0, 5.0, 5.0, 5.0]]])
    rc, _, _, _ = device_refine(ctx, samples, starts, 2)
    assert rc == L.ERR_INVALID_ARG
    with pytest.raises(O.OracleError):
        O.lloyd_refine(samples, starts, 2)


def test_shape_limits(ctx):
    rc, *_ = device_refine(ctx, np.zeros((8, 17)), np.zeros((1, 2, 17)), 1)
    assert rc == L.ERR_UNSUPPORTED


@pytest.mark.parametrize("seed,training,restarts,iterations", [(42, 2048, 4, 8), (7, 1024, 2, 5), (3, 4096, 1, 3)])
def test_profile_codebook_built_on_device(ctx, seed, training, restarts, iterations):
    lib = L.lib()
    lib.pkv_constants_cache_clear()    # the next profile must build (on the device)
    p = C.c_void_p()
    L.check(lib.pkv_fib_profile_create(ctx.ptr, 64, 4, 32, seed, training, restarts, iterations, C.byref(p)),
            "pkv_fib_profile_create")
    try:
        cb = np.zeros(128, np.float32)
        rot = np.zeros(64 * 64, np.float64)
        L.check(lib.pkv_profile_constants(p, cb.ctypes.data, cb.nbytes, rot.ctypes.data, rot.nbytes),
                "pkv_profile_constants")
    finally:
        lib.pkv_profile_destroy(p)
    want = O.fib_codebook(64, 4, 32, seed, training, restarts, iterations)
    want_cb = want[0] if isinstance(want, tuple) else want
    assert np.array_equal(cb.view(np.uint32), np.asarray(want_cb, np.float32).reshape(-1).view(np.uint32))
