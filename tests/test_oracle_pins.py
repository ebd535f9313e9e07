"""What the mathematics pins in the oracle's derived constants.

No file of the reference holds the values of its seeded constants (QJL
matrix, stored rotation, Lloyd codebook), so they cannot be compared with
golden vectors.  What can be shown is that they do not depend on the pieces
the oracle restates without bit-identity guarantees:

* the ziggurat table (rand_distr 0.4.3 ziggurat_tables.py recursion): the
  oracle builds the correctly rounded table (every exp / log call of the
  recursion correctly rounded); a libm that rounds one hard call the other
  way (this host's glibc 2.35 does, at F[94]) changes no seed-42 constant;
* the draws behind every seed-42 constant: no accept / reject comparison
  that involves exp or log is within many ulps of flipping, and every log
  whose value enters a drawn number directly (the ziggurat tail) is
  correctly rounded, so the normal / gamma streams do not hinge on libm;
* the Lloyd codebook: bit-identical when every initial codeword coordinate
  and every restart's rotated start moves by a relative 1e-12 or 1e-10
  (the inverse CDFs of statrs and nalgebra's k x k QR, restated to ~1e-12);
* the stored rotation: the config-1 FB2 bytes (1,228,800 vectors) are
  unchanged when every entry of the rotation moves by 1 or 4 ulp (the
  nalgebra QR, restated in its reflector order to the last few ulp).
The remaining residual -- the exact draw stream of rand's samplers as
restated -- is pinned by the known-answer tests of test_oracle_rng.py.
"""
import math
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from oracle import oracle as O

mpmath = pytest.importorskip("mpmath")
from mpmath.libmp import round_nearest, to_float  # noqa: E402

SEED = 42


def correctly_rounded(fn, x: float) -> float:
    """Nearest double to fn(x) (x an exact double), at 200 bits."""
    with mpmath.workprec(200):
        return to_float(fn(mpmath.mpf(x))._mpf_, rnd=round_nearest)


def zig_recursion(exp, log):
    R, V = 3.6541528853610088, 0.00492867323399

    def f(x):
        return exp(-x * x / 2.0)

    x = [0.0] * 257
    x[0] = V / f(R)
    x[1] = R
    for i in range(2, 256):
        x[i] = math.sqrt(-2.0 * log(V / x[i - 1] + f(x[i - 1])))
    return x, [f(v) for v in x], R


def test_ziggurat_table_is_the_correctly_rounded_table():
    """The oracle's table is the recursion with correctly rounded exp / log
    (mpmath at 200 bits, rounded to nearest), through "%.18f" (correctly
    rounded both ways in glibc and CPython)."""
    x, fx, R = zig_recursion(lambda t: correctly_rounded(mpmath.exp, t),
                             lambda y: correctly_rounded(mpmath.log, y))
    zx, zf, zr = O.zig_tables()
    assert np.array_equal(zx, np.array([float("%.18f" % v) for v in x]))
    assert np.array_equal(zf, np.array([float("%.18f" % v) for v in fx]))
    assert zr == float("%.18f" % R)


def test_glibc_table_differs_at_one_entry_that_no_seed42_constant_uses():
    """This host's glibc exp (2.35) rounds one call of the recursion the
    other way (its argument lies 0.0024 ulp from a midpoint): F[94] moves by
    1 ulp.  Which of the two tables rand's generator printed depends on the
    libm it ran on; every seed-42 constant is the same under both."""
    x, fx, _ = zig_recursion(math.exp, math.log)
    cx, cf, _ = zig_recursion(lambda t: correctly_rounded(mpmath.exp, t),
                              lambda y: correctly_rounded(mpmath.log, y))
    assert x == cx
    assert [i for i in range(257) if fx[i] != cf[i]] == [94]
    lib = O.lib()

    def constants():
        cb, _, _ = O.fib_codebook(64, 4, 32, SEED, 2048, 4, 8)
        rot, gauss = O.stored_rotation(64, SEED)
        return [cb, rot, gauss, *O.turbo_constants(64, 32, SEED), *O.turbo_constants(128, 32, SEED)]

    cr = constants()
    lib.ora_set_zig_glibc(1)
    try:
        assert O.zig_tables()[1][94] != float("%.18f" % cf[94])
        gl = constants()
    finally:
        lib.ora_set_zig_glibc(0)
    for a, b in zip(cr, gl):
        assert np.array_equal(a, b)


def test_seed42_draws_do_not_hinge_on_libm_last_bits():
    lib = O.lib()
    lib.ora_track_reset(1)
    try:
        O.fib_codebook(64, 4, 32, SEED, 2048, 4, 8)
        O.stored_rotation(64, SEED)
        O.turbo_constants(64, 32, SEED)
        O.turbo_constants(128, 32, SEED)
        margin = lib.ora_track_margin()
        args, vals = np.zeros(4096), np.zeros(4096)
        n = lib.ora_track_tail_logs(args.ctypes.data, vals.ctypes.data, 4096)
    finally:
        lib.ora_track_reset(0)
    # a libm within 1 ulp moves either side by at most ~2^-52 relative
    assert margin > 2.0 ** -40, margin
    assert 0 < n <= 4096
    for a, v in zip(args[:n], vals[:n]):
        assert v == correctly_rounded(mpmath.log, float(a))


@pytest.mark.parametrize("rel", [1e-12, 1e-10])
def test_codebook_invariant_to_initial_codeword_perturbation(rel):
    lib = O.lib()
    cb0, init0, _ = O.fib_codebook(64, 4, 32, SEED, 2048, 4, 8)
    lib.ora_set_codebook_perturbation(rel)
    try:
        cb1, init1, _ = O.fib_codebook(64, 4, 32, SEED, 2048, 4, 8)
    finally:
        lib.ora_set_codebook_perturbation(0.0)
    assert init1 != init0                      # the perturbation reached the start
    assert np.array_equal(cb0.view(np.uint32), cb1.view(np.uint32))


@pytest.mark.slow
def test_config1_fb2_bytes_invariant_to_rotation_perturbation():
    from provekv_amd import synth
    corpus = synth.corpus_tokens(1, 24, 32, 800, 64)
    x = np.ascontiguousarray(corpus.reshape(-1, 64))
    cb, rot = O.fib_constants(SEED)
    chunks = np.array_split(np.arange(x.shape[0]), 16)

    def encode(r):
        with ThreadPoolExecutor(8) as ex:
            parts = list(ex.map(lambda idx: O.fib_encode_batch(x[idx], cb, r)[19:], chunks))
        return b"".join(parts)

    base = encode(rot)
    sign = np.where(np.random.RandomState(1).rand(*rot.shape) < 0.5, -1.0, 1.0)
    for ulps in (1, 4):
        moved = rot + sign * ulps * np.spacing(rot)
        assert not np.array_equal(moved, rot)
        assert encode(moved) == base, ulps
