"""Pins of the oracle's RNG chain against published known answers.

Sources of the expected values: RFC 7539 section A.1 test vector 1 (ChaCha20,
zero key and nonce); the 8-round zero-key keystream of the ChaCha test-vector
draft (draft-strombergson-chacha-test-vectors, TC1); rand_core 0.6's
value-breakage test of seed_from_u64(0) and rand_chacha 0.3's
test_chacha_construction; the literals of rand_distr 0.4's
ziggurat_tables.rs.  Moments and tail checks pin the sampler's use of them.
"""
import numpy as np

from oracle import oracle as O


def test_chacha20_rfc7539_a1():
    w = O.chacha_words([0] * 8, 20, 16)
    expect = [0xade0b876, 0x903df1a0, 0xe56a5d40, 0x28bd8653, 0xb819d2bd, 0x1aed8da0, 0xccef36a8,
              0xc70d778b, 0x7c5941da, 0x8d485751, 0x3fe02477, 0x374ad8b8, 0xf4b8436a, 0x1ca11815,
              0x69b687c3, 0x8665eeb2]
    assert [int(x) for x in w] == expect


def test_chacha8_zero_key_tc1():
    w = O.chacha_words([0] * 8, 8, 16)
    assert w.astype("<u4").tobytes()[:64].hex() == (
        "3e00ef2f895f40d67f5bb8e81f09a5a12c840ec3ce9a7f3b181be188ef711a1e"
        "984ce172b9216f419f445367456d5619314a42a3da86b001387bfdb80e0cfe42")


def test_chacha_block_counter_continues():
    # the second 64-byte block is the first block of counter 1: skipping 16
    # words must equal generating 32 and dropping 16
    a = O.chacha_words([1, 2, 3, 4, 5, 6, 7, 8], 8, 32)
    b = O.chacha_words([1, 2, 3, 4, 5, 6, 7, 8], 8, 16, skip=16)
    assert np.array_equal(a[16:], b)


def test_rand_core_seed_from_u64_value():
    k = O.seed_key(0)
    assert int(k[0]) | (int(k[1]) << 32) == 5029875928683246316


def test_rand_chacha_construction_value():
    # ChaChaRng (20 rounds) from_seed([0,0,0,0,0,0,0,0,1,0,...,2,...,3,...])
    assert int(O.chacha_words([0, 0, 1, 0, 2, 0, 3, 0], 20, 1)[0]) == 137206642


def test_ziggurat_table_literals():
    x, f, r = O.zig_tables()
    assert "%.18f" % r == "3.654152885361008796"
    assert "%.18f" % x[0] == "3.910757959537090045"
    assert "%.18f" % x[1] == "3.654152885361008796"
    assert "%.18f" % x[2] == "3.449278298560964462"
    assert "%.18f" % f[0] == "0.000477467764586655"
    assert "%.18f" % f[1] == "0.001260285930498598"
    assert "%.18f" % f[2] == "0.002609072746106363"
    assert x[256] == 0.0 and f[256] == 1.0
    assert np.all(np.diff(x[1:]) < 0)


def test_normal_moments_and_tail():
    z = O.normal_f64(7, 400_000)
    assert abs(z.mean()) < 0.01
    assert abs(z.std() - 1.0) < 0.01
    assert abs((z ** 3).mean()) < 0.03
    assert abs((z ** 4).mean() - 3.0) < 0.05
    # the zero_case tail beyond R = 3.654 is exercised and lands there
    tail = np.abs(z) > 3.654152885361009
    assert 0 < tail.sum() < 200   # expected 2.6e-4 * 4e5 ~ 103


def test_gamma_moments():
    for shape in (2.0, 30.0):
        g = O.gamma_f64(11, shape, 200_000)
        assert abs(g.mean() - shape) < 0.02 * shape
        assert abs(g.var() - shape) < 0.05 * shape
        assert g.min() > 0
