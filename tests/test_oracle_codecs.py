"""Oracle codec pins: the reference's own literal unit tests, closed forms,
size receipts and brute force on small inputs."""
import math
import struct

import numpy as np
import pytest

from oracle import oracle as O

SEED = 42


def test_bitpack_literal_fallback_rs_389():
    # gpu-backend/src/fallback.rs:389-397: [0,1,2,3,0,1,2,3] @ 2 bits -> 0b11100100
    packed = O.pack_bits([0, 1, 2, 3, 0, 1, 2, 3], 2)
    assert len(packed) == 2 and packed[0] == 0b11100100


@pytest.mark.parametrize("bits", [1, 3, 5, 7, 12, 16])
def test_bitpack_round_trip_and_padding(bits):
    rng = np.random.RandomState(bits)
    n = 37
    vals = rng.randint(0, 1 << bits, size=n)
    data = O.pack_bits(vals, bits)
    assert len(data) == (n * bits + 7) // 8
    assert np.array_equal(O.unpack_bits(data, n, bits), vals)
    if (n * bits) % 8:
        bad = bytearray(data)
        bad[-1] |= 0x80
        with pytest.raises(O.OracleError):
            O.unpack_bits(bytes(bad), n, bits)


def test_codebook_lookup_exact_and_ties_fallback_rs_409_443():
    cb = np.array([[1, 0, 0, 0], [0, 0, 0, 1], [0, 1, 0, 0], [0, 0, 1, 0]], np.float32)
    assert O.nearest_codeword_k4([1, 0, 0, 0], cb) == 0
    assert O.nearest_codeword_k4([0, 0, 0, 1], cb) == 1
    assert O.nearest_codeword_k4([0, 1, 0, 0], cb) == 2
    assert O.nearest_codeword_k4([0, 0, 1, 0], cb) == 3
    # equidistant -> lowest index (strict <)
    cb2 = np.array([[1, 0, 0, 0], [0, 1, 0, 0]], np.float32)
    assert O.nearest_codeword_k4([1, 1, 0, 0], cb2) == 0


def _lcg_values(seed, count):
    out = []
    s = seed
    for _ in range(count):
        s = (s * 6364136223846793005 + 1442695040888963407) & (2 ** 64 - 1)
        v = (s >> 32) & 0xFFFFFFFF
        if v >= 2 ** 31:
            v -= 2 ** 32
        out.append(np.float32(np.float32(v) / np.float32(2147483647)) * np.float32(0.5))
    return np.array(out, np.float32)


def test_avx2_order_matches_scalar_on_lcg_data_simd_nearest_rs():
    # simd_nearest.rs tests: AVX2 == scalar on LCG seeds (lib.rs:251-314 inputs)
    for seed in range(16):
        vals = _lcg_values(0xDEADBEEF + seed, 32 * 4 + 4 * 40)
        cb = vals[:128].reshape(32, 4)
        for b in range(40):
            s = vals[128 + 4 * b: 132 + 4 * b]
            assert O.nearest_codeword_k4(s, cb) == O.nearest_codeword_scalar(s, cb, 4)


def test_avx2_intrinsics_equal_pairwise_restatement():
    """The oracle's AVX2 argmin (the instructions of simd_nearest.rs:44-92,
    used by the CPU baseline) returns the pairwise scalar restatement's index
    on random samples and on near-ties built on codeword bisectors."""
    cb = O.fib_constants(SEED)[0]
    rng = np.random.RandomState(11)
    S = (rng.randn(20000, 4) * 0.2).astype(np.float32)
    for i in range(4000):
        a, b = rng.choice(32, 2, replace=False)
        t = 0.5 + rng.choice([0.0, 1e-8, -1e-8, 1e-7])
        S[i] = (t * cb[a] + (1 - t) * cb[b]).astype(np.float32)
    for s in S:
        assert O.nearest_codeword_k4_avx2(s, cb) == O.nearest_codeword_k4(s, cb)


def test_argmin_brute_force_small():
    rng = np.random.RandomState(3)
    for _ in range(2000):
        cb = rng.randn(32, 4).astype(np.float32) * 0.2
        s = rng.randn(4).astype(np.float32) * 0.2
        e = (cb - s).astype(np.float32)
        q = (e * e).astype(np.float32)
        d = ((q[:, 0] + q[:, 1]).astype(np.float32) + (q[:, 2] + q[:, 3]).astype(np.float32)).astype(np.float32)
        assert O.nearest_codeword_k4(s, cb) == int(np.argmin(d))


def test_f16_against_numpy():
    rng = np.random.RandomState(5)
    vals = np.concatenate([rng.uniform(-70000, 70000, 20000), rng.uniform(-1e-4, 1e-4, 20000),
                           [0.0, -0.0, 65504.0, 65519.99, 65520.0, 2 ** -24, 2 ** -25, 3 * 2 ** -26, np.inf,
                            -np.inf]]).astype(np.float32)
    for v in vals:
        h = O.f32_to_f16(float(v))
        assert h == int(np.array([v], np.float32).astype(np.float16).view(np.uint16)[0]), v
        ref = float(np.array([h], np.uint16).view(np.float16).astype(np.float32)[0])
        got = O.f16_to_f32(h)
        assert (got == ref) or (math.isnan(got) and math.isnan(ref))


def test_hadamard_e0_and_inverse():
    signs, _ = O.turbo_constants(64, 0, SEED)
    assert set(np.unique(signs)) <= {-1.0, 1.0}
    e0 = np.zeros(64, np.float32)
    e0[0] = 1
    y = O.turbo_rotate(signs, e0)
    assert np.allclose(np.abs(y), 0.125, atol=0)        # fallback.rs:312-335 closed form
    # Sylvester H_64 / 8 applied to (x * signs)
    H = np.array([[1.0]])
    while H.shape[0] < 64:
        H = np.block([[H, H], [H, -H]])
    x = np.random.RandomState(1).randn(64).astype(np.float32)
    ref = (H @ (x.astype(np.float64) * signs)) / 8.0
    assert np.allclose(O.turbo_rotate(signs, x), ref, rtol=1e-5, atol=1e-6)
    back = O.turbo_rotate_inverse(signs, O.turbo_rotate(signs, x))
    assert np.allclose(back, x, atol=1e-5)


def test_angle_bins_special_cases():
    signs = np.ones(64, np.float32)
    # choose x so that the rotated pair (y0, y1) is a known point: rotate back
    cases = {(1.0, 0.0): 4, (0.0, 1.0): 6, (0.0, -1.0): 2, (-1.0, 0.0): 0, (0.0, 0.0): 4,
             (1.0, 1.0): 5, (-1.0, -1.0): 1}
    for (a, b), want in cases.items():
        y = np.zeros(64, np.float32)
        y[0], y[1] = a, b
        x = O.turbo_rotate_inverse(signs, y)
        yy = O.turbo_rotate(signs, x)
        if not (yy[0] == a and yy[1] == b):
            continue   # not exactly representable after two transforms
        G = np.zeros((32, 64), np.float32)
        _, idx, _ = O.turbo_encode_vector(x, signs, G)
        assert idx[0] == want, ((a, b), idx[0])


def test_turbo_sizes_match_receipts():
    # encoded_size.rs: 4*pairs + ceil(pairs*bits/8) + ceil(m/8)
    assert O.turbo_payload_len(64, 4, 32, 1, 0) == 144
    assert O.turbo_payload_len(64, 4, 32, 1, 1) == 56
    assert O.turbo_payload_len(128, 4, 32, 1, 0) == 284
    assert O.turbo_payload_len(128, 4, 32, 1, 1) == 100
    # CLAIMS.json pins: shells 6,194,976 (lossless) / 2,410,272 (lossy) per agent
    assert 43008 * 144 + 48 * 38 == 6194976
    assert 43008 * 56 + 48 * 38 == 2410272
    # pool 14,746,512 = 1,228,800 * 12 + 48 * 19
    assert 1228800 * 12 + 48 * 19 == 14746512


def test_turbo_blob_layout_and_round_trip():
    x = np.random.RandomState(2).randn(16, 64).astype(np.float32)
    blob = O.turbo_encode_batch(x, SEED)
    assert len(blob) == 38 + 16 * 144
    assert blob[:4] == b"TQB1" and struct.unpack_from("<H", blob, 4)[0] == 1
    assert struct.unpack_from("<H", blob, 6)[0] == 1 and blob[8] == 2 and blob[14] == 3 and blob[15] == 0
    assert struct.unpack_from("<I", blob, 10)[0] == 64 and struct.unpack_from("<I", blob, 18)[0] == 32
    assert struct.unpack_from("<Q", blob, 22)[0] == SEED
    assert struct.unpack_from("<I", blob, 30)[0] == 16 and struct.unpack_from("<I", blob, 34)[0] == 144
    # f32 radii are the pair norms of the rotated vector
    signs, G = O.turbo_constants(64, 32, SEED)
    y = O.turbo_rotate(signs, x[0])
    r = np.frombuffer(blob[38:38 + 128], np.float32)
    assert np.allclose(r, np.sqrt(y[0::2].astype(np.float64) ** 2 + y[1::2] ** 2), rtol=1e-6)
    dec = O.turbo_decode_batch(blob, 64, SEED)
    assert dec.shape == (16, 64)
    lossy = O.turbo_encode_batch(x, SEED, radii_codec=1)
    assert len(lossy) == 38 + 16 * 56 and lossy[15] == 1
    dl = O.turbo_decode_batch(lossy, 64, SEED)
    assert np.linalg.norm(dl - dec) / np.linalg.norm(dec) < 0.05   # wire.rs lossy radii < 5%


def test_turbo_qjl_signs_brute_force():
    signs, G = O.turbo_constants(64, 32, SEED)
    x = np.random.RandomState(4).randn(64).astype(np.float32)
    radii, idx, sb = O.turbo_encode_vector(x, signs, G)
    blob = O.turbo_encode_batch(x[None, :], SEED)
    rec = O.turbo_decode_batch(blob, 64, SEED)[0]
    res = (x - rec).astype(np.float32)
    for j in range(32):
        acc = np.float32(0)
        for c in range(64):
            acc = np.float32(acc + np.float32(G[j, c] * res[c]))
        assert bool((sb[j // 8] >> (j % 8)) & 1) == bool(acc >= 0)


def test_turbo_decode_rejects():
    x = np.random.RandomState(2).randn(4, 64).astype(np.float32)
    blob = bytearray(O.turbo_encode_batch(x, SEED))
    for mutate in (lambda b: b.__setitem__(0, ord("X")), lambda b: b.__setitem__(14, 4),
                   lambda b: b.__setitem__(22, 7), lambda b: b.extend(b"\0"),
                   lambda b: struct.pack_into("<f", b, 38, -1.0)):
        bad = bytearray(blob)
        mutate(bad)
        with pytest.raises(O.OracleError):
            O.turbo_decode_batch(bytes(bad), 64, SEED)


def test_turbo_decode_trailing_bytes_checked_after_vectors():
    """wire.rs:489-498 rejects a short buffer before any vector, cursor.finish()
    (wire.rs:566) rejects trailing bytes only after every vector: a blob with a
    corrupt vector AND trailing bytes reports the vector."""
    x = np.random.RandomState(2).randn(6, 64).astype(np.float32)
    blob = bytearray(O.turbo_encode_batch(x, SEED))
    both = bytearray(blob)
    struct.pack_into("<f", both, 38 + 144 * 4 + 8, -1.0)   # vector 4: negative radius
    both.extend(b"\0\0")
    with pytest.raises(O.OracleError) as e:
        O.turbo_decode_batch(bytes(both), 64, SEED)
    assert e.value.kind == "malformed" and e.value.index == 4
    with pytest.raises(O.OracleError) as e:                 # trailing bytes alone
        O.turbo_decode_batch(bytes(blob) + b"\0", 64, SEED)
    assert e.value.kind == "malformed"
    with pytest.raises(O.OracleError):                      # short by one byte
        O.turbo_decode_batch(bytes(blob[:-1]), 64, SEED)


@pytest.mark.parametrize("dim", [64, 128])
def test_qjl_sum_order_fixture(dim):
    """tests/golden/qjl_sum_order.npz: for each vector the oracle's sign bit of
    the stored projection is the sign of the reference's sequential sum, and
    summing the lane groups in rotated order gives the other sign -- so a
    kernel that hands partial sums on in any other order fails on them."""
    import os
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "qjl_sum_order.npz"))
    x, proj, refdot = f[f"x{dim}"], f[f"proj{dim}"], f[f"refdot{dim}"]
    signs, G = O.turbo_constants(dim, 32, SEED)
    plen = O.turbo_payload_len(dim)
    blob = O.turbo_encode_batch(x, SEED, signs=signs, G=G)
    rec = O.turbo_decode_batch(blob, dim, SEED, signs=signs)
    groups = 2 if dim == 64 else 4
    for i in range(len(x)):
        j = int(proj[i])
        p = (G[j] * (x[i] - rec[i]).astype(np.float32)).astype(np.float32)
        seq = np.float32(0)
        for v in p:
            seq = np.float32(seq + v)
        w = dim // groups
        alt = np.float32(0)
        for v in np.concatenate([p[w:], p[:w]]):
            alt = np.float32(alt + v)
        assert seq == refdot[i] and (seq >= 0) != (alt >= 0)
        sb = blob[38 + i * plen + plen - 4:38 + (i + 1) * plen]
        assert bool((sb[j // 8] >> (j % 8)) & 1) == bool(seq >= 0)


def test_turbo_lossy_equal_radii_span_clamp():
    # BlockLogU8: equal radii -> span clamps to EPSILON on encode, 0 on decode
    x = np.zeros((4, 64), np.float32)
    blob = O.turbo_encode_batch(x, SEED, radii_codec=1)
    p = blob[38:38 + 56]
    assert all(v == 0 for v in p[:32])
    mn, mx = struct.unpack_from("<ff", p, 32)
    assert mn == mx == np.float32(np.log(np.float32(1.1754944e-38)))


def test_qr_rotation_invariants():
    m, g = O.stored_rotation(64, SEED)
    assert np.abs(m @ m.T - np.eye(64)).max() < 1e-13
    R = m.T @ g
    assert np.abs(np.tril(R, -1)).max() < 1e-12
    assert np.all(np.diag(R) > 0)           # Q is THE Q of the Gaussian matrix


def test_roberts_kronecker_and_radius_closed_forms():
    # profile_digest.rs:51 -- beta_{d,k} literal 0.7 is for (d=8, k=4): (4/6)*1 + 1 ... check d=64:
    from scipy import stats
    d, k, n = 64, 4, 32
    beta = (k / (k + 2)) * ((d - k - 2) / 2) + 1
    for idx in (1, 7, 16, 32):
        q = (idx - 0.5) / n
        want = math.sqrt(stats.beta.ppf(q, k / 2, beta))
        assert abs(O.radius_quantile(d, k, idx, n) - want) < 1e-12
    for p in (1e-12, 0.01, 0.3, 0.5, 0.77, 1 - 1e-12):
        assert abs(O.inv_norm_cdf(p) - stats.norm.ppf(p)) < 1e-12 * max(1, abs(stats.norm.ppf(p)))
    dirs = O.roberts_kronecker(4, 32)
    assert np.allclose(np.linalg.norm(dirs, axis=1), 1.0)
    # phi solves phi^5 = phi + 1 (the k=4 Roberts constant)
    phi = 1.1673039782614187
    assert abs(phi ** 5 - phi - 1) < 1e-12


def test_codebook_training_improves():
    cb, init_mse, train_mse = O.fib_codebook()
    assert cb.shape == (32, 4) and np.all(np.isfinite(cb))
    assert train_mse <= init_mse                      # paper_smoke_regression.rs:20
    assert np.linalg.norm(cb, axis=1).max() < 1.0
    cb2, _, _ = O.fib_codebook()
    assert np.array_equal(cb, cb2)                    # codebook_determinism.rs


def test_fib_blob_layout_and_round_trip():
    cb, _, _ = O.fib_codebook()
    rot, _ = O.stored_rotation(64, SEED)
    x = np.random.RandomState(9).randn(16, 64).astype(np.float32)
    blob = O.fib_encode_batch(x, cb, rot)
    assert len(blob) == 19 + 16 * 12                  # codec.rs:1126-1127
    assert blob[:3] == b"FB2" and blob[3] == 1 and blob[4] == 5 and blob[5] == 0
    assert struct.unpack_from("<I", blob, 6)[0] == 16 and struct.unpack_from("<I", blob, 10)[0] == 16
    assert blob[14] == 0 and struct.unpack_from("<HH", blob, 15) == (2, 10)
    for v in range(16):   # norm bytes: f16(f32(||x||_f64)), pinned without RNG
        h = struct.unpack_from("<H", blob, 19 + 12 * v)[0]
        nrm = np.float32(np.sqrt(np.sum(x[v].astype(np.float64) ** 2)))
        assert h == int(np.array([nrm], np.float32).astype(np.float16).view(np.uint16)[0])
    dec = O.fib_decode_batch(blob, cb, rot)
    assert dec.shape == (16, 64)
    cos = np.sum(dec * x, axis=1) / np.linalg.norm(dec, axis=1) / np.linalg.norm(x, axis=1)
    assert cos.min() > 0.7
    # trailing bytes are accepted (codec.rs:380-386)
    assert np.array_equal(O.fib_decode_batch(blob + b"\0\0", cb, rot), dec)


def test_fib_errors():
    cb, _, _ = O.fib_codebook()
    rot, _ = O.stored_rotation(64, SEED)
    x = np.random.RandomState(9).randn(8, 64).astype(np.float32)
    z = x.copy()
    z[3] = 0
    with pytest.raises(O.OracleError) as e:
        O.fib_encode_batch(z, cb, rot)
    assert e.value.kind == "zero_norm" and e.value.index == 3
    nf = x.copy()
    nf[5, 7] = np.nan
    with pytest.raises(O.OracleError) as e:
        O.fib_encode_batch(nf, cb, rot)
    assert e.value.kind == "nonfinite_input" and e.value.index == 5
    big = x.copy()
    big[2] *= 1e6
    with pytest.raises(O.OracleError) as e:
        O.fib_encode_batch(big, cb, rot)
    assert e.value.kind == "norm_unrepresentable"
