"""GPU parity of the per-vector KVecCodec methods (TQW1 / FB1 records)
through the C ABI (pkv_encode_vectors / pkv_decode_vectors) against the CPU
oracle.  Bar: record bytes bit-exact, decoded f32 bit-exact, and the
rejected record index equal to the oracle's."""
import struct

import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd import synth
from provekv_amd.codec import DecompressionFailed, FibQuantAdapter, RadiiCompression, TurboQuantAdapter

pytestmark = pytest.mark.gpu
SEED = 42


def kv_vectors(seed, n, dim=64):
    K, V = synth.kv_cache(seed, 1, 4, (n + 7) // 8, dim)
    return np.ascontiguousarray(np.concatenate([K.reshape(-1, dim), V.reshape(-1, dim)])[:n])


def same_f32(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


@pytest.fixture(scope="module")
def fib(ctx):
    ad = FibQuantAdapter(64, 4, 32, 2048, 4, 8)
    cb, rot = O.fib_constants(SEED)   # the oracle's own constants
    return ad, cb.reshape(32, 4), rot.reshape(64, 64)


@pytest.mark.parametrize("n", [1, 3, 64, 257, 1000])
def test_tqw1_encode_decode_bit_exact(ctx, n):
    x = kv_vectors(n, n)
    for rc in (RadiiCompression.Lossless, RadiiCompression.Lossy):   # TQW1 ignores the radii policy
        ad = TurboQuantAdapter(64, 4, 32, rc)
        recs = ad.encode_batch(x, SEED)
        ref = O.turbo_encode_tqw1(x, SEED)
        assert recs == ref
        assert ad.encode(x[n - 1], SEED) == ref[-1]
        dec = ad.decode_batch(recs, SEED)
        assert same_f32(dec, O.turbo_decode_tqw1(ref, 64, SEED))
        assert same_f32(ad.decode(recs[0], SEED), dec[0])


@pytest.mark.parametrize("bits,proj,mode", [(4, 64, 1), (4, 32, 0), (8, 32, 1)])
def test_tqw1_other_profiles(ctx, bits, proj, mode):
    x = kv_vectors(7, 130)
    prof = ctx.turbo_profile(64, bits, proj, SEED, mode)
    recs = prof.encode_vectors(x, each=True)
    ref = O.turbo_encode_tqw1(x, SEED, bits=bits, proj=proj, mode=mode)
    assert recs == ref
    assert same_f32(prof.decode_vectors(recs, each=True),
                    O.turbo_decode_tqw1(ref, 64, SEED, bits=bits, proj=proj, mode=mode))


def test_tqw1_dim128(ctx):
    x = kv_vectors(8, 70, 128)
    ad = TurboQuantAdapter(128, 4, 32)
    recs = ad.encode_batch(x, SEED)
    assert recs == O.turbo_encode_tqw1(x, SEED)
    assert same_f32(ad.decode_batch(recs, SEED), O.turbo_decode_tqw1(recs, 128, SEED))


def test_tqw1_rejections_report_the_reference_index(ctx):
    prof = ctx.turbo_profile(64, 4, 32, SEED, 1)
    recs = O.turbo_encode_tqw1(kv_vectors(9, 40), SEED)

    def mut(i, f):
        r = [bytearray(t) for t in recs]
        f(r[i])
        return [bytes(t) for t in r]

    cases = [
        mut(17, lambda r: r.__setitem__(slice(0, 4), b"BAD!")),
        mut(3, lambda r: struct.pack_into("<H", r, 4, 2)),
        recs[:5] + [recs[5] + b"\0"] + recs[6:],
        mut(30, lambda r: struct.pack_into("<Q", r, 22, 8)),
        mut(11, lambda r: r.__setitem__(9, 1)),
        mut(12, lambda r: r.__setitem__(15, 1)),
        mut(0, lambda r: struct.pack_into("<Q", r, 38, 145)),
        mut(21, lambda r: struct.pack_into("<f", r, 46 + 8, -1.0)),
        mut(39, lambda r: struct.pack_into("<f", r, 46, float("inf"))),
        recs[:2] + [recs[2][:45]] + recs[3:],
    ]
    for recs_bad in cases:
        with pytest.raises(O.OracleError) as want:
            O.turbo_decode_tqw1(recs_bad, 64, SEED)
        with pytest.raises(L.PkvError) as got:
            prof.decode_vectors(recs_bad, each=True)
        assert got.value.status == L.ERR_CORRUPT_PAYLOAD and got.value.index == want.value.index
    with pytest.raises(DecompressionFailed):
        TurboQuantAdapter(64, 4, 32).decode(b'{"polar_code": {}}', SEED)


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 257, 1000])
def test_fb1_encode_bit_exact(ctx, fib, n):
    ad, cb, rot = fib
    x = kv_vectors(200 + n, n)
    assert ad.encode_batch(x, SEED) == O.fib_encode_fb1(x, cb, rot, each=False)
    each = ad.build_quantizer(SEED).encode_vectors(x, each=True)
    assert each == O.fib_encode_fb1(x, cb, rot, each=True)
    assert ad.encode(x[0], SEED) == each[0]


@pytest.mark.parametrize("n", [1, 5, 257, 1000])
def test_fb1_decode_bit_exact(ctx, fib, n):
    ad, cb, rot = fib
    recs = O.fib_encode_fb1(kv_vectors(300 + n, n), cb, rot, each=False)
    assert same_f32(ad.decode_batch(recs, SEED), O.fib_decode_fb1(recs, cb, rot, each=False))
    f64 = ad.build_quantizer(SEED).decode_vectors(recs, each=True)
    assert same_f32(f64, O.fib_decode_fb1(recs, cb, rot, each=True))
    assert same_f32(ad.decode(recs[-1], SEED), f64[-1])


def test_fb1_each_encode_bit_exact_at_scale(ctx, fib):
    """Per-vector (FibQuantizer::encode) semantics on 200,000 config-1-shaped
    vectors: the matrix-core keys decide most blocks, the exact path the
    rest; every record equals the oracle's per-vector encode."""
    ad, cb, rot = fib
    x = np.ascontiguousarray(synth.corpus_tokens(5, 2, 32, 1600, 64).reshape(-1, 64)[:200_000])
    got = ad.build_quantizer(SEED).encode_vectors(x, each=True)
    want = O.fib_encode_fb1(x, cb, rot, each=True)
    assert len(got) == len(want)
    bad = [i for i, (g, w) in enumerate(zip(got, want)) if g != w]
    assert not bad, (len(bad), bad[:5])


def test_fib_profile_shapes_outside_fib_k4_n32_are_refused(ctx):
    with pytest.raises(L.PkvError) as e:
        ctx.fib_profile(128, 4, 32, SEED)
    assert e.value.status == L.ERR_UNSUPPORTED


@pytest.mark.parametrize("dim,k,n", [(0, 2, 8), (8, 0, 8), (10, 4, 8), (8, 2, 1), (8, 8, 8), (8194, 2, 8),
                                     (256, 128, 1 << 20)])
def test_fib_profile_invalid_parts_rejected(ctx, dim, k, n):
    """fib-quant/tests/profile_digest.rs:19-36 and profile_resource_bounds.rs
    (FibQuantProfileV1::paper_default): zero dimension, zero block dim, a
    dimension the block does not divide, a one-codeword codebook, block dim
    equal to the dimension, an oversized rotation matrix and oversized
    codebook values are invalid, not merely unsupported."""
    with pytest.raises(L.PkvError) as e:
        ctx.fib_profile(dim, k, n, SEED)
    assert e.value.status == L.ERR_INVALID_ARG


def test_fb1_each_encode_near_ties(ctx, fib):
    """Blocks on codeword bisectors (within 1e-7 .. 1e-9 of the tie): the
    matrix-core gap test leaves them to the exact path under both
    semantics, and the bytes must match the reference's."""
    ad, cb, rot = fib
    rng = np.random.RandomState(23)
    cb64 = cb.astype(np.float64)
    xs = []
    for _ in range(300):
        rho = np.zeros(64)
        for b in range(16):
            w1, w2 = rng.choice(32, 2, replace=False)
            t = 0.5 + rng.choice([0.0, 1e-9, -1e-9, 1e-7])
            rho[4 * b:4 * b + 4] = t * cb64[w1] + (1 - t) * cb64[w2]
        xs.append(rot.T @ rho * rng.uniform(0.5, 4.0))
    x = np.array(xs, np.float32)
    prof = ad.build_quantizer(SEED)
    assert prof.encode_vectors(x, each=True) == O.fib_encode_fb1(x, cb, rot, each=True)
    assert prof.encode_vectors(x, each=False) == O.fib_encode_fb1(x, cb, rot, each=False)


def test_fb1_rejections_and_precedence(ctx, fib):
    ad, cb, rot = fib
    prof = ad.build_quantizer(SEED)
    recs = O.fib_encode_fb1(kv_vectors(12, 50), cb, rot, each=False)
    bad_magic = bytes([ord("X"), ord("B"), ord("1"), 1, 5, 0, 0, 0, 16, 0, 0])
    wrong_ilen = b"FB1" + bytes([1, 5]) + struct.pack("<I", 16) + struct.pack("<H", 2) + b"\0\0\0"
    bc17 = b"FB1" + bytes([1, 5]) + struct.pack("<I", 17) + struct.pack("<H", 2) + recs[0][11:13] + b"\0" * 11
    zero_norm = recs[9][:11] + b"\0\0" + recs[9][13:]
    nlen3 = recs[4][:9] + struct.pack("<H", 3) + recs[4][11:] + b"\0"
    b20 = recs[10][:4] + bytes([4]) + struct.pack("<I", 20) + recs[10][9:]   # 20 x 4 bits: parses, wrong profile
    fb2_magic = b"FB2" + recs[30][3:]
    cases = [
        recs[:7] + [bad_magic] + recs[8:],
        recs[:7] + [b"FB1\1"] + recs[8:],
        recs[:20] + [wrong_ilen] + recs[21:],
        recs[:33] + [bc17] + recs[34:],
        recs[:9] + [zero_norm] + recs[10:],
        recs[:4] + [nlen3] + recs[5:],
        recs[:9] + [zero_norm] + recs[10:40] + [recs[40][:22]] + recs[41:],   # batch: parse failure 40 wins
        # same record length (packed layout): parse failure at 30, header mismatch at 10
        recs[:10] + [b20] + recs[11:30] + [fb2_magic] + recs[31:],
    ]
    for recs_bad in cases:
        for each in (True, False):
            with pytest.raises(O.OracleError) as want:
                O.fib_decode_fb1(recs_bad, cb, rot, each=each)
            with pytest.raises(L.PkvError) as got:
                prof.decode_vectors(recs_bad, each=each)
            assert got.value.status == L.ERR_CORRUPT_PAYLOAD and got.value.index == want.value.index, (each,)
