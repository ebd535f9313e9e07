"""GPU parity: libpkv_hip.so (through the C ABI) against the CPU oracle.

Bar: TQB1 / FB2 bytes bit-exact; decoded f32 within 1e-6 relative
(per vector, max|d| / max|ref|) -- the kernels are in fact expected to match
the oracle bit for bit, and the tests report exact equality separately.
"""
import struct

import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd import synth
from provekv_amd.codec import (CompressionFailed, DecompressionFailed, FibQuantAdapter, RadiiCompression,
                               TurboQuantAdapter)

pytestmark = pytest.mark.gpu
SEED = 42


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.maximum(np.abs(b).max(axis=-1), 1e-30)
    return (np.abs(a - b).max(axis=-1) / den).max()


def kv_vectors(seed, n, dim=64):
    K, V = synth.kv_cache(seed, 1, 4, (n + 7) // 8, dim)
    x = np.concatenate([K.reshape(-1, dim), V.reshape(-1, dim)])[:n]
    assert x.shape == (n, dim)
    return np.ascontiguousarray(x)


@pytest.mark.parametrize("n", [1, 3, 4, 63, 64, 65, 255, 256, 257, 1000])
@pytest.mark.parametrize("lossy", [False, True])
def test_turbo_encode_decode_bit_exact(ctx, n, lossy):
    x = kv_vectors(n, n)
    ad = TurboQuantAdapter(64, 4, 32, RadiiCompression.Lossy if lossy else RadiiCompression.Lossless)
    blob = ad.encode_batch_compact(x, SEED)
    ref = O.turbo_encode_batch(x, SEED, radii_codec=1 if lossy else 0)
    assert blob == ref
    dec = ad.decode_batch_compact(blob, SEED)
    dref = O.turbo_decode_batch(ref, 64, SEED)
    assert rel_err(dec, dref) <= 1e-6
    assert np.array_equal(dec.view(np.uint32), dref.view(np.uint32))


def test_turbo_dim128_bit_exact(ctx):
    x = kv_vectors(5, 300, 128)
    for lossy in (False, True):
        ad = TurboQuantAdapter(128, 4, 32, RadiiCompression.Lossy if lossy else RadiiCompression.Lossless)
        blob = ad.encode_batch_compact(x, SEED)
        assert blob == O.turbo_encode_batch(x, SEED, radii_codec=int(lossy))
        dec = ad.decode_batch_compact(blob, SEED)
        dref = O.turbo_decode_batch(blob, 128, SEED)
        assert rel_err(dec, dref) <= 1e-6
        assert np.array_equal(dec.view(np.uint32), dref.view(np.uint32))


@pytest.mark.parametrize("n", [1, 15, 16, 17, 63, 257, 1000])
def test_turbo_dim128_group_sizes(ctx, n):
    """Head_dim 128 encodes 16 vectors per wave (four lanes each): partial
    groups and tiles, both radii codecs, bit-exact."""
    x = kv_vectors(900 + n, n, 128)
    for rc in (0, 1):
        ad = TurboQuantAdapter(128, 4, 32, RadiiCompression.Lossy if rc else RadiiCompression.Lossless)
        blob = ad.encode_batch_compact(x, SEED)
        assert blob == O.turbo_encode_batch(x, SEED, radii_codec=rc)
        assert np.array_equal(ad.decode_batch_compact(blob, SEED).view(np.uint32),
                              O.turbo_decode_batch(blob, 128, SEED).view(np.uint32))


def test_turbo_dim128_edge_inputs_and_projections(ctx):
    rng = np.random.RandomState(8)
    x = rng.randn(80, 128).astype(np.float32)
    x[0] = 0.0                      # zero residual: every QJL sign takes the exact path
    x[1] = -0.0
    x[2, ::2] = 0.0
    x[3] = 1e-30
    x[4] = np.float32(1e18)
    x[5, :] = np.arange(128, dtype=np.float32)
    x[6] = 1.0                      # a constant vector: one non-zero Hadamard coefficient
    for proj in (32, 64):
        prof = ctx.turbo_profile(128, 4, proj, SEED, 1)
        for rc in (L.RADII_F32, L.RADII_LOG_U8):
            assert prof.encode_batch_compact(x, rc) == O.turbo_encode_batch(x, SEED, proj=proj, radii_codec=rc)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("bits,mode", [(8, 1), (9, 1), (6, 0), (4, 0), (2, 1), (1, 0)])
def test_turbo_other_bit_widths(ctx, dim, bits, mode):
    """Generic polar bit widths (the kernels specialise pbits 3): bytes and
    decodes bit for bit, both radii codecs."""
    x = kv_vectors(7 + bits, 200, dim)
    prof = ctx.turbo_profile(dim, bits, 32, SEED, mode)
    for rc in (L.RADII_F32, L.RADII_LOG_U8):
        blob = prof.encode_batch_compact(x, rc)
        assert blob == O.turbo_encode_batch(x, SEED, bits=bits, mode=mode, radii_codec=rc)
        dec = prof.decode_batch_compact(blob)
        dref = O.turbo_decode_batch(blob, dim, SEED, bits=bits, mode=mode)
        assert rel_err(dec, dref) <= 1e-6
        assert np.array_equal(dec.view(np.uint32), dref.view(np.uint32))


def test_turbo_edge_inputs(ctx):
    rng = np.random.RandomState(3)
    x = rng.randn(64, 64).astype(np.float32)
    x[0] = 0.0                      # all-zero vector: r = 0, theta = 0 -> bin 4
    x[1] = -0.0
    x[2, ::2] = 0.0                 # many pairs on the octant lines
    x[3] = 1e-30                    # tiny values (denormal products)
    x[4] = np.float32(1e18)
    x[5, :] = np.arange(64, dtype=np.float32)
    ad = TurboQuantAdapter(64, 4, 32)
    assert ad.encode_batch_compact(x, SEED) == O.turbo_encode_batch(x, SEED)
    adl = TurboQuantAdapter(64, 4, 32, RadiiCompression.Lossy)
    assert adl.encode_batch_compact(x, SEED) == O.turbo_encode_batch(x, SEED, radii_codec=1)


def test_turbo_errors(ctx):
    ad = TurboQuantAdapter(64, 4, 32)
    x = kv_vectors(11, 100)
    bad = x.copy()
    bad[37, 5] = np.inf
    with pytest.raises(CompressionFailed, match="non-finite input.*vector 37"):
        ad.encode_batch_compact(bad, SEED)
    with pytest.raises(O.OracleError) as e:
        O.turbo_encode_batch(bad, SEED)
    assert e.value.index == 37
    huge = x.copy()
    huge[12] = 3e38                  # rotated values overflow -> non-finite radius
    with pytest.raises(CompressionFailed, match="non-finite radius"):
        ad.encode_batch_compact(huge, SEED)
    with pytest.raises(CompressionFailed):
        ad.encode_batch_compact(np.zeros((0, 64), np.float32), SEED)
    blob = bytearray(ad.encode_batch_compact(x, SEED))
    neg = bytearray(blob)
    struct.pack_into("<f", neg, 38 + 144 * 9 + 4, -1.0)
    with pytest.raises(DecompressionFailed, match="vector 9"):
        ad.decode_batch_compact(bytes(neg), SEED)
    with pytest.raises(DecompressionFailed):
        ad.decode_batch_compact(bytes(blob) + b"\0", SEED)     # trailing bytes
    with pytest.raises(DecompressionFailed):
        ad.decode_batch_compact(bytes(blob[:-1]), SEED)         # short buffer
    # a corrupt vector and trailing bytes: the vector is reported, as the
    # reference validates every vector before cursor.finish() (wire.rs:566)
    with pytest.raises(DecompressionFailed, match="vector 9"):
        ad.decode_batch_compact(bytes(neg) + b"\0\0", SEED)
    with pytest.raises(O.OracleError) as e:
        O.turbo_decode_batch(bytes(neg) + b"\0\0", 64, SEED)
    assert e.value.index == 9
    with pytest.raises(DecompressionFailed):
        ad.decode_batch_compact(bytes(blob), SEED + 1)          # seed mismatch


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 64, 257, 1000])
def test_fib_encode_decode_bit_exact(ctx, n):
    x = kv_vectors(100 + n, n)
    ad = FibQuantAdapter(64, 4, 32, 2048, 4, 8)
    blob = ad.encode_batch_compact(x, SEED)
    prof = ad.build_quantizer(SEED)
    cb, rot = prof.constants()
    ref = O.fib_encode_batch(x, cb.reshape(32, 4), rot.reshape(64, 64))
    assert blob == ref
    dec = ad.decode_batch_compact(blob, SEED)
    dref = O.fib_decode_batch(ref, cb.reshape(32, 4), rot.reshape(64, 64))
    assert rel_err(dec, dref) <= 1e-6
    assert np.array_equal(dec.view(np.uint32), dref.view(np.uint32))


def test_fib_errors(ctx):
    ad = FibQuantAdapter(64, 4, 32, 2048, 4, 8)
    x = kv_vectors(21, 50)
    z = x.copy()
    z[7] = 0
    z[30] *= 1e6     # later failure of another kind: validation pass wins
    with pytest.raises(CompressionFailed, match="zero norm.*vector 7"):
        ad.encode_batch_compact(z, SEED)
    nf = x.copy()
    nf[44, 1] = np.nan
    with pytest.raises(CompressionFailed, match="non-finite input.*vector 44"):
        ad.encode_batch_compact(nf, SEED)
    big = x.copy()
    big[30] *= 1e6
    with pytest.raises(CompressionFailed, match="fp16.*vector 30"):
        ad.encode_batch_compact(big, SEED)
    blob = bytearray(ad.encode_batch_compact(x, SEED))
    zero_norm = bytearray(blob)
    zero_norm[19 + 12 * 3] = 0
    zero_norm[19 + 12 * 3 + 1] = 0
    with pytest.raises(DecompressionFailed, match="vector 3"):
        ad.decode_batch_compact(bytes(zero_norm), SEED)
    hdr = bytearray(blob)
    hdr[4] = 6
    with pytest.raises(DecompressionFailed):
        ad.decode_batch_compact(bytes(hdr), SEED)
    # trailing bytes are accepted (fib-quant/src/codec.rs:380-386)
    out = ad.decode_batch_compact(bytes(blob) + b"\1\2\3", SEED)
    assert out.shape == (50, 64)


def test_fib_encode_near_ties_take_exact_path(ctx):
    """Vectors whose rotated blocks sit on the bisector of two codewords: the
    approximate argmin cannot decide them, the exact path must, and the bytes
    must still equal the reference's."""
    ad = FibQuantAdapter(64, 4, 32, 2048, 4, 8)
    prof = ad.build_quantizer(SEED)
    cb, rot = prof.constants()
    cb = cb.reshape(32, 4).astype(np.float64)
    rot = rot.reshape(64, 64)
    rng = np.random.RandomState(17)
    xs = []
    for _ in range(300):
        rho = np.zeros(64)
        for b in range(16):
            w1, w2 = rng.choice(32, 2, replace=False)
            t = 0.5 + rng.choice([0.0, 1e-9, -1e-9, 1e-7, 3e-6])
            rho[4 * b:4 * b + 4] = t * cb[w1] + (1 - t) * cb[w2]
        x = rot.T @ rho
        xs.append(x * rng.uniform(0.5, 4.0))
    x = np.array(xs, np.float32)
    blob = ad.encode_batch_compact(x, SEED)
    assert blob == O.fib_encode_batch(x, cb.astype(np.float32), rot)
