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
from provekv_amd import device as D
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
def test_qjl_sign_follows_reference_sum_order(ctx, dim):
    """Vectors whose QJL dot for one projection is so close to zero that its
    sign depends on the summation order (tests/golden/qjl_sum_order.npz, built
    by the oracle): the kernels must reproduce the reference's one sequential
    sum (qjl.rs:203-220) -- alone, batched, and at every lane position of a
    32-vector (d64) / 16-vector (d128) group, both radii codecs."""
    import os
    f = np.load(os.path.join(os.path.dirname(__file__), "golden", "qjl_sum_order.npz"))
    x = f[f"x{dim}"]
    rng = np.random.RandomState(dim)
    filler = rng.randn(40, dim).astype(np.float32)
    batches = [x[i:i + 1] for i in range(len(x))] + [x]
    for pos in range(0, 32 if dim == 64 else 16, 5):   # the tricky vectors at lane position pos
        batches.append(np.concatenate([filler[:pos], x, filler[:7]]))
    prof = ctx.turbo_profile(dim, 4, 32, SEED, 1)
    for rc in (L.RADII_F32, L.RADII_LOG_U8):
        for b in batches:
            b = np.ascontiguousarray(b)
            assert prof.encode_batch_compact(b, rc) == O.turbo_encode_batch(b, SEED, radii_codec=rc)


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


@pytest.mark.parametrize("n", [1, 3, 1000])
def test_write_header_matches_encoded_blobs(ctx, n):
    """pkv_write_header: the header bytes of the blob an n-vector encode
    writes (TQB1 with both radii codecs, QJL and PolarOnly, other polar
    widths; FB2), equal to the oracle's blobs; an empty batch and a short
    buffer are rejected."""
    lib = L.lib()
    x = kv_vectors(50 + n, n)
    cases = []
    for bits, mode in ((4, 1), (6, 0), (2, 1)):
        prof = ctx.turbo_profile(64, bits, 32, SEED, mode)
        for rc in (L.RADII_F32, L.RADII_LOG_U8):
            cases.append((prof, rc, O.turbo_encode_batch(x, SEED, bits=bits, mode=mode, radii_codec=rc)[:38]))
    cb, rot = O.fib_constants(SEED)
    fprof = ctx.fib_profile_with_constants(cb, rot)
    cases.append((fprof, L.RADII_LOG_U8, O.fib_encode_batch(x, cb.reshape(32, 4), rot.reshape(64, 64))[:19]))
    for prof, rc, want in cases:
        buf = np.zeros(64, np.uint8)
        assert lib.pkv_header_len(prof._ptr) == len(want)
        assert lib.pkv_write_header(prof._ptr, rc, n, buf.ctypes.data, buf.size) == 0
        assert bytes(buf[:len(want)]) == want
        assert lib.pkv_write_header(prof._ptr, rc, 0, buf.ctypes.data, buf.size) == L.ERR_EMPTY_BATCH
        assert lib.pkv_write_header(prof._ptr, rc, n, buf.ctypes.data, len(want) - 1) == L.ERR_CAPACITY


def test_turbo_profile_parameters_rejected_like_the_reference(ctx):
    """turbo-quant/tests/invalid_inputs.rs:17-27 (TurboQuantizer::new,
    turbo.rs:148-164): an odd dimension and a QJL profile of 1 bit are
    invalid; a valid profile outside what the kernels implement (dim 8) is
    reported as unsupported, not as invalid."""
    for dim, bits in ((7, 8), (8, 1)):
        with pytest.raises(L.PkvError) as e:
            ctx.turbo_profile(dim, bits, 8, 42, 1)
        assert e.value.status == L.ERR_INVALID_ARG
    with pytest.raises(L.PkvError) as e:
        ctx.turbo_profile(8, 8, 8, 42, 1)
    assert e.value.status == L.ERR_UNSUPPORTED


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
    cb, rot = O.fib_constants(SEED)   # the oracle's own codebook and rotation
    ref = O.fib_encode_batch(x, cb.reshape(32, 4), rot.reshape(64, 64))
    assert blob == ref
    dec = ad.decode_batch_compact(blob, SEED)
    dref = O.fib_decode_batch(ref, cb.reshape(32, 4), rot.reshape(64, 64))
    assert rel_err(dec, dref) <= 1e-6
    assert np.array_equal(dec.view(np.uint32), dref.view(np.uint32))


def test_fib_valu_decode_fallback(ctx):
    """A codebook with exact 0.0 components (and a subnormal one): the matrix
    core returns a product 0 x (negative) as +0.0 where f32 multiplication
    gives -0.0, so the profile's product check sends its decode to the VALU
    kernel.  Bytes and decodes (f32, and bf16 fanned out to two caches) must
    still be the oracle's, run on the same codebook."""
    import torch
    cb, rot = O.fib_constants(SEED)
    cb = cb.copy()
    cb[3, 1] = 0.0
    cb[20, 2] = 0.0
    cb[7, 0] = np.float32(1e-39)
    prof = ctx.fib_profile_with_constants(cb, rot)
    try:
        assert prof.fib_decode_path() == "valu"
        x = kv_vectors(31, 1000)
        blob = prof.encode_batch_compact(x)
        assert blob == O.fib_encode_batch(x, cb, rot)
        dref = O.fib_decode_batch(blob, cb, rot)
        assert np.array_equal(prof.decode_batch_compact(blob).view(np.uint32), dref.view(np.uint32))
        n = x.shape[0]
        wire = torch.from_numpy(np.frombuffer(blob, np.uint8).copy()).cuda()
        segs = D.segments([D.contiguous_segment(0, n, 64, 0)])
        out = torch.empty(2 * n * 64, dtype=torch.bfloat16, device="cuda")
        st = torch.empty(2, dtype=torch.int32, device="cuda")
        prof.decode_segments(wire, segs, out, status=st, fanout=2, fanout_stride=n * 64)
        torch.cuda.synchronize()
        assert prof.status_error(st.cpu().numpy().view(np.uint32), segs) is None
        want = torch.from_numpy(dref.reshape(-1)).to(torch.bfloat16)
        for c in range(2):
            assert torch.equal(out[c * n * 64:(c + 1) * n * 64].cpu().view(torch.int16), want.view(torch.int16))
    finally:
        prof.close()
    # the seed-42 profile itself decodes on the matrix cores
    assert ctx.fib_profile(64, 4, 32, SEED).fib_decode_path() == "matrix"


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
    # every element the smallest subnormal: the norm underflows fp16
    # (fib-quant/tests/norm_payload_rejection.rs:13-19), batch and per vector
    tiny = x.copy()
    tiny[12] = np.frombuffer(np.uint32(1).tobytes(), np.float32)[0]
    with pytest.raises(CompressionFailed, match="fp16.*vector 12"):
        ad.encode_batch_compact(tiny, SEED)
    with pytest.raises(CompressionFailed, match="fp16"):
        ad.encode(tiny[12], SEED)
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
    cb, rot = O.fib_constants(SEED)
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


def test_fib_encode_full_wave_lists(ctx):
    """300,000 vectors with every block near a codeword bisector: every
    vector is undecided, each encode wave lists 32 per unit, and a wave with
    more than two units redoes a full list in the middle of its unit loop
    (the path ordinary data never takes) as well as after its last unit; the
    bytes must still equal the reference's."""
    ad = FibQuantAdapter(64, 4, 32, 2048, 4, 8)
    cb, rot = O.fib_constants(SEED)
    cb = cb.reshape(32, 4).astype(np.float64)
    rot = rot.reshape(64, 64)
    rng = np.random.RandomState(29)
    n = 300_000
    w1 = rng.randint(0, 32, (n, 16))
    w2 = (w1 + rng.randint(1, 32, (n, 16))) % 32
    t = 0.5 + rng.choice([0.0, 1e-9, -1e-9, 1e-7], (n, 16))
    rho = t[..., None] * cb[w1] + (1 - t[..., None]) * cb[w2]
    x = ((rho.reshape(n, 64) @ rot) * rng.uniform(0.5, 4.0, (n, 1))).astype(np.float32)
    blob = ad.encode_batch_compact(x, SEED)
    assert blob == O.fib_encode_batch(x, cb.astype(np.float32), rot)
