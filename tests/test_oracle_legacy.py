"""Oracle pins for the legacy per-vector formats behind KVecCodec::encode /
decode: TQW1 (turbo-quant/src/wire.rs:44-256) and compact FB1
(fib-quant/src/codec.rs:81-176).

Header layouts are pinned by the reference's own tests
(turbo-quant/tests/wire_format.rs, fib-quant/tests/compact_bytes_roundtrip.rs);
payload bytes by the independently pinned TQB1 / FB2 paths; the f64 fib
decode (FibQuantizer::decode, codec.rs:506-537) by an exact rational
evaluation of the same sum."""
import struct
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O

SEED = 42
# turbo-quant/tests/wire_format.rs:3-7
RESERVED_OFFSET, RESERVED2_OFFSET, SEED_OFFSET, PAYLOAD_LEN_OFFSET, PAYLOAD_START_OFFSET = 9, 15, 22, 38, 46


def _x(seed, n, d=64):
    return np.random.RandomState(seed).randn(n, d).astype(np.float32)


@pytest.fixture(scope="module")
def fib_consts():
    cb, _, _ = O.fib_codebook()
    rot, _ = O.stored_rotation(64, SEED)
    return cb, rot


# ---------------------------------------------------------------- TQW1
def test_tqw1_layout_offsets_and_payload():
    x = _x(1, 9)
    recs = O.turbo_encode_tqw1(x, SEED)
    # proveKV/src/codec.rs:234-237: "TQW1 (per-vector header): 46 + 136 = 182
    # bytes/vector" at head_dim 64, 32 projections, b = 2
    assert len(O.turbo_encode_tqw1(x[:1], SEED, bits=2)[0]) == 182
    blob = O.turbo_encode_batch(x, SEED)          # TQB1, f32 radii
    for i, r in enumerate(recs):
        assert len(r) == 46 + 144
        assert r[:4] == b"TQW1" and struct.unpack_from("<HH", r, 4) == (1, 1) and r[8] == 1
        assert r[RESERVED_OFFSET] == 0 and r[RESERVED2_OFFSET:RESERVED2_OFFSET + 3] == b"\0\0\0"
        assert struct.unpack_from("<I", r, 10)[0] == 64 and r[14] == 3
        assert struct.unpack_from("<I", r, 18)[0] == 32
        assert struct.unpack_from("<Q", r, SEED_OFFSET)[0] == SEED
        assert struct.unpack_from("<II", r, 30) == (32, 32)
        assert struct.unpack_from("<Q", r, PAYLOAD_LEN_OFFSET)[0] == 144
        assert r[PAYLOAD_START_OFFSET:] == blob[38 + 144 * i:38 + 144 * (i + 1)]


def test_tqw1_decode_equals_tqb1_decode():
    x = _x(2, 40)
    recs = O.turbo_encode_tqw1(x, SEED)
    a = O.turbo_decode_tqw1(recs, 64, SEED)
    b = O.turbo_decode_batch(O.turbo_encode_batch(x, SEED), 64, SEED)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_tqw1_polar_only_sign_count_zero():
    x = _x(3, 5)
    recs = O.turbo_encode_tqw1(x, SEED, bits=4, mode=0)
    assert struct.unpack_from("<I", recs[0], 18)[0] == 32       # projections() even without QJL
    assert struct.unpack_from("<I", recs[0], 34)[0] == 0
    assert len(recs[0]) == 46 + 128 + 16
    O.turbo_decode_tqw1(recs, 64, SEED, bits=4, mode=0)


def _tqw1_rejected(recs, i=0, **kw):
    with pytest.raises(O.OracleError) as e:
        O.turbo_decode_tqw1(recs, kw.pop("dim", 64), kw.pop("seed", SEED), **kw)
    assert e.value.index == i


def test_tqw1_rejections_wire_format_rs():
    recs = O.turbo_encode_tqw1(_x(4, 6), SEED)

    def mut(i, f):
        r = [bytearray(t) for t in recs]
        f(r[i])
        return [bytes(t) for t in r]

    _tqw1_rejected(mut(2, lambda r: r.__setitem__(slice(0, 4), b"BAD!")), 2)        # wrong_magic_rejected
    _tqw1_rejected(mut(1, lambda r: struct.pack_into("<H", r, 4, 2)), 1)             # wrong_version_rejected
    _tqw1_rejected(recs[:3] + [recs[3] + b"\0"] + recs[4:], 3)                       # trailing_byte_rejected
    _tqw1_rejected(recs, 0, dim=128)                                                 # dimension_mismatch
    _tqw1_rejected(recs, 0, bits=3)                                                  # bit_width_mismatch
    _tqw1_rejected(recs, 0, proj=64)                                                 # projection_mismatch
    _tqw1_rejected(mut(5, lambda r: struct.pack_into("<Q", r, SEED_OFFSET, 8)), 5)   # seed_mismatch
    _tqw1_rejected(mut(4, lambda r: r.__setitem__(RESERVED_OFFSET, 1)), 4)           # reserved_bytes
    _tqw1_rejected(mut(4, lambda r: r.__setitem__(RESERVED2_OFFSET, 1)), 4)
    _tqw1_rejected(mut(0, lambda r: struct.pack_into("<Q", r, PAYLOAD_LEN_OFFSET, 143)), 0)   # payload_length
    _tqw1_rejected(mut(0, lambda r: struct.pack_into("<Q", r, PAYLOAD_LEN_OFFSET, 145)), 0)
    _tqw1_rejected(mut(1, lambda r: struct.pack_into("<f", r, 46 + 8, -1.0)), 1)     # validate_for radius
    _tqw1_rejected(mut(1, lambda r: struct.pack_into("<f", r, 46, float("nan"))), 1)
    _tqw1_rejected(recs[:2] + [recs[2][:45]] + recs[3:], 2)                          # short record


def test_tqw1_qjl_padding_bits_rejected():
    # wire_format.rs qjl_padding_bits_rejected: projections not a multiple of 8
    x = _x(5, 2)
    recs = O.turbo_encode_tqw1(x, SEED, bits=4, proj=33)
    sign_off = PAYLOAD_START_OFFSET + 32 * 4 + 12
    last = sign_off + 5 - 1
    r = bytearray(recs[1])
    r[last] |= 0b1111_1110
    _tqw1_rejected([recs[0], bytes(r)], 1, proj=33)
    O.turbo_decode_tqw1(recs, 64, SEED, proj=33)


# ---------------------------------------------------------------- FB1
def test_fb1_layout_and_payload(fib_consts):
    cb, rot = fib_consts
    x = _x(6, 20)
    recs = O.fib_encode_fb1(x, cb, rot, each=False)
    blob = O.fib_encode_batch(x, cb, rot)
    # fib-quant/src/codec.rs:78-80 ("23 bytes per block") and the header
    # literal of compact_bytes_roundtrip.rs: "FB1", 1, 5, u32 16, u16 2
    hdr = b"FB1" + bytes([1, 5]) + struct.pack("<I", 16) + struct.pack("<H", 2)
    for i, r in enumerate(recs):
        assert len(r) == 23 and r[:11] == hdr
        assert r[11:] == blob[19 + 12 * i:19 + 12 * (i + 1)]


def test_fb1_each_uses_per_vector_normalisation(fib_consts):
    cb, rot = fib_consts
    x = _x(7, 64)
    each = O.fib_encode_fb1(x, cb, rot, each=True)
    for i in range(0, 64, 7):   # FibQuantizer::encode == encode_batch of one vector (n < 4)
        assert each[i][11:] == O.fib_encode_batch(x[i:i + 1], cb, rot)[19:]
    # batch of >= 4 takes the f32-rounded normalisation; tiny batches the f64 one
    small = O.fib_encode_fb1(x[:3], cb, rot, each=False)
    assert small == each[:3]


def test_fb1_rejections_compact_bytes_roundtrip_rs(fib_consts):
    cb, rot = fib_consts
    good = O.fib_encode_fb1(_x(8, 4), cb, rot, each=True)
    bad_magic = bytes([ord("X"), ord("B"), ord("1"), 1, 5, 0, 0, 0, 16, 0, 0])
    truncated = b"FB1" + bytes([1])
    wrong_ilen = b"FB1" + bytes([1, 5]) + struct.pack("<I", 16) + struct.pack("<H", 2) + b"\0\0" + b"\0"
    bc17 = b"FB1" + bytes([1, 5]) + struct.pack("<I", 17) + struct.pack("<H", 2) + good[0][11:13] + b"\0" * 11
    bad_version = bytes([ord("F"), ord("B"), ord("1"), 2]) + good[0][4:]
    for bad in (bad_magic, truncated, wrong_ilen, bc17, bad_version):
        for each in (True, False):
            with pytest.raises(O.OracleError) as e:
                O.fib_decode_fb1(good[:2] + [bad] + good[2:], cb, rot, each=each)
            assert e.value.index == 2


def test_fb1_batch_parse_errors_take_precedence(fib_consts):
    cb, rot = fib_consts
    recs = O.fib_encode_fb1(_x(9, 8), cb, rot, each=False)
    zero_norm = recs[2][:11] + b"\0\0" + recs[2][13:]          # parses, fails decode_norm
    short = recs[5][:22]                                       # fails from_compact_bytes
    mixed = recs[:2] + [zero_norm] + recs[3:5] + [short] + recs[6:]
    with pytest.raises(O.OracleError) as e:
        O.fib_decode_fb1(mixed, cb, rot, each=False)           # decode_batch: parse pass first
    assert e.value.index == 5
    with pytest.raises(O.OracleError) as e:
        O.fib_decode_fb1(mixed, cb, rot, each=True)            # decode per record: first failure
    assert e.value.index == 2


def test_fb1_same_length_header_failures_are_classified(fib_consts):
    cb, rot = fib_consts
    recs = O.fib_encode_fb1(_x(13, 40), cb, rot, each=False)
    b20 = recs[10][:4] + bytes([4]) + struct.pack("<I", 20) + recs[10][9:]   # parses (20 x 4 bits = 10 B)
    fb2_magic = b"FB2" + recs[30][3:]                                       # fails from_compact_bytes
    mixed = recs[:10] + [b20] + recs[11:30] + [fb2_magic] + recs[31:]
    assert len(b20) == len(fb2_magic) == 23
    with pytest.raises(O.OracleError) as e:
        O.fib_decode_fb1(mixed, cb, rot, each=False)
    assert e.value.index == 30
    with pytest.raises(O.OracleError) as e:
        O.fib_decode_fb1(mixed, cb, rot, each=True)
    assert e.value.index == 10


def test_fb1_batch_decode_equals_fb2_decode(fib_consts):
    cb, rot = fib_consts
    x = _x(10, 30)
    a = O.fib_decode_fb1(O.fib_encode_fb1(x, cb, rot, each=False), cb, rot, each=False)
    b = O.fib_decode_batch(O.fib_encode_batch(x, cb, rot), cb, rot)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_fb1_each_decode_is_the_f64_rotation(fib_consts):
    """out[col] = f32(sum_row M[row][col] * f64(c[row]) * norm) in f64, checked
    against the exact rational value: the f64 sum's error (< 64 u sum|M c|,
    u = 2^-53) is far below half an f32 ulp, so the f32 result must be the
    exact value rounded to nearest, up to that margin."""
    cb, rot = fib_consts
    x = _x(11, 6)
    recs = O.fib_encode_fb1(x, cb, rot, each=True)
    out = O.fib_decode_fb1(recs, cb, rot, each=True)
    fast = O.fib_decode_fb1(recs, cb, rot, each=False)
    M = [[Fraction(float(v)) for v in row] for row in rot]
    differ = 0
    for i, r in enumerate(recs):
        h = struct.unpack_from("<H", r, 11)[0]
        nv = Fraction(float(np.array([h], np.uint16).view(np.float16)[0]))
        bits = int.from_bytes(r[13:23], "little")
        c = []
        for b in range(16):
            c.extend(Fraction(float(v)) for v in cb[(bits >> (5 * b)) & 31])
        for col in range(64):
            exact = sum(M[row][col] * c[row] for row in range(64)) * nv
            mag = sum(abs(M[row][col] * c[row]) for row in range(64)) * nv
            got = Fraction(float(out[i, col]))
            ulp = Fraction(float(np.spacing(np.abs(out[i, col]))))
            assert abs(got - exact) <= ulp / 2 + mag * Fraction(65, 2 ** 53), (i, col)
            differ += int(out[i, col] != fast[i, col])
    assert differ > 0   # the f32 decode_batch_fast path really is a different computation
