"""GPU parity for scoring on compressed codes (TurboQuantizer::prepare_query /
inner_product_estimate_prepared / score_batch_prepared, turbo-quant/src/
turbo.rs:316-381; AttentionScale of KvShadowCache::attention_scores_with_options,
kv.rs:269-320), through the C ABI, against the CPU oracle.

Bar: bit-exact.  The prepared queries (rotation + QJL projection) and every
score are compared as raw f32 bits with the oracle's sequential restatement;
errors must name the same query / code the oracle names.
"""
import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd import synth
from provekv_amd.device import segments

pytestmark = pytest.mark.gpu
SEED = 42

# (dim, bits, proj, mode): bits counts the QJL bit when mode = 1
PROFILES = [(64, 4, 32, 1), (64, 3, 32, 0), (64, 4, 64, 1), (128, 4, 32, 1), (128, 3, 32, 0), (128, 4, 64, 1),
            (64, 5, 32, 1), (128, 2, 32, 0)]


def _keys(seed, n, dim):
    K, V = synth.kv_cache(seed, 1, 4, (n + 7) // 8, dim)
    return np.ascontiguousarray(np.concatenate([K.reshape(-1, dim), V.reshape(-1, dim)])[:n])


def _queries(seed, nq, dim):
    return np.random.RandomState(seed).randn(nq, dim).astype(np.float32)


def _bits_equal(a, b):
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _profile(ctx, dim, bits, proj, mode):
    return ctx.turbo_profile(dim, bits, proj, SEED, mode)


@pytest.mark.parametrize("dim,bits,proj,mode", PROFILES)
def test_prepare_queries_bit_exact(ctx, dim, bits, proj, mode):
    import torch
    prof = _profile(ctx, dim, bits, proj, mode)
    q = _queries(dim + bits, 37, dim)
    q[3] = 0.0                                    # all-zero query: zero signs kept as the reference folds them
    dq = torch.from_numpy(q).cuda()
    prep = prof.prepare_queries(dq).cpu().numpy()
    ref = O.turbo_prepare_queries(q, SEED, proj=proj, mode=mode)
    assert prep.shape == (37, dim + (proj if mode else 0))
    assert _bits_equal(prep, ref)


@pytest.mark.parametrize("dim,bits,proj,mode", PROFILES)
@pytest.mark.parametrize("lossy", [False, True])
def test_score_batch_bit_exact(ctx, dim, bits, proj, mode, lossy):
    prof = _profile(ctx, dim, bits, proj, mode)
    x = _keys(dim * 3 + bits, 333, dim)
    blob = O.turbo_encode_batch(x, SEED, bits=bits, proj=proj, mode=mode, radii_codec=int(lossy))
    q = _queries(7, 5, dim)
    got = prof.score_batch(blob, q)
    ref = O.turbo_score(blob, O.turbo_prepare_queries(q, SEED, proj=proj, mode=mode), dim, SEED,
                        bits=bits, proj=proj, mode=mode)
    assert _bits_equal(got, ref)


def _empty_blob(dim=64, **kw):
    """A valid 0-code TQB1 blob: a 1-code header with its count set to 0."""
    hdr = O.turbo_encode_batch(np.ones((1, dim), np.float32), SEED, **kw)[:38]
    return hdr[:30] + (0).to_bytes(4, "little") + hdr[34:38]


@pytest.mark.parametrize("n", [0, 1, 63, 64, 65, 256, 257])
def test_score_batch_sizes(ctx, n):
    prof = _profile(ctx, 64, 4, 32, 1)
    blob = O.turbo_encode_batch(_keys(n + 1, n, 64), SEED) if n else _empty_blob()
    q = _queries(n, 3, 64)
    got = prof.score_batch(blob, q)
    assert got.shape == (3, n)
    if n:
        assert _bits_equal(got, O.turbo_score(blob, O.turbo_prepare_queries(q, SEED), 64, SEED))


def test_post_scale_is_applied_after_the_score(ctx):
    """AttentionScale::ByHeadDim: each score times 1/sqrt(head_dim) (kv.rs:305-318)."""
    prof = _profile(ctx, 128, 4, 32, 1)
    x = _keys(11, 200, 128)
    blob = O.turbo_encode_batch(x, SEED)
    q = _queries(12, 4, 128)
    scale = np.float32(1.0) / np.sqrt(np.float32(128.0))
    got = prof.score_batch(blob, q, post_scale=float(scale))
    ref = O.turbo_score(blob, O.turbo_prepare_queries(q, SEED), 128, SEED) * scale
    assert _bits_equal(got, ref)


def test_score_segments_strided_columns(ctx):
    """Several blobs in one launch; codes of segment s land at strided score
    columns (token-major, head-interleaved like a [T, H] logits row)."""
    import torch
    prof = _profile(ctx, 64, 4, 32, 1)
    H, T = 4, 150
    blobs, rows, off = [], [], 0
    for h in range(H):
        b = O.turbo_encode_batch(_keys(100 + h, T, 64), SEED, radii_codec=h % 2)
        rows.append((h, H, 0, off, T, 1))                # col(i) = h + i * H
        blobs.append(b)
        off += len(b)
    wire = torch.from_numpy(np.frombuffer(b"".join(blobs), np.uint8).copy()).cuda()
    q = _queries(5, 6, 64)
    prep = prof.prepare_queries(torch.from_numpy(q).cuda())
    ld = H * T + 3
    scores = torch.full((6 * ld,), 7.0, dtype=torch.float32, device="cuda")
    status = torch.zeros(2 * H, dtype=torch.int32, device="cuda")
    segs = segments(rows)
    for h in range(H):   # radii codec differs per blob: one launch per codec
        sel = segs[h:h + 1]
        prof.score_segments(wire, sel, prep, scores, ld, radii=h % 2, status=status[2 * h:2 * h + 2])
    torch.cuda.synchronize()
    assert prof.score_status_error(status.cpu().numpy().view(np.uint32)) is None
    got = scores.cpu().numpy().reshape(6, ld)
    pref = O.turbo_prepare_queries(q, SEED)
    for h in range(H):
        ref = O.turbo_score(blobs[h], pref, 64, SEED)
        assert _bits_equal(got[:, h:H * T:H], ref)
    assert np.all(got[:, H * T:] == 7.0)            # columns past the codes untouched


def test_score_segments_one_launch_many_blobs(ctx):
    import torch
    prof = _profile(ctx, 128, 4, 32, 1)
    sizes = [1, 64, 300, 0, 513]
    blobs = [O.turbo_encode_batch(_keys(50 + i, n, 128), SEED) if n else None for i, n in enumerate(sizes)]
    raw, rows, off, col = [], [], 0, 0
    for n, b in zip(sizes, blobs):
        if b is None:
            b = _empty_blob(128)
        rows.append((col, 1, 1, off, n, 1))
        raw.append(b)
        off += len(b)
        col += n
    wire = torch.from_numpy(np.frombuffer(b"".join(raw), np.uint8).copy()).cuda()
    q = _queries(9, 3, 128)
    prep = prof.prepare_queries(torch.from_numpy(q).cuda())
    scores = torch.zeros(3 * col, dtype=torch.float32, device="cuda")
    status = torch.zeros(2 * len(sizes), dtype=torch.int32, device="cuda")
    prof.score_segments(wire, segments(rows), prep, scores, col, status=status)
    torch.cuda.synchronize()
    assert prof.score_status_error(status.cpu().numpy().view(np.uint32)) is None
    got = scores.cpu().numpy().reshape(3, col)
    pref = O.turbo_prepare_queries(q, SEED)
    c = 0
    for n, b in zip(sizes, blobs):
        if n:
            assert _bits_equal(got[:, c:c + n], O.turbo_score(b, pref, 128, SEED))
        c += n


def test_score_segments_query_groups(ctx):
    """GQA layout: segment s = one KV head's keys, scored against its own
    group of G query heads (prepared rows s*G .. s*G+G-1); scores[g][s*T + t]."""
    import torch
    prof = _profile(ctx, 128, 4, 32, 1)
    S, T, G = 3, 200, 4
    blobs = [O.turbo_encode_batch(_keys(70 + s, T, 128), SEED, radii_codec=1) for s in range(S)]
    offs = np.cumsum([0] + [len(b) for b in blobs])
    wire = torch.from_numpy(np.frombuffer(b"".join(blobs), np.uint8).copy()).cuda()
    q = _queries(77, S * G, 128)
    prep = prof.prepare_queries(torch.from_numpy(q).cuda())
    scores = torch.zeros(G * S * T, dtype=torch.float32, device="cuda")
    status = torch.zeros(2 * S, dtype=torch.int32, device="cuda")
    segs = segments([(s * T, 1, 1, offs[s], T, 1) for s in range(S)])
    prof.score_segments(wire, segs, prep, scores, S * T, radii=L.RADII_LOG_U8, status=status, nq=G, query_stride=G)
    torch.cuda.synchronize()
    assert prof.score_status_error(status.cpu().numpy().view(np.uint32)) is None
    got = scores.cpu().numpy().reshape(G, S * T)
    pref = O.turbo_prepare_queries(q, SEED)
    for s in range(S):
        assert _bits_equal(got[:, s * T:(s + 1) * T], O.turbo_score(blobs[s], pref[s * G:(s + 1) * G], 128, SEED))
    with pytest.raises(L.PkvError) as e:                    # the last group would run past the prepared rows
        prof.score_segments(wire, segs, prep[:S * G - 1], scores, S * T, radii=L.RADII_LOG_U8, nq=G, query_stride=G)
    assert e.value.status == L.ERR_DIM_MISMATCH


def test_nonfinite_query_is_reported_by_index(ctx):
    prof = _profile(ctx, 64, 4, 32, 1)
    blob = O.turbo_encode_batch(_keys(3, 10, 64), SEED)
    q = _queries(3, 4, 64)
    q[2, 5] = np.nan
    with pytest.raises(O.OracleError) as eo:
        O.turbo_prepare_queries(q, SEED)
    with pytest.raises(L.PkvError) as e:
        prof.score_batch(blob, q)
    assert e.value.status == L.ERR_NONFINITE_INPUT and e.value.index == eo.value.index == 2


def test_overflowing_score_is_reported_by_code(ctx):
    """Radii ~1e18 against queries ~1e21: only code 9's score overflows."""
    prof = _profile(ctx, 64, 4, 32, 1)
    x = _keys(6, 64, 64)
    x[9] *= np.float32(1e18)
    blob = O.turbo_encode_batch(x, SEED)
    q = _queries(6, 5, 64) * np.float32(1e21)
    with pytest.raises(O.OracleError) as eo:
        O.turbo_score(blob, O.turbo_prepare_queries(q, SEED), 64, SEED)
    with pytest.raises(L.PkvError) as e:
        prof.score_batch(blob, q)
    assert e.value.status == L.ERR_CORRUPT_PAYLOAD and e.value.index == eo.value.index == 9


def test_rejected_code_precedes_nonfinite_score(ctx):
    """A corrupt radius at code 40 is reported even though code 9's score
    overflows first: the blob is validated before any score."""
    prof = _profile(ctx, 64, 4, 32, 1)
    x = _keys(6, 64, 64)
    x[9] *= np.float32(1e18)
    blob = bytearray(O.turbo_encode_batch(x, SEED))
    plen = prof.payload_len()
    blob[38 + 40 * plen + 4 * 3: 38 + 40 * plen + 4 * 4] = np.float32(-1.0).tobytes()   # radius 3 of code 40 < 0
    q = _queries(6, 5, 64) * np.float32(1e21)
    with pytest.raises(O.OracleError) as eo:
        O.turbo_score(bytes(blob), O.turbo_prepare_queries(q, SEED), 64, SEED)
    with pytest.raises(L.PkvError) as e:
        prof.score_batch(bytes(blob), q)
    assert e.value.status == L.ERR_CORRUPT_PAYLOAD and e.value.index == eo.value.index == 40


def test_header_mismatch_writes_no_score(ctx):
    import torch
    prof = _profile(ctx, 64, 4, 32, 1)
    blob = bytearray(O.turbo_encode_batch(_keys(8, 20, 64), SEED))
    blob[22] ^= 1                                           # seed field
    wire = torch.from_numpy(np.frombuffer(bytes(blob), np.uint8).copy()).cuda()
    prep = prof.prepare_queries(torch.from_numpy(_queries(8, 2, 64)).cuda())
    scores = torch.full((40,), 3.0, dtype=torch.float32, device="cuda")
    status = torch.zeros(2, dtype=torch.int32, device="cuda")
    prof.score_segments(wire, segments([(0, 1, 1, 0, 20, 1)]), prep, scores, 20, status=status)
    torch.cuda.synchronize()
    err = prof.score_status_error(status.cpu().numpy().view(np.uint32))
    assert err is not None and err.status == L.ERR_CORRUPT_PAYLOAD
    assert torch.all(scores == 3.0)


def test_score_segments_rejects_bad_extents(ctx):
    import torch
    prof = _profile(ctx, 64, 4, 32, 1)
    blob = O.turbo_encode_batch(_keys(8, 20, 64), SEED)
    wire = torch.from_numpy(np.frombuffer(blob, np.uint8).copy()).cuda()
    prep = prof.prepare_queries(torch.from_numpy(_queries(8, 2, 64)).cuda())
    scores = torch.zeros(40, dtype=torch.float32, device="cuda")
    with pytest.raises(L.PkvError) as e:                    # column 20 >= ld
        prof.score_segments(wire, segments([(1, 1, 1, 0, 20, 1)]), prep, scores, 20)
    assert e.value.status == L.ERR_DIM_MISMATCH
    with pytest.raises(L.PkvError) as e:                    # second row past the buffer
        prof.score_segments(wire, segments([(0, 1, 1, 0, 20, 1)]), prep, scores[:39], 20)
    assert e.value.status == L.ERR_DIM_MISMATCH
    with pytest.raises(L.PkvError) as e:
        prof.score_segments(wire, segments([(0, 1, 1, 0, 20, 1)]), prep, scores, 20, post_scale=float("inf"))
    assert e.value.status == L.ERR_INVALID_ARG
