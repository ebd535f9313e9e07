"""Randomised segment tables through pkv_encode_segments / pkv_decode_segments_ex:
strided vector layouts (group, outer and inner strides, gaps), blobs at odd
byte offsets with gaps between them, f32 and bf16 inputs, f32 / bf16 / f16
outputs with fan-out.  Every blob must equal the oracle's batch encode of the
vectors its segment addresses, every decoded vector the oracle decode (in the
output dtype, RNE) at each of its fan-out positions, and every element no
segment addresses must keep its sentinel.  Seeds are fixed."""
import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd.device import segments

pytestmark = pytest.mark.gpu
SEED = 42


def _layout(rng, nseg, dim, align, max_n=600, allow_empty=False):
    """Random non-overlapping strided segments; returns rows and the extent."""
    rows, cursor = [], int(rng.randint(0, 4)) * align
    for _ in range(nseg):
        n = int(rng.randint(0 if allow_empty else 1, max_n))
        g = int(rng.choice([1, max(n, 1), int(rng.randint(1, 40))]))
        si = dim * int(rng.randint(1, 3))
        so = si * g + align * int(rng.randint(0, 3))
        eo = cursor
        if n:
            end = eo + ((n - 1) // g) * so + (min(g, n) - 1) * si + dim
        else:
            end = eo
        rows.append([eo, so, si, 0, n, g])
        cursor = end + align * int(rng.randint(0, 5))
    return rows, cursor


def _positions(row, dim):
    eo, so, si, _, n, g = row
    i = np.arange(n, dtype=np.int64)
    return eo + (i // g) * so + (i % g) * si


def _codec(ctx, kind, dim, lossy):
    if kind == "fib":
        prof = ctx.fib_profile(dim, 4, 32, SEED)
        cb, rot = O.fib_constants(SEED)
        cb, rot = cb.reshape(32, 4), rot.reshape(dim, dim)
        return prof, L.RADII_F32, (lambda x: O.fib_encode_batch(x, cb, rot)), (lambda b: O.fib_decode_batch(b, cb, rot))
    prof = ctx.turbo_profile(dim, 4, 32, SEED)
    radii = L.RADII_LOG_U8 if lossy else L.RADII_F32
    return (prof, radii, (lambda x: O.turbo_encode_batch(x, SEED, radii_codec=int(lossy))),
            (lambda b: O.turbo_decode_batch(b, dim, SEED)))


CASES = [("turbo", 64, False, "float32", "float32", 1, 0), ("turbo", 64, True, "bfloat16", "bfloat16", 2, 1),
         ("turbo", 128, True, "float32", "float16", 3, 2), ("turbo", 128, False, "bfloat16", "float32", 2, 3),
         ("fib", 64, False, "float32", "float32", 1, 4), ("fib", 64, False, "bfloat16", "float16", 3, 5)]


@pytest.mark.parametrize("kind,dim,lossy,in_dt,out_dt,fanout,seed", CASES)
def test_random_segment_tables(ctx, kind, dim, lossy, in_dt, out_dt, fanout, seed):
    import torch
    rng = np.random.RandomState(100 + seed)
    prof, radii, enc, dec = _codec(ctx, kind, dim, lossy)
    tin, tout = getattr(torch, in_dt), getattr(torch, out_dt)
    align_in = 8 if in_dt == "bfloat16" else 4
    rows, extent = _layout(rng, int(rng.randint(3, 9)), dim, align_in)
    x = (rng.randn(extent) * rng.lognormal(0, 0.5, extent)).astype(np.float32)
    xin = torch.from_numpy(x).to(tin)
    xf = xin.to(torch.float32).numpy()          # what the encoder sees (bf16 upcast exactly)
    # blobs back to back at odd offsets
    woff, blobs_ref = int(rng.randint(0, 7)), []
    for r in rows:
        r[3] = woff
        ref = enc(np.ascontiguousarray(xf[_positions(r, dim)[:, None] + np.arange(dim)]))
        blobs_ref.append(ref)
        woff += len(ref) + int(rng.randint(0, 7))
    segs = segments(rows)
    wire = torch.full((woff + 3,), 0xA5, dtype=torch.uint8, device="cuda")
    st = torch.zeros(2 * len(rows), dtype=torch.int32, device="cuda")
    prof.encode_segments(xin.cuda(), segs, wire, radii=radii, status=st)
    torch.cuda.synchronize()
    assert prof.status_error(st.cpu().numpy().view(np.uint32), segs) is None
    w = wire.cpu().numpy()
    for r, ref in zip(rows, blobs_ref):
        assert w[r[3]:r[3] + len(ref)].tobytes() == ref
    # decode the same blobs into another strided layout of the output dtype
    drows, dext = _layout(rng, len(rows), dim, 4)
    for dr, r in zip(drows, rows):   # keep the vector count of each blob
        n = r[4]
        dr[4], dr[3] = n, r[3]
        g = dr[5] if dr[5] <= max(n, 1) else n
        dr[5] = max(g, 1)
        dr[1] = dr[2] * dr[5] + 4 * int(rng.randint(0, 3))
    # re-pack the decode layout without overlaps after the edits above
    cur = 0
    for dr in drows:
        dr[0] = cur
        n, g, so, si = dr[4], dr[5], dr[1], dr[2]
        cur = dr[0] + ((n - 1) // g) * so + (min(g, n) - 1) * si + dim + 4 * int(rng.randint(0, 4))
    stride = (cur + 3) // 4 * 4
    out = torch.full((stride * fanout,), 7.0, dtype=tout, device="cuda")
    dsegs = segments(drows)
    dst = torch.zeros(2 * len(drows), dtype=torch.int32, device="cuda")
    prof.decode_segments(wire, dsegs, out, radii=radii, status=dst, fanout=fanout, fanout_stride=stride)
    torch.cuda.synchronize()
    assert prof.status_error(dst.cpu().numpy().view(np.uint32), dsegs) is None
    got = out.cpu()
    touched = np.zeros(stride, bool)
    for dr, ref in zip(drows, blobs_ref):
        want = torch.from_numpy(np.ascontiguousarray(dec(ref).reshape(-1, dim))).to(tout)
        idx = _positions(dr, dim)[:, None] + np.arange(dim)
        touched[idx.reshape(-1)] = True
        for k in range(fanout):
            rows_got = got[k * stride:(k + 1) * stride][torch.from_numpy(idx.reshape(-1))].reshape(-1, dim)
            bits = torch.int32 if out_dt == "float32" else torch.int16
            assert torch.equal(rows_got.view(bits), want.view(bits))
    for k in range(fanout):
        rest = got[k * stride:(k + 1) * stride][torch.from_numpy(~touched)]
        assert torch.all(rest == 7.0)


@pytest.mark.parametrize("kind", ["fib", "turbo"])
def test_header_only_blobs(ctx, kind):
    """A blob that holds no vectors (n = 0): both batched decoders accept it
    (fib-quant/src/codec.rs:323-402, turbo-quant/src/wire.rs:401-568) and
    decode_batch_fast(&[]) returns nothing (fib-quant/tests/
    decode_batch_fast_parity.rs:52-60).  The compact decode returns no
    vectors; between two non-empty blobs of one segment table it decodes to
    nothing while the others decode as the oracle's; its header is still
    checked."""
    import torch
    from provekv_amd.device import segments
    prof, radii, enc, dec = _codec(ctx, kind, 64, False)
    hl = int(L.lib().pkv_header_len(prof._ptr))
    nfield = 10 if kind == "fib" else 30          # the u32 vector count in the header
    rng = np.random.RandomState(9)
    xa, xb = rng.randn(5, 64).astype(np.float32), rng.randn(7, 64).astype(np.float32)
    ba, bb = enc(xa), enc(xb)
    empty = bytearray(ba[:hl])
    empty[nfield:nfield + 4] = b"\0\0\0\0"
    assert prof.decode_batch_compact(bytes(empty)).shape == (0, 64)
    wire = torch.from_numpy(np.frombuffer(ba + bytes(empty) + bb, np.uint8).copy()).cuda()
    segs = segments([(0, 64, 64, 0, 5, 1), (5 * 64, 64, 64, len(ba), 0, 1), (5 * 64, 64, 64, len(ba) + hl, 7, 1)])
    want = np.concatenate([dec(ba), dec(bb)]).reshape(-1)
    for corrupt in (False, True):
        if corrupt:
            wire[len(ba)] ^= 0xFF                    # the empty blob's magic
        out = torch.full((12 * 64,), 7.0, dtype=torch.float32, device="cuda")
        st = torch.zeros(6, dtype=torch.int32, device="cuda")
        prof.decode_segments(wire, segs, out, radii=radii, status=st)
        torch.cuda.synchronize()
        err = prof.status_error(st.cpu().numpy().view(np.uint32), segs)
        if not corrupt:
            assert err is None
            assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))
        else:
            assert err is not None and err.segment == 1 and err.status == L.ERR_CORRUPT_PAYLOAD


@pytest.mark.parametrize("kind", ["fib", "turbo"])
def test_calls_without_status_words_fail_closed(ctx, kind):
    """Without the caller's status words (d_status = NULL) a segment call
    reports a rejected blob or input itself, as the reference's decode /
    encode return the error: the call waits for its kernels and returns the
    error's code (the segment and vector are in the status words, for a
    caller that passes them); a clean call returns normally with the same
    bytes."""
    import torch
    prof, radii, enc, dec = _codec(ctx, kind, 64, False)
    rng = np.random.RandomState(11)
    xa, xb = rng.randn(9, 64).astype(np.float32), rng.randn(6, 64).astype(np.float32)
    ba, bb = enc(xa), enc(xb)
    segs = segments([(0, 64, 64, 0, 9, 1), (9 * 64, 64, 64, len(ba), 6, 1)])
    wire = torch.from_numpy(np.frombuffer(ba + bb, np.uint8).copy()).cuda()
    out = torch.zeros(15 * 64, dtype=torch.float32, device="cuda")
    prof.decode_segments(wire, segs, out, radii=radii)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), np.concatenate([dec(ba), dec(bb)]).reshape(-1).view(np.uint32))
    wire[len(ba)] ^= 0xFF                                   # the second blob's magic
    with pytest.raises(L.PkvError) as e:
        prof.decode_segments(wire, segs, out, radii=radii)
    assert e.value.status == L.ERR_CORRUPT_PAYLOAD
    # encode: a non-finite input in the second segment
    x = np.concatenate([xa, xb])
    x[11, 5] = np.inf
    inp = torch.from_numpy(x.reshape(-1)).cuda()
    wout = torch.empty(len(ba) + len(bb), dtype=torch.uint8, device="cuda")
    with pytest.raises(L.PkvError) as e:
        prof.encode_segments(inp, segs, wout, radii=radii)
    assert e.value.status == L.ERR_NONFINITE_INPUT
    x[11, 5] = 0.5
    inp = torch.from_numpy(x.reshape(-1)).cuda()
    prof.encode_segments(inp, segs, wout, radii=radii)
    assert wout.cpu().numpy().tobytes()[:len(ba)] == ba
