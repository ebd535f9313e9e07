"""GPU tests of the library's stream handling: a device-resident segment
table uploaded on one stream and reused by a call on another stream.

The library keeps uploaded segment tables and reuses a table a later call
brings again (every step of a serving loop).  A call on another stream must
not read the table before the upload on the first stream has landed; these
tests queue a long spin ahead of the upload so that the second stream's
kernel would start first if nothing ordered it, and compare both decodes
with the oracle bit for bit.
"""
import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import device as D
from provekv_amd import synth

pytestmark = pytest.mark.gpu
SEED = 42


def _vectors(seed, n, dim=64):
    K, V = synth.kv_cache(seed, 1, 4, (n + 7) // 8, dim)
    return np.ascontiguousarray(np.concatenate([K.reshape(-1, dim), V.reshape(-1, dim)])[:n])


@pytest.mark.parametrize("codec", ["turbo", "fib"])
def test_table_reused_on_second_stream_waits_for_upload(ctx, codec):
    import torch
    n = 3000
    x = _vectors(77, n)
    if codec == "turbo":
        prof = ctx.turbo_profile(64, 4, 32, SEED, 1)
        blob = O.turbo_encode_batch(x, SEED)
        want = O.turbo_decode_batch(blob, 64, SEED)
    else:
        prof = ctx.fib_profile(64, 4, 32, SEED)
        cb, rot = O.fib_codebook(seed=SEED)[0], O.stored_rotation(64, SEED)[0]
        blob = O.fib_encode_batch(x, cb, rot)
        want = O.fib_decode_batch(blob, cb, rot)
    # an element offset no other test uses, so the first call uploads a new table
    off = 4 * 1237 + (0 if codec == "turbo" else 64)
    wire = torch.from_numpy(np.frombuffer(blob, np.uint8).copy()).cuda()
    segs = D.segments([D.contiguous_segment(off, n, 64, 0)])
    outs = [torch.full((off + n * 64,), np.nan, dtype=torch.float32, device="cuda") for _ in range(2)]
    stats = [torch.empty(2, dtype=torch.int32, device="cuda") for _ in range(2)]
    torch.cuda.synchronize()
    a, b = torch.cuda.Stream(), torch.cuda.Stream()   # default priority
    with torch.cuda.stream(a):
        torch.cuda._sleep(100_000_000)   # work queued ahead of the upload on stream a
    prof.decode_segments(wire, segs, outs[0], status=stats[0], stream=a)   # uploads the table on a
    prof.decode_segments(wire, segs, outs[1], status=stats[1], stream=b)   # reuses it on b
    torch.cuda.synchronize()
    for o, s in zip(outs, stats):
        assert prof.status_error(s.cpu().numpy().view(np.uint32), segs) is None
        got = o[off:].cpu().numpy().reshape(n, 64)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        assert np.isnan(o[:off].cpu().numpy()).all()   # nothing written before the segment
