"""GPU test of pkv_decode_segments_noalloc, called through the C ABI: the
entry point that allocates nothing (segment table, tile prefix and status
words in the library's fixed per-GPU scratch) must decode exactly what
pkv_decode_segments_ex decodes, bit for bit, on consecutive calls of
different sizes, and report the same status words."""
import ctypes as C

import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd import device as D
from provekv_amd import synth
from provekv_amd.pool import DeviceKVCache, TwoTierPlan

pytestmark = pytest.mark.gpu
SEED = 42


def _dtype_code(t):
    import torch
    return {torch.float32: L.DT_F32, torch.bfloat16: L.DT_BF16, torch.float16: L.DT_F16}[t.dtype]


def _noalloc(prof, wire, segs, out, radii, fanout, fanout_stride, status, stream):
    segs = np.ascontiguousarray(segs, dtype=D.SEG_DTYPE)
    return L.lib().pkv_decode_segments_noalloc(
        prof.ctx.ptr, prof.ptr, radii, wire.data_ptr(), wire.numel(), segs.ctypes.data, len(segs), out.data_ptr(),
        _dtype_code(out), out.numel(), fanout, fanout_stride, None if status is None else status.data_ptr(),
        C.c_void_p(stream.cuda_stream))


def _bits(t):
    import torch
    return t.view(torch.int32) if t.element_size() == 4 else t.view(torch.int16)


def _rehydrate_both_ways(ctx, layers, heads, prefix, agents, dtype, copies, lossy, corpus_seed, with_status):
    """Encode a two-tier plan, rehydrate it into two caches (existing entry
    point / no-allocation entry point) and compare them and the status words."""
    import torch
    plan = TwoTierPlan(ctx, layers, heads, 64, prefix, agents, seed=SEED, lossy=lossy)
    corpus = synth.corpus_tokens(corpus_seed, layers, heads, plan.tokens, 64)
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    bufs = plan.alloc()
    plan.encode(dev, bufs)
    torch.cuda.synchronize()
    plan.check(bufs, decode=False)
    caches = [DeviceKVCache(layers, heads, plan.tokens, 64, dtype=dtype, copies=copies) for _ in range(2)]
    for c in caches:
        c.buf.fill_(float("nan"))
    firsts, t = [], prefix
    for nt in agents:
        firsts.append(t)
        t += nt
    stream = torch.cuda.current_stream()
    tiers = [(plan.fib, bufs["pool_wire"], caches[0].segments_for(plan.pool, [0]), L.RADII_F32),
             (plan.turbo, bufs["shell_wire"], caches[0].segments_for(plan.shells, firsts), plan.radii)]
    for prof, wire, segs, radii in tiers:
        st_a = torch.full((2 * len(segs),), -7, dtype=torch.int32, device="cuda")
        st_b = torch.full((2 * len(segs),), -7, dtype=torch.int32, device="cuda") if with_status else None
        prof.decode_segments(wire, segs, caches[0].buf.view(-1), radii=radii, status=st_a, fanout=copies,
                             fanout_stride=caches[0].copy_stride)
        rc = _noalloc(prof, wire, segs, caches[1].buf.view(-1), radii, copies, caches[1].copy_stride, st_b, stream)
        assert rc == L.OK, L.status_string(rc)
        torch.cuda.synchronize()
        assert prof.status_error(st_a.cpu().numpy().view(np.uint32), segs) is None
        if with_status:
            assert torch.equal(st_a, st_b)
    torch.cuda.synchronize()
    assert torch.equal(_bits(caches[0].buf), _bits(caches[1].buf))
    assert not torch.isnan(caches[1].buf.float()).any()
    # the first pool blob against the oracle (its own constants), every copy
    cb, rot = O.fib_codebook(seed=SEED)[0], O.stored_rotation(64, SEED)[0]
    want = O.fib_decode_batch(plan.blob(bufs, "pool", 0), cb, rot)
    want = torch.from_numpy(np.ascontiguousarray(want.reshape(prefix, heads, 64).transpose(1, 0, 2))).to(dtype)
    for k in range(copies):
        assert torch.equal(_bits(caches[1].buf[k, 0, 0, :, :prefix, :].cpu()), _bits(want))
    return plan, bufs


def test_noalloc_matches_decode_segments_ex_two_calls(ctx):
    import torch
    # first call: the larger table (f32 caches, 3 copies, lossless shells, caller's status words)
    _rehydrate_both_ways(ctx, 4, 8, 200, [30, 20, 10], torch.float32, 3, False, 5, True)
    # second call: a smaller table over the same scratch (bf16, 1 copy, lossy shells, status in the scratch)
    _rehydrate_both_ways(ctx, 2, 4, 50, [7], torch.bfloat16, 1, True, 6, False)


def test_noalloc_rejects_header_like_decode_segments_ex(ctx):
    """A corrupt blob header: both entry points leave the segment's output
    untouched and report the same status words."""
    import torch
    plan, bufs = _rehydrate_both_ways(ctx, 2, 4, 40, [6, 6], torch.float32, 2, False, 7, True)
    wire = bufs["pool_wire"].clone()
    _, _, _, off, _ = plan.pool.blob_offsets[1]
    wire[off] = ord("X")   # FB2 magic of blob 1
    caches = [DeviceKVCache(2, 4, plan.tokens, 64, copies=2) for _ in range(2)]
    segs = caches[0].segments_for(plan.pool, [0])
    sts = [torch.full((2 * len(segs),), -7, dtype=torch.int32, device="cuda") for _ in range(2)]
    plan.fib.decode_segments(wire, segs, caches[0].buf.view(-1), status=sts[0], fanout=2,
                             fanout_stride=caches[0].copy_stride)
    rc = _noalloc(plan.fib, wire, segs, caches[1].buf.view(-1), L.RADII_F32, 2, caches[1].copy_stride, sts[1],
                  torch.cuda.current_stream())
    assert rc == L.OK
    torch.cuda.synchronize()
    assert torch.equal(sts[0], sts[1])
    err = plan.fib.status_error(sts[1].cpu().numpy().view(np.uint32), segs)
    assert err is not None and err.status == L.ERR_CORRUPT_PAYLOAD and err.segment == 1
    assert torch.equal(caches[0].buf.view(torch.int32), caches[1].buf.view(torch.int32))


def test_noalloc_rejects_tables_beyond_its_scratch(ctx):
    import torch
    prof = ctx.turbo_profile(64, 4, 32, SEED, 1)
    n = L.NOALLOC_MAX_SEGMENTS + 1
    segs = D.segments([(0, 0, 64, 0, 0, 1)] * n)
    wire = torch.zeros(38 * n, dtype=torch.uint8, device="cuda")
    out = torch.zeros(64, dtype=torch.float32, device="cuda")
    rc = _noalloc(prof, wire, segs, out, L.RADII_F32, 1, 0, None, torch.cuda.current_stream())
    assert rc == L.ERR_SCRATCH_LIMIT
    assert "scratch" in L.status_string(rc)
