"""GPU test of pkv_decode_segments_noalloc, called through the C ABI: the
entry point that allocates nothing (segment table and tile prefix in the
library's fixed per-GPU scratch) must decode exactly what
pkv_decode_segments_ex decodes, bit for bit, on consecutive calls of
different sizes, and report the same status words; it refuses to run without
status words (a rejected blob would otherwise pass silently) and under graph
capture, and its calls from two streams and two contexts of one GPU, which
share the scratch, are ordered on the device."""
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


def _rehydrate_both_ways(ctx, layers, heads, prefix, agents, dtype, copies, lossy, corpus_seed):
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
        st_b = torch.full((2 * len(segs),), -7, dtype=torch.int32, device="cuda")
        prof.decode_segments(wire, segs, caches[0].buf.view(-1), radii=radii, status=st_a, fanout=copies,
                             fanout_stride=caches[0].copy_stride)
        rc = _noalloc(prof, wire, segs, caches[1].buf.view(-1), radii, copies, caches[1].copy_stride, st_b, stream)
        assert rc == L.OK, L.status_string(rc)
        torch.cuda.synchronize()
        assert prof.status_error(st_a.cpu().numpy().view(np.uint32), segs) is None
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
    # first call: the larger table (f32 caches, 3 copies, lossless shells)
    _rehydrate_both_ways(ctx, 4, 8, 200, [30, 20, 10], torch.float32, 3, False, 5)
    # second call: a smaller table over the same scratch (bf16, 1 copy, lossy shells)
    _rehydrate_both_ways(ctx, 2, 4, 50, [7], torch.bfloat16, 1, True, 6)


def test_noalloc_rejects_header_like_decode_segments_ex(ctx):
    """A corrupt blob header: both entry points leave the segment's output
    untouched and report the same status words."""
    import torch
    plan, bufs = _rehydrate_both_ways(ctx, 2, 4, 40, [6, 6], torch.float32, 2, False, 7)
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
    st = torch.zeros(2 * n, dtype=torch.int32, device="cuda")
    rc = _noalloc(prof, wire, segs, out, L.RADII_F32, 1, 0, st, torch.cuda.current_stream())
    assert rc == L.ERR_SCRATCH_LIMIT
    assert "scratch" in L.status_string(rc)


def _corrupt_pool(ctx):
    import torch
    plan, bufs = _rehydrate_both_ways(ctx, 2, 4, 40, [6, 6], torch.float32, 1, False, 8)
    wire = bufs["pool_wire"].clone()
    _, _, _, off, _ = plan.pool.blob_offsets[1]
    wire[off] = ord("X")   # FB2 magic of blob 1
    cache = DeviceKVCache(2, 4, plan.tokens, 64, copies=1)
    return plan, wire, cache, cache.segments_for(plan.pool, [0])


def test_noalloc_refuses_to_run_without_status_words(ctx):
    """Fails closed: with no status words a rejected blob could not be
    reported, so the call refuses before any work and writes nothing."""
    import torch
    plan, wire, cache, segs = _corrupt_pool(ctx)
    cache.buf.fill_(float("nan"))
    rc = _noalloc(plan.fib, wire, segs, cache.buf.view(-1), L.RADII_F32, 1, cache.copy_stride, None,
                  torch.cuda.current_stream())
    assert rc == L.ERR_INVALID_ARG
    torch.cuda.synchronize()
    assert torch.isnan(cache.buf).all()


def test_noalloc_refuses_graph_capture(ctx):
    """The table is copied from host memory on every call, which a graph could
    not replay: under capture the call returns UNSUPPORTED and enqueues nothing."""
    import torch
    plan, wire, cache, segs = _corrupt_pool(ctx)
    st = torch.full((2 * len(segs),), -7, dtype=torch.int32, device="cuda")
    x = torch.zeros(16, device="cuda")
    g = torch.cuda.CUDAGraph()
    codes = []
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        x.add_(1.0)
        codes.append(_noalloc(plan.fib, wire, segs, cache.buf.view(-1), L.RADII_F32, 1, cache.copy_stride, st,
                              torch.cuda.current_stream()))
    torch.cuda.synchronize()
    assert codes == [L.ERR_UNSUPPORTED]
    assert (st == -7).all()
    del g


def test_noalloc_two_streams_and_two_contexts(ctx):
    """Calls that share the per-GPU scratch from two streams, and from a second
    context on the same device, issued back to back with no host wait between
    them: each must decode what pkv_decode_segments_ex decodes."""
    import torch
    from provekv_amd.device import Context
    ctx2 = Context(0)
    try:
        jobs = []
        for c, (layers, heads, prefix, agents, seed) in zip(
                (ctx, ctx2, ctx, ctx2),
                ((4, 8, 300, [40, 12], 11), (3, 4, 120, [9], 12), (2, 8, 64, [5, 5, 5], 13), (5, 2, 90, [3], 14))):
            plan = TwoTierPlan(c, layers, heads, 64, prefix, agents, seed=SEED)
            corpus = synth.corpus_tokens(seed, layers, heads, plan.tokens, 64)
            bufs = plan.alloc()
            plan.encode(torch.from_numpy(corpus.reshape(-1)).cuda(), bufs)
            firsts, t = [], prefix
            for nt in agents:
                firsts.append(t)
                t += nt
            caches = [DeviceKVCache(layers, heads, plan.tokens, 64, copies=2) for _ in range(2)]
            for cc in caches:
                cc.buf.fill_(float("nan"))
            jobs.append((plan, bufs, caches, firsts))
        calls = []
        for plan, bufs, caches, firsts in jobs:
            for prof, wire, segs, radii in ((plan.fib, bufs["pool_wire"], caches[1].segments_for(plan.pool, [0]),
                                             L.RADII_F32),
                                            (plan.turbo, bufs["shell_wire"],
                                             caches[1].segments_for(plan.shells, firsts), plan.radii)):
                st = torch.full((2 * len(segs),), -7, dtype=torch.int32, device="cuda")
                calls.append((prof, wire, segs, radii, caches[1], st))
        torch.cuda.synchronize()   # inputs, caches and status words ready before the side streams use them
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        stats = []
        for j, (prof, wire, segs, radii, cache, st) in enumerate(calls):
            rc = _noalloc(prof, wire, segs, cache.buf.view(-1), radii, 2, cache.copy_stride, st, streams[(j // 2) % 2])
            assert rc == L.OK, L.status_string(rc)
            stats.append((prof, st, segs))
        torch.cuda.synchronize()
        for prof, st, segs in stats:
            assert prof.status_error(st.cpu().numpy().view(np.uint32), segs) is None
        for plan, bufs, caches, firsts in jobs:
            plan.fib.decode_segments(bufs["pool_wire"], caches[0].segments_for(plan.pool, [0]), caches[0].buf.view(-1),
                                     fanout=2, fanout_stride=caches[0].copy_stride)
            plan.turbo.decode_segments(bufs["shell_wire"], caches[0].segments_for(plan.shells, firsts),
                                       caches[0].buf.view(-1), radii=plan.radii, fanout=2,
                                       fanout_stride=caches[0].copy_stride)
        torch.cuda.synchronize()
        for plan, bufs, caches, firsts in jobs:
            assert torch.equal(_bits(caches[0].buf), _bits(caches[1].buf))
            assert not torch.isnan(caches[1].buf).any()
    finally:
        torch.cuda.synchronize()
        ctx2.close()
