"""GPU parity of the batched two-tier path (all (owner, layer, K|V) blobs in
one launch per tier) against per-blob oracle calls on the gathered vectors,
plus the receipt byte math at the N=8 SmolLM2 shape."""
import ctypes
import struct

import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd import synth
from provekv_amd.device import SEG_DTYPE, Profile
from provekv_amd.pool import TwoTierPlan

pytestmark = pytest.mark.gpu
SEED = 42


def gather(corpus, t0, nt, layer, side):
    # proveKV/src/pool.rs:246-257: token-major, head-minor
    return np.ascontiguousarray(corpus[t0:t0 + nt, layer, :, side, :].reshape(-1, corpus.shape[-1]))


@pytest.mark.parametrize("lossy", [False, True])
def test_two_tier_small_bit_exact(ctx, lossy):
    import torch
    layers, heads, dim, prefix, agents = 3, 4, 64, 37, [5, 1, 9]
    corpus = synth.corpus_tokens(3, layers, heads, prefix + sum(agents), dim)
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=SEED, lossy=lossy)
    bufs = plan.alloc()
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    plan.encode(dev, bufs)
    plan.decode(bufs)
    torch.cuda.synchronize()
    plan.check(bufs)
    cb, rot = O.fib_constants(SEED)
    cb = cb.reshape(32, 4)
    rot = rot.reshape(dim, dim)
    pool_out = bufs["pool_out"].cpu().numpy()
    for i, (_, layer, side, _, ln) in enumerate(plan.pool.blob_offsets):
        x = gather(corpus, 0, prefix, layer, side)
        ref = O.fib_encode_batch(x, cb, rot)
        assert plan.blob(bufs, "pool", i) == ref
        n = x.shape[0]
        got = pool_out[plan.pool.dec[i]["elem_offset"]:][: n * dim].reshape(n, dim)
        assert np.array_equal(got, O.fib_decode_batch(ref, cb, rot))
    shell_out = bufs["shell_out"].cpu().numpy()
    t = prefix
    k = 0
    for nt in agents:
        for layer in range(layers):
            for side in (0, 1):
                x = gather(corpus, t, nt, layer, side)
                ref = O.turbo_encode_batch(x, SEED, radii_codec=int(lossy))
                assert plan.blob(bufs, "shell", k) == ref
                n = x.shape[0]
                got = shell_out[plan.shells.dec[k]["elem_offset"]:][: n * dim].reshape(n, dim)
                assert np.array_equal(got, O.turbo_decode_batch(ref, dim, SEED))
                k += 1
        t += nt


def test_smollm2_n8_receipt_bytes(ctx):
    """CLAIMS.json:34-37,61-64: pool 14,746,512 B; shells 6,194,976 B (TQB1)
    / 2,410,272 B (TQB1-L) per agent; system 64,306,320 / 34,028,688 B."""
    for lossy, shell, system in ((False, 6194976, 64306320), (True, 2410272, 34028688)):
        plan = TwoTierPlan(ctx, 24, 32, 64, 800, [28] * 8, seed=SEED, lossy=lossy)
        b = plan.compressed_bytes()
        assert b["pool"] == 14746512
        assert b["per_agent_shell"] == shell
        assert b["total"] == system


def _patched_cache(plan, corpus, layers, heads, dim, prefix, agents, lossy):
    """Oracle decodes placed like patch_cache_with_multi_agent_kv
    (proveKV/scripts/ppl_validate_multi_agent.py:226-272): [layer][K|V][H][T][D] f32."""
    T = prefix + sum(agents)
    cb, rot = O.fib_constants(SEED)
    cb, rot = cb.reshape(32, 4), rot.reshape(dim, dim)
    ref = np.zeros((layers, 2, heads, T, dim), np.float32)
    owners = [(0, prefix, "fib")]
    t = prefix
    for nt in agents:
        owners.append((t, nt, "turbo"))
        t += nt
    for t0, nt, kind in owners:
        for layer in range(layers):
            for side in (0, 1):
                x = gather(corpus, t0, nt, layer, side)
                if kind == "fib":
                    dec = O.fib_decode_batch(O.fib_encode_batch(x, cb, rot), cb, rot)
                else:
                    dec = O.turbo_decode_batch(O.turbo_encode_batch(x, SEED, radii_codec=int(lossy)), dim, SEED)
                ref[layer, side, :, t0:t0 + nt, :] = dec.reshape(nt, heads, dim).transpose(1, 0, 2)
    return ref


@pytest.mark.parametrize("dtype,copies,lossy", [("float32", 1, False), ("bfloat16", 2, False),
                                                ("float16", 3, True)])
def test_rehydrate_into_cache_layout(ctx, dtype, copies, lossy):
    """Fused rehydrate: both tiers decoded straight into [1, H, T, D] per
    layer, in the cache dtype (RNE of the f32 decode), into `copies` caches."""
    import torch
    from provekv_amd.pool import DeviceKVCache
    layers, heads, dim, prefix, agents = 2, 4, 64, 21, [3, 6]
    corpus = synth.corpus_tokens(5, layers, heads, prefix + sum(agents), dim)
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=SEED, lossy=lossy)
    bufs = plan.alloc()
    plan.encode(torch.from_numpy(corpus.reshape(-1)).cuda(), bufs)
    tdt = getattr(torch, dtype)
    cache = DeviceKVCache(layers, heads, prefix + sum(agents), dim, dtype=tdt, copies=copies)
    cache.buf.fill_(7.0)
    plan.rehydrate(bufs, cache)
    torch.cuda.synchronize()
    plan.check_rehydrate(bufs)
    assert cache.seq_len() == prefix + sum(agents) and cache.num_layers() == layers
    ref = torch.from_numpy(_patched_cache(plan, corpus, layers, heads, dim, prefix, agents, lossy)).to(tdt)
    got = cache.buf.cpu()
    for c in range(copies):
        assert torch.equal(got[c].view(torch.int16 if dtype != "float32" else torch.int32),
                           ref.view(torch.int16 if dtype != "float32" else torch.int32))
    assert tuple(cache.keys(1, copies - 1).shape) == (1, heads, prefix + sum(agents), dim)


@pytest.mark.parametrize("lossy", [False, True])
def test_build_and_rehydrate_two_streams(ctx, lossy):
    """The whole step with the shell tier on a second stream: encode bytes and
    the rehydrated caches equal the one-stream step bit for bit, and work
    queued on the main stream afterwards sees both tiers (the join)."""
    import torch
    from provekv_amd.pool import DeviceKVCache
    layers, heads, dim, prefix, agents = 3, 8, 64, 150, [20, 33, 7]
    corpus = synth.corpus_tokens(9, layers, heads, prefix + sum(agents), dim)
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=SEED, lossy=lossy)
    caches, wires = [], []
    side = torch.cuda.Stream()
    for use_side in (False, True):
        bufs = plan.alloc()
        cache = DeviceKVCache(layers, heads, prefix + sum(agents), dim, copies=3)
        cache.buf.fill_(7.0)
        main = torch.cuda.Stream()
        with torch.cuda.stream(main):
            for _ in range(2):   # back to back: the second step reuses every buffer
                plan.build_and_rehydrate(dev, bufs, cache, stream=main, side=side if use_side else None)
            snap = cache.buf.clone()   # queued on main after the join
        torch.cuda.synchronize()
        plan.check(bufs, decode=False)
        plan.check_rehydrate(bufs)
        caches.append(snap.cpu())
        wires.append((bufs["pool_wire"].cpu(), bufs["shell_wire"].cpu()))
    assert torch.equal(caches[0].view(torch.int32), caches[1].view(torch.int32))
    assert torch.equal(wires[0][0], wires[1][0]) and torch.equal(wires[0][1], wires[1][1])
    ref = torch.from_numpy(_patched_cache(plan, corpus, layers, heads, dim, prefix, agents, lossy))
    assert torch.equal(caches[1][0].view(torch.int32), ref.view(torch.int32))


@pytest.mark.parametrize("max_workgroups", [1, 3, 64])
def test_bounded_turbo_decode_matches_full_grid(ctx, max_workgroups):
    """pkv_decode_segments_bounded: a grid of a few workgroups looping over
    every half-tile writes the same cache as one workgroup per half-tile,
    and reports a corrupt vector the same way."""
    import torch
    from provekv_amd.pool import DeviceKVCache
    layers, heads, dim, prefix, agents = 2, 8, 64, 10, [40, 17, 300]
    corpus = synth.corpus_tokens(11, layers, heads, prefix + sum(agents), dim)
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=SEED)
    bufs = plan.alloc()
    plan.encode(torch.from_numpy(corpus.reshape(-1)).cuda(), bufs)
    plen = plan.turbo.payload_len()
    # corrupt one radius of vector 123 of blob 5 (a negative radius)
    _, _, _, off, _ = plan.shells.blob_offsets[5]
    pos = off + 38 + 123 * plen + 4 * 7
    bufs["shell_wire"][pos:pos + 4] = torch.from_numpy(np.frombuffer(np.float32(-2.0).tobytes(), np.uint8).copy()).cuda()
    outs, stats = [], []
    for bound in (0, max_workgroups):
        cache = DeviceKVCache(layers, heads, prefix + sum(agents), dim, copies=2)
        cache.buf.fill_(3.0)
        plan._cache_tables(bufs, cache)
        _, sseg = plan._cache_segs
        st = torch.zeros(2 * len(sseg), dtype=torch.int32, device="cuda")
        plan.turbo.decode_segments(bufs["shell_wire"], sseg, cache.buf.view(-1), status=st, fanout=2,
                                   fanout_stride=cache.copy_stride, max_workgroups=bound)
        torch.cuda.synchronize()
        outs.append(cache.buf.cpu())
        stats.append(st.cpu().numpy().view(np.uint32).copy())
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))
    assert np.array_equal(stats[0], stats[1])
    err = plan.turbo.status_error(stats[1], sseg)
    assert err is not None and err.segment == 5 and err.index == 123


@pytest.mark.parametrize("max_workgroups", [1, 5, 64, 640])
def test_bounded_fib_encode_matches_full_grid(ctx, max_workgroups):
    """pkv_encode_segments_bounded: the fib encode's persistent grid held to a
    few workgroups (each wave then walks more units, and its list of
    undecided vectors spans them) writes the same FB2 blobs as the full grid,
    equal to the oracle's, and reports a non-finite input the same way; the
    turbo encode ignores the bound."""
    import torch
    layers, heads, dim, prefix, agents = 3, 8, 64, 500, [30, 7]
    corpus = synth.corpus_tokens(13, layers, heads, prefix + sum(agents), dim)
    corpus[5, 1, 3, 1, 17] = np.inf   # token 5, layer 1, head 3, V: pool blob (layer 1, V), vector 5 * 8 + 3
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=SEED)
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    wires, stats, swires = [], [], []
    for bound in (0, max_workgroups):
        bufs = plan.alloc()
        st = torch.zeros(2 * len(plan.pool.enc), dtype=torch.int32, device="cuda")
        plan.fib.encode_segments(dev, plan.pool.enc, bufs["pool_wire"], status=st, max_workgroups=bound)
        plan.turbo.encode_segments(dev, plan.shells.enc, bufs["shell_wire"], radii=plan.radii,
                                   status=bufs["shell_status"], max_workgroups=bound)
        torch.cuda.synchronize()
        wires.append(bufs["pool_wire"].cpu())
        swires.append(bufs["shell_wire"].cpu())
        stats.append(st.cpu().numpy().view(np.uint32).copy())
    assert torch.equal(wires[0], wires[1]) and torch.equal(swires[0], swires[1])
    assert np.array_equal(stats[0], stats[1])
    err = plan.fib.status_error(stats[1], plan.pool.enc)
    assert err is not None and err.index == 5 * heads + 3
    cb, rot = O.fib_constants(SEED)
    for b, (_, layer, side, off, nbytes) in enumerate(plan.pool.blob_offsets):
        if (layer, side) == (1, 1):
            continue   # the rejected blob
        x = np.ascontiguousarray(corpus[:prefix, layer, :, side, :]).reshape(-1, dim)
        assert bytes(wires[1][off:off + nbytes].numpy()) == O.fib_encode_batch(x, cb.reshape(32, 4),
                                                                              rot.reshape(64, 64))


@pytest.mark.parametrize("max_workgroups,copies", [(1, 2), (3, 1), (7, 2), (5, 8)])
def test_bounded_fib_decode_matches_full_grid(ctx, max_workgroups, copies):
    """The fib matrix-core decode on a bounded grid (workgroups looping over
    the tiles of every segment, staged fan-out stores or direct ones) writes
    the same cache as one workgroup per tile, and reports a corrupt norm the
    same way."""
    import torch
    from provekv_amd.pool import DeviceKVCache
    layers, heads, dim, prefix, agents = 2, 8, 64, 300, [5]
    corpus = synth.corpus_tokens(12, layers, heads, prefix + sum(agents), dim)
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=SEED)
    bufs = plan.alloc()
    plan.encode(torch.from_numpy(corpus.reshape(-1)).cuda(), bufs)
    plen = plan.fib.payload_len()
    # an infinite f16 norm for vector 1000 of blob 2 (FB2 header: 19 bytes)
    _, _, _, off, _ = plan.pool.blob_offsets[2]
    pos = off + 19 + 1000 * plen
    bufs["pool_wire"][pos:pos + 2] = torch.tensor([0x00, 0x7C], dtype=torch.uint8, device="cuda")
    outs, stats = [], []
    for bound in (0, max_workgroups):
        cache = DeviceKVCache(layers, heads, prefix + sum(agents), dim, copies=copies)
        cache.buf.fill_(3.0)
        plan._cache_tables(bufs, cache)
        pseg, _ = plan._cache_segs
        st = torch.zeros(2 * len(pseg), dtype=torch.int32, device="cuda")
        plan.fib.decode_segments(bufs["pool_wire"], pseg, cache.buf.view(-1), status=st, fanout=copies,
                                 fanout_stride=cache.copy_stride, max_workgroups=bound)
        torch.cuda.synchronize()
        outs.append(cache.buf.cpu())
        stats.append(st.cpu().numpy().view(np.uint32).copy())
    assert torch.equal(outs[0].view(torch.int32), outs[1].view(torch.int32))
    assert np.array_equal(stats[0], stats[1])
    err = plan.fib.status_error(stats[1], pseg)
    assert err is not None and err.segment == 2 and err.index == 1000
    # every other vector is the oracle's decode
    cb, rot = O.fib_constants(SEED)
    want = O.fib_decode_batch(plan.blob(bufs, "pool", 0), cb.reshape(32, 4), rot.reshape(64, 64)).reshape(prefix, heads, dim)
    got = outs[1][0, 0, 0, :, :prefix, :].permute(1, 0, 2).numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("heads,prefix,copies,bound", [(8, 256, 3, 0), (32, 96, 8, 0), (16, 48, 2, 5),
                                                       (4, 128, 8, 3)])
def test_whole_tile_fanout_rehydrate(ctx, heads, prefix, copies, bound):
    """Pool blobs of T tokens x G heads whose vector count is a multiple of
    256 (whole decode tiles, no partial last tile), 2 to 8 cache copies,
    full and bounded grids: every copy equals the oracle's decode, and a
    corrupt norm is reported at its own vector index with its rows left
    untouched."""
    import torch
    from provekv_amd.pool import DeviceKVCache
    layers, dim, agents = 2, 64, [5]
    assert (prefix * heads) % 256 == 0
    corpus = synth.corpus_tokens(31, layers, heads, prefix + sum(agents), dim)
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=SEED)
    bufs = plan.alloc()
    plan.encode(torch.from_numpy(corpus.reshape(-1)).cuda(), bufs)
    plen = plan.fib.payload_len()
    bad_v = 3 * heads + 1                       # token 3, head 1 of blob 1 (layer 0, V)
    _, _, _, off, _ = plan.pool.blob_offsets[1]
    pos = off + 19 + bad_v * plen
    bufs["pool_wire"][pos:pos + 2] = torch.tensor([0x00, 0x7C], dtype=torch.uint8, device="cuda")
    cache = DeviceKVCache(layers, heads, prefix + sum(agents), dim, copies=copies)
    cache.buf.fill_(5.0)
    plan._cache_tables(bufs, cache)
    pseg, _ = plan._cache_segs
    st = torch.zeros(2 * len(pseg), dtype=torch.int32, device="cuda")
    plan.fib.decode_segments(bufs["pool_wire"], pseg, cache.buf.view(-1), status=st, fanout=copies,
                             fanout_stride=cache.copy_stride, max_workgroups=bound)
    torch.cuda.synchronize()
    err = plan.fib.status_error(st.cpu().numpy().view(np.uint32), pseg)
    assert err is not None and err.segment == 1 and err.index == bad_v
    got = cache.buf.cpu()
    cb, rot = O.fib_constants(SEED)
    for k, (_, layer, side, _, _) in enumerate(plan.pool.blob_offsets):
        want = O.fib_decode_batch(plan.blob(bufs, "pool", k) if k != 1 else _restore(plan, bufs, k, bad_v),
                                  cb.reshape(32, 4), rot.reshape(64, 64)).reshape(prefix, heads, dim)
        for c in range(copies):
            g = got[c, layer, side, :, :prefix, :].permute(1, 0, 2).numpy()
            if k == 1:   # the corrupt vector's row is left untouched
                assert np.all(g[3, 1] == 5.0)
                g = g.copy()
                g[3, 1] = want[3, 1]
            assert np.array_equal(g.view(np.uint32), want.view(np.uint32)), (k, c)


def _restore(plan, bufs, k, v):
    """Blob k with vector v's norm made finite again (for the oracle's decode)."""
    b = bytearray(plan.blob(bufs, "pool", k))
    plen = plan.fib.payload_len()
    b[19 + v * plen:19 + v * plen + 2] = bytes([0x00, 0x3C])   # f16 1.0
    return bytes(b)


def test_cache_target_append(ctx):
    """CacheTarget (proveKV/src/pool.rs:646-658): append one token's [H * D]
    key / value at a position in every copy."""
    import torch
    from provekv_amd.pool import DeviceKVCache
    cache = DeviceKVCache(3, 2, 8, 64, dtype=torch.bfloat16, copies=2)
    k = np.arange(128, dtype=np.float32) / 7
    cache.append_key(1, 5, k)
    cache.append_value(2, 6, -k)
    assert cache.seq_len() == 7 and cache.num_layers() == 3
    want = torch.from_numpy(k.reshape(2, 64)).to(torch.bfloat16)
    assert torch.equal(cache.keys(1, 1)[0, :, 5, :].cpu(), want)
    assert torch.equal(cache.values(2, 0)[0, :, 6, :].cpu(), -want)
    with pytest.raises(IndexError):
        cache.append_key(3, 0, k)


def test_decode_output_dtype_rounding_edges(ctx):
    """With an identity rotation and a unit f16 norm the decode returns the
    codebook entries exactly, so planted values check the bf16 / f16
    conversion against torch's own (round to nearest even): ties, f16
    subnormals, the f16 overflow threshold, zeros."""
    import torch
    vals = [1 + 2 ** -8, 1 + 3 * 2 ** -8, -(1 + 2 ** -8), 1 + 2 ** -11, 1 + 3 * 2 ** -11, 65504.0, 65519.0,
            65520.0, 1e5, -1e5, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 1e-6, -1e-7, 2.0 ** -126, 0.0, -0.0,
            1 / 3, np.pi, -np.e, 3.4e38, 1.5 * 2 ** -14, 2 ** -14 - 2 ** -25]
    rng = np.random.RandomState(1)
    rest = rng.randn(128 - len(vals)) * 10.0 ** rng.randint(-8, 6, 128 - len(vals))
    cb = np.array(vals + list(rest), np.float32).reshape(32, 4)
    rot = np.ascontiguousarray(np.eye(64))
    ptr = ctypes.c_void_p()
    L.check(L.lib().pkv_fib_profile_create_with_constants(ctx.ptr, 64, 4, 32, cb.ctypes.data, rot.ctypes.data,
                                                          ctypes.byref(ptr)), "pkv_fib_profile_create_with_constants")
    prof = Profile(ctx, ptr, L.CODEC_FIB, 64)
    n = 8
    blob = bytearray(b"FB2" + bytes([1, 5, 0]) + struct.pack("<II", 16, n) + bytes([0]) + struct.pack("<HH", 2, 10))
    for v in range(n):
        idx = sum(((v * 16 + b) % 32) << (5 * b) for b in range(16))
        blob += struct.pack("<H", 0x3C00) + idx.to_bytes(10, "little")
    wire = torch.frombuffer(blob, dtype=torch.uint8).cuda()
    want32 = O.fib_decode_batch(bytes(blob), cb, rot)   # the codebook entries, but -0.0 + 0.0 = +0.0
    assert np.array_equal(want32[0], np.where(cb[:16].reshape(64) == 0, 0.0, cb[:16].reshape(64)))
    segs = np.array([(0, 0, 64, 0, n, n)], dtype=SEG_DTYPE)
    for tdt in (torch.float32, torch.bfloat16, torch.float16):
        out = torch.empty(n * 64, dtype=tdt, device="cuda")
        prof.decode_segments(wire, segs, out)
        torch.cuda.synchronize()
        want = torch.from_numpy(want32).reshape(-1).to(tdt)
        bits = torch.int32 if tdt == torch.float32 else torch.int16
        assert torch.equal(out.cpu().view(bits), want.view(bits)), tdt


def _config4_like(layers, heads, tokens, seed=4):
    """Config 4's value distribution (K scales LogNormal(0, 0.7), 4 outlier
    channels x10 per head, V ~ N(0, 1)) as bf16 (RNE) in the [L][K|V][H][T][D]
    layout, plus the exact f32 upcast the CPU side consumes."""
    import torch
    K, V = synth.kv_cache(seed, layers, heads, tokens, 128, k_sigma=0.7, outliers=4, outlier_mult=10.0,
                          v_scale=1.0)
    x = np.stack([K, V], axis=1)                                    # [L][2][H][T][D]
    xb = torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16)
    return xb, xb.to(torch.float32).numpy()


def test_config4_bf16_d128_lossy_bit_exact(ctx):
    """Config 4 at reduced size: bf16 input upcast in-kernel, Hadamard dim 128,
    b = 4 with QJL, BlockLogU8 radii; one TQB1-L blob per (layer, K|V) in one
    launch; bytes and decodes equal the oracle on the f32 upcast."""
    import torch
    layers, heads, tokens = 2, 3, 150
    xb, x32 = _config4_like(layers, heads, tokens)
    prof = ctx.turbo_profile(128, 4, 32, SEED)
    n = heads * tokens
    plen = prof.payload_len(L.RADII_LOG_U8)
    assert plen == 100                                              # d/2 + 8 + ceil(64*3/8) + 4
    blob = 38 + n * plen
    segs = np.array([((b * n) * 128, 0, 128, b * blob, n, n) for b in range(2 * layers)], dtype=SEG_DTYPE)
    wire = torch.empty(2 * layers * blob, dtype=torch.uint8, device="cuda")
    st = torch.empty(2 * len(segs), dtype=torch.int32, device="cuda")
    prof.encode_segments(xb.reshape(-1).cuda(), segs, wire, radii=L.RADII_LOG_U8, status=st)
    out = torch.empty(2 * layers * n * 128, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(st)
    prof.decode_segments(wire, segs, out, radii=L.RADII_LOG_U8, status=dst)
    torch.cuda.synchronize()
    for s_ in (st, dst):
        err = prof.status_error(s_.cpu().numpy().view(np.uint32), segs)
        assert err is None, err
    w = wire.cpu().numpy().tobytes()
    got = out.cpu().numpy().reshape(2 * layers, n, 128)
    for b in range(2 * layers):
        ref = O.turbo_encode_batch(x32.reshape(2 * layers, n, 128)[b], SEED, radii_codec=1)
        assert w[b * blob:(b + 1) * blob] == ref, b
        assert np.array_equal(got[b].view(np.uint32), O.turbo_decode_batch(ref, 128, SEED).view(np.uint32))
