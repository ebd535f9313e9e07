"""Full-size GPU parity: every BASELINE.json configuration at its real shape,
through the C ABI, against the CPU oracle run with its OWN profile constants
(O.fib_constants: codebook + rotation built by the oracle's restated RNG, QR
and Lloyd; O.turbo_constants: signs + QJL matrix) -- never the product's.

  config 0  turbo b=4 lossless, K and V [32 heads, 1024 tokens, 64] [H][T][D]
            (data seed 0): 2 TQB1 blobs, 65,536 vectors, every byte and decode
  config 1  fib_k4_n32 pool 24 layers x {K,V} x 32 heads x 800 tokens (seed 1):
            48 FB2 blobs in one launch, 1,228,800 vectors, every byte and decode
  config 2  turbo shells N=8 x 28 tokens x 24 layers x {K,V} x 32 heads (seed 2):
            384 blobs in one launch, lossless and lossy, every byte and decode
  config 3  pool + 8 shells (seed 3) built and rehydrated into 8 f32 caches
            [1, H, T, D] per layer: every blob byte, cache copy 0 against the
            oracle decodes, copies 1-7 equal to copy 0
  config 4  Llama-3-8B KV 32 x {K,V} x 8 heads x 32768 tokens x 128, bf16 in,
            TQB1-L (seeded on the device, 4.3 GB): one full-size launch each
            way; one vector of every 64-vector workgroup tile of all 64 blobs
            (262,144 vectors, the position inside the tile cycling over all
            64) against the oracle bit for bit, every header, and
            size-independent checks over all 16.8 M vectors

Bars: wire bytes and decodes bit-exact (decode within 1e-6 relative is the
stated bar; exact equality is what is checked).  Oracle calls run on a thread
pool (ctypes releases the GIL); constants are built on the main thread first.
"""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd import device as D
from provekv_amd import synth
from provekv_amd.pool import DeviceKVCache, TwoTierPlan

pytestmark = pytest.mark.gpu
SEED = 42
THREADS = 8
LAYERS, HEADS, DIM, PREFIX, AGENTS = 24, 32, 64, 800, [28] * 8


def pmap(fn, items):
    with ThreadPoolExecutor(THREADS) as ex:
        return list(ex.map(fn, items))


def turbo_consts(dim=64):
    signs, G = O.turbo_constants(dim, 32, SEED)
    return signs, G


def check_blobs(wire_host: np.ndarray, blob_offsets, inputs, encode, decode, dec_host=None, dec_offsets=None):
    """Every blob's bytes against the oracle encode of its input vectors; its
    decode (when given) against the oracle decode."""
    def one(k):
        _, _, _, off, ln = blob_offsets[k]
        ref = encode(inputs(k))
        got = wire_host[off:off + ln].tobytes()
        if got != ref:
            return f"blob {k}: bytes differ"
        if dec_host is not None:
            want = decode(ref)
            o0 = dec_offsets[k]
            got_d = dec_host[o0:o0 + want.size].reshape(want.shape)
            if not np.array_equal(got_d.view(np.uint32), want.view(np.uint32)):
                return f"blob {k}: decode differs"
        return None
    errs = [e for e in pmap(one, range(len(blob_offsets))) if e]
    assert not errs, errs[:5]


def test_config0_single_layer_turbo_full(ctx):
    import torch
    K, V = synth.kv_cache(0, 1, 32, 1024, DIM)
    x = np.ascontiguousarray(np.stack([K[0], V[0]]))          # [K|V][H][T][D]
    n = 32 * 1024
    prof = ctx.turbo_profile(DIM, 4, 32, SEED, 1)
    blob = prof.blob_len(n)
    segs = D.segments([D.contiguous_segment(0, n, DIM, 0), D.contiguous_segment(n * DIM, n, DIM, blob)])
    dev = torch.from_numpy(x.reshape(-1)).cuda()
    wire = torch.empty(2 * blob, dtype=torch.uint8, device="cuda")
    out = torch.empty(2 * n * DIM, dtype=torch.float32, device="cuda")
    st = torch.empty(4, dtype=torch.int32, device="cuda")
    prof.encode_segments(dev, segs, wire, status=st)
    prof.decode_segments(wire, segs, out, status=st)
    torch.cuda.synchronize()
    assert prof.status_error(st.cpu().numpy().view(np.uint32), segs) is None
    signs, G = turbo_consts()
    w = wire.cpu().numpy()
    o = out.cpu().numpy()
    offs = [(None, 0, s, s * blob, blob) for s in range(2)]
    check_blobs(w, offs, lambda k: x[k].reshape(-1, DIM),
                lambda v: O.turbo_encode_batch(v, SEED, signs=signs, G=G),
                lambda b: O.turbo_decode_batch(b, DIM, SEED, signs=signs), o, [0, n * DIM])


def _plan_inputs(corpus, tier):
    """Input vectors of blob k of a tier: token-major, head-minor (pool.rs:246-257)."""
    owners = {}
    def inputs(k):
        name, layer, side, _, _ = tier.blob_offsets[k]
        t0, nt = owners[name]
        return np.ascontiguousarray(corpus[t0:t0 + nt, layer, :, side, :]).reshape(-1, corpus.shape[-1])
    return owners, inputs


def test_config1_fib_pool_full(ctx):
    import torch
    corpus = synth.corpus_tokens(1, LAYERS, HEADS, PREFIX, DIM)
    plan = TwoTierPlan(ctx, LAYERS, HEADS, DIM, PREFIX, [], seed=SEED)
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    wire = torch.empty(plan.pool.wire_bytes, dtype=torch.uint8, device="cuda")
    out = torch.empty(plan.pool.out_elems, dtype=torch.float32, device="cuda")
    st = torch.empty(2 * len(plan.pool.enc), dtype=torch.int32, device="cuda")
    dst = torch.empty(2 * len(plan.pool.dec), dtype=torch.int32, device="cuda")
    plan.fib.encode_segments(dev, plan.pool.enc, wire, status=st)
    plan.fib.decode_segments(wire, plan.pool.dec, out, status=dst)
    torch.cuda.synchronize()
    assert plan.fib.status_error(st.cpu().numpy().view(np.uint32), plan.pool.enc) is None
    assert plan.fib.status_error(dst.cpu().numpy().view(np.uint32), plan.pool.dec) is None
    assert plan.pool.wire_bytes == 14_746_512                     # CLAIMS.json pool receipt
    cb, rot = O.fib_constants(SEED)
    owners, inputs = _plan_inputs(corpus, plan.pool)
    owners["pool"] = (0, PREFIX)
    check_blobs(wire.cpu().numpy(), plan.pool.blob_offsets, inputs,
                lambda v: O.fib_encode_batch(v, cb, rot), lambda b: O.fib_decode_batch(b, cb, rot),
                out.cpu().numpy(), [int(s["elem_offset"]) for s in plan.pool.dec])


@pytest.mark.parametrize("lossy", [False, True])
def test_config2_turbo_shells_full(ctx, lossy):
    import torch
    corpus = synth.corpus_tokens(2, LAYERS, HEADS, sum(AGENTS), DIM)
    plan = TwoTierPlan(ctx, LAYERS, HEADS, DIM, 0, AGENTS, seed=SEED, lossy=lossy)
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    wire = torch.empty(plan.shells.wire_bytes, dtype=torch.uint8, device="cuda")
    out = torch.empty(plan.shells.out_elems, dtype=torch.float32, device="cuda")
    st = torch.empty(2 * len(plan.shells.enc), dtype=torch.int32, device="cuda")
    plan.turbo.encode_segments(dev, plan.shells.enc, wire, radii=plan.radii, status=st)
    torch.cuda.synchronize()
    assert plan.turbo.status_error(st.cpu().numpy().view(np.uint32), plan.shells.enc) is None
    plan.turbo.decode_segments(wire, plan.shells.dec, out, radii=plan.radii, status=st)
    torch.cuda.synchronize()
    assert plan.turbo.status_error(st.cpu().numpy().view(np.uint32), plan.shells.dec) is None
    assert plan.shells.wire_bytes == (19_282_176 if lossy else 49_559_808)   # receipts
    signs, G = turbo_consts()
    owners, inputs = _plan_inputs(corpus, plan.shells)
    t = 0
    for a, nt in enumerate(AGENTS):
        owners[f"agent{a}"] = (t, nt)
        t += nt
    rc = L.RADII_LOG_U8 if lossy else L.RADII_F32
    check_blobs(wire.cpu().numpy(), plan.shells.blob_offsets, inputs,
                lambda v: O.turbo_encode_batch(v, SEED, radii_codec=rc, signs=signs, G=G),
                lambda b: O.turbo_decode_batch(b, DIM, SEED, signs=signs),
                out.cpu().numpy(), [int(s["elem_offset"]) for s in plan.shells.dec])


def test_config3_two_tier_rehydrate_8_caches_full(ctx):
    import torch
    T = PREFIX + sum(AGENTS)
    corpus = synth.corpus_tokens(3, LAYERS, HEADS, T, DIM)
    plan = TwoTierPlan(ctx, LAYERS, HEADS, DIM, PREFIX, AGENTS, seed=SEED)
    bufs = plan.alloc()
    cache = DeviceKVCache(LAYERS, HEADS, T, DIM, dtype=torch.float32, copies=8)
    cache.buf.fill_(float("nan"))
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    side = torch.cuda.Stream()
    plan.build_and_rehydrate(dev, bufs, cache, stream=torch.cuda.current_stream(), side=side)
    torch.cuda.synchronize()
    plan.check(bufs, decode=False)
    plan.check_rehydrate(bufs)
    assert plan.compressed_bytes()["total"] == 64_306_320                    # CLAIMS.json compressed_total
    cb, rot = O.fib_constants(SEED)
    signs, G = turbo_consts()
    ref = np.empty((LAYERS, 2, HEADS, T, DIM), np.float32)
    for tier, wkey, enc, dec, firsts in (
            (plan.pool, "pool_wire", lambda v: O.fib_encode_batch(v, cb, rot),
             lambda b: O.fib_decode_batch(b, cb, rot), {"pool": (0, PREFIX)}),
            (plan.shells, "shell_wire", lambda v: O.turbo_encode_batch(v, SEED, signs=signs, G=G),
             lambda b: O.turbo_decode_batch(b, DIM, SEED, signs=signs),
             {f"agent{a}": (PREFIX + 28 * a, 28) for a in range(8)})):
        owners, inputs = _plan_inputs(corpus, tier)
        owners.update(firsts)
        w = bufs[wkey].cpu().numpy()

        def one(k, tier=tier, w=w, enc=enc, dec=dec, inputs=inputs, owners=owners):
            name, layer, side_, off, ln = tier.blob_offsets[k]
            b = enc(inputs(k))
            t0, nt = owners[name]
            ref[layer, side_, :, t0:t0 + nt, :] = dec(b).reshape(nt, HEADS, DIM).transpose(1, 0, 2)
            return w[off:off + ln].tobytes() == b
        ok = pmap(one, range(len(tier.blob_offsets)))
        assert all(ok), [k for k, v in enumerate(ok) if not v][:5]
    got0 = cache.buf[0].cpu().numpy()
    assert np.array_equal(got0.view(np.uint32), ref.view(np.uint32))
    for c in range(1, 8):
        assert torch.equal(cache.buf[c].view(torch.int32), cache.buf[0].view(torch.int32)), c


def test_config4_llama_bf16_lossy_full_size(ctx):
    import torch
    Lr, H, T, Dd = 32, 8, 32768, 128
    n = H * T
    x = synth.device_kv_bf16(4, Lr, H, T, Dd)                       # [L][K|V][H][T][D] bf16
    prof = ctx.turbo_profile(Dd, 4, 32, SEED, 1)
    plen = prof.payload_len(L.RADII_LOG_U8)
    blob = prof.blob_len(n, L.RADII_LOG_U8)
    assert plen == 100
    nb = 2 * Lr
    segs = D.segments([D.contiguous_segment(k * n * Dd, n, Dd, k * blob) for k in range(nb)])
    wire = torch.empty(nb * blob, dtype=torch.uint8, device="cuda")
    st = torch.empty(2 * nb, dtype=torch.int32, device="cuda")
    flat = x.view(-1)
    prof.encode_segments(flat, segs, wire, radii=L.RADII_LOG_U8, status=st)
    torch.cuda.synchronize()
    assert prof.status_error(st.cpu().numpy().view(np.uint32), segs) is None
    out = torch.empty(nb * n * Dd, dtype=torch.float32, device="cuda")
    prof.decode_segments(wire, segs, out, radii=L.RADII_LOG_U8, status=st)
    torch.cuda.synchronize()
    assert prof.status_error(st.cpu().numpy().view(np.uint32), segs) is None
    assert wire.numel() == 1_677_724_032                            # 64 x 38 + 16.8 M x 100
    signs, G = turbo_consts(Dd)
    # one vector of every 64-vector workgroup tile of every blob, bit for bit
    # against the oracle: the encode and decode grids give each workgroup 64
    # consecutive vectors (four waves of 16), and the vector taken inside a
    # tile cycles through all 64 positions (lane groups, waves) over the tiles
    tiles = n // 64
    hdr_ref = None
    for k in range(nb):
        idx = (np.arange(tiles, dtype=np.int64) * 64 + (np.arange(tiles) * 29 + k * 7) % 64).astype(np.int64)
        ti = torch.from_numpy(idx).cuda()
        xs = flat[k * n * Dd:(k + 1) * n * Dd].view(n, Dd)[ti].float().cpu().numpy()   # exact bf16 upcast
        ref = O.turbo_encode_batch(xs, SEED, radii_codec=1, signs=signs, G=G)
        wb = wire[k * blob:(k + 1) * blob]
        hdr = wb[:38].cpu().numpy().copy()
        hdr[30:34] = np.frombuffer(np.uint32(tiles).tobytes(), np.uint8)
        assert hdr.tobytes() == ref[:38], k
        pay = wb[38:].view(n, plen)[ti].cpu().numpy()
        assert pay.tobytes() == ref[38:], k
        dref = O.turbo_decode_batch(ref, Dd, SEED, signs=signs)
        got = out[k * n * Dd:(k + 1) * n * Dd].view(n, Dd)[ti].cpu().numpy()
        assert np.array_equal(got.view(np.uint32), dref.view(np.uint32)), k
        hdr_ref = hdr_ref or ref[:30]
    # every header: the same 30 leading bytes, n and payload length (size-independent)
    heads = wire.view(nb, blob)[:, :38].cpu().numpy()
    assert all(h[:30].tobytes() == hdr_ref for h in heads)
    assert np.all(heads[:, 30:34].copy().view(np.uint32) == n)
    assert np.all(heads[:, 34:38].copy().view(np.uint32) == plen)
    # and every decoded vector is finite and points the way its input does
    xf = flat.view(nb * n, Dd)
    of = out.view(nb * n, Dd)
    cos_min = 1.0
    for c0 in range(0, nb * n, 1 << 22):
        a, b = xf[c0:c0 + (1 << 22)].float(), of[c0:c0 + (1 << 22)]
        assert torch.isfinite(b).all()
        cos = (a * b).sum(1) / (a.norm(dim=1) * b.norm(dim=1)).clamp_min(1e-30)
        cos_min = min(cos_min, float(cos.min()))
    assert cos_min > 0.5, cos_min
