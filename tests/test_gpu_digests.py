"""BLAKE3 digests on the device against the oracle (bit-exact).

* pkv_blake3 (host bytes through the device) on the published test vectors;
* pkv_blake3_ranges over one buffer: empty ranges, every length class around
  the block (64), chunk (1024) and pass (16, 64 and 4096 chunks) boundaries,
  with the first pass on four lanes per chunk and on one,
  every start alignment, a range ending at the last byte of a buffer whose
  size is not a multiple of 4, overlapping ranges;
* a two-tier build: every blob's payload digest (CompressedBlock::new) and
  every layer digest (PoolLayer / ShellLayer::compute_digest) against the
  oracle over the wire bytes copied back;
* quant-codec-core's digest types (digest_stability.rs) and profile digests;
* argument errors.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import _lib as L
from provekv_amd import synth
from provekv_amd.kvcodec import ArtifactDigest, CodecProfileDigest, DeviceKvCodec
from provekv_amd.pool import TwoTierPlan

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
VECTORS = json.load(open(os.path.join(HERE, "golden", "blake3_vectors.json")))


def test_blake3_host_bytes_known_answers(ctx):
    for v in VECTORS["vectors"]:
        data = bytes(i % 251 for i in range(v["input_len"]))
        assert ctx.blake3(data).hex() == v["hash"], v["input_len"]
    for v in VECTORS["ascii"]:
        assert ctx.blake3(v["input"].encode()).hex() == v["hash"]


def _ranges(buf_len: int, rng):
    lens = [0, 1, 2, 3, 4, 5, 63, 64, 65, 127, 128, 1000, 1023, 1024, 1025, 2047, 2048, 2049, 3073,
            15 * 1024 + 1, 16 * 1024 - 1, 16 * 1024, 16 * 1024 + 1, 17 * 1024,
            63 * 1024 + 1, 64 * 1024 - 1, 64 * 1024, 64 * 1024 + 1, 65 * 1024 + 7,
            1024 * 1024, 1024 * 1024 + 1,
            4096 * 1024, 4096 * 1024 + 1, 4100 * 1024 + 5]
    out = []
    for ln in lens:
        for align in range(4):
            off = int(rng.integers(0, (buf_len - ln) // 4 + 1)) * 4 + align
            off = min(off, buf_len - ln)
            out.append((off, ln))
    out += [(buf_len, 0), (buf_len - 1, 1), (buf_len - 3, 3), (buf_len - 1027, 1027), (0, buf_len),
            (1, buf_len - 1), (2, buf_len - 2), (3, buf_len - 3)]
    return out


def _chunks(ranges):
    return sum(max(1, (ln + 1023) // 1024) for _, ln in ranges)


@pytest.mark.parametrize("mode", ["quad", "lane"])
def test_ranges_match_oracle(ctx, mode):
    """Both first-pass forms: a call of fewer than 32 Ki chunks runs four
    lanes per chunk, a larger one one lane per chunk."""
    import torch
    rng = np.random.default_rng(11)
    n = 4100 * 1024 + 4099           # not a multiple of 4
    host = rng.integers(0, 256, n, dtype=np.uint8)
    buf = torch.from_numpy(host).cuda()
    ranges = _ranges(n, rng)
    if mode == "quad":
        keep, total = [], 0
        for r in ranges:
            if total + _chunks([r]) < 32 * 1024:
                keep.append(r)
                total += _chunks([r])
        ranges = keep
        assert _chunks(ranges) < 32 * 1024 and any(ln > 4096 * 1024 for _, ln in ranges)
    else:
        assert _chunks(ranges) >= 32 * 1024
    print(f"{len(ranges)} ranges over {n} bytes", flush=True)
    got = ctx.blake3_ranges(buf, ranges)
    torch.cuda.synchronize()
    want = O.blake3_ranges(host, ranges)
    bad = [ranges[i] for i in range(len(ranges)) if not np.array_equal(got[i].cpu().numpy(), want[i])]
    assert not bad, bad[:8]


def test_ranges_lane_mode_match_oracle(ctx):
    """32 Ki chunks or more in one call (here: 40 overlapping ranges of
    ~4.1 MB) take the one-lane-per-chunk first pass; fewer take four lanes
    per chunk (the other range tests here)."""
    import torch
    rng = np.random.default_rng(13)
    n = 5 * 1024 * 1024 + 3
    host = rng.integers(0, 256, n, dtype=np.uint8)
    buf = torch.from_numpy(host).cuda()
    ranges = [(int(a), 4100 * 1024 + int(b)) for a, b in zip(rng.integers(0, 900_000, 40), rng.integers(0, 2048, 40))]
    assert sum((ln + 1023) // 1024 for _, ln in ranges) >= 32 * 1024
    got = ctx.blake3_ranges(buf, ranges).cpu().numpy()
    assert np.array_equal(got, O.blake3_ranges(host, ranges))


def test_ranges_twice_and_reused_output(ctx):
    """Back-to-back calls on one stream (the ring slot and its chaining-value
    scratch reused) give the same digests; a smaller second table too."""
    import torch
    rng = np.random.default_rng(12)
    host = rng.integers(0, 256, 300_000, dtype=np.uint8)
    buf = torch.from_numpy(host).cuda()
    big = [(int(o), int(l)) for o, l in zip(rng.integers(0, 1000, 40), rng.integers(0, 299_000, 40))]
    small = big[:3]
    out = torch.full((40, 32), 0xA5, dtype=torch.uint8, device="cuda")
    for table in (big, small, big):
        ctx.blake3_ranges(buf, table, out=out)
        torch.cuda.synchronize()
        assert np.array_equal(out[:len(table)].cpu().numpy(), O.blake3_ranges(host, table))


@pytest.mark.parametrize("lossy,two_streams", [(False, False), (True, False), (False, True)])
def test_two_tier_digests_match_oracle(ctx, lossy, two_streams):
    """Twice in a row (the second call reuses the first call's table slots),
    outputs spoiled in between."""
    import torch
    layers, heads, dim, prefix, agents = 3, 8, 64, 200, [12, 40, 8]
    corpus = synth.corpus_tokens(5, layers, heads, prefix + sum(agents), dim)
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=42, lossy=lossy)
    bufs = plan.alloc()
    plan.encode(torch.from_numpy(corpus.reshape(-1)).cuda(), bufs)
    side = torch.cuda.Stream() if two_streams else None
    plan.digests(bufs, side=side)
    torch.cuda.synchronize()
    for k in ("pool_digests", "shell_digests", "pool_layer_digests", "shell_layer_digests"):
        bufs[k].fill_(0x5A)
    plan.digests(bufs, side=side)
    torch.cuda.synchronize()
    plan.check(bufs, decode=False)
    rep = plan.digest_report(bufs)
    for tier, name in ((plan.pool, "pool"), (plan.shells, "shell")):
        wire = bufs[f"{name}_wire"].cpu().numpy()
        for i in range(len(tier.blob_offsets) // 2):
            owner, layer, _, ko, kl = tier.blob_offsets[2 * i]
            _, _, _, vo, vl = tier.blob_offsets[2 * i + 1]
            kd, vd = O.blake3(wire[ko:ko + kl].tobytes()), O.blake3(wire[vo:vo + vl].tobytes())
            entry = [e for e in rep[owner] if e["layer_index"] == layer][0]
            assert entry["key_payload_digest"] == kd.hex()
            assert entry["value_payload_digest"] == vd.hex()
            assert entry["block_digest"] == O.layer_digest(layer, kd, vd).hex()
            if owner == "pool":
                assert entry["num_blocks"] == prefix * heads   # one FB2 block per (token, head)
    assert sorted(rep) == ["agent0", "agent1", "agent2", "pool"]


def test_layer_digests_entry_layout(ctx):
    import torch
    rng = np.random.default_rng(4)
    kv = rng.integers(0, 256, (10, 2, 32), dtype=np.uint8)
    got = ctx.layer_digests(torch.from_numpy(kv).cuda(), layers=4).cpu().numpy()
    for i in range(10):
        assert got[i].tobytes() == O.layer_digest(i % 4, kv[i, 0].tobytes(), kv[i, 1].tobytes())


def test_digest_types(ctx):
    # quant-codec-core/tests/digest_stability.rs
    a = CodecProfileDigest.from_parts([b"codec", b"v1", b"profile"], ctx)
    b = CodecProfileDigest.from_parts([b"codec", b"v1", b"profile"], ctx)
    c = CodecProfileDigest.from_parts([b"codecv1", b"profile"], ctx)
    assert a == b and a != c and len(str(a)) == 64
    parts = b"".join(len(p).to_bytes(8, "little") + p for p in (b"codec", b"v1", b"profile"))
    assert a.as_bytes() == O.blake3(parts)
    assert CodecProfileDigest.from_canonical_bytes(b"mock", ctx).as_bytes() == O.blake3(b"mock")
    art = ArtifactDigest.from_canonical_bytes(b"mock", ctx)
    assert art.as_bytes() == O.blake3(b"mock") and art != CodecProfileDigest(art.as_bytes())


def test_profile_digests(ctx):
    turbo = ctx.turbo_profile(64, 4, 32, 42)
    fib = ctx.fib_profile(64, 4, 32, 42)
    dt = DeviceKvCodec(turbo, "turbo_8bit_batched")
    dtl = DeviceKvCodec(turbo, "turbo_8bit_batched_lossy", radii=L.RADII_LOG_U8)
    dfib = DeviceKvCodec(fib, "fib_k4_n32_batched")
    d1 = dt.profile_digest()
    assert d1 == dt.profile_digest()
    parts = dt.canonical_profile_parts()
    assert d1.as_bytes() == O.blake3(b"".join(len(p).to_bytes(8, "little") + p for p in parts))
    others = {dtl.profile_digest(), dfib.profile_digest(),
              DeviceKvCodec(ctx.turbo_profile(64, 4, 32, 43), "turbo_8bit_batched").profile_digest()}
    assert d1 not in others and len(others) == 3


def test_argument_errors(ctx):
    import torch
    buf = torch.zeros(100, dtype=torch.uint8, device="cuda")
    with pytest.raises(L.PkvError) as e:
        ctx.blake3_ranges(buf, [(90, 11)])
    assert e.value.status == L.ERR_INVALID_ARG
    with pytest.raises(L.PkvError):
        ctx.blake3_ranges(buf, [(101, 0)])
    out = torch.zeros(80, dtype=torch.uint8, device="cuda")
    with pytest.raises(L.PkvError):
        ctx.blake3_ranges(buf, [(0, 10)], out=out[1:33])
    with pytest.raises(L.PkvError):
        ctx.layer_digests(torch.zeros((2, 2, 32), dtype=torch.uint8, device="cuda"), layers=0)


def test_tier_digests_equal_the_two_calls(ctx):
    """pkv_blake3_tier_digests (the digests of one tier in one call) writes
    the bytes of pkv_blake3_ranges followed by pkv_blake3_layer_digests;
    layers == 0 and an unaligned output are rejected."""
    import torch
    rng = np.random.RandomState(11)
    data = rng.randint(0, 256, size=300_000).astype(np.uint8)
    buf = torch.from_numpy(data).cuda()
    lens = rng.randint(0, 9000, size=12)
    offs = [int(rng.randint(0, len(data) - l)) for l in lens]
    ranges = np.array(list(zip(offs, lens)), np.uint64)        # 6 entries of (key, value)
    blob = torch.zeros((6, 2, 32), dtype=torch.uint8, device="cuda")
    layer = torch.zeros((6, 32), dtype=torch.uint8, device="cuda")
    ctx.tier_digests(buf, ranges, 3, blob, layer)
    want_blob = ctx.blake3_ranges(buf, ranges)
    want_layer = ctx.layer_digests(want_blob.reshape(6, 2, 32).contiguous(), 3)
    torch.cuda.synchronize()
    assert torch.equal(blob.reshape(12, 32).cpu(), want_blob.cpu())
    assert torch.equal(layer.cpu(), want_layer.cpu())
    for i in range(6):   # and the oracle's text digest, entry i being layer i % 3
        k, v = data[offs[2 * i]:offs[2 * i] + lens[2 * i]], data[offs[2 * i + 1]:offs[2 * i + 1] + lens[2 * i + 1]]
        assert layer[i].cpu().numpy().tobytes() == O.layer_digest(i % 3, O.blake3(k.tobytes()), O.blake3(v.tobytes()))
    with pytest.raises(L.PkvError):
        ctx.tier_digests(buf, ranges, 0, blob, layer)
    big = torch.zeros(8 * 64 + 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(L.PkvError):
        ctx.tier_digests(buf, ranges, 3, big[1:1 + 6 * 64], layer)


def test_same_table_on_two_streams(ctx):
    """One range table digested alternately on two streams, with a long
    kernel queued ahead on each: a call reuses a table slot (and its
    chaining-value scratch) only after an earlier call on its own stream, so
    both streams' digests stay correct."""
    import torch
    rng = np.random.default_rng(21)
    host = rng.integers(0, 256, 3_000_000, dtype=np.uint8)
    buf = torch.from_numpy(host).cuda()
    table = [(int(o), int(l)) for o, l in zip(rng.integers(0, 10_000, 24), rng.integers(60_000, 2_900_000, 24))]
    want = O.blake3_ranges(host, table)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    outs = [torch.empty((24, 32), dtype=torch.uint8, device="cuda") for _ in range(2)]
    for _ in range(4):
        for o in outs:
            o.fill_(0xA5)
        torch.cuda.synchronize()
        for st, o in zip((s1, s2), outs):
            with torch.cuda.stream(st):
                torch.cuda._sleep(2_000_000)
            ctx.blake3_ranges(buf, table, out=o, stream=st)
        torch.cuda.synchronize()
        for o in outs:
            assert np.array_equal(o.cpu().numpy(), want)
