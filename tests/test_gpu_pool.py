"""GPU parity of the batched two-tier path (all (owner, layer, K|V) blobs in
one launch per tier) against per-blob oracle calls on the gathered vectors,
plus the receipt byte math at the N=8 SmolLM2 shape."""
import numpy as np
import pytest

from oracle import oracle as O
from provekv_amd import synth
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
    cb, rot = plan.fib.constants()
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
