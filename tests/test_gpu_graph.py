"""The two-tier step (shell encode, shell rehydrate on a second stream beside
the pool encode, pool rehydrate) captured into a HIP graph replays to the
eager step's bytes.

The graph is replayed several times, with the program's own eager steps and
synchronisations between the replays, and every replay's outputs -- both
wires, every cache copy and all status words -- are compared with the eager
result after the outputs were overwritten with garbage, so a replay that
skips a node cannot pass.
"""
import numpy as np
import pytest

from provekv_amd import synth
from provekv_amd.pool import DeviceKVCache, TwoTierPlan

pytestmark = pytest.mark.gpu
SEED = 42


def _outputs(bufs, cache):
    keys = ("pool_wire", "shell_wire", "pool_status", "shell_status", "pool_cstatus", "shell_cstatus")
    return {k: bufs[k].cpu().numpy().copy() for k in keys} | {"cache": cache.buf.cpu().numpy().copy()}


def _spoil(bufs, cache):
    for k in ("pool_wire", "shell_wire"):
        bufs[k].fill_(0xA5)
    for k in ("pool_status", "shell_status", "pool_cstatus", "shell_cstatus"):
        bufs[k].fill_(0x5A5A5A5A)
    cache.buf.fill_(float("nan"))


@pytest.mark.parametrize("lossy", [False, True])
def test_two_tier_step_graph_replays_match_eager(ctx, lossy):
    import torch
    layers, heads, dim, prefix, agents = 3, 8, 64, 96, [12, 20, 8]
    corpus = synth.corpus_tokens(7, layers, heads, prefix + sum(agents), dim)
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=SEED, lossy=lossy)
    bufs = plan.alloc()
    cache = DeviceKVCache(layers, heads, plan.tokens, dim, dtype=torch.float32, copies=3)
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    side = torch.cuda.Stream()

    def step(stream):
        plan.build_and_rehydrate(dev, bufs, cache, stream=stream, side=side, side_workgroups=64)

    main = torch.cuda.current_stream()
    for _ in range(3):   # eager warm-up: tables uploaded and seen complete
        step(main)
    torch.cuda.synchronize()
    plan.check(bufs, decode=False)
    plan.check_rehydrate(bufs)
    want = _outputs(bufs, cache)
    assert np.isfinite(want["cache"]).all()

    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=cap):
        step(torch.cuda.current_stream())
    torch.cuda.synchronize()

    for _ in range(3):
        _spoil(bufs, cache)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = _outputs(bufs, cache)
        for k, v in want.items():
            assert np.array_equal(v.view(np.uint8), got[k].view(np.uint8)), k
        # the program's own eager work between replays
        _spoil(bufs, cache)
        step(main)
        torch.cuda.synchronize()
        got = _outputs(bufs, cache)
        assert np.array_equal(want["cache"].view(np.uint8), got["cache"].view(np.uint8))
