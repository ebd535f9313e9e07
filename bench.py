"""Benchmark: proveKV codec hot path on one MI355X.

Default workload: the SmolLM2-1.7B-shape N=8 pool --
24 layers x 32 KV heads x head_dim 64, an 800-token shared prefix in the
fib_k4_n32 cold tier (FB2) and 8 agents x 28 unique tokens in the turbo b=4
hot tier (TQB1, lossless radii).  One step = build the pool + all 8 shells
(encode: 2 launches) and rehydrate the pool once and every shell (decode:
2 launches), inputs resident in HBM.

value = f32 KV bytes of the context (402,653,184 B) / the GPU time of one step
(events at the two ends of K back-to-back steps).  kernels_ms: a second pass
with events between the four calls.
roofline = the dominant kernel's algorithmic bytes per launch / its mean
duration (HIP events on the launch stream) against 8 TB/s.
cpu_baseline = the C oracle (a one-thread restatement of the reference Rust
codecs) timed on a bounded sample of the same workload on the host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(corpus: np.ndarray, plan, budget_s: float = 16.0) -> dict:
    """Oracle (one thread) encode + decode of sampled (layer, K|V) blobs of
    both tiers, scaled to the f32-KV GB/s of the whole workload."""
    from oracle import oracle as O
    cb, rot = plan.fib.constants()
    cb = cb.reshape(32, 4)
    rot = rot.reshape(plan.dim, plan.dim)
    layers, dim = plan.layers, plan.dim
    # fib: one (layer, K) blob of the prefix, truncated to a fixed vector count
    x_pool = np.ascontiguousarray(corpus[:plan.prefix, 0, :, 0, :].reshape(-1, dim))[:25600]
    x_shell = np.ascontiguousarray(corpus[plan.prefix:plan.prefix + plan.agent_tokens[0], 0, :, 0, :]
                                   .reshape(-1, dim))
    t0 = time.perf_counter()
    blob = O.fib_encode_batch(x_pool, cb, rot)
    t1 = time.perf_counter()
    O.fib_decode_batch(blob, cb, rot)
    t2 = time.perf_counter()
    reps = 0
    t3 = time.perf_counter()
    while True:
        tb = O.turbo_encode_batch(x_shell, plan.fib.params["seed"], radii_codec=plan.radii)
        O.turbo_decode_batch(tb, dim, plan.fib.params["seed"])
        reps += 1
        if time.perf_counter() - t3 > budget_s / 2:
            break
    t4 = time.perf_counter()
    fib_s_per_vec = ((t1 - t0) + (t2 - t1)) / x_pool.shape[0]
    turbo_s_per_vec = (t4 - t3) / (reps * x_shell.shape[0])
    n_pool = plan.prefix * plan.heads * layers * 2
    n_shell = sum(plan.agent_tokens) * plan.heads * layers * 2
    total_s = n_pool * fib_s_per_vec + n_shell * turbo_s_per_vec
    f32_bytes = (n_pool + n_shell) * dim * 4
    return {"value": round(f32_bytes / total_s / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": (f"oracle/pkv_oracle.c, 1 thread: fib FB2 encode+decode of {x_pool.shape[0]} pool vectors "
                       f"({(t2 - t0):.2f} s) and turbo TQB1 encode+decode of {x_shell.shape[0]} shell vectors x "
                       f"{reps} reps ({(t4 - t3):.2f} s), scaled to the {n_pool}+{n_shell}-vector workload"),
            "encode_decode_s_projected": round(total_s, 2)}


# the kernel each timed span is about (fib_encode's span also holds the exact
# fixup kernel, turbo/fib spans a status fill of a few microseconds)
KERNEL_SYMBOL = {"fib_encode": "fib_encode_kernel<64>", "turbo_encode": "turbo_encode_qjl_kernel<3>",
                 "fib_decode": "fib_decode_mfma_kernel<64>", "turbo_decode": "turbo_decode_split_kernel<3>"}
SINGLE_KERNEL = ("fib_decode", "turbo_encode", "turbo_decode")


def profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC
    summary (calibrated FETCH_SIZE + WRITE_SIZE), or None."""
    path = os.path.join(ROOT, "profiles", "codec_kernels_config3.md")
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.strip().rsplit(" ", 1)
        if line.startswith("traffic_bytes ") and len(parts) == 2:
            name = parts[0][len("traffic_bytes "):]
            if name == KERNEL_SYMBOL[kernel]:
                return int(parts[1])
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--lossy", action="store_true", help="TQB1-L shells (BlockLogU8 radii)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run a 256 MiB device copy (reference kernel for rocprofv3 --pmc byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)

    import torch
    from provekv_amd import synth
    from provekv_amd.device import default_context
    from provekv_amd.pool import TwoTierPlan

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU"}))
        sys.exit(1)
    layers, heads, dim, prefix, agents = 24, 32, 64, 800, [28] * 8
    log(f"[bench] generating synthetic corpus ({prefix + sum(agents)} tokens x {layers}L x {heads}H x 2 x {dim})")
    corpus = synth.corpus_tokens(3, layers, heads, prefix + sum(agents), dim)
    ctx = default_context()
    log("[bench] building profiles (fib codebook + rotation, turbo signs + QJL)")
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=42, lossy=args.lossy)
    bufs = plan.alloc()
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    stream = torch.cuda.current_stream()

    def step(evs=None):
        if evs is None:
            plan.encode(dev, bufs)
            plan.decode(bufs)
            return
        e = evs
        e[0].record(stream)
        plan.fib.encode_segments(dev, plan.pool.enc, bufs["pool_wire"], status=bufs["pool_status"])
        e[1].record(stream)
        plan.turbo.encode_segments(dev, plan.shells.enc, bufs["shell_wire"], radii=plan.radii,
                                   status=bufs["shell_status"])
        e[2].record(stream)
        plan.fib.decode_segments(bufs["pool_wire"], plan.pool.dec, bufs["pool_out"], status=bufs["pool_dstatus"])
        e[3].record(stream)
        plan.turbo.decode_segments(bufs["shell_wire"], plan.shells.dec, bufs["shell_out"], radii=plan.radii,
                                   status=bufs["shell_dstatus"])
        e[4].record(stream)

    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    plan.check(bufs)
    # timed region: K whole steps, events only at its two ends
    log(f"[bench] timing {args.steps} steps")
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    t_start.record(stream)
    for _ in range(args.steps):
        step()
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_gpu_ms = t_start.elapsed_time(t_end) / args.steps
    plan.check(bufs)
    # per-op breakdown from a separate pass with events between the launches
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(5)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    for k in range(args.steps):
        step(evs[k])
    torch.cuda.synchronize()
    names = ["fib_encode", "turbo_encode", "fib_decode", "turbo_decode"]
    per = {n: float(np.mean([evs[k][i].elapsed_time(evs[k][i + 1]) for k in range(args.steps)]))
           for i, n in enumerate(names)}
    n_pool = prefix * heads * layers * 2
    n_shell = sum(agents) * heads * layers * 2
    f32_pool = n_pool * dim * 4
    f32_shell = n_shell * dim * 4
    wire_pool = plan.pool.wire_bytes
    wire_shell = plan.shells.wire_bytes
    alg = {"fib_encode": f32_pool + wire_pool, "turbo_encode": f32_shell + wire_shell,
           "fib_decode": f32_pool + wire_pool, "turbo_decode": f32_shell + wire_shell}
    kern_gbs = {n: alg[n] / (per[n] * 1e-3) / 1e9 for n in names}
    step_ms = wall / args.steps * 1e3
    f32_total = f32_pool + f32_shell
    value = f32_total / (step_gpu_ms * 1e-3) / 1e9
    # roofline: the longest span made of one codec kernel
    dom = max(SINGLE_KERNEL, key=lambda n: per[n])
    total_alg = sum(alg.values())
    out = {
        "metric": "KV codec encode+decode GB/s (f32 in) and % HBM peak, SmolLM2-1.7B-shape N=8 pool",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_gpu_ms, 4),
        "ms_per_step_wall": round(step_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded log-normal K with outlier channels, Gaussian V)",
        "config": {"workload": "config3: N=8 two-tier pool, 24L x 32H x d64, 800-token fib_k4_n32 prefix + "
                               "8 x 28-token turbo b=4 shells" + (" (TQB1-L lossy radii)" if args.lossy else
                                                                  " (TQB1 lossless radii)"),
                   "layers": layers, "kv_heads": heads, "head_dim": dim, "prefix_tokens": prefix,
                   "agents": len(agents), "agent_tokens": agents[0], "seed": 42},
        "hbm_fraction_codec": round(total_alg / (step_gpu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "kernels_ms": {n: round(per[n], 4) for n in names},
        "kernels_gbs": {n: round(kern_gbs[n], 1) for n in names},
        "roofline": {"bound": "hbm", "kernel": KERNEL_SYMBOL[dom], "achieved": round(kern_gbs[dom], 1),
                     "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kern_gbs[dom] / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(dom),
                     "algorithmic_bytes": alg[dom]},
        "compressed_bytes": plan.compressed_bytes(),
    }
    # STREAM-style copy: the achievable HBM bandwidth on this box
    src = torch.empty(1 << 28, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record(stream)
    for _ in range(10):
        dst.copy_(src)
    c1.record(stream)
    torch.cuda.synchronize()
    out["copy_gbs"] = round(2 * src.numel() * 10 / (c0.elapsed_time(c1) * 1e-3) / 1e9, 1)
    if args.copy_calib:
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
    del src, dst
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle, bounded sample)")
        out["cpu_baseline"] = cpu_baseline(corpus, plan)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
