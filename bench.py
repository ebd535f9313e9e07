"""Benchmark: proveKV codec hot path on one MI355X.

Workloads (`--workload`, default config3):

  config3  the metric's configuration: the SmolLM2-1.7B-shape N=8 pool -- 24
           layers x 32 KV heads x head_dim 64, an 800-token shared prefix in
           the fib_k4_n32 cold tier (FB2) and 8 agents x 28 unique tokens in the
           turbo b=4 hot tier (TQB1, lossless radii).  One step = build the
           pool + all 8 shells (encode: 2 launches) and rehydrate all 8 agents'
           full 1024-token KV -- pool and every shell decoded once and written
           to each agent's cache -- into HuggingFace-layout KV caches ([1, H,
           T, D] per layer and K|V, f32; decode: 2 launches; 3,221,225,472 B
           written).  The shell encode runs first, then the shell rehydrate on
           a second stream (on at most --side-workgroups workgroups) beside the
           pool encode (on at most --pool-workgroups), then the pool rehydrate
           (`--serial-tiers`: in order).
  config0  one layer, turbo b=4 lossless: K and V [32 heads, 1024 tokens, 64]
           (seed 0) -> 2 TQB1 blobs -> f32
  config1  fib_k4_n32 pool: 24 layers x {K,V} x 32 heads x 800 tokens (seed 1)
           -> 48 FB2 blobs in one launch -> f32 [tokens][heads][dim] per blob
  config2  turbo b=4 shells: 8 agents x 28 tokens x 24 layers x {K,V} x 32
           heads (seed 2) -> 384 TQB1 blobs in one launch, lossless and
           lossy (BlockLogU8) radii -> f32
  config4  Llama-3-8B KV: 32 layers x {K,V} x 8 heads x 32768 tokens x 128,
           bf16 in (generated on the device, seed 4), turbo b=4 + BlockLogU8
           radii -> 64 TQB1-L blobs -> f32
  legacy   per-vector KVecCodec records (TQW1 / FB1), host buffers
  score    attention scores on config-4 compressed keys

value = the workload's f32 KV bytes (the metric's "f32 in"; config 4: the
f32-equivalent bytes) / GPU time of one step (events at the two ends of K
back-to-back steps; inputs and outputs resident in HBM).  configs 0-2 and 4:
one step = encode + decode (the fused round trip); their K steps are queued
behind a GPU spin, so the events measure the GPU's time and not the host's
launch rate.  kernels_ms: a second pass with events between the launches.
roofline = the dominant kernel's algorithmic bytes per launch / its mean
duration (HIP events on its launch stream) against 8 TB/s; `traffic` = its
HBM bytes per launch from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
summary of the same workload, when there is one.
cpu_baseline = the C oracle (a restatement of the reference Rust CPU codecs,
oracle/pkv_oracle.c, -O3, AVX2 argmin) encoding + decoding the same blobs on
the host with profile constants prebuilt: one thread, and a thread per blob
on all the host cores this process may use (up to 16, the reference's rayon
tasks per (layer, K|V), proveKV/src/pool.rs:299-309); `value` is the
all-cores figure; the profile-constant build time is reported separately.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
                       [--workload config3|config0|config1|config2|config4|legacy|score]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

HBM_PEAK_GBS = 8000.0
VALU_PEAK_OPS = 256 * 4 * 16 * 2.4e9   # f32 lane-ops/s without packed FP32 (157.3 TFLOP/s / 4)
SEED = 42
MAX_CPU_THREADS = 16
ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# ================================================================ helpers
def need_gpu():
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU"}))
        sys.exit(1)


def cpu_info() -> dict:
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"nproc": os.cpu_count(), "usable": usable, "model": model,
            "threads": max(1, min(MAX_CPU_THREADS, usable))}


def cpu_baseline(jobs, job_bytes, total_bytes, what, budget_s=12.0) -> dict:
    """Oracle encode + decode of the workload's blobs on the host.  jobs[i]()
    encodes and decodes blob i; job_bytes[i] is its f32 KV bytes; the jobs
    cover total_bytes (or a stated sample of it).  One thread runs jobs in
    order until budget_s is spent (at least one); then a pool of the host's
    usable cores (<= 16) runs every job once.  GB/s of f32 KV, scaled to the
    whole workload."""
    info = cpu_info()
    t0 = time.perf_counter()
    done_bytes = 0
    k = 0
    while k < len(jobs):
        jobs[k]()
        done_bytes += job_bytes[k]
        k += 1
        if time.perf_counter() - t0 > budget_s:
            break
    t1 = time.perf_counter()
    single = done_bytes / (t1 - t0) / 1e9
    threads = info["threads"]
    with ThreadPoolExecutor(threads) as ex:
        t2 = time.perf_counter()
        list(ex.map(lambda f: f(), jobs))
        t3 = time.perf_counter()
    allc = sum(job_bytes) / (t3 - t2) / 1e9
    return {"value": round(allc, 4), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": (f"{what}: oracle/pkv_oracle.c (-O3, AVX2 argmin) encode + decode; 1 thread ran {k} of "
                       f"{len(jobs)} jobs ({done_bytes} B of f32 KV) in {t1 - t0:.2f} s; {threads} threads ran all "
                       f"{len(jobs)} jobs ({sum(job_bytes)} B) in {t3 - t2:.2f} s; workload {total_bytes} B"),
            "single_thread": {"value": round(single, 4), "unit": "GB/s", "cores": 1},
            "host": {"nproc": info["nproc"], "usable_cores": info["usable"], "model": info["model"]},
            "projected_s": {"single_thread": round(total_bytes / (single * 1e9), 2),
                            "all_cores": round(total_bytes / (allc * 1e9), 3)}}


def fib_constants_build_s() -> float:
    """One build of the fib_k4_n32 profile constants (Lloyd codebook + Haar
    rotation) by the oracle -- the cost the reference pays on every adapter
    call (FibQuantAdapter::build_quantizer, proveKV/src/codec.rs:471-499)."""
    from oracle import oracle as O
    t0 = time.perf_counter()
    O.fib_codebook(64, 4, 32, SEED, 2048, 4, 8)
    O.stored_rotation(64, SEED)
    return round(time.perf_counter() - t0, 4)


def profiled_traffic(summary: str, kernel: str):
    """HBM bytes per launch of `kernel` from a committed rocprofv3 PMC summary
    (calibrated FETCH_SIZE + WRITE_SIZE: lines `traffic_bytes <kernel> <B>`)."""
    path = os.path.join(ROOT, "profiles", summary)
    if not os.path.exists(path):
        return None
    for line in open(path):
        parts = line.strip().rsplit(" ", 1)
        if line.startswith("traffic_bytes ") and len(parts) == 2 and parts[0][len("traffic_bytes "):] == kernel:
            return int(parts[1])
    return None


def roofline(kernel: str, alg_bytes: int, ms: float, summary: str, tag: str = "") -> dict:
    """`tag` picks a labelled row of the summary (" [lossy]" where one run
    launches the same kernel for two workloads)."""
    gbs = alg_bytes / (ms * 1e-3) / 1e9
    return {"bound": "hbm", "kernel": kernel, "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": profiled_traffic(summary, kernel + tag),
            "algorithmic_bytes": int(alg_bytes)}


def copy_gbs(stream) -> float:
    """STREAM-style 256 MiB device copy: the achievable HBM bandwidth here."""
    import torch
    src = torch.empty(1 << 28, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    c0.record(stream)
    for _ in range(10):
        dst.copy_(src)
    c1.record(stream)
    torch.cuda.synchronize()
    return round(2 * src.numel() * 10 / (c0.elapsed_time(c1) * 1e-3) / 1e9, 1)


def copy_calib():
    """Two 256 MiB device copies: the reference kernel for the rocprofv3
    FETCH_SIZE / WRITE_SIZE byte calibration."""
    import torch
    src = torch.empty(1 << 28, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(2):
        dst.copy_(src)
    torch.cuda.synchronize()


def time_steps_queued(step, steps: int, stream) -> float:
    """ms per step of `steps` back-to-back steps, all enqueued behind a GPU
    spin before the GPU reaches them (the measurement is the GPU's time, not
    the host's launch rate); the spin is lengthened until the first event is
    still pending once everything is queued."""
    import torch
    spin = 20_000_000
    for _ in range(3):   # 20 M, 80 M, 320 M spin cycles
        t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            torch.cuda._sleep(spin)
        t_start.record(stream)
        for _ in range(steps):
            step()
        t_end.record(stream)
        queued_in_time = not t_start.query()
        torch.cuda.synchronize()
        if queued_in_time:
            return t_start.elapsed_time(t_end) / steps
        spin *= 4
    raise RuntimeError("could not queue the steps ahead of the GPU")


def kernel_ms(launches, steps: int, stream) -> list:
    """Mean GPU ms of each launch of a step (events between the launches, on
    the launch stream), over `steps` steps queued behind a spin."""
    import torch
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(launches) + 1)] for _ in range(steps)]
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        torch.cuda._sleep(50_000_000)
    for k in range(steps):
        evs[k][0].record(stream)
        for i, fn in enumerate(launches):
            fn()
            evs[k][i + 1].record(stream)
    torch.cuda.synchronize()
    return [float(np.mean([evs[k][i].elapsed_time(evs[k][i + 1]) for k in range(steps)]))
            for i in range(len(launches))]


def check_status(prof, status, segs):
    err = prof.status_error(status.cpu().numpy().view(np.uint32), segs)
    if err is not None:
        raise err


def pmap(fn, items, threads=8):
    with ThreadPoolExecutor(threads) as ex:
        return list(ex.map(fn, items))


# ================================================================ configs 0, 1, 2, 4
def codec_workload(args, *, name, metric, prof, radii, inp, segs, wire, out, f32_bytes, enc_alg, dec_alg,
                   kernels, summary, parity, cpu, data, config, dtype="f32", tag=""):
    """Encode all segments into `wire`, decode them into `out`: timed as the
    fused round trip (value) and per kernel."""
    import torch
    stream = torch.cuda.current_stream()
    est = torch.empty(2 * len(segs), dtype=torch.int32, device="cuda")
    dst = torch.empty_like(est)

    def enc():
        prof.encode_segments(inp, segs, wire, radii=radii, status=est)

    def dec():
        prof.decode_segments(wire, segs, out, radii=radii, status=dst)

    def step():
        enc()
        dec()

    log(f"[bench] {name}: {len(segs)} blobs, warmup {args.warmup}")
    for _ in range(max(1, args.warmup)):
        step()
    torch.cuda.synchronize()
    check_status(prof, est, segs)
    check_status(prof, dst, segs)
    log("[bench] parity spot check against the oracle")
    parity_ok = parity()
    if not parity_ok:
        raise AssertionError(f"{name}: GPU bytes or decodes differ from the oracle")
    log(f"[bench] timing {args.steps} steps")
    t0 = time.perf_counter()
    step_ms = time_steps_queued(step, args.steps, stream)
    wall = time.perf_counter() - t0
    enc_ms, dec_ms = kernel_ms([enc, dec], args.steps, stream)
    check_status(prof, est, segs)
    check_status(prof, dst, segs)
    dom = 0 if enc_ms >= dec_ms else 1
    res = {
        "metric": metric,
        "value": round(f32_bytes / (step_ms * 1e-3) / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": dtype, "data": data, "config": config,
        "hbm_fraction_codec": round((enc_alg + dec_alg) / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "kernels_ms": {"encode": round(enc_ms, 4), "decode": round(dec_ms, 4)},
        "kernels_gbs": {"encode": round(enc_alg / (enc_ms * 1e-3) / 1e9, 1),
                        "decode": round(dec_alg / (dec_ms * 1e-3) / 1e9, 1)},
        "algorithmic_bytes": {"encode": int(enc_alg), "decode": int(dec_alg)},
        "roofline": roofline(kernels[dom], (enc_alg, dec_alg)[dom], (enc_ms, dec_ms)[dom], summary, tag),
        "roofline_other": roofline(kernels[1 - dom], (enc_alg, dec_alg)[1 - dom], (enc_ms, dec_ms)[1 - dom],
                                   summary, tag),
        "parity_checked": True,
        "wall_s_timed": round(wall, 3),
        "copy_gbs": copy_gbs(stream),
    }
    if args.copy_calib:
        copy_calib()
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle)")
        res["cpu_baseline"] = cpu()
        res["cpu_baseline"]["constants_build_s"] = fib_constants_build_s()
    return res


def _turbo_jobs(xs_list, radii, dim=64):
    """Oracle encode + decode of each input batch (turbo b=4, QJL-32, seed 42)."""
    from oracle import oracle as O
    signs, G = O.turbo_constants(dim, 32, SEED)

    def job(x):
        return lambda: O.turbo_decode_batch(O.turbo_encode_batch(x, SEED, radii_codec=radii, signs=signs, G=G),
                                            dim, SEED, signs=signs)
    return [job(x) for x in xs_list], [x.size * 4 for x in xs_list]


def _fib_jobs(xs_list):
    from oracle import oracle as O
    cb, rot = O.fib_constants(SEED)

    def job(x):
        return lambda: O.fib_decode_batch(O.fib_encode_batch(x, cb, rot), cb, rot)
    return [job(x) for x in xs_list], [x.size * 4 for x in xs_list]


def _blob_parity(prof, wire, out, segs, blob_inputs, picks, encode_ref, decode_ref, dim):
    """Blobs `picks`: wire bytes and decodes (segment layout of `segs`: one
    contiguous [n][dim] block per blob) against the oracle."""
    w = wire.cpu().numpy()
    o = out.cpu().numpy()

    def one(b):
        s = segs[b]
        n = int(s["n_vectors"])
        ref = encode_ref(blob_inputs(b))
        off = int(s["wire_offset"])
        if w[off:off + len(ref)].tobytes() != ref:
            return False
        want = decode_ref(ref)
        e0 = int(s["elem_offset"])
        return np.array_equal(o[e0:e0 + n * dim].view(np.uint32), want.reshape(-1).view(np.uint32))
    return all(pmap(one, picks))


def bench_config0(args):
    import torch
    from oracle import oracle as O
    from provekv_amd import _lib as L
    from provekv_amd import device as D
    from provekv_amd import synth
    need_gpu()
    K, V = synth.kv_cache(0, 1, 32, 1024, 64)
    x = np.ascontiguousarray(np.stack([K[0], V[0]]))                      # [K|V][H][T][D]
    n = 32 * 1024
    ctx = D.default_context()
    prof = ctx.turbo_profile(64, 4, 32, SEED, 1)
    blob = prof.blob_len(n)
    segs = D.segments([D.contiguous_segment(0, n, 64, 0), D.contiguous_segment(n * 64, n, 64, blob)])
    inp = torch.from_numpy(x.reshape(-1)).cuda()
    wire = torch.empty(2 * blob, dtype=torch.uint8, device="cuda")
    out = torch.empty(2 * n * 64, dtype=torch.float32, device="cuda")
    signs, G = O.turbo_constants(64, 32, SEED)
    xs = [x[0].reshape(-1, 64), x[1].reshape(-1, 64)]
    chunks = [c for v in xs for c in np.split(v, 8)]                      # rayon's per-vector split
    jobs, jb = _turbo_jobs([np.ascontiguousarray(c) for c in chunks], 0)
    res = codec_workload(
        args, name="config0", prof=prof, radii=L.RADII_F32, inp=inp, segs=segs, wire=wire, out=out,
        metric="KV codec encode+decode GB/s (f32 in) and % HBM peak, config 0 (single-layer turbo b=4 round trip)",
        f32_bytes=x.nbytes, enc_alg=x.nbytes + 2 * blob, dec_alg=2 * blob + x.nbytes,
        kernels=("turbo_encode_qjl_kernel<3, false>", "turbo_decode_split_kernel<3>"),
        summary="codec_kernels_config0.md",
        parity=lambda: _blob_parity(prof, wire, out, segs, lambda b: xs[b], [0, 1],
                                    lambda v: O.turbo_encode_batch(v, SEED, signs=signs, G=G),
                                    lambda bb: O.turbo_decode_batch(bb, 64, SEED, signs=signs), 64),
        cpu=lambda: cpu_baseline(jobs, jb, x.nbytes, "config 0, 16 chunks of 4096 vectors"),
        data="synthetic (seed 0: log-normal K channel scales with 2 outlier channels x8 per head, V = 0.5 N(0,1))",
        config={"workload": "config0: K and V [32 heads, 1024 tokens, 64] [H][T][D], turbo b=4 (3-bit angles + "
                            "QJL-32), f32 radii, TQB1 round trip", "blobs": 2, "vectors": 2 * n, "seed": SEED})
    print(json.dumps(res), flush=True)


def bench_config1(args):
    import torch
    from oracle import oracle as O
    from provekv_amd import _lib as L
    from provekv_amd import synth
    from provekv_amd.device import default_context
    from provekv_amd.pool import TwoTierPlan
    need_gpu()
    layers, heads, dim, prefix = 24, 32, 64, 800
    log("[bench] generating the config-1 corpus (seed 1)")
    corpus = synth.corpus_tokens(1, layers, heads, prefix, dim)
    ctx = default_context()
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, [], seed=SEED)
    prof, tier = plan.fib, plan.pool
    inp = torch.from_numpy(corpus.reshape(-1)).cuda()
    wire = torch.empty(tier.wire_bytes, dtype=torch.uint8, device="cuda")
    out = torch.empty(tier.out_elems, dtype=torch.float32, device="cuda")
    cb, rot = O.fib_constants(SEED)

    def blob_in(b):
        _, layer, side, _, _ = tier.blob_offsets[b]
        return np.ascontiguousarray(corpus[:, layer, :, side, :]).reshape(-1, dim)
    jobs, jb = _fib_jobs([blob_in(b) for b in range(len(tier.blob_offsets))])
    f32 = corpus.nbytes

    class Prof:   # encode reads the corpus layout (tier.enc), decode writes [T][H][D] per blob (tier.dec)
        status_error = prof.status_error

        @staticmethod
        def encode_segments(i, s, w, radii, status):
            prof.encode_segments(i, tier.enc, w, status=status)

        @staticmethod
        def decode_segments(w, s, o, radii, status):
            prof.decode_segments(w, tier.dec, o, status=status)
    res = codec_workload(
        args, name="config1", prof=Prof, radii=L.RADII_F32, inp=inp, segs=tier.dec, wire=wire, out=out,
        metric="KV codec encode+decode GB/s (f32 in) and % HBM peak, config 1 (fib_k4_n32 cold pool)",
        f32_bytes=f32, enc_alg=f32 + tier.wire_bytes, dec_alg=tier.wire_bytes + f32,
        kernels=("fib_encode_kernel<64, false>", "fib_decode_mfma_kernel<64, false>"),
        summary="codec_kernels_config1.md",
        parity=lambda: _blob_parity(prof, wire, out, tier.dec, blob_in, [0, 1, 23, 46, 47],
                                    lambda v: O.fib_encode_batch(v, cb, rot),
                                    lambda bb: O.fib_decode_batch(bb, cb, rot), dim),
        cpu=lambda: cpu_baseline(jobs, jb, f32, "config 1, the 48 pool blobs"),
        data="synthetic (seed 1: log-normal K channel scales with 2 outlier channels x8 per head, V = 0.5 N(0,1))",
        config={"workload": "config1: fib_k4_n32 pool 24L x {K,V} x 32H x 800 tokens x d64 -> 48 FB2 blobs "
                            "(one launch) -> f32 [T][H][D] per blob", "blobs": len(tier.enc),
                "vectors": int(tier.enc["n_vectors"].sum()), "wire_bytes": tier.wire_bytes, "seed": SEED})
    print(json.dumps(res), flush=True)


def bench_config2(args):
    import torch
    from oracle import oracle as O
    from provekv_amd import _lib as L
    from provekv_amd import synth
    from provekv_amd.device import default_context
    from provekv_amd.pool import TwoTierPlan
    need_gpu()
    layers, heads, dim, agents = 24, 32, 64, [28] * 8
    log("[bench] generating the config-2 corpus (seed 2)")
    corpus = synth.corpus_tokens(2, layers, heads, sum(agents), dim)
    ctx = default_context()
    inp = torch.from_numpy(corpus.reshape(-1)).cuda()
    signs, G = O.turbo_constants(dim, 32, SEED)
    lines = {}
    for lossy in (False, True):
        plan = TwoTierPlan(ctx, layers, heads, dim, 0, agents, seed=SEED, lossy=lossy)
        prof, tier = plan.turbo, plan.shells
        wire = torch.empty(tier.wire_bytes, dtype=torch.uint8, device="cuda")
        out = torch.empty(tier.out_elems, dtype=torch.float32, device="cuda")
        rc = plan.radii

        def blob_in(b, tier=tier):
            name, layer, side, _, _ = tier.blob_offsets[b]
            a = int(name[5:])
            return np.ascontiguousarray(corpus[28 * a:28 * a + 28, layer, :, side, :]).reshape(-1, dim)
        jobs, jb = _turbo_jobs([blob_in(b) for b in range(len(tier.blob_offsets))], rc)

        class Prof:
            status_error = prof.status_error

            @staticmethod
            def encode_segments(i, s, w, radii, status, prof=prof, tier=tier):
                prof.encode_segments(i, tier.enc, w, radii=radii, status=status)

            @staticmethod
            def decode_segments(w, s, o, radii, status, prof=prof, tier=tier):
                prof.decode_segments(w, tier.dec, o, radii=radii, status=status)
        f32 = corpus.nbytes
        lines[lossy] = codec_workload(
            args, name=f"config2 ({'lossy' if lossy else 'lossless'})", prof=Prof, radii=rc, inp=inp,
            segs=tier.dec, wire=wire, out=out,
            metric="KV codec encode+decode GB/s (f32 in) and % HBM peak, config 2 (N=8 turbo b=4 shells)",
            f32_bytes=f32, enc_alg=f32 + tier.wire_bytes, dec_alg=tier.wire_bytes + f32,
            kernels=("turbo_encode_qjl_kernel<3, false>", "turbo_decode_split_kernel<3>"),
            summary="codec_kernels_config2.md", tag=" [lossy]" if lossy else " [lossless]",
            parity=lambda prof=prof, wire=wire, out=out, tier=tier, blob_in=blob_in, rc=rc: _blob_parity(
                prof, wire, out, tier.dec, blob_in, [0, 1, 191, 383],
                lambda v: O.turbo_encode_batch(v, SEED, radii_codec=rc, signs=signs, G=G),
                lambda bb: O.turbo_decode_batch(bb, dim, SEED, signs=signs), dim),
            cpu=lambda jobs=jobs, jb=jb: cpu_baseline(jobs, jb, f32, "config 2, the 384 shell blobs"),
            data="synthetic (seed 2: log-normal K channel scales with 2 outlier channels x8 per head, "
                 "V = 0.5 N(0,1))",
            config={"workload": f"config2: 8 agents x 28 tokens x 24L x {{K,V}} x 32H x d64 -> 384 TQB1"
                                f"{'-L (BlockLogU8 radii)' if lossy else ' (f32 radii)'} blobs (one launch) -> f32",
                    "blobs": len(tier.enc), "vectors": int(tier.enc["n_vectors"].sum()),
                    "wire_bytes": tier.wire_bytes, "radii": "BlockLogU8" if lossy else "f32", "seed": SEED})
    res = lines[False]
    res["lossy"] = {k: lines[True][k] for k in ("value", "ms_per_step", "kernels_ms", "kernels_gbs", "roofline",
                                                "hbm_fraction_codec", "config", "cpu_baseline") if k in lines[True]}
    print(json.dumps(res), flush=True)


def bench_config4(args):
    import torch
    from oracle import oracle as O
    from provekv_amd import _lib as L
    from provekv_amd import device as D
    from provekv_amd import synth
    need_gpu()
    layers, heads, tokens, dim = 32, 8, 32768, 128
    n = heads * tokens
    log("[bench] generating the config-4 KV on the device (bf16, seed 4)")
    x = synth.device_kv_bf16(4, layers, heads, tokens, dim)               # [L][K|V][H][T][D]
    flat = x.view(-1)
    ctx = D.default_context()
    prof = ctx.turbo_profile(dim, 4, 32, SEED, 1)
    rc = L.RADII_LOG_U8
    blob = prof.blob_len(n, rc)
    nb = 2 * layers
    segs = D.segments([D.contiguous_segment(b * n * dim, n, dim, b * blob) for b in range(nb)])
    wire = torch.empty(nb * blob, dtype=torch.uint8, device="cuda")
    out = torch.empty(nb * n * dim, dtype=torch.float32, device="cuda")
    signs, G = O.turbo_constants(dim, 32, SEED)
    rng = np.random.RandomState(4)
    picks = (0, 21, 42, 63)
    samp = {b: np.sort(rng.choice(n, 2048, replace=False)) for b in picks}
    plen = prof.payload_len(rc)

    def parity():
        ok = True
        for b in picks:
            ti = torch.from_numpy(samp[b]).cuda()
            xs = flat[b * n * dim:(b + 1) * n * dim].view(n, dim)[ti].float().cpu().numpy()
            ref = O.turbo_encode_batch(xs, SEED, radii_codec=rc, signs=signs, G=G)
            got = wire[b * blob + 38:(b + 1) * blob].view(n, plen)[ti].cpu().numpy()
            ok &= got.tobytes() == ref[38:]
            dec = out[b * n * dim:(b + 1) * n * dim].view(n, dim)[ti].cpu().numpy()
            ok &= np.array_equal(dec.view(np.uint32), O.turbo_decode_batch(ref, dim, SEED, signs=signs).view(np.uint32))
        return ok

    # CPU sample: 8192 vectors of every blob (the f32 upcast of the bf16 input)
    cs = [np.ascontiguousarray(flat[b * n * dim:(b * n + 8192) * dim].view(8192, dim).float().cpu().numpy())
          for b in range(nb)]
    jobs, jb = _turbo_jobs(cs, rc, dim)
    f32 = nb * n * dim * 4
    res = codec_workload(
        args, name="config4", prof=prof, radii=rc, inp=flat, segs=segs, wire=wire, out=out,
        metric="KV codec encode+decode GB/s (f32-equivalent KV) and % HBM peak, config 4 (Llama-3-8B shape)",
        f32_bytes=f32, enc_alg=nb * n * dim * 2 + wire.numel(), dec_alg=wire.numel() + f32,
        kernels=("turbo_encode_qjl128_kernel<3, false>", "turbo_decode_split128_kernel<3>"),
        summary="codec_kernels_config4.md", parity=parity,
        cpu=lambda: cpu_baseline(jobs, jb, f32, "config 4, the first 8192 vectors of each of the 64 blobs "
                                 "(f32 upcast of the bf16 input)", budget_s=10.0),
        data="synthetic (seed 4, generated on the GPU: K = LogNormal(0, 0.7) channel scales with 4 outlier "
             "channels x10 per head times N(0,1), V = N(0,1), rounded to bf16)",
        config={"workload": "config4: 32L x {K,V} x 8 KV heads x 32768 tokens x d128, bf16 in, turbo b=4 QJL-32, "
                            "TQB1-L (BlockLogU8 radii) -> f32", "blobs": nb, "vectors": nb * n,
                "wire_bytes": int(wire.numel()), "seed": SEED},
        dtype="f32 arithmetic on bf16 input")
    print(json.dumps(res), flush=True)


# ================================================================ config 3 (the metric)
def spot_check_cache(plan, bufs, cache, corpus):
    """The rehydrated cache against the oracle (its own constants) on one pool
    blob and one shell blob (layer 0, K), every cache copy."""
    import torch
    from oracle import oracle as O
    cb, rot = O.fib_constants(SEED)
    heads, dim = plan.heads, plan.dim
    checks = [(0, plan.prefix, O.fib_decode_batch(plan.blob(bufs, "pool", 0), cb, rot)),
              (plan.prefix, plan.agent_tokens[0], O.turbo_decode_batch(plan.blob(bufs, "shell", 0), dim, SEED))]
    for t0, nt, dec in checks:
        want = torch.from_numpy(np.ascontiguousarray(dec.reshape(nt, heads, dim).transpose(1, 0, 2)))
        want = want.to(cache.buf.dtype)
        for c in range(cache.copies):
            got = cache.buf[c, 0, 0, :, t0:t0 + nt, :].cpu()
            if not torch.equal(got, want):
                raise AssertionError(f"rehydrated cache differs from the oracle (copy {c}, tokens {t0}..)")
    # the encoded bytes of those blobs
    x_pool = np.ascontiguousarray(corpus[:plan.prefix, 0, :, 0, :]).reshape(-1, dim)
    if plan.blob(bufs, "pool", 0) != O.fib_encode_batch(x_pool, cb, rot):
        raise AssertionError("pool blob 0 differs from the oracle")
    x_sh = np.ascontiguousarray(corpus[plan.prefix:plan.prefix + plan.agent_tokens[0], 0, :, 0, :]).reshape(-1, dim)
    if plan.blob(bufs, "shell", 0) != O.turbo_encode_batch(x_sh, SEED, radii_codec=plan.radii):
        raise AssertionError("shell blob 0 differs from the oracle")


def bench_config3(args):
    import torch
    from provekv_amd import synth
    from provekv_amd.device import default_context
    from provekv_amd.pool import DeviceKVCache, TwoTierPlan
    need_gpu()
    kernel = {"fib_encode": "fib_encode_kernel<64, false>", "turbo_encode": "turbo_encode_qjl_kernel<3, false>",
              "fib_decode": "fib_decode_mfma_kernel<64, true>" if args.copies > 1 else
                            "fib_decode_mfma_kernel<64, false>",
              "turbo_decode": "turbo_decode_split_kernel<3>"}
    layers, heads, dim, prefix, agents = 24, 32, 64, 800, [28] * 8
    log(f"[bench] generating synthetic corpus ({prefix + sum(agents)} tokens x {layers}L x {heads}H x 2 x {dim})")
    corpus = synth.corpus_tokens(3, layers, heads, prefix + sum(agents), dim)
    ctx = default_context()
    log("[bench] building profiles (fib codebook + rotation, turbo signs + QJL)")
    plan = TwoTierPlan(ctx, layers, heads, dim, prefix, agents, seed=SEED, lossy=args.lossy)
    bufs = plan.alloc()
    cache_dtype = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[args.cache_dtype]
    cache = DeviceKVCache(layers, heads, plan.tokens, dim, dtype=cache_dtype, copies=args.copies)
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    stream = torch.cuda.current_stream()
    side = None if args.serial_tiers else torch.cuda.Stream()   # default priority

    def step():
        plan.build_and_rehydrate(dev, bufs, cache, stream=stream, side=side, side_workgroups=args.side_workgroups,
                                 pool_workgroups=args.pool_workgroups)

    def launches():
        pseg, sseg = plan._cache_segs
        out = cache.buf.view(-1)
        return [
            lambda: plan.fib.encode_segments(dev, plan.pool.enc, bufs["pool_wire"], status=bufs["pool_status"]),
            lambda: plan.turbo.encode_segments(dev, plan.shells.enc, bufs["shell_wire"], radii=plan.radii,
                                               status=bufs["shell_status"]),
            lambda: plan.fib.decode_segments(bufs["pool_wire"], pseg, out, status=bufs["pool_cstatus"],
                                             fanout=cache.copies, fanout_stride=cache.copy_stride),
            lambda: plan.turbo.decode_segments(bufs["shell_wire"], sseg, out, radii=plan.radii,
                                               status=bufs["shell_cstatus"], fanout=cache.copies,
                                               fanout_stride=cache.copy_stride)]

    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    plan.check(bufs, decode=False)
    plan.check_rehydrate(bufs)
    spot_check_cache(plan, bufs, cache, corpus)
    run_step, graph_ok = step, None
    if args.graph:
        # one step captured into a HIP graph (both streams): a replay issues the
        # same kernels without the host launch path between them
        log("[bench] capturing one step into a HIP graph")
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=torch.cuda.Stream()):
            plan.build_and_rehydrate(dev, bufs, cache, stream=torch.cuda.current_stream(), side=side,
                                     side_workgroups=args.side_workgroups, pool_workgroups=args.pool_workgroups)
        torch.cuda.synchronize()
        # a replay must reproduce the eager step's bytes: outputs spoiled first
        names_out = ("pool_wire", "shell_wire", "pool_status", "shell_status", "pool_cstatus", "shell_cstatus")
        step()
        torch.cuda.synchronize()
        want = [bufs[k].clone() for k in names_out] + [cache.buf.clone()]
        for k in names_out:
            bufs[k].fill_(0x5A)
        cache.buf.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        got = [bufs[k] for k in names_out] + [cache.buf]
        graph_ok = all(torch.equal(a.view(torch.uint8), b.view(torch.uint8)) for a, b in zip(want, got))
        del want
        if not graph_ok:
            raise AssertionError("config3: the graph replay differs from the eager step")
        run_step = graph.replay
    # timed region: K whole steps, events only at its two ends
    log(f"[bench] timing {args.steps} steps")
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    t_start.record(stream)
    for _ in range(args.steps):
        run_step()
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_gpu_ms = t_start.elapsed_time(t_end) / args.steps
    plan.check(bufs, decode=False)
    plan.check_rehydrate(bufs)
    # per-op breakdown from a separate pass with events between the four launches
    names = ["fib_encode", "turbo_encode", "fib_decode", "turbo_decode"]
    per = dict(zip(names, kernel_ms(launches(), args.steps, stream)))
    n_pool = prefix * heads * layers * 2
    n_shell = sum(agents) * heads * layers * 2
    f32_pool = n_pool * dim * 4
    f32_shell = n_shell * dim * 4
    wire_pool = plan.pool.wire_bytes
    wire_shell = plan.shells.wire_bytes
    out_scale = args.copies * cache.buf.element_size() / 4   # cache bytes written per f32 input byte
    alg = {"fib_encode": f32_pool + wire_pool, "turbo_encode": f32_shell + wire_shell,
           "fib_decode": int(f32_pool * out_scale) + wire_pool, "turbo_decode": int(f32_shell * out_scale) + wire_shell}
    kern_gbs = {n: alg[n] / (per[n] * 1e-3) / 1e9 for n in names}
    f32_total = f32_pool + f32_shell
    value = f32_total / (step_gpu_ms * 1e-3) / 1e9
    dom = max(("fib_decode", "turbo_encode", "turbo_decode", "fib_encode"), key=lambda n: per[n])
    summary = "codec_kernels_config3.md"
    out = {
        "metric": "KV codec encode+decode GB/s (f32 in) and % HBM peak, SmolLM2-1.7B-shape N=8 pool",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_gpu_ms, 4),
        "ms_per_step_wall": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded log-normal K with outlier channels, Gaussian V)",
        "config": {"workload": "config3: N=8 two-tier pool, 24L x 32H x d64, 800-token fib_k4_n32 prefix + "
                               "8 x 28-token turbo b=4 shells" + (" (TQB1-L lossy radii)" if args.lossy else
                                                                  " (TQB1 lossless radii)") +
                               f", rehydrated into {args.copies} x [1,H,T,D] {args.cache_dtype} KV cache(s)",
                   "layers": layers, "kv_heads": heads, "head_dim": dim, "prefix_tokens": prefix,
                   "agents": len(agents), "agent_tokens": agents[0], "seed": SEED,
                   "cache_dtype": args.cache_dtype, "cache_copies": args.copies,
                   "tier_streams": 1 if args.serial_tiers else 2,
                   "hip_graph": graph_ok is not None,
                   "side_workgroups": None if args.serial_tiers else args.side_workgroups,
                   "pool_workgroups": None if args.serial_tiers else args.pool_workgroups},
        "hbm_fraction_codec": round(sum(alg.values()) / (step_gpu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "kernels_ms": {n: round(per[n], 4) for n in names},
        "kernels_gbs": {n: round(kern_gbs[n], 1) for n in names},
        "roofline": roofline(kernel[dom], alg[dom], per[dom], summary),
        "roofline_all": {n: roofline(kernel[n], alg[n], per[n], summary) for n in names},
        "graph_replay_matches_eager": graph_ok,
        "compressed_bytes": plan.compressed_bytes(),
        "rehydrated_bytes": cache.buf.numel() * cache.buf.element_size(),
        "copy_gbs": copy_gbs(stream),
    }
    if args.copy_calib:
        copy_calib()
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (oracle, the whole workload: 48 pool + 384 shell blobs)")
        jobs, jb = [], []
        for b in range(len(plan.pool.blob_offsets)):
            _, layer, side_, _, _ = plan.pool.blob_offsets[b]
            xb = np.ascontiguousarray(corpus[:prefix, layer, :, side_, :]).reshape(-1, dim)
            j, s = _fib_jobs([xb])
            jobs += j
            jb += s
        xs = []
        for b in range(len(plan.shells.blob_offsets)):
            name, layer, side_, _, _ = plan.shells.blob_offsets[b]
            t0_ = prefix + 28 * int(name[5:])
            xs.append(np.ascontiguousarray(corpus[t0_:t0_ + 28, layer, :, side_, :]).reshape(-1, dim))
        j, s = _turbo_jobs(xs, plan.radii)
        jobs += j
        jb += s
        out["cpu_baseline"] = cpu_baseline(jobs, jb, f32_total, "config 3 (decode once, no cache fan-out)")
        out["cpu_baseline"]["constants_build_s"] = fib_constants_build_s()
    print(json.dumps(out), flush=True)


# ================================================================ legacy records
def bench_legacy(args):
    """Per-vector KVecCodec records through the host-buffer entry points
    (pkv_encode_vectors / pkv_decode_vectors, PCIe copies included): a
    config-1-sized pool as FB1 records and config-2-sized shells as TQW1
    records.  Prints one JSON line; the kernel durations come from rocprofv3."""
    import ctypes as C

    from oracle import oracle as O
    from provekv_amd import _lib as L
    from provekv_amd import synth
    from provekv_amd.device import default_context
    need_gpu()
    ctx = default_context()
    fib = ctx.fib_profile(64, 4, 32, SEED)
    tur = ctx.turbo_profile(64, 4, 32, SEED, 1)
    log("[bench] generating config-1 / config-2 shaped vectors")
    x1 = np.ascontiguousarray(synth.corpus_tokens(1, 24, 32, 800, 64).reshape(-1, 64))
    x2 = np.ascontiguousarray(synth.corpus_tokens(2, 24, 32, 224, 64).reshape(-1, 64))

    def enc(prof, x, each):
        n, rec = x.shape[0], prof.record_len()
        out = np.empty(n * rec, np.uint8)
        ln, err = C.c_uint64(), L.Error()
        rc = L.lib().pkv_encode_vectors(ctx.ptr, prof.ptr, int(each), x.ctypes.data, n, out.ctypes.data, out.size,
                                        C.byref(ln), C.byref(err))
        if rc:
            raise L.PkvError(rc, "pkv_encode_vectors", err.segment, err.index)
        return out

    def dec(prof, recs, n, each):
        off = np.arange(n + 1, dtype=np.uint64) * np.uint64(prof.record_len())
        out = np.empty((n, 64), np.float32)
        err = L.Error()
        rc = L.lib().pkv_decode_vectors(ctx.ptr, prof.ptr, int(each), recs.ctypes.data, off.ctypes.data, n,
                                        out.ctypes.data, n, C.byref(err))
        if rc:
            raise L.PkvError(rc, "pkv_decode_vectors", err.segment, err.index)
        return out

    def timed(fn):
        fn()
        best = float("inf")
        for _ in range(args.steps):
            t0 = time.perf_counter()
            r = fn()
            best = min(best, time.perf_counter() - t0)
        return r, best

    ops = {}
    r_fib, t = timed(lambda: enc(fib, x1, False))
    ops["fib_fb1_encode_batch"] = (x1.shape[0], t)
    _, t = timed(lambda: enc(fib, x1, True))
    ops["fib_fb1_encode_each"] = (x1.shape[0], t)
    d_fast, t = timed(lambda: dec(fib, r_fib, x1.shape[0], False))
    ops["fib_fb1_decode_batch"] = (x1.shape[0], t)
    d_f64, t = timed(lambda: dec(fib, r_fib, x1.shape[0], True))
    ops["fib_fb1_decode_each_f64"] = (x1.shape[0], t)
    r_tur, t = timed(lambda: enc(tur, x2, True))
    ops["turbo_tqw1_encode"] = (x2.shape[0], t)
    d_tur, t = timed(lambda: dec(tur, r_tur, x2.shape[0], True))
    ops["turbo_tqw1_decode"] = (x2.shape[0], t)
    # parity spot check against the oracle (its own constants) on the first records
    m = 2000
    cb, rot = O.fib_constants(SEED)
    rec1 = fib.record_len()
    ref = O.fib_encode_fb1(x1[:m], cb, rot, each=False)
    parity = b"".join(ref) == r_fib[:m * rec1].tobytes()
    parity &= np.array_equal(O.fib_decode_fb1(ref, cb, rot, each=True).view(np.uint32), d_f64[:m].view(np.uint32))
    rec2 = tur.record_len()
    ref2 = O.turbo_encode_tqw1(x2[:m], SEED)
    parity &= b"".join(ref2) == r_tur[:m * rec2].tobytes()
    parity &= np.array_equal(O.turbo_decode_tqw1(ref2, 64, SEED).view(np.uint32), d_tur[:m].view(np.uint32))
    out = {"workload": "legacy per-vector records (KVecCodec::encode/decode): config-1 pool as 1,228,800 FB1 "
                       "records, config-2 shells as 344,064 TQW1 records, host buffers (PCIe included)",
           "unit": "GB/s of f32 KV", "steps": args.steps, "parity_first_2000": bool(parity),
           "ops": {k: {"vectors": n, "ms": round(t * 1e3, 3), "gbs": round(n * 256 / t / 1e9, 2)}
                   for k, (n, t) in ops.items()}}
    if args.copy_calib:
        copy_calib()
    print(json.dumps(out), flush=True)


# ================================================================ scoring
def bench_score(args):
    """Scoring on compressed keys (TurboQuantizer::inner_product_estimate_prepared,
    the attention logits of KvShadowCache::attention_scores, turbo-quant/src/
    kv.rs:269-320) at the config-4 shape: the K half of Llama-3-8B's KV
    (32 layers x 8 KV heads x 32768 tokens, head_dim 128) as TQB1-L blobs
    resident in HBM, one blob per (layer, KV head); each blob scored against
    its GQA group of 4 query heads (32 query heads / 8 KV heads), scale
    1/sqrt(128).  One step = prepare the 1024 queries + one scoring launch.
    value = query-key scores per second.  Parity: sampled codes of several
    blobs against the C oracle, bit for bit."""
    import torch
    from oracle import oracle as O
    from provekv_amd import _lib as L
    from provekv_amd import synth
    from provekv_amd.device import SEG_DTYPE, default_context
    need_gpu()
    layers, kv_heads, tokens, dim, group = 32, 8, 32768, 128, 4
    log("[bench] generating the config-4 keys on the device (bf16, seed 4)")
    kv = synth.device_kv_bf16(4, layers, kv_heads, tokens, dim)
    x = kv[:, 0].contiguous().view(-1)                                    # K: [L][H][T][D]
    del kv
    nseg = layers * kv_heads
    ctx = default_context()
    prof = ctx.turbo_profile(dim, 4, 32, SEED)
    est = torch.empty(2 * nseg, dtype=torch.int32, device="cuda")
    wires = {}
    for radii in (L.RADII_LOG_U8, L.RADII_F32):
        plen_r = prof.payload_len(radii)
        blob_r = 38 + tokens * plen_r
        segs = np.array([(b * tokens * dim, 0, dim, b * blob_r, tokens, tokens) for b in range(nseg)],
                        dtype=SEG_DTYPE)
        w = torch.empty(nseg * blob_r, dtype=torch.uint8, device="cuda")
        log(f"[bench] encoding {nseg} key blobs x {tokens} tokens, radii codec {radii} (untimed)")
        prof.encode_segments(x, segs, w, radii=radii, status=est)
        torch.cuda.synchronize()
        check_status(prof, est, segs)
        wires[radii] = (w, plen_r, blob_r)
    del x
    wire, plen, blob = wires[L.RADII_LOG_U8]
    nq = nseg * group
    rng = np.random.RandomState(11)
    qh = rng.randn(nq, dim).astype(np.float32)
    q = torch.from_numpy(qh).cuda()
    W = prof.prepared_len()
    prep = torch.empty((nq, W), dtype=torch.float32, device="cuda")
    ld = nseg * tokens
    scores = torch.empty(group * ld, dtype=torch.float32, device="cuda")
    seg_tabs = {r: np.array([(b * tokens, 1, 1, b * wires[r][2], tokens, 1) for b in range(nseg)], dtype=SEG_DTYPE)
                for r in wires}
    pst = torch.empty(2, dtype=torch.int32, device="cuda")
    sst = torch.empty(2 * nseg, dtype=torch.int32, device="cuda")
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dim)))
    stream = torch.cuda.current_stream()

    def prep_fn():
        prof.prepare_queries(q, prep, status=pst)

    def score_fn(radii=L.RADII_LOG_U8):
        prof.score_segments(wires[radii][0], seg_tabs[radii], prep, scores, ld, radii=radii, post_scale=scale,
                            status=sst, nq=group, query_stride=group)

    for _ in range(max(1, args.warmup)):
        prep_fn()
        score_fn()
    torch.cuda.synchronize()
    perr = prof.status_error(pst.cpu().numpy().view(np.uint32))
    serr = prof.score_status_error(sst.cpu().numpy().view(np.uint32))
    if perr is not None or serr is not None:
        raise perr or serr
    steps = max(1, args.steps)
    log(f"[bench] timing {steps} steps")
    step_ms = time_steps_queued(lambda: (prep_fn(), score_fn()), steps, stream)
    prep_ms, score_ms = kernel_ms([prep_fn, score_fn], steps, stream)
    score32_ms, = kernel_ms([lambda: score_fn(L.RADII_F32)], steps, stream)
    torch.cuda.synchronize()
    serr = prof.score_status_error(sst.cpu().numpy().view(np.uint32))
    if serr is not None:
        raise serr
    w32, plen32, blob32 = wires[L.RADII_F32]
    alg32 = nseg * blob32 + nseg * tokens * group * 4 + nq * prof.prepared_len() * 4
    score_fn()   # TQB1-L scores for the parity sample
    torch.cuda.synchronize()
    pref = O.turbo_prepare_queries(qh, SEED)
    parity = np.array_equal(prep.cpu().numpy().view(np.uint32), pref.view(np.uint32))
    got_all = scores.reshape(group, ld)
    samp = np.random.RandomState(5)
    for b in (0, 1, nseg // 2, nseg - 1):
        idx = np.sort(samp.choice(tokens, 256, replace=False))
        w = wire[b * blob:(b + 1) * blob].cpu().numpy()
        sub = w[:38].copy()
        sub[30:34] = np.frombuffer(np.uint32(len(idx)).tobytes(), np.uint8)
        sub = sub.tobytes() + w[38:].reshape(tokens, plen)[idx].tobytes()
        ref = O.turbo_score(sub, pref[b * group:(b + 1) * group], dim, SEED) * np.float32(scale)
        got = got_all[:, b * tokens:(b + 1) * tokens][:, idx].cpu().numpy()
        parity &= np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    pairs = nseg * tokens * group
    wire_bytes = nseg * blob
    alg = wire_bytes + pairs * 4 + nq * W * 4
    lane_ops = pairs * ((dim // 2) * 3 + 32)   # per pair: table offset, mul, add (+ LDS read); 32 QJL FMAs
    cpu = None
    if not args.no_cpu_baseline:
        n_s = 20000
        w0 = wire[:blob].cpu().numpy()
        sub = w0[:38].copy()
        sub[30:34] = np.frombuffer(np.uint32(n_s).tobytes(), np.uint8)
        sub = sub.tobytes() + w0[38:38 + n_s * plen].tobytes()
        info = cpu_info()
        reps, t_cpu = 0, 0.0
        while t_cpu < 8.0:
            c0 = time.perf_counter()
            O.turbo_score(sub, pref[:group], dim, SEED)
            t_cpu += time.perf_counter() - c0
            reps += 1
        single = reps * n_s * group / t_cpu
        th = info["threads"]
        c0 = time.perf_counter()
        pmap(lambda _: O.turbo_score(sub, pref[:group], dim, SEED), range(4 * th), th)
        allc = 4 * th * n_s * group / (time.perf_counter() - c0)
        cpu = {"value": round(allc, 1), "unit": "scores/s", "cores": th, "kind": "port",
               "sample": f"({n_s} codes of blob 0 x {group} queries) through the C oracle's ora_turbo_score "
                         f"(validation + sequential estimator): 1 thread {reps} reps in {t_cpu:.2f} s; {th} threads "
                         f"{4 * th} reps",
               "single_thread": {"value": round(single, 1), "unit": "scores/s", "cores": 1},
               "host": {"nproc": info["nproc"], "usable_cores": info["usable"], "model": info["model"]}}
    res = {"metric": "compressed-domain attention scores per second (TQB1-L keys, GQA 4)",
           "value": round(pairs / (step_ms * 1e-3), 1), "unit": "scores/s", "n_gpus": 1, "steps": steps,
           "warmup": args.warmup, "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f32",
           "data": "synthetic (seed 4 config-4 keys generated on the GPU, bf16; Gaussian queries)",
           "config": {"workload": "score: config-4 keys (32L x 8 KV heads x 32768 tokens x d128, turbo b=4 QJL-32, "
                                  "TQB1-L) x GQA groups of 4 query heads, scale 1/sqrt(128)",
                      "blobs": nseg, "codes_per_blob": tokens, "queries": nq, "wire_bytes": wire_bytes},
           "kernels_ms": {"prepare": round(prep_ms, 4), "score": round(score_ms, 4),
                          "score_f32_radii": round(score32_ms, 4)},
           "f32_radii": {"scores_per_s": round(pairs / (score32_ms * 1e-3), 1),
                         "hbm_gbs": round(alg32 / (score32_ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(alg32 / (score32_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                         "algorithmic_bytes": alg32},
           "roofline": {"bound": "valu", "kernel": "turbo_score_lut_kernel<128, 32, true, 3>",
                        "achieved": round(lane_ops / (score_ms * 1e-3) / 1e12, 2),
                        "peak": round(VALU_PEAK_OPS / 1e12, 2), "unit": "T lane-ops/s",
                        "frac": round(lane_ops / (score_ms * 1e-3) / VALU_PEAK_OPS, 4),
                        "hbm_gbs": round(alg / (score_ms * 1e-3) / 1e9, 1),
                        "hbm_frac": round(alg / (score_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                        "algorithmic_bytes": alg, "lane_ops": lane_ops},
           "cpu_baseline": cpu, "parity_sampled": bool(parity)}
    if args.copy_calib:
        copy_calib()
    print(json.dumps(res), flush=True)


# ================================================================ digests
B3_LANE_OPS_PER_BLOCK = 7 * 8 * 12 + 8   # BLAKE3 compression: rounds x G x ops, + output xors


def bench_digest(args):
    """BLAKE3 digests of a build (row a19: CompressedBlock::new of every blob,
    PoolLayer / ShellLayer::compute_digest of every layer) on config 3's pool
    and shell wires, where the encode left them; plus a bulk case (512 ranges
    of 1 MiB) that fills the GPU.  Every digest is compared with the oracle.
    Prints one JSON line; VALU-bound, so the roofline is the VALU issue rate."""
    import torch

    from oracle import oracle as O
    from provekv_amd import synth
    from provekv_amd.device import default_context
    from provekv_amd.pool import TwoTierPlan
    need_gpu()
    ctx = default_context()
    stream = torch.cuda.current_stream()
    log("[bench] digest: config-3 build")
    plan = TwoTierPlan(ctx, 24, 32, 64, 800, [28] * 8, seed=SEED)
    bufs = plan.alloc()
    corpus = torch.from_numpy(synth.corpus_tokens(3, 24, 32, plan.tokens, 64).reshape(-1)).cuda()
    plan.encode(corpus, bufs)
    plan.digests(bufs)
    torch.cuda.synchronize()
    plan.check(bufs, decode=False)
    # parity: every payload and layer digest against the oracle
    rep = plan.digest_report(bufs)
    parity = True
    wires = {}
    for tier, name in ((plan.pool, "pool"), (plan.shells, "shell")):
        wire = bufs[f"{name}_wire"].cpu().numpy()
        wires[name] = wire
        rg = np.array([(o, ln) for _, _, _, o, ln in tier.blob_offsets], np.uint64)
        ref = O.blake3_ranges(wire, rg)
        for i in range(len(rg) // 2):
            owner, layer = tier.blob_offsets[2 * i][:2]
            e = [x for x in rep[owner] if x["layer_index"] == layer][0]
            parity &= e["key_payload_digest"] == ref[2 * i].tobytes().hex()
            parity &= e["value_payload_digest"] == ref[2 * i + 1].tobytes().hex()
            parity &= e["block_digest"] == O.layer_digest(layer, ref[2 * i].tobytes(), ref[2 * i + 1].tobytes()).hex()
    log(f"[bench] digest parity vs oracle: {parity}")
    for _ in range(args.warmup):
        plan.digests(bufs)
    torch.cuda.synchronize()
    wire_bytes = plan.pool.wire_bytes + plan.shells.wire_bytes

    def timed(fn, steps):
        # events around back-to-back calls: each call takes a private table
        # slot and may wait on the host for that slot's last use, so the
        # calls cannot all be queued behind a spin first
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record(stream)
        for _ in range(steps):
            fn()
        t1.record(stream)
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps

    side = None if args.serial_tiers else torch.cuda.Stream()
    for _ in range(max(1, args.warmup)):
        plan.digests(bufs, stream=stream, side=side)
    ms = timed(lambda: plan.digests(bufs, stream=stream, side=side), args.steps)
    # bulk: 512 x 1 MiB
    bulk = torch.randint(0, 256, (512 << 20,), dtype=torch.uint8, device="cuda")
    brg = np.array([(i << 20, 1 << 20) for i in range(512)], np.uint64)
    bout = torch.empty((512, 32), dtype=torch.uint8, device="cuda")
    for _ in range(max(1, args.warmup)):
        ctx.blake3_ranges(bulk, brg, out=bout)
    torch.cuda.synchronize()
    host = bulk[: 8 << 20].cpu().numpy()
    parity &= np.array_equal(bout[:8].cpu().numpy(), O.blake3_ranges(host, brg[:8]))
    bms = timed(lambda: ctx.blake3_ranges(bulk, brg, out=bout), max(3, args.steps // 4))
    bulk_bytes = 512 << 20

    def valu(nbytes, t_ms):
        blocks = (nbytes + 63) // 64
        ops = blocks * B3_LANE_OPS_PER_BLOCK / (t_ms * 1e-3)
        return {"bound": "valu", "achieved": round(ops / 1e12, 2), "peak": round(VALU_PEAK_OPS / 1e12, 2),
                "unit": "T lane-ops/s", "frac": round(ops / VALU_PEAK_OPS, 4),
                "gbs_at_peak": round(VALU_PEAK_OPS / B3_LANE_OPS_PER_BLOCK * 64 / 1e9, 1)}

    res = {"metric": "BLAKE3 digests of encoded KV (payload + layer digests), GB/s of hashed bytes",
           "workload": "digest", "unit": "GB/s", "steps": args.steps, "warmup": args.warmup,
           "parity_all_digests": bool(parity),
           "config3": {"ranges": len(plan.pool.blob_offsets) + len(plan.shells.blob_offsets),
                       "tiers": "one stream" if side is None else "pool and shell tiers on two streams",
                       "bytes": int(wire_bytes), "ms_per_call": round(ms, 4),
                       "gbs": round(wire_bytes / (ms * 1e-3) / 1e9, 1), "roofline": valu(wire_bytes, ms)},
           "bulk_512x1MiB": {"bytes": bulk_bytes, "ms_per_call": round(bms, 4),
                             "gbs": round(bulk_bytes / (bms * 1e-3) / 1e9, 1), "roofline": valu(bulk_bytes, bms)}}
    if not args.no_cpu_baseline:
        log("[bench] digest: CPU baseline (oracle BLAKE3, config-3 wires)")
        jobs, job_bytes = [], []
        for tier, name in ((plan.pool, "pool"), (plan.shells, "shell")):
            for _, _, _, o, ln in tier.blob_offsets:
                blob = wires[name][o:o + ln].tobytes()
                jobs.append(lambda b=blob: O.blake3(b))
                job_bytes.append(ln)
        info = cpu_info()
        t0 = time.perf_counter()
        for j in jobs:
            j()
        t1 = time.perf_counter()
        with ThreadPoolExecutor(info["threads"]) as ex:
            t2 = time.perf_counter()
            list(ex.map(lambda f: f(), jobs))
            t3 = time.perf_counter()
        res["cpu_baseline"] = {"value": round(wire_bytes / (t3 - t2) / 1e9, 3), "unit": "GB/s",
                               "cores": info["threads"], "kind": "port",
                               "sample": f"oracle/blake3_oracle.c (portable C, -O3) over all {len(jobs)} config-3 "
                                         f"blobs ({wire_bytes} B), {info['threads']} threads in {t3 - t2:.3f} s",
                               "single_thread": {"value": round(wire_bytes / (t1 - t0) / 1e9, 3), "unit": "GB/s",
                                                 "cores": 1},
                               "host": {"nproc": info["nproc"], "model": info["model"]}}
    print(json.dumps(res), flush=True)


# ================================================================ main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=("config3", "pool", "config0", "config1", "config2", "config4", "legacy",
                                           "score", "digest"), default="config3",
                    help="config3 (alias pool): the metric (default); config0/1/2/4: the other BASELINE "
                         "configurations; legacy: per-vector TQW1 / FB1 records; score: attention scores on "
                         "config-4 compressed keys; digest: BLAKE3 payload and layer digests of the config-3 "
                         "build")
    ap.add_argument("--lossy", action="store_true", help="config3: TQB1-L shells (BlockLogU8 radii)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run a 256 MiB device copy (reference kernel for rocprofv3 --pmc byte counters)")
    ap.add_argument("--cache-dtype", choices=("f32", "bf16", "f16"), default="f32",
                    help="config3: dtype of the KV cache the rehydrate writes (default f32, the metric's)")
    ap.add_argument("--copies", type=int, default=8,
                    help="config3: KV caches filled from one decode: all 8 agents' full 1024-token KV (default 8)")
    ap.add_argument("--serial-tiers", action="store_true",
                    help="config3: the pool tier and the shell tier one after the other on one stream (default: "
                         "the shell tier on a second stream, concurrent with the pool tier)")
    ap.add_argument("--graph", action="store_true",
                    help="config3: replay one captured HIP graph per step instead of launching it eagerly "
                         "(checked against the eager step's bytes; slower here: 0.92 against 0.87 ms)")
    ap.add_argument("--side-workgroups", type=int, default=512,
                    help="config3: workgroups of the shell-tier rehydrate while it overlaps the pool encode")
    ap.add_argument("--pool-workgroups", type=int, default=640,
                    help="config3: workgroups of the pool encode while the shell-tier rehydrate runs beside it "
                         "(0: every workgroup slot)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)
    {"config3": bench_config3, "pool": bench_config3, "config0": bench_config0, "config1": bench_config1,
     "config2": bench_config2, "config4": bench_config4, "legacy": bench_legacy,
     "score": bench_score, "digest": bench_digest}[args.workload](args)


if __name__ == "__main__":
    main()
