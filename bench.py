"""Benchmark: proveKV codec hot path on one MI355X.

Default workload: the SmolLM2-1.7B-shape N=8 pool --
24 layers x 32 KV heads x head_dim 64, an 800-token shared prefix in the
fib_k4_n32 cold tier (FB2) and 8 agents x 28 unique tokens in the turbo b=4
hot tier (TQB1, lossless radii).  One step = build the pool + all 8 shells
(encode: 2 launches) and rehydrate all 8 agents' full 1024-token KV -- pool
and every shell, decoded once and written to each agent's cache -- straight
into HuggingFace-layout KV caches ([1, H, T, D] per layer and K|V, f32;
decode: 2 launches; 3,221,225,472 B written), inputs resident in HBM.  The
shell encode runs first, then the shell rehydrate on a second stream (on at
most --side-workgroups workgroups) beside the pool encode, then the pool
rehydrate (`--serial-tiers`: the four launches in order on one stream).

value = f32 KV bytes of the context (402,653,184 B, the metric's "f32 in") /
the GPU time of one step (events at the two ends of K back-to-back steps).  kernels_ms: a second pass
with events between the four calls.
roofline = the dominant kernel's algorithmic bytes per launch / its mean
duration (HIP events on the launch stream) against 8 TB/s.
cpu_baseline = the C oracle (a one-thread restatement of the reference Rust
codecs) timed on a bounded sample of the same workload on the host.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--lossy]
                       [--workload pool|legacy|config4|score]
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
    cb, rot = O.fib_constants(plan.fib.params["seed"])   # the oracle's own constants
    cb = cb.reshape(32, 4)
    rot = rot.reshape(plan.dim, plan.dim)
    layers, dim = plan.layers, plan.dim
    # fib: one (layer, K) blob of the prefix, truncated to a fixed vector count
    x_pool = np.ascontiguousarray(corpus[:plan.prefix, 0, :, 0, :].reshape(-1, dim))[:25600]
    x_shell = np.ascontiguousarray(corpus[plan.prefix:plan.prefix + plan.agent_tokens[0], 0, :, 0, :]
                                   .reshape(-1, dim))
    freps = 0
    t0 = time.perf_counter()
    while True:
        blob = O.fib_encode_batch(x_pool, cb, rot)
        O.fib_decode_batch(blob, cb, rot)
        freps += 1
        if time.perf_counter() - t0 > budget_s / 2:
            break
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
    fib_s_per_vec = (t2 - t0) / (freps * x_pool.shape[0])
    turbo_s_per_vec = (t4 - t3) / (reps * x_shell.shape[0])
    n_pool = plan.prefix * plan.heads * layers * 2
    n_shell = sum(plan.agent_tokens) * plan.heads * layers * 2
    total_s = n_pool * fib_s_per_vec + n_shell * turbo_s_per_vec
    f32_bytes = (n_pool + n_shell) * dim * 4
    return {"value": round(f32_bytes / total_s / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": (f"oracle/pkv_oracle.c, 1 thread: fib FB2 encode+decode of {x_pool.shape[0]} pool vectors x "
                       f"{freps} reps ({(t2 - t0):.2f} s) and turbo TQB1 encode+decode of {x_shell.shape[0]} shell vectors x "
                       f"{reps} reps ({(t4 - t3):.2f} s), scaled to the {n_pool}+{n_shell}-vector workload"),
            "encode_decode_s_projected": round(total_s, 2)}


def spot_check_cache(plan, bufs, cache, corpus):
    """Parity spot check of the rehydrated cache against the oracle on one
    pool blob and one shell blob (layer 0, K): the cache rows must be the
    oracle decode (rounded to the cache dtype) in every copy."""
    import torch
    from oracle import oracle as O
    cb, rot = O.fib_constants(plan.fib.params["seed"])   # the oracle's own constants
    cb, rot = cb.reshape(32, 4), rot.reshape(plan.dim, plan.dim)
    heads, dim = plan.heads, plan.dim
    checks = [(0, plan.prefix, O.fib_decode_batch(plan.blob(bufs, "pool", 0), cb, rot))]
    checks.append((plan.prefix, plan.agent_tokens[0],
                   O.turbo_decode_batch(plan.blob(bufs, "shell", 0), dim, plan.fib.params["seed"])))
    for t0, nt, dec in checks:
        want = torch.from_numpy(np.ascontiguousarray(dec.reshape(nt, heads, dim).transpose(1, 0, 2)))
        want = want.to(cache.buf.dtype)
        for c in range(cache.copies):
            got = cache.buf[c, 0, 0, :, t0:t0 + nt, :].cpu()
            if not torch.equal(got, want):
                raise AssertionError(f"rehydrated cache differs from the oracle (copy {c}, tokens {t0}..)")


# the kernel each timed span is about (fib_encode's span also holds the exact
# fixup kernel, turbo/fib spans a status fill of a few microseconds)
KERNEL_SYMBOL = {"fib_encode": "fib_encode_kernel<64>", "turbo_encode": "turbo_encode_qjl_kernel<3>",
                 "fib_decode": "fib_decode_mfma_kernel<64, true>", "turbo_decode": "turbo_decode_split_kernel<3>"}
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


def bench_legacy(args):
    """Per-vector KVecCodec records through the host-buffer entry points
    (pkv_encode_vectors / pkv_decode_vectors, PCIe copies included): a
    config-1-sized pool as FB1 records and config-2-sized shells as TQW1
    records.  Prints one JSON line; the kernel durations come from rocprofv3."""
    import ctypes as C

    import torch
    from oracle import oracle as O
    from provekv_amd import _lib as L
    from provekv_amd import synth
    from provekv_amd.device import default_context

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU"}))
        sys.exit(1)
    ctx = default_context()
    fib = ctx.fib_profile(64, 4, 32, 42)
    tur = ctx.turbo_profile(64, 4, 32, 42, 1)
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
    # parity spot check against the oracle on the first records
    m = 2000
    cb, rot = O.fib_constants(42)
    cb, rot = cb.reshape(32, 4), rot.reshape(64, 64)
    rec1 = fib.record_len()
    ref = O.fib_encode_fb1(x1[:m], cb, rot, each=False)
    parity = b"".join(ref) == r_fib[:m * rec1].tobytes()
    parity &= np.array_equal(O.fib_decode_fb1(ref, cb, rot, each=True).view(np.uint32), d_f64[:m].view(np.uint32))
    rec2 = tur.record_len()
    ref2 = O.turbo_encode_tqw1(x2[:m], 42)
    parity &= b"".join(ref2) == r_tur[:m * rec2].tobytes()
    parity &= np.array_equal(O.turbo_decode_tqw1(ref2, 64, 42).view(np.uint32), d_tur[:m].view(np.uint32))
    out = {"workload": "legacy per-vector records (KVecCodec::encode/decode): config-1 pool as 1,228,800 FB1 "
                       "records, config-2 shells as 344,064 TQW1 records, host buffers (PCIe included)",
           "unit": "GB/s of f32 KV", "steps": args.steps, "parity_first_2000": bool(parity),
           "ops": {k: {"vectors": n, "ms": round(t * 1e3, 3), "gbs": round(n * 256 / t / 1e9, 2)}
                   for k, (n, t) in ops.items()}}
    if args.copy_calib:   # the reference kernel for rocprofv3 --pmc byte counters
        src = torch.empty(1 << 28, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps(out), flush=True)


def bench_config4(args):
    """BASELINE config 4 at full size: Llama-3-8B KV (32 layers x K|V x 8 KV
    heads x 32768 tokens x head_dim 128) as bf16, turbo b = 4 with Hadamard
    dim 128 and BlockLogU8 radii, one TQB1-L blob per (layer, K|V) in one
    launch, then decode to f32.  The seeded generator produces two layers'
    values on the host (bf16, RNE); they are tiled over the 32 layers on the
    device (per-vector cost does not depend on the values' layer).  value =
    f32-equivalent KV bytes (8,589,934,592) / GPU time of encode + decode.
    Parity: sampled vectors of several blobs against the oracle on the f32
    upcast."""
    import torch
    from oracle import oracle as O
    from provekv_amd import _lib as L
    from provekv_amd import synth
    from provekv_amd.device import SEG_DTYPE, default_context

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU"}))
        sys.exit(1)
    layers, heads, tokens, dim, gen_layers = 32, 8, 32768, 128, 2
    log(f"[bench] generating {gen_layers} layers of config-4 values (bf16)")
    K, V = synth.kv_cache(4, gen_layers, heads, tokens, dim, k_sigma=0.7, outliers=4, outlier_mult=10.0,
                          v_scale=1.0)
    block = torch.from_numpy(np.ascontiguousarray(np.stack([K, V], axis=1))).to(torch.bfloat16)
    del K, V
    n = heads * tokens
    x = torch.empty((layers // gen_layers, gen_layers * 2 * n * dim), dtype=torch.bfloat16, device="cuda")
    x[:] = block.reshape(1, -1).cuda()
    x = x.reshape(-1)
    ctx = default_context()
    prof = ctx.turbo_profile(dim, 4, 32, 42)
    plen = prof.payload_len(L.RADII_LOG_U8)
    blob = 38 + n * plen
    nseg = 2 * layers
    segs = np.array([(b * n * dim, 0, dim, b * blob, n, n) for b in range(nseg)], dtype=SEG_DTYPE)
    wire = torch.empty(nseg * blob, dtype=torch.uint8, device="cuda")
    out = torch.empty(nseg * n * dim, dtype=torch.float32, device="cuda")
    est = torch.empty(2 * nseg, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(est)
    stream = torch.cuda.current_stream()

    def step(ev=None):
        if ev is not None:
            ev[0].record(stream)
        prof.encode_segments(x, segs, wire, radii=L.RADII_LOG_U8, status=est)
        if ev is not None:
            ev[1].record(stream)
        prof.decode_segments(wire, segs, out, radii=L.RADII_LOG_U8, status=dst)
        if ev is not None:
            ev[2].record(stream)

    log(f"[bench] config 4: {nseg} blobs x {n} vectors, warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    for s_ in (est, dst):
        err = prof.status_error(s_.cpu().numpy().view(np.uint32), segs)
        if err is not None:
            raise err
    steps = max(1, min(args.steps, 5))
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    step_ms = t0.elapsed_time(t1) / steps
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for k in range(steps):
        step(evs[k])
    torch.cuda.synchronize()
    enc_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in evs]))
    dec_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in evs]))
    # sampled parity: 512 vectors of four blobs, bytes and decodes vs the oracle
    rng = np.random.RandomState(4)
    parity = True
    for b in (0, 1, nseg - 2, nseg - 1):
        idx = np.sort(rng.choice(n, 512, replace=False))
        gb = b % (2 * gen_layers)
        xs = block.reshape(2 * gen_layers, n, dim)[gb][idx].to(torch.float32).numpy()
        ref = O.turbo_encode_batch(xs, 42, radii_codec=1)
        w = wire[b * blob + 38:(b + 1) * blob].cpu().numpy().reshape(n, plen)[idx]
        parity &= w.tobytes() == ref[38:]
        got = out[b * n * dim:(b + 1) * n * dim].reshape(n, dim)[idx].cpu().numpy()
        parity &= np.array_equal(got.view(np.uint32), O.turbo_decode_batch(ref, dim, 42).view(np.uint32))
    f32_bytes = nseg * n * dim * 4
    wire_bytes = nseg * blob
    enc_alg = nseg * n * dim * 2 + wire_bytes
    dec_alg = wire_bytes + f32_bytes
    dom, dom_ms, dom_alg = ("encode", enc_ms, enc_alg) if enc_ms >= dec_ms else ("decode", dec_ms, dec_alg)
    res = {"metric": "KV codec encode+decode GB/s (f32-equivalent KV) and % HBM peak, Llama-3-8B shape",
           "value": round(f32_bytes / (step_ms * 1e-3) / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps,
           "ms_per_step": round(step_ms, 3), "dtype": "f32 arithmetic on bf16 input",
           "data": f"synthetic (seeded config-4 distribution, {gen_layers} generated layers tiled over {layers})",
           "config": {"workload": "config4: 32L x K|V x 8 KV heads x 32768 tokens x d128, bf16 in, turbo b=4 "
                                  "QJL-32, TQB1-L (BlockLogU8 radii)", "blobs": nseg, "vectors_per_blob": n,
                      "wire_bytes": wire_bytes},
           "kernels_ms": {"encode": round(enc_ms, 3), "decode": round(dec_ms, 3)},
           "kernels_gbs": {"encode": round(enc_alg / (enc_ms * 1e-3) / 1e9, 1),
                           "decode": round(dec_alg / (dec_ms * 1e-3) / 1e9, 1)},
           "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(dom_alg / (dom_ms * 1e-3) / 1e9, 1),
                        "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(dom_alg / (dom_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                        "algorithmic_bytes": dom_alg},
           "parity_sampled_2048": bool(parity)}
    if args.copy_calib:   # the reference kernel for rocprofv3 --pmc byte counters
        src = torch.empty(1 << 28, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps(res), flush=True)


VALU_PEAK_OPS = 256 * 4 * 16 * 2.4e9   # f32 lane-ops/s without packed FP32 (157.3 TFLOP/s / 4)


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

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU"}))
        sys.exit(1)
    layers, kv_heads, tokens, dim, group, gen_layers = 32, 8, 32768, 128, 4, 2
    log(f"[bench] generating {gen_layers} layers of config-4 keys")
    K, _ = synth.kv_cache(4, gen_layers, kv_heads, tokens, dim, k_sigma=0.7, outliers=4, outlier_mult=10.0,
                          v_scale=1.0)
    block = torch.from_numpy(np.ascontiguousarray(K)).to(torch.bfloat16)   # [gl, H, T, D]
    del K
    nseg = layers * kv_heads
    x = torch.empty((layers // gen_layers, block.numel()), dtype=torch.bfloat16, device="cuda")
    x[:] = block.reshape(1, -1).cuda()
    x = x.reshape(-1)
    ctx = default_context()
    prof = ctx.turbo_profile(dim, 4, 32, 42)
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
        err = prof.status_error(est.cpu().numpy().view(np.uint32), segs)
        if err is not None:
            raise err
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
    ssegs = np.array([(b * tokens, 1, 1, b * blob, tokens, 1) for b in range(nseg)], dtype=SEG_DTYPE)
    pst = torch.empty(2, dtype=torch.int32, device="cuda")
    sst = torch.empty(2 * nseg, dtype=torch.int32, device="cuda")
    scale = float(np.float32(1.0) / np.sqrt(np.float32(dim)))
    stream = torch.cuda.current_stream()

    def step(ev=None, radii=L.RADII_LOG_U8):
        w, _, blob_r = wires[radii]
        sg = ssegs if radii == L.RADII_LOG_U8 else np.array(
            [(b * tokens, 1, 1, b * blob_r, tokens, 1) for b in range(nseg)], dtype=SEG_DTYPE)
        if ev is not None:
            ev[0].record(stream)
        prof.prepare_queries(q, prep, status=pst)
        if ev is not None:
            ev[1].record(stream)
        prof.score_segments(w, sg, prep, scores, ld, radii=radii, post_scale=scale, status=sst,
                            nq=group, query_stride=group)
        if ev is not None:
            ev[2].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    perr = prof.status_error(pst.cpu().numpy().view(np.uint32))
    serr = prof.score_status_error(sst.cpu().numpy().view(np.uint32))
    if perr is not None or serr is not None:
        raise perr or serr
    steps = max(1, args.steps)
    log(f"[bench] timing {steps} steps")
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    step_ms = t0.elapsed_time(t1) / steps
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for k in range(steps):
        step(evs[k])
    torch.cuda.synchronize()
    prep_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in evs]))
    score_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in evs]))
    # the same keys with f32 radii (TQB1 lossless: the in-memory TurboCode form)
    for k in range(max(1, args.warmup)):
        step(radii=L.RADII_F32)
    evs32 = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for k in range(steps):
        step(evs32[k], radii=L.RADII_F32)
    torch.cuda.synchronize()
    serr = prof.score_status_error(sst.cpu().numpy().view(np.uint32))
    if serr is not None:
        raise serr
    score32_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in evs32]))
    w32, plen32, blob32 = wires[L.RADII_F32]
    alg32 = nseg * blob32 + nseg * tokens * group * 4 + nq * prof.prepared_len() * 4
    # the timed region above left TQB1-L scores in `scores`: rerun one TQB1-L step for the parity sample
    step()
    torch.cuda.synchronize()
    # sampled parity: 256 codes of four blobs, every query of the group, bit for bit
    pref = O.turbo_prepare_queries(qh, 42)
    parity = np.array_equal(prep.cpu().numpy().view(np.uint32), pref.view(np.uint32))
    got_all = scores.reshape(group, ld)
    samp = np.random.RandomState(5)
    for b in (0, 1, nseg // 2, nseg - 1):
        idx = np.sort(samp.choice(tokens, 256, replace=False))
        w = wire[b * blob:(b + 1) * blob].cpu().numpy()
        sub = w[:38].copy()
        sub[30:34] = np.frombuffer(np.uint32(len(idx)).tobytes(), np.uint8)
        sub = sub.tobytes() + w[38:].reshape(tokens, plen)[idx].tobytes()
        ref = O.turbo_score(sub, pref[b * group:(b + 1) * group], dim, 42) * np.float32(scale)
        got = got_all[:, b * tokens:(b + 1) * tokens][:, idx].cpu().numpy()
        parity &= np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    pairs = nseg * tokens * group
    wire_bytes = nseg * blob
    alg = wire_bytes + pairs * 4 + nq * W * 4
    lane_ops = pairs * ((dim // 2) * 3 + 32)   # per pair: table offset, mul, add (+ LDS read); 32 QJL FMAs
    # CPU baseline: the oracle (one thread) scoring a bounded sample
    cpu = None
    if not args.no_cpu_baseline:
        n_s = 20000
        w0 = wire[:blob].cpu().numpy()
        sub = w0[:38].copy()
        sub[30:34] = np.frombuffer(np.uint32(n_s).tobytes(), np.uint8)
        sub = sub.tobytes() + w0[38:38 + n_s * plen].tobytes()
        reps, t_cpu = 0, 0.0
        while t_cpu < 10.0:
            c0 = time.perf_counter()
            O.turbo_score(sub, pref[:group], dim, 42)
            t_cpu += time.perf_counter() - c0
            reps += 1
        cpu = {"value": round(reps * n_s * group / t_cpu, 1), "unit": "scores/s", "cores": 1, "kind": "port",
               "sample": f"{reps} x ({n_s} codes of blob 0 x {group} queries) through the C oracle's "
                         "ora_turbo_score (validation + sequential estimator)"}
    res = {"metric": "compressed-domain attention scores per second (TQB1-L keys, GQA 4)",
           "value": round(pairs / (step_ms * 1e-3), 1), "unit": "scores/s", "n_gpus": 1, "steps": steps,
           "warmup": args.warmup, "ms_per_step": round(step_ms, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f32",
           "data": f"synthetic (seeded config-4 keys, {gen_layers} generated layers tiled over {layers}; "
                   "Gaussian queries)",
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
    if args.copy_calib:   # the reference kernel for rocprofv3 --pmc byte counters
        src = torch.empty(1 << 28, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
    print(json.dumps(res), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--lossy", action="store_true", help="TQB1-L shells (BlockLogU8 radii)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calib", action="store_true",
                    help="also run a 256 MiB device copy (reference kernel for rocprofv3 --pmc byte counters)")
    ap.add_argument("--cache-dtype", choices=("f32", "bf16", "f16"), default="f32",
                    help="dtype of the KV cache the rehydrate writes (default f32, the metric's)")
    ap.add_argument("--copies", type=int, default=8,
                    help="KV caches filled from one decode: config 3 rehydrates all 8 agents' full 1024-token "
                         "KV (default 8)")
    ap.add_argument("--serial-tiers", action="store_true",
                    help="run the pool tier and the shell tier one after the other on one stream (default: the "
                         "shell tier on a second stream, concurrent with the pool tier)")
    ap.add_argument("--side-workgroups", type=int, default=192,
                    help="workgroups of the shell-tier rehydrate while it overlaps the pool encode")
    ap.add_argument("--workload", choices=("pool", "legacy", "config4", "score"), default="pool",
                    help="pool: the config-3 metric (default); legacy: per-vector TQW1 / FB1 records; "
                         "config4: Llama-3-8B shape, bf16, d128, TQB1-L; score: attention scores on "
                         "config-4 compressed keys")
    args = ap.parse_args()
    if args.copies == 1:   # one cache: the fib decode stores directly (no LDS staging)
        KERNEL_SYMBOL["fib_decode"] = "fib_decode_mfma_kernel<64, false>"
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1",
                          "n_gpus": args.gpus}), flush=True)
        sys.exit(2)
    if args.workload == "legacy":
        bench_legacy(args)
        return
    if args.workload == "config4":
        bench_config4(args)
        return
    if args.workload == "score":
        bench_score(args)
        return

    import torch
    from provekv_amd import synth
    from provekv_amd.device import default_context
    from provekv_amd.pool import DeviceKVCache, TwoTierPlan

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
    cache_dtype = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[args.cache_dtype]
    cache = DeviceKVCache(layers, heads, plan.tokens, dim, dtype=cache_dtype, copies=args.copies)
    dev = torch.from_numpy(corpus.reshape(-1)).cuda()
    stream = torch.cuda.current_stream()
    side = None if args.serial_tiers else torch.cuda.Stream()   # default priority

    def step(evs=None):
        if evs is None:
            plan.build_and_rehydrate(dev, bufs, cache, stream=stream, side=side,
                                     side_workgroups=args.side_workgroups)
            return
        e = evs
        pseg, sseg = plan._cache_segs
        out = cache.buf.view(-1)
        e[0].record(stream)
        plan.fib.encode_segments(dev, plan.pool.enc, bufs["pool_wire"], status=bufs["pool_status"])
        e[1].record(stream)
        plan.turbo.encode_segments(dev, plan.shells.enc, bufs["shell_wire"], radii=plan.radii,
                                   status=bufs["shell_status"])
        e[2].record(stream)
        plan.fib.decode_segments(bufs["pool_wire"], pseg, out, status=bufs["pool_cstatus"], fanout=cache.copies,
                                 fanout_stride=cache.copy_stride)
        e[3].record(stream)
        plan.turbo.decode_segments(bufs["shell_wire"], sseg, out, radii=plan.radii, status=bufs["shell_cstatus"],
                                   fanout=cache.copies, fanout_stride=cache.copy_stride)
        e[4].record(stream)

    log(f"[bench] warmup {args.warmup}")
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    plan.check(bufs, decode=False)
    plan.check_rehydrate(bufs)
    spot_check_cache(plan, bufs, cache, corpus)
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
    plan.check(bufs, decode=False)
    plan.check_rehydrate(bufs)
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
    out_scale = args.copies * cache.buf.element_size() / 4   # cache bytes written per f32 input byte
    alg = {"fib_encode": f32_pool + wire_pool, "turbo_encode": f32_shell + wire_shell,
           "fib_decode": int(f32_pool * out_scale) + wire_pool, "turbo_decode": int(f32_shell * out_scale) + wire_shell}
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
                                                                  " (TQB1 lossless radii)") +
                               f", rehydrated into {args.copies} x [1,H,T,D] {args.cache_dtype} KV cache(s)",
                   "layers": layers, "kv_heads": heads, "head_dim": dim, "prefix_tokens": prefix,
                   "agents": len(agents), "agent_tokens": agents[0], "seed": 42,
                   "cache_dtype": args.cache_dtype, "cache_copies": args.copies,
                   "tier_streams": 1 if args.serial_tiers else 2,
                   "side_workgroups": None if args.serial_tiers else args.side_workgroups},
        "hbm_fraction_codec": round(total_alg / (step_gpu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "kernels_ms": {n: round(per[n], 4) for n in names},
        "kernels_gbs": {n: round(kern_gbs[n], 1) for n in names},
        "roofline": {"bound": "hbm", "kernel": KERNEL_SYMBOL[dom], "achieved": round(kern_gbs[dom], 1),
                     "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(kern_gbs[dom] / HBM_PEAK_GBS, 4),
                     "traffic": profiled_traffic(dom),
                     "algorithmic_bytes": alg[dom]},
        "compressed_bytes": plan.compressed_bytes(),
        "rehydrated_bytes": cache.buf.numel() * cache.buf.element_size(),
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
