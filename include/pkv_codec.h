/*
 * pkv_codec.h -- C ABI of libpkv_hip.so, the MI355X (gfx950) implementation of
 * proveKV's codec hot path: turbo-quant TQB1, fib-quant fib_k4_n32 FB2 and the
 * batched pool / shell rehydrate.
 *
 * The library replaces the reference's `gpu-backend` crate
 * (gpu-backend/src/lib.rs:24-249) underneath the unchanged Rust codec
 * adapters.  Each entry point below names the reference interface it
 * replaces.  Conventions:
 *   - every function returns a pkv status code (PKV_OK == 0); nothing throws
 *     or aborts across the boundary;
 *   - device pointers are plain `void*` / `uint8_t*` / `float*` into memory the
 *     caller allocated on the context's device; the library never frees caller
 *     memory;
 *   - `stream` is a hipStream_t passed as `void*` (NULL = the null stream);
 *     kernels are enqueued on it and completion is the caller's to wait for;
 *   - profiles are immutable after creation and may be shared across threads.
 * Wire formats are byte-identical to the reference: FB2
 * (fib-quant/src/codec.rs:195-320) and TQB1 (turbo-quant/src/wire.rs:267-398).
 */
#ifndef PKV_CODEC_H
#define PKV_CODEC_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status */
enum pkv_status {
    PKV_OK = 0,
    PKV_ERR_INVALID_ARG = 1,        /* ProveKvError::InvalidPolicy / bad call  */
    PKV_ERR_DIM_MISMATCH = 2,       /* ProveKvError::DimensionMismatch          */
    PKV_ERR_OOM = 3,                /* GpuError::OutOfMemory                    */
    PKV_ERR_DEVICE = 4,             /* GpuError::CudaError (HIP runtime error)  */
    PKV_ERR_CORRUPT_PAYLOAD = 5,    /* DecompressionFailed / CorruptPayload     */
    PKV_ERR_UNSUPPORTED = 6,        /* profile outside what the kernels handle  */
    PKV_ERR_NONFINITE_INPUT = 7,    /* NonFiniteInput                           */
    PKV_ERR_ZERO_NORM = 8,          /* FibQuantError::ZeroNorm                  */
    PKV_ERR_NORM_UNREPRESENTABLE = 9, /* encode_norm: not a finite positive f16 */
    PKV_ERR_EMPTY_BATCH = 10,       /* "empty batch" (wire encode_batch)        */
    PKV_ERR_CAPACITY = 11,          /* caller buffer too small                  */
    PKV_ERR_NONFINITE_CODE = 12,    /* turbo encode: radius / residual not finite */
    PKV_ERR_SCRATCH_LIMIT = 13      /* beyond the fixed scratch of pkv_decode_segments_noalloc */
};

/* Returns a static, human-readable name for a status code. */
const char* pkv_status_string(int status);

/* Detail of the first failure of a batched call. */
typedef struct pkv_error {
    int32_t status;      /* pkv_status                                  */
    int32_t segment;     /* failing segment, -1 when not segment-bound  */
    uint64_t index;      /* failing vector inside the segment           */
} pkv_error;

/* ---------------------------------------------------------------- context */
typedef struct pkv_ctx pkv_ctx;
typedef struct pkv_profile pkv_profile;

/* Replaces GpuContext::init / is_available (gpu-backend/src/lib.rs:41-58):
 * binds a context to HIP device `device` (an index, 0 = first).  The first
 * context on a device also runs the device checks the encodes' proofs rest
 * on: it measures the BlockLogU8 log bound (pkv_radii_log_bound) and checks
 * that the f16 matrix cores keep subnormal operands (the QJL acceptance
 * bound assumes it); PKV_ERR_UNSUPPORTED if they do not. */
int pkv_ctx_create(int device, pkv_ctx** out);
void pkv_ctx_destroy(pkv_ctx* ctx);
/* 1 if a gfx950 device is usable, 0 otherwise (never errors). */
int pkv_device_available(void);

/* ---------------------------------------------------------------- profiles */
enum pkv_codec_kind { PKV_CODEC_TURBO = 1, PKV_CODEC_FIB = 2 };
enum pkv_turbo_mode { PKV_TURBO_POLAR_ONLY = 0, PKV_TURBO_POLAR_WITH_QJL = 1 };
enum pkv_radii_codec { PKV_RADII_F32 = 0, PKV_RADII_LOG_U8 = 1 };
enum pkv_dtype { PKV_F32 = 0, PKV_BF16 = 1, PKV_F16 = 2 };

/* Replaces TurboQuantizer::new_with_mode (turbo-quant/src/turbo.rs:124-188)
 * as built by TurboQuantAdapter (proveKV/src/codec.rs:249-250): FastHadamard
 * signs and the QJL matrix are derived from `seed` exactly like the reference
 * and kept resident on the device.  dim must be 64 or 128. */
int pkv_turbo_profile_create(pkv_ctx* ctx, uint32_t dim, uint32_t bits, uint32_t projections,
                             uint64_t seed, int mode, pkv_profile** out);
/* Same, with the constants supplied by the caller (a Rust host that already
 * holds `FastHadamardRotation::signs` and `QjlQuantizer::projection_matrix`);
 * signs: dim floats (+-1), qjl: projections*dim floats row-major. */
int pkv_turbo_profile_create_with_constants(pkv_ctx* ctx, uint32_t dim, uint32_t bits,
                                            uint32_t projections, uint64_t seed, int mode,
                                            const float* signs, const float* qjl,
                                            pkv_profile** out);

/* Replaces FibQuantAdapter::build_quantizer (proveKV/src/codec.rs:471-499):
 * paper_default profile with the adapter's training overrides; the codebook
 * and the f64 rotation are built once per process and uploaded (the host
 * draws the training samples and restart starts, the Lloyd-Max iterations of
 * a codebook not built yet run on this context's device, pkv_lloyd_refine).
 * The kernels implement fib_k4_n32 at head_dim 64 (dim 64, k 4, n 32);
 * other shapes return PKV_ERR_UNSUPPORTED. */
int pkv_fib_profile_create(pkv_ctx* ctx, uint32_t dim, uint32_t k, uint32_t n, uint64_t seed,
                           uint32_t training_samples, uint32_t lloyd_restarts,
                           uint32_t lloyd_iterations, pkv_profile** out);
/* Same, with FibCodebookV1::codewords (n*k f32 row-major) and
 * StoredRotation::matrix (dim*dim f64 row-major) supplied by the caller. */
int pkv_fib_profile_create_with_constants(pkv_ctx* ctx, uint32_t dim, uint32_t k, uint32_t n,
                                          const float* codebook, const double* rotation,
                                          pkv_profile** out);
void pkv_profile_destroy(pkv_profile* prof);

/* Which kernel decodes a fib profile: 1 = the matrix-core decode (every
 * product f32(Pi)[r][col] * c[w][r % 4] it can form was checked equal to f32
 * multiplication when the profile was created), 0 = the VALU decode (some
 * product differed, e.g. a -0.0 product that the matrix core returns as +0.0),
 * -1 = not a fib profile.  Both produce the bytes of decode_batch_fast
 * (fib-quant/src/codec.rs:797-844); this only reports which one runs. */
int pkv_fib_decode_path(const pkv_profile* prof);

/* Host-only constant generators (no device needed): the exact constants
 * pkv_turbo_profile_create / pkv_fib_profile_create derive from a seed.
 * turbo: signs[dim], qjl[projections*dim] (NULL skips);
 * fib: codebook[n*k], rotation[dim*dim] (row-major), optional MSEs. */
int pkv_turbo_constants(uint32_t dim, uint32_t projections, uint64_t seed, float* signs, float* qjl);
int pkv_fib_constants(uint32_t dim, uint32_t k, uint32_t n, uint64_t seed, uint32_t training_samples,
                      uint32_t lloyd_restarts, uint32_t lloyd_iterations, float* codebook,
                      double* rotation, double* init_mse, double* training_mse);

/* Profile-constant service.  The reference rebuilds a quantizer's constants
 * on every adapter call (FibQuantAdapter::build_quantizer,
 * proveKV/src/codec.rs:471-499, called 2x per layer in a pool build and per
 * decompress, pool.rs:225, 265-266, 517-519; TurboQuantizer::new per turbo
 * call, codec.rs:249, 296).  This library builds each distinct profile's
 * constants (codebook, rotation, signs, QJL matrix) once per process, keyed
 * by every parameter they depend on, and shares them across contexts and
 * the host-only generators.  Stats: lookups served from the cache, builds,
 * distinct entries; clear() drops them (the next request rebuilds). */
void pkv_constants_cache_stats(uint64_t* hits, uint64_t* misses, uint64_t* entries);
void pkv_constants_cache_clear(void);

/* Copies the profile constants out (host memory).  turbo: a = signs[dim],
 * b = float qjl[proj*dim]; fib: a = float codebook[n*k], b = double rot[dim*dim]. */
int pkv_profile_constants(const pkv_profile* prof, void* a, size_t a_bytes, void* b, size_t b_bytes);

/* Wire sizing: per-vector payload bytes, header bytes (38 TQB1 / 19 FB2) and
 * the blob size of an n-vector batch. radii_codec is ignored for fib. */
uint32_t pkv_payload_len(const pkv_profile* prof, int radii_codec);
uint32_t pkv_header_len(const pkv_profile* prof);
uint64_t pkv_blob_len(const pkv_profile* prof, int radii_codec, uint64_t n_vectors);

/* The blob header an encode of n_vectors writes, byte for byte, into
 * out[0 .. pkv_header_len(prof)), for a caller that lays blobs out itself.
 * Replaces the header half of TurboCodeWireV1::encode_batch
 * (turbo-quant/src/wire.rs:291-346: "TQB1", version, rotation, variant, dim,
 * bits, radii codec, projections, seed, n, payload length) and of
 * FibCodeV1::encode_batch (fib-quant/src/codec.rs:225-296: "FB2", version,
 * bits, block count, n, norm format, norm / index lengths).  EMPTY_BATCH for
 * n_vectors == 0 (the encodes reject an empty batch), CAPACITY when cap is
 * short; radii_codec is ignored for fib. */
int pkv_write_header(const pkv_profile* prof, int radii_codec, uint64_t n_vectors, uint8_t* out, uint64_t cap);

/* ---------------------------------------------------------------- segments
 * One segment = one FB2/TQB1 blob <-> n_vectors dim-sized f32 (or bf16)
 * vectors of a strided tensor.  Vector i of the segment starts at element
 *     elem_offset + (i / group) * stride_outer + (i % group) * stride_inner
 * which expresses the proveKV gather order (vector i = token * H + head;
 * proveKV/src/pool.rs:246-257, shell.rs:250-262) and the decode re-layout
 * (pool.rs:538-558, flatten_heads_tokens 19-33) without a copy.  The blob
 * (header included) starts at byte wire_offset of the wire buffer.
 * All (agent, layer, K|V) batches of a pool or of N shells go in ONE launch. */
typedef struct pkv_seg {
    uint64_t elem_offset;
    uint64_t stride_outer;
    uint64_t stride_inner;
    uint64_t wire_offset;
    uint32_t n_vectors;
    uint32_t group;
} pkv_seg;

/* Per-segment status words written by the kernels (2 per segment): word 0 =
 * first input-validation failure, word 1 = first later failure, each packed
 * as (vector_index << 4) | kind; 0xFFFFFFFF = none.  pkv_segments_status()
 * turns them into a pkv_error following the reference's precedence: segments
 * in order; within a fib segment an input-validation failure precedes a norm
 * failure (FibQuantizer::encode_batch, fib-quant/src/codec.rs:592-610 before
 * 694-704: every segment is taken as a batch of >= 4 vectors, the pool and
 * shell case); within a turbo segment the first failing vector wins. */
int pkv_segments_status(const pkv_profile* prof, const uint32_t* host_status, uint32_t nseg,
                        pkv_error* err);

/* Encode every segment: writes complete blobs (header + payloads) into
 * d_wire.  Replaces the per-(layer, K|V) loops of TurboQuantAdapter /
 * FibQuantAdapter::encode_batch_compact (proveKV/src/codec.rs:248-291,
 * 513-525) driven by materialize_shell / SharedKVPool::build_with_policy.
 * d_status: 2*nseg uint32 device words, or NULL.  With status words the call
 * is asynchronous and a rejected input is reported only there
 * (pkv_segments_status); with NULL it waits for its kernels and returns the
 * first error's code itself, as the reference's encode does (not under graph
 * capture: PKV_ERR_UNSUPPORTED).  The call validates the segment table
 * against in_elems / wire_bytes before launching. */
int pkv_encode_segments(pkv_ctx* ctx, const pkv_profile* prof, int radii_codec, int in_dtype,
                        const void* d_in, uint64_t in_elems, const pkv_seg* segs, uint32_t nseg,
                        uint8_t* d_wire, uint64_t wire_bytes, uint32_t* d_status, void* stream);

/* pkv_encode_segments on a bounded share of the GPU: the fib encode, a
 * persistent grid that otherwise takes every workgroup slot of the device,
 * runs on at most max_workgroups workgroups (0: no bound), its waves stepping
 * over more 32-vector units, so a kernel queued on another stream (the shell
 * rehydrate of the same step) keeps compute units beside it.  Turbo encodes
 * (one workgroup per tile group) launch as by pkv_encode_segments.  No
 * counterpart in the reference (its tiers run one after the other); for
 * callers that overlap the pool and shell tiers of one pool build. */
int pkv_encode_segments_bounded(pkv_ctx* ctx, const pkv_profile* prof, int radii_codec, int in_dtype,
                                const void* d_in, uint64_t in_elems, const pkv_seg* segs, uint32_t nseg,
                                uint8_t* d_wire, uint64_t wire_bytes, uint32_t max_workgroups,
                                uint32_t* d_status, void* stream);

/* Decode every segment into f32 at the segment's strided positions.
 * radii_codec: the TQB1 radii codec the caller expects (ignored for fib);
 * each header is checked against the profile and the segment on the device
 * (a mismatch marks the segment corrupt and leaves its output untouched).
 * d_status as in pkv_encode_segments: a NULL one makes the call wait and
 * return a rejected blob's error, so it never fails open.
 * Replaces decode_batch_compact (proveKV/src/codec.rs:295-326, 530-569) under
 * SharedKVPool::decompress_layer (pool.rs:471-614) and
 * AgentShell::decompress_all_layers_with_seed (shell.rs:92-141). */
int pkv_decode_segments(pkv_ctx* ctx, const pkv_profile* prof, int radii_codec,
                        const uint8_t* d_wire, uint64_t wire_bytes, const pkv_seg* segs,
                        uint32_t nseg, float* d_out, uint64_t out_elems, uint32_t* d_status,
                        void* stream);

/* Decode straight into a framework KV-cache layout.  Same as
 * pkv_decode_segments, plus:
 *   out_dtype  PKV_F32, PKV_BF16 or PKV_F16: the f32 decode rounded to nearest
 *              even, the conversion the reference harness applies when it
 *              patches decoded K/V into a bf16 / fp16 HuggingFace cache
 *              (`torch.tensor(..., dtype=k.dtype)`,
 *              proveKV/scripts/ppl_validate_multi_agent.py:226-272);
 *   fanout     every decoded vector is written `fanout` times, copy k at
 *              element offset + k * fanout_stride: one decode of the shared
 *              pool feeds the caches of several agents (rehydrate fan-out).
 * With group = H, stride_outer = D, stride_inner = T * D a segment writes a
 * layer's [1, H, T, D] K or V tensor at token offset elem_offset / D: the
 * re-layout of flatten_heads_tokens (proveKV/src/pool.rs:19-33) and the cache
 * patch fused into the decode.  Offsets, strides and fanout_stride are
 * multiples of 4 elements; d_out is 16-byte aligned; out_elems counts
 * elements of out_dtype. */
int pkv_decode_segments_ex(pkv_ctx* ctx, const pkv_profile* prof, int radii_codec,
                           const uint8_t* d_wire, uint64_t wire_bytes, const pkv_seg* segs,
                           uint32_t nseg, void* d_out, int out_dtype, uint64_t out_elems,
                           uint32_t fanout, uint64_t fanout_stride, uint32_t* d_status,
                           void* stream);

/* pkv_decode_segments_ex on a bounded share of the GPU: the head_dim-64
 * turbo decode and the fib matrix-core decode run on at most max_workgroups
 * workgroups (0: no bound), each looping over the blob tiles, so a kernel
 * queued on another stream (the other tier's encode) gets the remaining
 * compute units instead of waiting behind a full grid.  Other profiles (and
 * the fib VALU decode, used only when a profile's matrix-core products fail
 * their check) decode as pkv_decode_segments_ex.  No
 * counterpart in the reference (its tiers run one after the other); for
 * callers that overlap the pool and shell tiers of one rehydrate. */
int pkv_decode_segments_bounded(pkv_ctx* ctx, const pkv_profile* prof, int radii_codec,
                                const uint8_t* d_wire, uint64_t wire_bytes, const pkv_seg* segs,
                                uint32_t nseg, void* d_out, int out_dtype, uint64_t out_elems,
                                uint32_t fanout, uint64_t fanout_stride, uint32_t max_workgroups,
                                uint32_t* d_status, void* stream);

/* pkv_decode_segments_ex without any allocation: no hipMalloc, hipFree or
 * other allocating call, here or in the kernels.  No counterpart in the
 * reference; for callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, checks, kernels
 * and results as pkv_decode_segments_ex, except:
 *   - d_status is required (2*nseg device words; NULL returns
 *     PKV_ERR_INVALID_ARG before any work): a rejected blob leaves its output
 *     untouched and is reported only there, so the call cannot fail open;
 *   - the segment table and its workgroup prefix live in one fixed device
 *     array of the library per GPU (about 176 KiB, held until the process
 *     ends), so nseg <= PKV_NOALLOC_MAX_SEGMENTS; a larger table returns
 *     PKV_ERR_SCRATCH_LIMIT before any work;
 *   - every call on a GPU shares that array.  The library orders the calls
 *     on the device: each waits (hipStreamWaitEvent, no host wait) for the
 *     previous call's kernel, on whatever stream or context of that GPU it
 *     ran, before it rewrites the table, so overlapping calls are correct but
 *     run one after the other;
 *   - the table is copied from the caller's host memory with hipMemcpyAsync
 *     on `stream` on every call (segs may be released when the call returns),
 *     which a captured graph could not replay: on a stream under HIP graph
 *     capture the call returns PKV_ERR_UNSUPPORTED. */
#define PKV_NOALLOC_MAX_SEGMENTS 4096u
int pkv_decode_segments_noalloc(pkv_ctx* ctx, const pkv_profile* prof, int radii_codec,
                                const uint8_t* d_wire, uint64_t wire_bytes, const pkv_seg* segs,
                                uint32_t nseg, void* d_out, int out_dtype, uint64_t out_elems,
                                uint32_t fanout, uint64_t fanout_stride, uint32_t* d_status,
                                void* stream);

/* ---------------------------------------------------------------- host-buffer
 * Drop-ins for the adapters' inherent batch methods: host slices in, wire
 * bytes out (and back), with the H2D / launch / D2H / sync inside, exactly the
 * contract of TurboQuantAdapter::encode_batch_compact /
 * decode_batch_compact (proveKV/src/codec.rs:248-326) and the FibQuantAdapter
 * pair (513-569).  vectors: n*dim f32 row-major.  For decode, the header is
 * parsed and validated on the host with the reference's checks
 * (turbo-quant/src/wire.rs:401-568; fib-quant/src/codec.rs:323-424).  A fib
 * payload without the FB2 magic is FibQuantAdapter::decode_batch_compact's
 * fallback (codec.rs:542-561): one FB1 record, or else one JSON FibCodeV1,
 * decoded as decode_batch_fast decodes it (one vector out). */
int pkv_encode_batch_compact(pkv_ctx* ctx, const pkv_profile* prof, int radii_codec,
                             const float* vectors, uint64_t n, uint8_t* out, uint64_t out_cap,
                             uint64_t* out_len, pkv_error* err);
int pkv_decode_batch_compact(pkv_ctx* ctx, const pkv_profile* prof, const uint8_t* payload,
                             uint64_t len, float* out, uint64_t out_cap_vectors, uint64_t* n_out,
                             pkv_error* err);

/* ---------------------------------------------------------------- per-vector
 * The KVecCodec trait's own methods (proveKV/src/codec.rs:8-66), whose wire
 * form is one self-describing record per vector: TQW1 for turbo
 * (TurboCodeWireV1::encode / decode, turbo-quant/src/wire.rs:44-256; always
 * f32 radii) and compact FB1 for fib (FibCodeV1::to_compact_bytes /
 * from_compact_bytes, fib-quant/src/codec.rs:81-176).  Legacy pools and
 * shells store these (pool.rs:569-603).  Records are fixed-size for a
 * profile: pkv_record_len bytes (190 = 46 + 144 TQW1, 23 = 11 + 12 FB1 at
 * head_dim 64). */
uint32_t pkv_record_len(const pkv_profile* prof);

/* Replaces TurboQuantAdapter::encode / KVecCodec::encode_batch (codec.rs:28-30,
 * 339-365; every vector encoded on its own) and FibQuantAdapter::encode
 * (each != 0, codec.rs:582-594: FibQuantizer::encode per vector, f64
 * normalisation) / encode_batch (each == 0, 596-610: FibQuantizer::encode_batch,
 * f32-rounded normalisation when n >= 4).  Writes n records back to back
 * (out_len = n * pkv_record_len).  Errors as pkv_encode_batch_compact. */
int pkv_encode_vectors(pkv_ctx* ctx, const pkv_profile* prof, int each, const float* vectors, uint64_t n,
                       uint8_t* out, uint64_t out_cap, uint64_t* out_len, pkv_error* err);

/* Replaces TurboQuantAdapter::decode / KVecCodec::decode_batch (codec.rs:367-405,
 * 34-37) and FibQuantAdapter::decode (each != 0, 612-637: FibQuantizer::decode,
 * f64 inverse rotation, codec.rs:506-537) / decode_batch (each == 0, 639-665:
 * every record parsed first, then decode_batch_fast).  Record i is
 * records[offsets[i] .. offsets[i + 1]) (n + 1 non-decreasing offsets, the
 * flattening of a `&[&[u8]]`).  A record without the TQW1 / FB1 magic is
 * the adapters' JSON fallback: the serde_json text of a TurboCode /
 * FibCodeV1 (see pkv_code_from_json), parsed and checked on the host and
 * decoded by the same kernels (fib profiles created with caller constants
 * cannot check the JSON digests: PKV_ERR_UNSUPPORTED; so do turbo
 * PolarOnly profiles, whose angle width the adapter's bits - 1 does not
 * match).  A rejected record gives PKV_ERR_CORRUPT_PAYLOAD with err->index =
 * the record the reference reports (fib decode_batch: every payload is
 * parsed, FB1 or JSON, before any is decoded). */
int pkv_decode_vectors(pkv_ctx* ctx, const pkv_profile* prof, int each, const uint8_t* records,
                       const uint64_t* offsets, uint64_t n, float* out, uint64_t out_cap_vectors, pkv_error* err);

/* ---------------------------------------------------------------- JSON codes
 * Before the compact records, proveKV stored a vector's code as the
 * serde_json text of turbo-quant's TurboCode {polar_code, residual_sketch}
 * (turbo-quant/src/turbo.rs:50-56, polar.rs:35-46, qjl.rs:41-50) or of
 * fib-quant's FibCodeV1 (fib-quant/src/codec.rs:31-54), and the adapters
 * still read it when a payload lacks the record magic:
 * TurboQuantAdapter::decode (proveKV/src/codec.rs:386-393; the trait's
 * decode_batch loops over it), FibQuantAdapter::decode (622-630),
 * decode_batch (650-658) and decode_batch_compact (552-561).
 * pkv_decode_vectors and pkv_decode_batch_compact take such payloads
 * directly; the helpers below are their host half. */

/* A codec profile by its parameters (host-only helpers; no device). */
typedef struct pkv_codec_params {
    int32_t kind;                  /* PKV_CODEC_TURBO or PKV_CODEC_FIB */
    uint32_t dim;
    uint32_t bits;                 /* turbo: the adapter's bits; its codes carry bits - 1 angle bits */
    uint32_t projections;          /* turbo: QJL projections */
    uint32_t k, n;                 /* fib: block dimension, codebook size */
    uint32_t training_samples, lloyd_restarts, lloyd_iterations;   /* fib: the adapter's overrides */
    uint64_t seed;
} pkv_codec_params;

/* Host only.  serde_json::from_slice of a JSON code (serde_json 1.0.150:
 * object or field array, unknown fields skipped, duplicate / missing fields,
 * trailing characters and out-of-range numbers rejected) followed by the
 * checks the adapter's decode applies before the arithmetic: turbo
 * PolarCode::validate_for(dim, bits - 1) (turbo-quant/src/polar.rs:107-152);
 * fib validate_code_header (fib-quant/src/codec.rs:926-975: schema, the
 * profile digest always, the codebook and rotation digests when not empty,
 * dimensions, index width, norm format) and the index / norm lengths
 * (bitpack.rs:47-66, codec.rs:1020-1031).  On success writes the payload of
 * the equivalent TQW1 / FB1 record (turbo: f32 radii, packed angle indices,
 * the sketch's signs when it holds one per projection -- the decode never
 * reads them; fib: fp16 norm, packed indices; *payload_len bytes, CAPACITY
 * when cap is short).  Errors: PKV_ERR_CORRUPT_PAYLOAD with *stage = 1 (the
 * text does not deserialize: the adapters' "code deserialize failed") or 2
 * (the code does not fit the profile: the decode's rejection);
 * PKV_ERR_INVALID_ARG for parameters no reference profile accepts. */
int pkv_code_from_json(const pkv_codec_params* params, const uint8_t* json, uint64_t len, uint8_t* payload,
                       uint64_t cap, uint64_t* payload_len, int* stage);

/* Host only.  The digest strings ("blake3:" + 64 hex digits, NUL-terminated,
 * 72 bytes each; NULL skips one) of a fib profile, as validate_code_header
 * compares them: FibQuantProfileV1::digest (fib-quant/src/profile.rs:256-262,
 * the adapter's profile, proveKV/src/codec.rs:471-499),
 * FibCodebookV1::compute_digest (codebook.rs:133-157, over the codewords,
 * the MSEs and the Lloyd report) and StoredRotation::digest
 * (rotation.rs:80-100), each json_digest (digest.rs:5-13).  Memoised per
 * profile; the first codebook digest runs the codebook build on the host
 * for its report (a few ms). */
int pkv_fib_digests(const pkv_codec_params* params, char* profile_digest, char* codebook_digest,
                    char* rotation_digest);

/* Parses a TQB1 / FB2 header against the profile (host memory) and reports
 * the number of vectors and the radii codec; PKV_ERR_CORRUPT_PAYLOAD on any
 * header mismatch the reference decoder rejects before reading a vector,
 * including a buffer shorter than the header's vectors.  Bytes after the last
 * TQB1 payload are not a header fault: the reference rejects them only after
 * every vector (cursor.finish(), turbo-quant/src/wire.rs:566), and so do
 * pkv_decode_batch_compact and pkv_turbo_score_batch; FB2 accepts them
 * (fib-quant/src/codec.rs:380-386). */
int pkv_parse_header(const pkv_profile* prof, const uint8_t* blob, uint64_t len,
                     uint64_t* n_vectors, int* radii_codec);

/* ---------------------------------------------------------------- scoring
 * Inner-product scores straight from TQB1 codes, without decoding them:
 * TurboQuantizer::prepare_query / inner_product_estimate_prepared /
 * score_batch_prepared (turbo-quant/src/turbo.rs:316-381), the scorer under
 * TurboIndex::search_prepared (index.rs:98-140) and
 * KvShadowCache::attention_scores_with_options (kv.rs:269-320).  Turbo
 * profiles only (head_dim 64 or 128). */

/* Floats per prepared query: dim (+ proj with QJL): [R q][G q]. */
uint32_t pkv_prepared_len(const pkv_profile* prof);

/* prepare_query (turbo.rs:322-338; PolarQuantizer::project_query, polar.rs:
 * 336-343; QjlQuantizer::project_query, qjl.rs:266-282) for nq device queries
 * d_queries[nq][dim] (f32) into d_prepared[nq][pkv_prepared_len].  d_status:
 * 2 device words (may be NULL); word 0 = (q << 4) | 0 for the first query
 * with a non-finite input, rotated or projected value (NonFiniteInput). */
int pkv_turbo_prepare_queries(pkv_ctx* ctx, const pkv_profile* prof, const float* d_queries, uint32_t nq,
                              float* d_prepared, uint32_t* d_status, void* stream);

/* inner_product_estimate_prepared of every code of every segment against
 * nq prepared queries, times post_scale (1.0f for the plain score; the
 * AttentionScale factor of attention_scores_with_options, applied after the
 * score's finiteness check, kv.rs:305-318):
 *     d_scores[q * ld + col(i)]  = score(code i of segment s, prepared row s * query_stride + q),
 *     col(i) = elem_offset + (i / group) * stride_outer + (i % group) * stride_inner
 * (the segment addressing of pkv_decode_segments, in score units; a
 * contiguous layout is group = 1, stride_outer = 1).  query_stride = 0: all
 * segments score the same nq queries; query_stride = nq: each (layer, KV
 * head) segment scores its own group of query heads (GQA).  d_prepared holds
 * prepared_rows rows of pkv_prepared_len floats.  Each blob's header is
 * checked as pkv_decode_segments does.  d_status: 2*nseg device words (may be
 * NULL): word 0 = a rejected header / code (no score written for it), word 1
 * = a non-finite score (turbo.rs:362-367); pkv_score_status resolves them. */
int pkv_turbo_score_segments(pkv_ctx* ctx, const pkv_profile* prof, int radii_codec, const uint8_t* d_wire,
                             uint64_t wire_bytes, const pkv_seg* segs, uint32_t nseg, const float* d_prepared,
                             uint64_t prepared_rows, uint32_t nq, uint64_t query_stride, float post_scale,
                             float* d_scores, uint64_t score_elems, uint64_t ld, uint32_t* d_status, void* stream);

/* Status words of pkv_turbo_score_segments -> pkv_error: per segment in
 * order, a rejected code (the blob is validated before any score) precedes a
 * non-finite score; both are PKV_ERR_CORRUPT_PAYLOAD (MalformedCode). */
int pkv_score_status(const uint32_t* host_status, uint32_t nseg, pkv_error* err);

/* Host-buffer form: one TQB1 blob and nq host queries -> scores[nq][n]
 * (row q = score_batch_prepared(prepare_query(queries[q]), codes)).  Errors:
 * a non-finite query (PKV_ERR_NONFINITE_INPUT, index = query) before any
 * rejected code or non-finite score (PKV_ERR_CORRUPT_PAYLOAD, index = code). */
int pkv_turbo_score_batch(pkv_ctx* ctx, const pkv_profile* prof, const uint8_t* payload, uint64_t len,
                          const float* queries, uint32_t nq, float post_scale, float* scores, uint64_t scores_cap,
                          uint64_t* n_out, pkv_error* err);

/* ---------------------------------------------------------------- diagnostics
 * Validation hook, no counterpart in the reference: the encode kernels take
 * their fast decisions from matrix-core approximations and keep them only
 * under a proven error bound (the rest is redone in the reference's exact
 * arithmetic).  This encodes n contiguous f32 device vectors into one blob
 * (the bytes pkv_encode_segments writes) and also writes the approximations
 * and bounds, so tests can measure how far inside the bound real data stays:
 *   fib:   d_diag[(v * 16 + b) * 32 + w] = approximate key of codeword w for
 *          block b of vector v, f32(|c_w|^2 + 1.25 - 2 c_w . rho'); a block's
 *          approximate argmin stands only when its two smallest keys (low 5
 *          bits replaced by the codeword index) differ by more than
 *          *threshold; n * 512 floats;
 *   turbo: (QJL profiles with polar bits <= 4, head_dim 64 / 128)
 *          d_diag[(v * proj + j) * 2 + 0] = matrix-core dot of projection j,
 *          [.. + 1] = its acceptance bound: the sign stands only when
 *          |dot| > bound; n * proj * 2 floats; *threshold = 0.
 * d_status: 2 words as in pkv_encode_segments (may be NULL). */
int pkv_encode_diagnostics(pkv_ctx* ctx, const pkv_profile* prof, int radii_codec, const float* d_in,
                           uint64_t n, uint8_t* d_wire, uint64_t wire_bytes, float* d_diag,
                           uint64_t diag_elems, float* threshold, uint32_t* d_status, void* stream);

/* Validation hook, no counterpart in the reference: the BlockLogU8 radii
 * encode (radius.rs:58-77) takes each code from a hardware log and keeps it
 * only when it lies farther from a rounding boundary than that log's error
 * bound allows (the rest, and the block's mn / mx, use the exact logf).  The
 * bound is measured on each device, over every normal positive float, when
 * the first context there is created.  out[e] (256 floats, host memory) =
 * the largest |hardware log - logf(v)| over every v whose logf(v) has a
 * biased f32 exponent <= e. */
int pkv_radii_log_bound(pkv_ctx* ctx, float* out);

/* read_fb2_n_blocks (proveKV/src/pool.rs:108-116): the n_blocks field of a
 * batched FB2 payload (bytes 10..14, little-endian) read without any profile
 * check, as PoolLayer::num_blocks does for a batched layer.  PKV_OK with *n,
 * or PKV_ERR_CORRUPT_PAYLOAD where the reference returns None (fewer than 14
 * bytes, or no "FB2" magic).  Host only. */
int pkv_fb2_n_blocks(const uint8_t* payload, uint64_t len, uint64_t* n);

/* Lloyd-Max refinement of a codebook on the context's device: every restart
 * at once, one workgroup each (refine_codebook's restart loop,
 * fib-quant/src/lloyd.rs:128-147: `iterations` rounds of assign_samples and
 * update_centroids with the SplitHighestDistortion repair, lloyd.rs:215-337,
 * then mse_for_codebook, 339-357), bit-identical to the host computation.
 * samples [ns][k] and starts [restarts][n][k] are f64 host arrays (the
 * training draws and each restart's start, which the host derives from the
 * seed); out_codebooks [restarts][n][k], out_mse [restarts] and *init_mse
 * (the MSE of starts[0]) are host outputs.  k <= 16, n <= 256, n*k <= 2048;
 * PKV_ERR_INVALID_ARG when an empty cell finds no donor
 * (EmptyCellRepairFailed).  pkv_fib_profile_create refines a codebook it
 * has not built yet in this process this way; the host generator
 * pkv_fib_constants refines on the host. */
int pkv_lloyd_refine(pkv_ctx* ctx, const double* samples, uint32_t ns, uint32_t k, uint32_t n,
                     const double* starts, uint32_t restarts, uint32_t iterations, double* out_codebooks,
                     double* out_mse, double* init_mse);

/* ---------------------------------------------------------------- digests
 * BLAKE3 (the unkeyed 32-byte hash of the blake3 crate, 1.8.5 in the
 * reference's lock file) computed on the device.  Digests are raw 32-byte
 * hashes; the reference prints them as lower-case hex. */
typedef struct pkv_range {
    uint64_t offset;   /* first byte, from the buffer start */
    uint64_t len;      /* bytes (0 allowed: the hash of the empty input) */
} pkv_range;

/* d_out[32 i .. 32 i + 32) = blake3(d_buf[ranges[i].offset .. + len]) for
 * every range, in one pass over the bytes where they lie (an encode's wire
 * buffer: one range per (layer, K|V) blob).  Replaces the payload digest of
 * CompressedBlock::new (proveKV/src/codec.rs:85-95), which SharedKVPool::
 * build_with_policy (pool.rs:268-275) and materialize_shell (shell.rs:280-282)
 * take of every blob after copying it to the host.  Ranges may overlap and
 * start at any byte; each must lie inside [0, buf_bytes).  d_out is 4-byte
 * aligned device memory.  n == 0 does nothing.  The range table is copied
 * from host memory on `stream`; it may be released when the call returns. */
int pkv_blake3_ranges(pkv_ctx* ctx, const uint8_t* d_buf, uint64_t buf_bytes, const pkv_range* ranges,
                      uint32_t n, uint8_t* d_out, void* stream);

/* Layer digests from payload digests: entry i of d_kv_digests is 64 bytes,
 * the key blob's digest then the value blob's, of layer i % layers (so a pool
 * is one run of `layers` entries, N shells N runs); d_out[32 i ..) =
 * blake3 of the compact JSON text
 *   {"key_digests":["<hex>"],"layer_index":L,"value_digests":["<hex>"]}
 * i.e. PoolLayer::compute_digest (proveKV/src/pool.rs:83-103) and
 * ShellLayer::compute_digest (shell.rs:48-66) of a batched layer (one key
 * block, one value block), whose serde_json object prints its keys sorted.
 * Both device pointers 4-byte aligned; layers >= 1. */
int pkv_blake3_layer_digests(pkv_ctx* ctx, const uint8_t* d_kv_digests, uint32_t n, uint32_t layers,
                             uint8_t* d_out, void* stream);

/* One tier of a build in one call: pkv_blake3_ranges over its 2 n blob
 * ranges (key, value, key, value, ... -- the pool's or the shells' blobs in
 * layer order) into d_blob_digests (n x 64 bytes), then
 * pkv_blake3_layer_digests of those into d_layer_digests (n x 32 bytes), on
 * `stream`.  Replaces the per-blob CompressedBlock::new digests and the
 * per-layer PoolLayer / ShellLayer::compute_digest of a pool or shell build
 * (proveKV/src/codec.rs:85-95, pool.rs:83-103, shell.rs:48-66); the same
 * bytes as the two calls, with one host round trip. */
int pkv_blake3_tier_digests(pkv_ctx* ctx, const uint8_t* d_buf, uint64_t buf_bytes, const pkv_range* ranges,
                            uint32_t n, uint32_t layers, uint8_t* d_blob_digests, uint8_t* d_layer_digests,
                            void* stream);

/* blake3 of host bytes, hashed on the context's device (copy in, the same
 * kernels, copy out, synchronise): blake3::hash over a host slice, as
 * CodecProfileDigest / ArtifactDigest::from_canonical_bytes and from_parts
 * (quant-codec-core/src/digest.rs:14-58) use it. */
int pkv_blake3(pkv_ctx* ctx, const void* data, uint64_t len, uint8_t out[32]);

/* ---------------------------------------------------------------- host math
 * Host builds of the exact scalar routines the kernels use (test hooks):
 * angle bins of (a[i], b[i]) for pbits, the encode kernels' octant fast path
 * (3-bit bin and whether the pair is safe for it, i.e. kept from the exact
 * formula), and logf / expf over arrays. */
void pkv_host_angle_bins(const float* a, const float* b, uint64_t n, uint32_t pbits, uint32_t* out);
void pkv_host_octant_bins(const float* a, const float* b, uint64_t n, uint32_t* bins, uint8_t* safe);
void pkv_host_logf(const float* x, uint64_t n, float* out);
void pkv_host_expf(const float* x, uint64_t n, float* out);
/* The fib encode redo's test that f32 rounds every value within |v| 2^-50
 * of v[i] like v[i] (1) or that the exact division must decide (0). */
void pkv_host_f32_stable_rel50(const double* v, uint64_t n, uint8_t* out);
/* BLAKE3 of host bytes on the host, with the compression the digest
 * kernels run (the fib digests' hash). */
void pkv_host_blake3(const void* data, uint64_t len, uint8_t out[32]);

#ifdef __cplusplus
}
#endif
#endif /* PKV_CODEC_H */
