// pkv_kernels.hip -- gfx950 kernels for proveKV's codec hot path.
//
// Work decomposition (all kernels): one workgroup = 4 waves = 256 vectors of
// ONE segment (one FB2/TQB1 blob); one lane owns one vector end to end.
// Every (agent, layer, K|V) segment of a call is in the same grid; a
// workgroup finds its segment by binary search over a prefix table.
//
// HBM traffic is staged through LDS so both sides stay coalesced whatever the
// strides of the f32 tensor and the byte alignment of the blob:
//   * f32 rows: 16 lanes cover one 256 B row with 16 B loads/stores; each lane
//     then reads its own row from LDS (row pitch dim+4 floats: conflict-free
//     ds_read_b128);
//   * wire bytes: a wave's 64 payloads are one contiguous byte range; it is
//     moved with aligned dword accesses and v_alignbyte, independent of the
//     38 B (TQB1) / 19 B (FB2) header offset.
//
// Arithmetic follows the reference operation by operation (compiled with
// -ffp-contract=off): the FWHT butterfly order of fwht_normalized
// (turbo-quant/src/rotation.rs:379-398), sequential f32 QJL dots
// (qjl.rs:215), sequential f64 norm / rotation sums (fib-quant/src/codec.rs:
// 1049-1057, rotation.rs:107-113), the AVX2 pairwise argmin order
// (gpu-backend/src/simd_nearest.rs:44-104) and the sequential f32 inverse
// rotation of decode_batch_fast (rotation.rs:136-149).  Host-libm
// transcendentals come from pkv_math.h.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <map>
#include <mutex>
#include <utility>

#include "pkv_internal.h"
#include "pkv_math.h"

namespace pkv {
namespace {

constexpr int WAVE = 64;
constexpr int WAVES = TILE / WAVE;

typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

__constant__ LogfEntry c_logf_tab[16] = {PKV_LOGF_TABLE};
__constant__ uint64_t c_exp2f_tab[32] = {PKV_EXP2F_TABLE};

// u / 255.0f for every u8 code u (radius.rs:139-143), correctly rounded by the
// compiler at build time: the decode reads it instead of dividing per radius.
struct Div255 {
    float v[256];
    constexpr Div255() : v() {
        for (int u = 0; u < 256; ++u) v[u] = static_cast<float>(u) / 255.0f;
    }
};
__constant__ Div255 c_div255 = Div255();

// Gap between cheap_logf (below) and logf, per magnitude of the result:
// g_logb[e] = the largest |cheap_logf(v) - logf(v)| over every normal positive
// float v whose logf(v) has biased exponent <= e, rounded up to f32.  Measured
// on each device, over all 2,130,706,432 such v, by launch_logf_bound before
// the library encodes anything there (pkv_ctx_create).
__device__ uint32_t g_logb_raw[256];
__device__ float g_logb[256];

// ------------------------------------------------------------ helpers
__device__ __forceinline__ uint32_t find_segment(const uint32_t* __restrict__ tile_start, uint32_t nseg,
                                                 uint32_t blk) {
    uint32_t lo = 0, hi = nseg;
    while (hi - lo > 1) {
        uint32_t mid = (lo + hi) >> 1;
        if (tile_start[mid] <= blk) lo = mid; else hi = mid;
    }
    return lo;
}

// Segment of workgroup tile blk: one load from the launch's per-tile map when
// it has one, otherwise a binary search of the tile prefix.
__device__ __forceinline__ uint32_t segment_of(const uint32_t* __restrict__ tile_seg,
                                               const uint32_t* __restrict__ tile_start, uint32_t nseg, uint32_t blk) {
    return tile_seg ? tile_seg[blk] : find_segment(tile_start, nseg, blk);
}

__device__ __forceinline__ uint64_t vec_elem_offset(const SegDev& s, uint64_t i) {
    return s.elem_offset + (i / s.group) * s.stride_outer + (i % s.group) * s.stride_inner;
}

__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
    const uint32_t lo = static_cast<uint32_t>(__shfl(static_cast<int>(v), src));
    const uint32_t hi = static_cast<uint32_t>(__shfl(static_cast<int>(v >> 32), src));
    return static_cast<uint64_t>(hi) << 32 | lo;
}

__device__ __forceinline__ void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ uint32_t lds_byte(const uint32_t* lds, uint32_t off) {
    return (lds[off >> 2] >> (8 * (off & 3))) & 0xffu;
}

// Move nbytes from LDS (LDS byte 0 == dst byte 0) to global memory at any
// byte alignment.  Needs one readable padding dword after the staged bytes.
__device__ void lds_to_global(uint8_t* __restrict__ dst, const uint32_t* lds, uint32_t nbytes, int lane) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(dst);
    uint32_t head = static_cast<uint32_t>((4u - (a & 3u)) & 3u);
    if (head > nbytes) head = nbytes;
    if (static_cast<uint32_t>(lane) < head) dst[lane] = static_cast<uint8_t>(lds_byte(lds, lane));
    const uint32_t body = (nbytes - head) >> 2;
    uint32_t* d32 = reinterpret_cast<uint32_t*>(dst + head);
    const uint32_t sh = head;   // 0..3
    for (uint32_t k = lane; k < body; k += WAVE) {
        const uint32_t q = (head >> 2) + k;    // head < 4, so q == k
        uint32_t w0 = lds[q], w1 = lds[q + 1];
        d32[k] = sh ? __builtin_amdgcn_alignbyte(w1, w0, sh) : w0;
    }
    const uint32_t t0 = head + (body << 2);
    const uint32_t tail = nbytes - t0;
    if (static_cast<uint32_t>(lane) < tail) dst[t0 + lane] = static_cast<uint8_t>(lds_byte(lds, t0 + lane));
}

// Move nbytes from global memory at any byte alignment into LDS (LDS byte 0 ==
// src byte 0).  Only aligned dwords holding at least one source byte are read;
// each lane issues up to BATCH loads before it waits on any of them.
template <uint32_t BATCH = 8>
__device__ void global_to_lds(uint32_t* lds, const uint8_t* __restrict__ src, uint32_t nbytes, int lane) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(src);
    const uint32_t* s32 = reinterpret_cast<const uint32_t*>(a & ~static_cast<uintptr_t>(3));
    const uint32_t sh = static_cast<uint32_t>(a & 3u);
    const uint32_t ndw = (nbytes + 3u) >> 2;
    // dwords of the aligned window [a & ~3, a + nbytes): the last one may be
    // the only reader of the tail bytes
    const uint32_t nwin = static_cast<uint32_t>(((a + nbytes + 3u) & ~static_cast<uintptr_t>(3)) -
                                                (a & ~static_cast<uintptr_t>(3))) >> 2;
    for (uint32_t k0 = 0; k0 < ndw; k0 += BATCH * WAVE) {
        uint32_t w0[BATCH], w1[BATCH];
#pragma unroll
        for (uint32_t j = 0; j < BATCH; ++j) {
            const uint32_t k = k0 + j * WAVE + static_cast<uint32_t>(lane);
            w0[j] = k < ndw ? s32[k] : 0u;
            w1[j] = (sh && k < ndw && k + 1 < nwin) ? s32[k + 1] : 0u;
        }
#pragma unroll
        for (uint32_t j = 0; j < BATCH; ++j) {
            const uint32_t k = k0 + j * WAVE + static_cast<uint32_t>(lane);
            if (k < ndw) lds[k] = sh ? __builtin_amdgcn_alignbyte(w1[j], w0[j], sh) : w0[j];
        }
    }
}

// Stage nv (<= 64) rows of DIM values (f32, or bf16 upcast) into LDS rows of
// pitch DIM+4 floats with 16-byte loads; each lane issues 8 loads before it
// waits on any of them.  Lane r computes row r's offset once; the loads fetch
// it with __shfl.
template <int DIM>
__device__ void stage_rows_in(float* stage, const void* __restrict__ in, bool bf16, const SegDev& s,
                              uint32_t v0, uint32_t nv, int lane) {
    constexpr int PITCH = DIM + 4;
    constexpr int BATCH = 8;
    const unsigned long long my_off = vec_elem_offset(s, v0 + min(static_cast<uint32_t>(lane), nv - 1));
    if (!bf16) {
        const float* fin = static_cast<const float*>(in);
        constexpr int Q = DIM / 4;       // float4 per row
        constexpr int RPI = WAVE / Q;    // rows per load instruction
        for (uint32_t r0 = 0; r0 < nv; r0 += RPI * BATCH) {
            float4 v[BATCH];
#pragma unroll
            for (int k = 0; k < BATCH; ++k) {
                const uint32_t r = r0 + k * RPI + lane / Q;
                const unsigned long long off = __shfl(my_off, static_cast<int>(r & 63u));
                if (r < nv) v[k] = *reinterpret_cast<const float4*>(fin + off + 4 * (lane % Q));
            }
#pragma unroll
            for (int k = 0; k < BATCH; ++k) {
                const uint32_t r = r0 + k * RPI + lane / Q;
                if (r < nv) *reinterpret_cast<float4*>(stage + r * PITCH + 4 * (lane % Q)) = v[k];
            }
        }
    } else {
        const uint16_t* hin = static_cast<const uint16_t*>(in);
        constexpr int Q = DIM / 8;       // uint4 (8 bf16) per row
        constexpr int RPI = WAVE / Q;
        for (uint32_t r0 = 0; r0 < nv; r0 += RPI * BATCH) {
            uint4 v[BATCH];
#pragma unroll
            for (int k = 0; k < BATCH; ++k) {
                const uint32_t r = r0 + k * RPI + lane / Q;
                const unsigned long long off = __shfl(my_off, static_cast<int>(r & 63u));
                if (r < nv) v[k] = *reinterpret_cast<const uint4*>(hin + off + 8 * (lane % Q));
            }
#pragma unroll
            for (int k = 0; k < BATCH; ++k) {
                const uint32_t r = r0 + k * RPI + lane / Q;
                if (r < nv) {
                    float* d = stage + r * PITCH + 8 * (lane % Q);
                    const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        d[2 * t] = u2f(w[t] << 16);
                        d[2 * t + 1] = u2f(w[t] & 0xffff0000u);
                    }
                }
            }
        }
    }
}

// f32 -> bfloat16 bits, round to nearest even (torch's / c10's conversion).
__device__ __forceinline__ uint32_t bf16_rne(float x) {
    const uint32_t u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;   // NaN stays a (quiet) NaN
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// f32 -> binary16 bits, round to nearest even (v_cvt_f16_f32 in the default mode).
__device__ __forceinline__ uint32_t f16_rne(float x) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

__device__ __forceinline__ uint32_t pack_out2(float a, float b, uint32_t dt) {
    return dt == PKV_BF16 ? bf16_rne(a) | (bf16_rne(b) << 16) : f16_rne(a) | (f16_rne(b) << 16);
}

// Store four consecutive values of one output vector at element offset `off`
// (a multiple of 4) in the decode's output dtype, in every fan-out copy.
// NT: non-temporal stores, for callers that write whole rows per instruction
// (the output is not read back by this launch); partial-row writers keep L2
// write-combining (non-temporal made them 1.6x slower).
template <bool NT = false>
__device__ __forceinline__ void store_out4(void* __restrict__ out, const LaunchCommon& lc, uint64_t off, float4 v) {
    if (lc.out_dtype == PKV_F32) {
        const v4f q = {v.x, v.y, v.z, v.w};
        for (uint32_t k = 0; k < lc.fanout; ++k, off += lc.fanout_stride) {
            v4f* p = reinterpret_cast<v4f*>(static_cast<float*>(out) + off);
            if (NT) __builtin_nontemporal_store(q, p); else *p = q;
        }
    } else {
        const v2u w = {pack_out2(v.x, v.y, lc.out_dtype), pack_out2(v.z, v.w, lc.out_dtype)};
        for (uint32_t k = 0; k < lc.fanout; ++k, off += lc.fanout_stride) {
            v2u* p = reinterpret_cast<v2u*>(static_cast<uint16_t*>(out) + off);
            if (NT) __builtin_nontemporal_store(w, p); else *p = w;
        }
    }
}

__device__ __forceinline__ void store_out1(void* __restrict__ out, const LaunchCommon& lc, uint64_t off, float v) {
    if (lc.out_dtype == PKV_F32) {
        for (uint32_t k = 0; k < lc.fanout; ++k, off += lc.fanout_stride) static_cast<float*>(out)[off] = v;
    } else {
        const uint16_t w = static_cast<uint16_t>(lc.out_dtype == PKV_BF16 ? bf16_rne(v) : f16_rne(v));
        for (uint32_t k = 0; k < lc.fanout; ++k, off += lc.fanout_stride) static_cast<uint16_t*>(out)[off] = w;
    }
}

// LDS rows (pitch DIM + 4) of nv vectors -> their output positions, 16 B per
// lane per store; rows whose bit is set in the skip masks are not written.
template <int DIM>
__device__ void stage_rows_out(void* __restrict__ out, const LaunchCommon& lc, const float* stage, const SegDev& s,
                               uint32_t v0, uint32_t nv, uint32_t skip_mask_lo, uint32_t skip_mask_hi, int lane) {
    constexpr int PITCH = DIM + 4;
    constexpr int Q = DIM / 4;
    for (uint32_t i = lane; i < nv * Q; i += WAVE) {
        uint32_t r = i / Q, c = i % Q;
        uint32_t skip = r < 32 ? (skip_mask_lo >> r) & 1u : (skip_mask_hi >> (r - 32)) & 1u;
        if (skip) continue;
        uint64_t off = vec_elem_offset(s, v0 + r);
        store_out4<true>(out, lc, off + 4 * c, *reinterpret_cast<const float4*>(stage + r * PITCH + 4 * c));
    }
}

// In-register fwht_normalized (turbo-quant/src/rotation.rs:379-398): stages
// step = 1, 2, 4, ...; (a + b, a - b) at (start+off, start+off+step).
template <int DIM>
__device__ __forceinline__ void fwht(float (&v)[DIM]) {
#pragma unroll
    for (int step = 1; step < DIM; step *= 2) {
#pragma unroll
        for (int start = 0; start < DIM; start += 2 * step) {
#pragma unroll
            for (int off = 0; off < step; ++off) {
                float a = v[start + off], b = v[start + off + step];
                v[start + off] = a + b;
                v[start + off + step] = a - b;
            }
        }
    }
}

// (n as f32).sqrt().recip(): 0.125 for 64; 1/f32(sqrt(128)) for 128.
template <int DIM>
__device__ __forceinline__ float fwht_scale() {
    return DIM == 64 ? 0.125f : 1.0f / __builtin_sqrtf(static_cast<float>(DIM));
}

__device__ __forceinline__ void status_fail(uint32_t* status, uint32_t seg, int word, uint32_t index,
                                            uint32_t kind) {
    atomicMin(status + 2 * seg + word, (index << 4) | kind);
}

// TQB1 header byte i (turbo-quant/src/wire.rs:267-346).
__device__ __forceinline__ uint32_t tqb1_byte(uint32_t i, uint32_t dim, uint32_t pbits, uint32_t radii,
                                              uint32_t proj, uint64_t seed, uint32_t n, uint32_t plen) {
    if (i < 4) return (0x31425154u >> (8 * i)) & 0xffu;          // "TQB1"
    if (i == 4) return 1u;
    if (i == 6) return 1u;                                       // FastHadamard
    if (i == 8) return 2u;
    if (i >= 10 && i < 14) return (dim >> (8 * (i - 10))) & 0xffu;
    if (i == 14) return pbits;
    if (i == 15) return radii ? 1u : 0u;
    if (i >= 18 && i < 22) return (proj >> (8 * (i - 18))) & 0xffu;
    if (i >= 22 && i < 30) return static_cast<uint32_t>(seed >> (8 * (i - 22))) & 0xffu;
    if (i >= 30 && i < 34) return (n >> (8 * (i - 30))) & 0xffu;
    if (i >= 34 && i < 38) return (plen >> (8 * (i - 34))) & 0xffu;
    return 0u;
}

// Bytes the TQB1 decoder checks (wire.rs:401-503): all but 9, 16, 17.
__device__ __forceinline__ bool tqb1_checked(uint32_t i) { return i < 38 && i != 9 && i != 16 && i != 17; }

// FB2 header byte i (fib-quant/src/codec.rs:195-320), n_blocks = n.
__device__ __forceinline__ uint32_t fb2_byte(uint32_t i, uint32_t bits, uint32_t blocks, uint32_t n,
                                             uint32_t ilen) {
    if (i < 3) return (0x324246u >> (8 * i)) & 0xffu;             // "FB2"
    if (i == 3) return 1u;
    if (i == 4) return bits;
    if (i >= 6 && i < 10) return (blocks >> (8 * (i - 6))) & 0xffu;
    if (i >= 10 && i < 14) return (n >> (8 * (i - 10))) & 0xffu;
    if (i == 15) return 2u;
    if (i == 17) return ilen & 0xffu;
    if (i == 18) return (ilen >> 8) & 0xffu;
    return 0u;
}

// Bytes the FB2 decoder checks (codec.rs:323-424): all but 5; the norm length
// only matters when there is at least one vector (decode_norm, 1025-1031).
__device__ __forceinline__ bool fb2_checked(uint32_t i, uint32_t n) {
    if (i == 5) return false;
    if ((i == 15 || i == 16) && n == 0) return false;
    return i < 19;
}

// ------------------------------------------------------------ turbo encode
template <int DIM, int PB>
__global__ __launch_bounds__(TILE) void turbo_encode_kernel(
    LaunchCommon lc, const void* __restrict__ in, uint8_t* __restrict__ wire,
    const float* __restrict__ signs, const float* __restrict__ qjl, const float* __restrict__ cs_tab,
    uint64_t seed, uint32_t pbits_rt, uint32_t proj, uint32_t mode) {
    constexpr int PITCH = DIM + 4;
    constexpr int PAIRS = DIM / 2;
    constexpr int WAVE_FLOATS = WAVE * PITCH + 8;
    extern __shared__ float smem[];
    __shared__ float cs_lds[512];
    __shared__ LogfEntry logf_lds[16];

    const uint32_t pbits = PB ? static_cast<uint32_t>(PB) : pbits_rt;
    const uint32_t levels = 1u << pbits;
    for (uint32_t t = threadIdx.x; t < 2 * levels; t += blockDim.x) cs_lds[t] = cs_tab[t];
    if (threadIdx.x < 16) logf_lds[threadIdx.x] = c_logf_tab[threadIdx.x];
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float* stage = smem + wave * WAVE_FLOATS;
    const uint32_t blk = blockIdx.x;
    const uint32_t sidx = segment_of(lc.tile_seg, lc.tile_start, lc.nseg, blk);
    const SegDev seg = lc.segs[sidx];
    const uint32_t tile = blk - lc.tile_start[sidx];
    const uint32_t v0 = tile * TILE + wave * WAVE;
    const uint32_t plen = lc.plen;
    uint8_t* blob = wire + seg.wire_offset;

    if (v0 < seg.n_vectors) {
        const uint32_t nv = min(static_cast<uint32_t>(WAVE), seg.n_vectors - v0);
        stage_rows_in<DIM>(stage, in, lc.in_bf16 != 0, seg, v0, nv, lane);
        wave_sync();

        const bool active = static_cast<uint32_t>(lane) < nv;
        const float* xr = stage + lane * PITCH;
        const float scale = fwht_scale<DIM>();
        // Lanes past the segment end compute on stale LDS; their results are
        // never stored.
        float y[DIM];
        bool finite = true;
#pragma unroll
        for (int c = 0; c < DIM; ++c) {
            float xv = xr[c];
            finite &= isfinite_f(xv);
            y[c] = xv * signs[c];
        }
        fwht<DIM>(y);
#pragma unroll
        for (int c = 0; c < DIM; ++c) y[c] *= scale;

        // radii and angle bins (polar.rs:246-266, 413-421): octant fast path;
        // pairs near an octant line (and every pair when pbits != 3) take the
        // exact libm formula in a rolled loop below.  Bins are kept packed
        // LSB-first exactly as the wire stores them (bitpack.rs:21-35).
        constexpr int NW = PB ? (PAIRS * PB + 31) / 32 : 1;
        float r[PAIRS];
        uint32_t bw[PB ? NW : 1];
        uint32_t bins_rt[PB ? 1 : PAIRS];
#pragma unroll
        for (int t = 0; t < (PB ? NW : 1); ++t) bw[t] = 0u;
        uint64_t slow = 0;
        bool rfinite = true;
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            float a = y[2 * i], b = y[2 * i + 1];
            float aa = a * a, bb = b * b;
            r[i] = __builtin_sqrtf(aa + bb);
            rfinite &= isfinite_f(r[i]);
            bool safe = false;
            if (PB == 3) {
                const uint32_t bin = octant_bin(a, b, safe);
                const int bit = 3 * i;
                bw[bit >> 5] |= bin << (bit & 31);
                if ((bit & 31) > 29) bw[(bit >> 5) + 1] |= bin >> (32 - (bit & 31));
            }
            if (!safe) slow |= 1ull << i;
        }
        if (slow) {
            for (int i = 0; i < PAIRS; ++i) {
                if (!((slow >> i) & 1ull)) continue;
                float a = 0.0f, b = 0.0f;
#pragma unroll
                for (int k = 0; k < PAIRS; ++k) {
                    a = (k == i) ? y[2 * k] : a;
                    b = (k == i) ? y[2 * k + 1] : b;
                }
                const uint32_t bin = angle_bin_exact(a, b, pbits);
                if (PB == 3) {
                    const uint32_t bit = 3u * static_cast<uint32_t>(i);
                    const uint32_t wd = bit >> 5, sh = bit & 31u;
#pragma unroll
                    for (int t = 0; t < (PB ? NW : 1); ++t) {
                        if (static_cast<uint32_t>(t) == wd) bw[t] = (bw[t] & ~(7u << sh)) | (bin << sh);
                        if (sh > 29 && static_cast<uint32_t>(t) == wd + 1)
                            bw[t] = (bw[t] & ~(7u >> (32 - sh))) | (bin >> (32 - sh));
                    }
                } else {
#pragma unroll
                    for (int k = 0; k < (PB ? 1 : PAIRS); ++k) bins_rt[k] = (k == i) ? bin : bins_rt[k];
                }
            }
        }
        auto bin_of = [&](int i) -> uint32_t {
            if (PB == 3) {
                const int bit = 3 * i;
                uint32_t v = bw[bit >> 5] >> (bit & 31);
                if ((bit & 31) > 29) v |= bw[(bit >> 5) + 1] << (32 - (bit & 31));
                return v & 7u;
            }
            return bins_rt[PB ? 0 : i];
        };

        uint32_t sbits0 = 0u, sbits1 = 0u;
        bool resfinite = true;
        if (mode) {
            // polar decode of the code just produced (polar.rs:272-278, 306-316)
#pragma unroll
            for (int i = 0; i < PAIRS; ++i) {
                const uint32_t bin = bin_of(i);
                y[2 * i] = r[i] * cs_lds[2 * bin];
                y[2 * i + 1] = r[i] * cs_lds[2 * bin + 1];
            }
            fwht<DIM>(y);
#pragma unroll
            for (int c = 0; c < DIM; ++c) {
                float z = (y[c] * scale) * signs[c];
                y[c] = xr[c] - z;                 // residual (turbo.rs:269-273)
                resfinite &= isfinite_f(y[c]);
            }
            // QJL sketch (qjl.rs:203-220): sequential f32 dot per row.
            for (uint32_t j = 0; j < proj; ++j) {
                const float* g = qjl + static_cast<size_t>(j) * DIM;
                float dot = 0.0f;
#pragma unroll
                for (int c = 0; c < DIM; ++c) dot = dot + g[c] * y[c];
                const uint32_t bit = dot >= 0.0f ? 1u << (j & 31) : 0u;
                if (j < 32) sbits0 |= bit; else sbits1 |= bit;
            }
        }

        // status: first failing vector (turbo encode is per-vector in order)
        if (active) {
            uint32_t vi = v0 + lane;
            if (!finite) status_fail(lc.status, sidx, 1, vi, KIND_NONFINITE_INPUT);
            else if (!rfinite) status_fail(lc.status, sidx, 1, vi, KIND_NONFINITE_RADIUS);
            else if (mode && !resfinite) status_fail(lc.status, sidx, 1, vi, KIND_NONFINITE_RESIDUAL);
        }
        wave_sync();   // every lane is done reading its staged row

        // payload into LDS (plen is a dword multiple for every profile the
        // host accepts; every field starts dword aligned).
        uint32_t* pw = reinterpret_cast<uint32_t*>(stage) + lane * (plen >> 2);
        if (active) {
            uint32_t w = 0;
            if (lc.radii == PKV_RADII_F32) {
#pragma unroll
                for (int i = 0; i < PAIRS; ++i) pw[w++] = f2u(r[i]);
            } else {
                // CompressedRadiiV1 BlockLogU8 (turbo-quant/src/radius.rs:58-77)
                float lg[PAIRS];
                float mn = u2f(0x7f800000u), mx = u2f(0xff800000u);
#pragma unroll
                for (int i = 0; i < PAIRS; ++i) {
                    float v = r[i] < 1.17549435e-38f ? 1.17549435e-38f : r[i];
                    lg[i] = og_logf_normal(v, logf_lds);
                    mn = __builtin_fminf(mn, lg[i]);
                    mx = __builtin_fmaxf(mx, lg[i]);
                }
                float span = __builtin_fmaxf(mx - mn, 1.1920929e-07f);
#pragma unroll
                for (int i = 0; i < PAIRS; i += 4) {
                    uint32_t packed = 0;
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        float nrm = (lg[i + t] - mn) / span;
                        nrm = nrm < 0.0f ? 0.0f : (nrm > 1.0f ? 1.0f : nrm);
                        float q = __builtin_roundf(nrm * 255.0f);
                        packed |= static_cast<uint32_t>(q) << (8 * t);
                    }
                    pw[w++] = packed;
                }
                pw[w++] = f2u(mn);
                pw[w++] = f2u(mx);
            }
            // angle indices, pbits each, LSB-first (bitpack.rs:21-35)
            if (PB == 3) {
#pragma unroll
                for (int t = 0; t < (PB ? NW : 1); ++t) pw[w++] = bw[t];
            } else {
                uint64_t acc = 0;
                uint32_t nb = 0;
                for (int i = 0; i < PAIRS; ++i) {
                    acc |= static_cast<uint64_t>(bin_of(i)) << nb;
                    nb += pbits;
                    if (nb >= 32) { pw[w++] = static_cast<uint32_t>(acc); acc >>= 32; nb -= 32; }
                }
                if (nb) pw[w++] = static_cast<uint32_t>(acc);
            }
            if (mode) {
                pw[w++] = sbits0;
                if (proj > 32) pw[w++] = sbits1;
            }
        }
        wave_sync();
        lds_to_global(blob + 38 + static_cast<uint64_t>(v0) * plen, reinterpret_cast<uint32_t*>(stage),
                      nv * plen, lane);
    }
    if (tile == 0 && threadIdx.x < 38) {
        blob[threadIdx.x] = static_cast<uint8_t>(
            tqb1_byte(threadIdx.x, DIM, pbits, lc.radii, proj, seed, seg.n_vectors, plen));
    }
}

// ------------------------------------------------------------ turbo encode, QJL on the matrix cores
// TurboQuantizer::encode with PolarWithQjl at head_dim 64 (turbo.rs:240-300).
// Two lanes per vector: lane (h, n) = (lane / 32, lane % 32) holds elements
// 32h .. 32h + 31 of vector n of a 32-vector tile.  The arithmetic is the
// reference's, operation for operation: FWHT stages 1..16 run in registers
// and stage 32 pairs the halves through v_permlane32_swap (same operands,
// same rounding); radii and angle bins are per pair; the residual is exact.
// Of the QJL sketch only the signs of the 32 (or 64) sequential f32 dots
// reach the wire (qjl.rs:203-220), so the dots come from the f16 matrix
// cores (v_mfma_f32_32x32x16_f16 on the halves of the scaled residual; lane
// (h, n) gives the B operand's column n, K step st covers dimensions
// 32h + 8st .. 32h + 8st + 7) and a sign is taken only past the proven bound
// at qjl_scale; the other dots are recomputed in the reference's order, the
// first half's partial sum handed to the second half.

// Value of the other half-wave's lane (l ^ 32).
__device__ __forceinline__ uint32_t partner(uint32_t x, int h) {
    const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return h ? p[0] : p[1];
}

// Value of the lane in the other 16-lane row of the same pair (l ^ 16).
__device__ __forceinline__ uint32_t partner16(uint32_t x, int q) {
    const auto p = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (q & 1) ? p[0] : p[1];
}

// fwht_normalized stages (turbo-quant/src/rotation.rs:379-398) on a vector
// split over the two halves of the wave: 32 elements per lane.
template <int FIRST = 1>
__device__ __forceinline__ void fwht_split(float (&v)[32], int h) {
#pragma unroll
    for (int step = FIRST; step < 32; step *= 2) {
#pragma unroll
        for (int start = 0; start < 32; start += 2 * step) {
#pragma unroll
            for (int off = 0; off < step; ++off) {
                const float a = v[start + off], b = v[start + off + step];
                v[start + off] = a + b;
                v[start + off + step] = a - b;
            }
        }
    }
    // step 32: element c (half 0) with c + 32 (half 1): (a + b, a - b).  A
    // v_permlane32_swap of two different elements v[c], v[c + 16] leaves (a, b)
    // of element c in the lanes of half 0 and (a, b) of element c + 16 in the
    // lanes of half 1, so every lane forms the same a + b and a - b; a second
    // swap returns each sum and difference to its own half.
    (void)h;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        auto p = __builtin_amdgcn_permlane32_swap(f2u(v[c]), f2u(v[c + 16]), false, false);
        const float a = u2f(p[0]), b = u2f(p[1]);
        p = __builtin_amdgcn_permlane32_swap(f2u(a + b), f2u(a - b), false, false);
        v[c] = u2f(p[0]);
        v[c + 16] = u2f(p[1]);
    }
}

// The sign flips of the rotation (x_c * s_c, s_c = +-1, exact) fused with
// the FWHT's first stage (step 1): (x0 s0 + x1 s1, x0 s0 - x1 s1) as two fmas
// around the exact product x1 s1 -- the same single roundings.
__device__ __forceinline__ void signs_stage1(float (&v)[32], const float (&sg)[32]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float t = v[2 * i + 1] * sg[2 * i + 1];
        const float a = v[2 * i];
        v[2 * i] = __builtin_fmaf(a, sg[2 * i], t);
        v[2 * i + 1] = __builtin_fmaf(a, sg[2 * i], -t);
    }
}

// The hardware log2 times ln 2 rounded to f32: within g_logb of logf.
__device__ __forceinline__ float cheap_logf(float v) { return __builtin_amdgcn_logf(v) * 0x1.62e430p-1f; }

// Correctly rounded sqrt of x >= 2^-96, +0, +inf or NaN: the hardware root s
// (v_sqrt_f32, within 1 ulp) moved to a neighbour s -+ 1 ulp when the exact
// remainder fma(-s', s, x) shows the root lies past the midpoint -- the
// fix-up of the compiler's own f32 sqrt expansion, without the rescaling it
// applies below 2^-96 or the +-0 / +inf select, which this fix-up already
// gets right (+0: the neighbours' remainders are NaN and -0; +inf: NaN).
// Below 2^-96 (callers route such inputs to __builtin_sqrtf) the remainder
// may underflow.
__device__ __forceinline__ float sqrt_normal(float x) {
    const float s = __builtin_amdgcn_sqrtf(x);
    const float sd = u2f(f2u(s) - 1u), su = u2f(f2u(s) + 1u);
    float r = __builtin_fmaf(-sd, s, x) <= 0.0f ? sd : s;
    r = __builtin_fmaf(-su, s, x) > 0.0f ? su : r;
    return r;
}

// CompressedRadiiV1 BlockLogU8 (turbo-quant/src/radius.rs:58-77) of one
// vector whose 64 radii sit 16 per lane on LPV = 2 (lanes l, l ^ 32; part =
// l >> 5) or LPV = 4 lanes (l, l ^ 16, l ^ 32, l ^ 48; part = l >> 4).
// Writes this lane's 16 codes (4 per word, radius 16 part + i in byte i) and
// the vector's mn, mx.  Every lane of the wave must call it.
//
// The reference takes v_i = max(r_i, FLT_MIN), l_i = logf(v_i), mn = min l_i,
// mx = max l_i, span = max(mx - mn, 2^-23) and
// code_i = roundf(fl(255 * clamp(fl(fl(l_i - mn) / span), 0, 1))).
// * logf is monotone non-decreasing on the normal floats (checked on every
//   one), so mn = logf(min v_i) and mx = logf(max v_i): two exact logs.
// * For the codes, t_i = fl(fl(cheap_logf(v_i) - mn) * fl(255 / span)) is
//   within 255 delta / span + 2 * 256 * 3.0001u (u = 2^-24) of the
//   reference's value P_i before roundf, with delta = g_logb of the larger of
//   |mn|, |mx| (every l_i lies between them): three roundings on each side,
//   of values at most 256 when the margin below is under 1/2.  When t_i is
//   farther than M = 255 delta / span (1 + 2^-10) + 1552u from every
//   half-integer, P_i lies in the same unit interval around rint(t_i), so
//   roundf(P_i) = rint(t_i) (t_i >= -M > -1/2 and t_i <= 255 + M; no ties).
//   The others -- every code when M >= 1/2, and a NaN t_i -- take the
//   reference's chain.
// * rint(t_i) comes from v_rndne_f32 and goes into its byte by
//   v_cvt_pk_u8_f32, exact for the integers 0..255 the decided codes have;
//   whether any code is undecided is a wave-wide OR of compare masks, and
//   only then does a lane rebuild its per-code flags.  A lane holding a
//   radius below FLT_MIN (zero, subnormal) or NaN takes the chain for every
//   code: there v_i = FLT_MIN (or NaN) differs from the radius the hardware
//   log sees.
template <int LPV>
__device__ __forceinline__ void block_log_u8(const float (&r)[16], int part, const LogfEntry* ltab, uint32_t (&code)[4],
                                             float& mn, float& mx) {
    constexpr float kMinPos = 1.17549435e-38f;
    // min / max of v_i = max(r_i, FLT_MIN): the same clamp applied to the
    // extremes of the radii (NaN radii skipped by fmin / fmax, as before)
    float rmin = u2f(0x7f800000u), rmax = u2f(0xff800000u);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        rmin = __builtin_fminf(rmin, r[i]);
        rmax = __builtin_fmaxf(rmax, r[i]);
    }
    const bool tiny = rmin < kMinPos;   // NaN radii show up as NaN codes below
    float vmin = tiny ? kMinPos : rmin;
    float vmax = rmax < kMinPos && rmax != u2f(0xff800000u) ? kMinPos : rmax;
    if constexpr (LPV == 4) {
        vmin = __builtin_fminf(vmin, u2f(partner16(f2u(vmin), part)));
        vmax = __builtin_fmaxf(vmax, u2f(partner16(f2u(vmax), part)));
    }
    vmin = __builtin_fminf(vmin, u2f(partner(f2u(vmin), LPV == 4 ? part >> 1 : part)));
    vmax = __builtin_fmaxf(vmax, u2f(partner(f2u(vmax), LPV == 4 ? part >> 1 : part)));
    // one exact log per lane: even parts the minimum, odd parts the maximum
    const float own = og_logf_normal((part & 1) ? vmax : vmin, ltab);
    const float other = u2f(LPV == 4 ? partner16(f2u(own), part) : partner(f2u(own), part));
    mn = (part & 1) ? other : own;
    mx = (part & 1) ? own : other;
    const float span = __builtin_fmaxf(mx - mn, 1.1920929e-07f);
    const float inv = 255.0f / span;
    const float big = __builtin_fmaxf(__builtin_fabsf(mn), __builtin_fabsf(mx));
    const float delta = g_logb[f2u(big) >> 23];
    const float margin = delta * inv * (1.0f + 0x1p-10f) + 0x1.84p-14f;   // 1552u >= 6 * 256 * 1.0001u
    const float thr = 0.5f - margin;   // decided when |t - rint(t)| < thr
    uint64_t undecided = __ballot(tiny);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t packed = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int i = 4 * w + t;
            const float tv = (cheap_logf(r[i]) - mn) * inv;
            const float k = __builtin_rintf(tv);
            undecided |= __ballot(!(__builtin_fabsf(tv - k) < thr));
            packed = __builtin_amdgcn_cvt_pk_u8_f32(k, static_cast<uint32_t>(t), packed);
        }
        code[w] = packed;
    }
    if (undecided) {
        uint32_t slow = tiny ? 0xffffu : 0u;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const float tv = (cheap_logf(r[i]) - mn) * inv;
            slow |= (__builtin_fabsf(tv - __builtin_rintf(tv)) < thr ? 0u : 1u) << i;
        }
        for (uint32_t m = slow; m; m &= m - 1u) {
            const uint32_t i = static_cast<uint32_t>(__ffs(m) - 1);
            float ri = r[0];   // r[i] by selects (a dynamic index would go through scratch)
#pragma unroll
            for (int j = 1; j < 16; ++j) ri = static_cast<uint32_t>(j) == i ? r[j] : ri;
            const float vi = ri < kMinPos ? kMinPos : ri;
            float nrm = (og_logf_normal(vi, ltab) - mn) / span;
            nrm = nrm < 0.0f ? 0.0f : (nrm > 1.0f ? 1.0f : nrm);
            const uint32_t q = static_cast<uint32_t>(__builtin_roundf(nrm * 255.0f));
            const uint32_t sh = 8u * (i & 3u), keep = ~(0xffu << sh);
#pragma unroll
            for (int w = 0; w < 4; ++w)
                code[w] = static_cast<uint32_t>(w) == (i >> 2) ? (code[w] & keep) | (q << sh) : code[w];
        }
    }
}

// Radii and angle bins (polar.rs:246-266, 413-421) of a lane's 16 pairs
// (y[2i], y[2i + 1]): r[i] = sqrt(fl(a^2) + fl(b^2)), the bins pbits apart
// in pk, rsum the lane's radius sum (its finiteness stands for every radius
// and input element).  At pbits = 3 a pair octant_bin_f passes takes the
// octant's bin and sqrt_normal's radius (its fl(a^2) + fl(b^2) >= 2^-94);
// the other pairs -- near an octant line or outside the covered range, every
// pair of a lane whose radius sum is not finite, every pair at other widths
// -- take angle_bin_exact and __builtin_sqrtf.  Every lane of the wave must
// call it.
template <int PB>
__device__ __forceinline__ void radii_bins(const float (&y)[32], uint32_t pbits, float (&r)[16], uint64_t& pk,
                                           float& rsum) {
    constexpr int HP = 16;
    uint64_t any_unsafe = 0;   // the wave's lanes with a pair that needs the exact formulas
    rsum = 0.0f;
    pk = 0;
    // octant_bin_f's bins, bit by bit: each pair shifts the sign bits of g,
    // a ^ b and b into a shift register (v_alignbit), ascending bit order,
    // pairs 0..9 and two bits of pair 10 into w0, the rest into w1; a bit
    // reversal then puts pair i at bits 3i (g), 3i + 1 (a ^ b), 3i + 2 (b),
    // and one xor per word turns them into octant_bin_f's (sign(g) ^ sign(a ^
    // b), sign(a ^ b), !sign(b)).
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int i = 0; i < HP; ++i) {
        const float a = y[2 * i], b = y[2 * i + 1];
        const float aa = a * a, bb = b * b;
        r[i] = sqrt_normal(aa + bb);
        rsum = rsum + r[i];
        bool uns = true;
        if constexpr (PB == 3) {
            const float fa = __builtin_fabsf(a), fb = __builtin_fabsf(b);
            const float g = fa - fb;
            const float mx = __builtin_fmaxf(__builtin_fmaxf(fa, fb), 0x1p-31f);
            const float m3 = __builtin_fminf(__builtin_fminf(fa, fb), __builtin_fabsf(g));
            uns = !(mx < m3 * 65536.0f);   // octant_bin_f's test
            const uint32_t src[3] = {f2u(g), f2u(a) ^ f2u(b), f2u(b)};
#pragma unroll
            for (int k = 0; k < 3; ++k) {
                if (3 * i + k < 32) w0 = __builtin_amdgcn_alignbit(w0, src[k], 31);
                else w1 = __builtin_amdgcn_alignbit(w1, src[k], 31);
            }
        }
        any_unsafe |= __ballot(uns);
    }
    if constexpr (PB == 3) {
        w0 = __builtin_bitreverse32(w0);
        w1 = __builtin_bitreverse32(w1) >> 16;
        w0 ^= ((w0 >> 1) & 0x49249249u) ^ 0x24924924u;   // bits 3i ^= 3i + 1; bits 3i + 2 flipped
        w1 ^= ((w1 >> 1) & 0x2492u) ^ 0x9249u;           // the same fields, one bit up (pair 10 straddles)
        pk = (static_cast<uint64_t>(w1) << 32) | w0;
    }
    const bool force = !isfinite_f(rsum);
    any_unsafe |= __ballot(force);
    if (any_unsafe) {
        // this lane's pairs again (the fast loop keeps only the wave's OR)
        const uint32_t levels = 1u << pbits;
        uint32_t slow = force ? 0xffffu : 0u;
#pragma unroll
        for (int i = 0; i < HP; ++i) {
            bool uns = true;
            if constexpr (PB == 3) (void)octant_bin_f(y[2 * i], y[2 * i + 1], uns);
            slow |= (uns ? 1u : 0u) << i;
        }
        for (uint32_t m = slow; m; m &= m - 1u) {
            const uint32_t i = static_cast<uint32_t>(__ffs(m) - 1);
            // pair i by selects (a dynamic index into y would go through scratch)
            float a = y[0], b = y[1];
#pragma unroll
            for (int j = 1; j < HP; ++j) {
                a = static_cast<uint32_t>(j) == i ? y[2 * j] : a;
                b = static_cast<uint32_t>(j) == i ? y[2 * j + 1] : b;
            }
            const uint64_t bin = angle_bin_exact(a, b, pbits);
            pk = (pk & ~(static_cast<uint64_t>(levels - 1u) << (i * pbits))) | (bin << (i * pbits));
            const float aa = a * a, bb = b * b;
            const float ri = __builtin_sqrtf(aa + bb);
#pragma unroll
            for (int j = 0; j < HP; ++j) r[j] = static_cast<uint32_t>(j) == i ? ri : r[j];
        }
    }
}

// QJL dots on the f16 matrix cores.  Per vector the residual is scaled by
// s = 2^k so that an upper bound of |x|_2 lies in [2^14, 2^15) (x = res * s,
// exact; qjl_scale), and
// split toward zero into f16 halves, x = xh + xl + ex with |ex| <= 2^-20 |x|
// + 2^-24; the host splits G = Gh + Gl + eG to nearest, |eG| <= 2^-22 |G| +
// 2^-25.  The matrix cores form acc = sum_c Gh xh + Gh xl + Gl xh (f16
// products are exact in f32, and subnormal f16 operands are kept: checked on
// the device by the test suite).  Per element, G x - (Gh xh + Gh xl + Gl xh)
// = eG x + Gh ex + Gl (x - xh), at most 28.1u |G||x| + 1.001 * 2^-25 |x| +
// 1.002 * 2^-24 |G| + 2^-49 (u = 2^-24); the 3d products accumulate with at
// most 3d roundings, taken at 2u each: 6.03d u sum|G x|; the reference's
// sequential f32 dot is within (d + 0.01)u sum|G_c res_c| of the exact one.
// With sum|G x| <= |g_j| |x| and |x| <= xn, the sign of acc is the sign of
// the reference's dot whenever |acc| > a_j xn + b_j (a_j, b_j built at
// turbo_qjl_mfma_constants with a (1 + 2^-10) margin, which also covers the
// rounding of the bound itself); the others are recomputed in the
// reference's order.
//
__device__ __forceinline__ v16f mfma16(const v4u& a, const v4u& b, const v16f& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}

__device__ __forceinline__ v4f mfma16x32(const v4u& a, const v4u& b, const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
}

// |res| rounded up: rn2 is the f32 sum of the squares (one fma each, then
// the lanes' partial sums added), within (1 + 35u) rn2 + 2^-144 of the exact
// one (relative roundings while normal, at most 2^-150 each while subnormal),
// so |res| <= sqrt(rn2) (1 + 19u) + 2^-72, which 1.0001 and 2^-70 cover.
__device__ __forceinline__ float qjl_norm_bound(float rn2) {
    return __builtin_fmaf(__builtin_sqrtf(rn2), 1.0001f, 0x1p-70f);
}

// 2^(14 - e) for the exponent e of rn >= |res| (clamped to [-60, 127]): every
// |x_c| = |res_c| 2^(14 - e) <= rn 2^(14 - e) < 2^15, inside the f16 range
// (and below 2^14 when rn < 2^-60).
__device__ __forceinline__ float qjl_scale(float rn) {
    int e = static_cast<int>((f2u(rn) >> 23) & 0xffu) - 127;
    e = e < -60 ? -60 : (e > 127 ? 127 : e);
    return u2f(static_cast<uint32_t>(127 + 14 - e) << 23);
}

// a - f32(f16 half `hi` of h), one v_fma_mix_f32 (exact: a's f16 truncation
// removed from a).
template <int HI>
__device__ __forceinline__ float sub_f16(float a, uint32_t h) {
    float r;
    if constexpr (HI)
        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(a));
    else
        asm("v_fma_mix_f32 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(h), "v"(a));
    return r;
}

// x = v[c0 + j] * sc, j = 0..7, as f16 halves toward zero: xh = f16(x),
// xl = f16(x - xh) (x - xh is exact in f32).
__device__ __forceinline__ void qjl_split8(const float (&v)[32], int c0, float sc, v4u& xh, v4u& xl) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const float a = v[c0 + 2 * t] * sc, b = v[c0 + 2 * t + 1] * sc;
        const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
        xh[t] = h;
        xl[t] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(sub_f16<0>(a, h), sub_f16<1>(b, h)));
    }
}

// DIAG: also write every projection's matrix-core dot and acceptance bound
// (divided by the residual's scale) to lc.diag[((vector * proj) + j) * 2 + {0, 1}].
template <int PB, bool DIAG>
__global__ __launch_bounds__(TILE) void turbo_encode_qjl_kernel(
    LaunchCommon lc, const void* __restrict__ in, uint8_t* __restrict__ wire, const float* __restrict__ signs,
    const float* __restrict__ qjl, const float* __restrict__ cs_tab, const uint32_t* __restrict__ qa,
    const float* __restrict__ qb, uint64_t seed, uint32_t pbits_rt, uint32_t proj) {
    constexpr int DIM = 64;
    constexpr int HP = 16;   // pairs per lane
    extern __shared__ uint32_t smem_u[];   // per wave: 32 payloads (+ f32 radii for BlockLogU8)
    __shared__ float cs_lds[512];
    __shared__ LogfEntry logf_lds[16];
    // the signs (+-1.0), then -sign * scale: the scale is 2^-3, so both are exact
    __shared__ __align__(16) float sg_lds[2 * DIM];

    const uint32_t pbits = PB ? static_cast<uint32_t>(PB) : pbits_rt;
    const uint32_t levels = 1u << pbits;
    for (uint32_t t = threadIdx.x; t < 2 * levels; t += blockDim.x) cs_lds[t] = cs_tab[t];
    if (threadIdx.x < 16) logf_lds[threadIdx.x] = c_logf_tab[threadIdx.x];
    for (uint32_t t = threadIdx.x; t < DIM; t += blockDim.x) {
        const float sv = signs[t];
        sg_lds[t] = sv;
        sg_lds[DIM + t] = -sv * fwht_scale<DIM>();
    }
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int h = lane >> 5, n = lane & 31;
    // two workgroups per TILE-vector tile, one 32-vector group per wave
    const uint32_t blk = blockIdx.x >> 1;
    const uint32_t sidx = segment_of(lc.tile_seg, lc.tile_start, lc.nseg, blk);
    const SegDev seg = lc.segs[sidx];
    const uint32_t tile = blk - lc.tile_start[sidx];
    const uint32_t plen = lc.plen, pwd = plen >> 2;
    const bool f32r = lc.radii == PKV_RADII_F32;
    // per vector: the payload, then (BlockLogU8 radii only) its 32 f32 radii
    const uint32_t vec_words = pwd + (f32r ? 0u : 32u);
    uint32_t* pay = smem_u + wave * (32 * vec_words + 4);
    uint8_t* blob = wire + seg.wire_offset;
    const bool bf16 = lc.in_bf16 != 0;
    const float scale = fwht_scale<DIM>();
    const uint32_t rwords = f32r ? 32u : 32u / 4 + 2;          // radii words in the payload
    const uint32_t bwords = (32u * pbits + 31) / 32;            // angle index words

    // this lane's 32 values of a 64-float LDS table (the signs, or -sign * scale)
    auto lds_half = [&](const float* tab, float (&v)[32]) {
        const float4* sp = reinterpret_cast<const float4*>(tab + 32 * h);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float4 q = sp[k];
            v[4 * k] = q.x; v[4 * k + 1] = q.y; v[4 * k + 2] = q.z; v[4 * k + 3] = q.w;
        }
    };

    do {
        const uint32_t t0 = tile * TILE + (blockIdx.x & 1u) * (TILE / 2) + 32u * static_cast<uint32_t>(wave);
        if (t0 >= seg.n_vectors) break;
        const uint32_t nv = min(32u, seg.n_vectors - t0);
        const bool active = static_cast<uint32_t>(n) < nv;   // other lanes repeat the last vector
        const uint64_t off = vec_elem_offset(seg, t0 + min(static_cast<uint32_t>(n), nv - 1)) + 32u * h;
        uint32_t* pv = pay + n * vec_words;          // this vector's payload
        uint32_t* rw = pv + (f32r ? 0u : pwd);       // its f32 radii

        float y[32];
        auto load_half = [&](float (&v)[32]) {
            if (!bf16) {
                const float4* src = reinterpret_cast<const float4*>(static_cast<const float*>(in) + off);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float4 q = src[k];
                    v[4 * k] = q.x; v[4 * k + 1] = q.y; v[4 * k + 2] = q.z; v[4 * k + 3] = q.w;
                }
            } else {
                const uint4* src = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(in) + off);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint4 q = src[k];
                    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        v[8 * k + 2 * t] = u2f(w[t] << 16);
                        v[8 * k + 2 * t + 1] = u2f(w[t] & 0xffff0000u);
                    }
                }
            }
        };
        load_half(y);
        {
            float sg[32];
            lds_half(sg_lds, sg);
            signs_stage1(y, sg);
        }
        fwht_split<2>(y, h);
#pragma unroll
        for (int c = 0; c < 32; ++c) y[c] *= scale;

        // zero this vector's angle index words: both halves OR into them
        if (h == 0 && active)
            for (uint32_t k = 0; k < bwords; ++k) pv[rwords + k] = 0u;
        wave_sync();

        // radii and angle bins (polar.rs:246-266, 413-421) of pairs 16h + i
        float r[HP];
        float rsum;
        uint64_t pk;
        radii_bins<PB>(y, pbits, r, pk, rsum);
        // A non-finite input makes every FWHT output, so every radius,
        // non-finite; a finite sum of the (non-negative) radii therefore
        // clears both checks.  Otherwise (or on an overflowing sum) they run
        // element by element.
        bool finite = true, rfinite = true;
        if (!isfinite_f(rsum)) {
            float x[32];
            load_half(x);
#pragma unroll
            for (int c = 0; c < 32; ++c) finite &= isfinite_f(x[c]);
#pragma unroll
            for (int i = 0; i < HP; ++i) rfinite &= isfinite_f(r[i]);
        }
        // angle indices, pbits each, LSB-first (bitpack.rs:21-35): this half's
        // 16 * pbits bits start at bit 16 * pbits * h
        if (active) {
            const uint32_t bit0 = 16u * pbits * static_cast<uint32_t>(h);
            const uint32_t nb = 16u * pbits;   // <= 128 bits: pk holds up to 64, pbits <= 4 here
            uint32_t* bwp = pv + rwords + (bit0 >> 5);
            const uint32_t sh = bit0 & 31u;
            const uint32_t w0 = static_cast<uint32_t>(pk << sh);
            const uint32_t w1 = static_cast<uint32_t>((pk << sh) >> 32) | (sh ? static_cast<uint32_t>(pk >> (64 - sh)) : 0u);
            const uint32_t w2 = sh ? static_cast<uint32_t>(pk >> (96 - sh)) : 0u;
            atomicOr(bwp, w0);
            if (sh + nb > 32) atomicOr(bwp + 1, w1);
            if (sh + nb > 64) atomicOr(bwp + 2, w2);
        }
        if (f32r) {
            if (active)
#pragma unroll
                for (int i = 0; i < HP; ++i) rw[16 * h + i] = f2u(r[i]);
        } else {
            // CompressedRadiiV1 BlockLogU8 (turbo-quant/src/radius.rs:58-77)
            uint32_t code[4];
            float mn, mx;
            block_log_u8<2>(r, h, logf_lds, code, mn, mx);
            if (active) {
#pragma unroll
                for (int w = 0; w < 4; ++w) pv[4 * h + w] = code[w];
                if (h == 0) {
                    pv[8] = f2u(mn);
                    pv[9] = f2u(mx);
                }
#pragma unroll
                for (int i = 0; i < HP; ++i) rw[16 * h + i] = f2u(r[i]);
            }
        }
        wave_sync();

        // polar decode of the code just produced (polar.rs:272-278, 306-316)
#pragma unroll
        for (int i = 0; i < HP; ++i) {
            const uint32_t bin = static_cast<uint32_t>(pk >> (static_cast<uint32_t>(i) * pbits)) & (levels - 1u);
            y[2 * i] = r[i] * cs_lds[2 * bin];
            y[2 * i + 1] = r[i] * cs_lds[2 * bin + 1];
        }
        fwht_split(y, h);
        // residual against x read again (turbo.rs:269-273)
        asm volatile("" ::: "memory");
        {
            // x - (y * scale) * sign: with the scale 2^-3, y * scale is exact
            // unless it is subnormal, and then the residual is the single
            // rounding of x - sign * y / 8, one fma with -sign * scale.  A wave
            // holding any |y| < 2^-123 (zeros included) takes the three
            // roundings' own order.
            float x[32];
            load_half(x);
            float ymin = __builtin_fabsf(y[0]);
#pragma unroll
            for (int c = 1; c < 32; ++c) ymin = __builtin_fminf(ymin, __builtin_fabsf(y[c]));
            if (__ballot(!(ymin >= 0x1p-123f)) == 0) {
                float ns[32];
                lds_half(sg_lds + DIM, ns);
#pragma unroll
                for (int c = 0; c < 32; ++c) y[c] = __builtin_fmaf(y[c], ns[c], x[c]);
            } else {
                float sg[32];
                lds_half(sg_lds, sg);
#pragma unroll
                for (int c = 0; c < 32; ++c) y[c] = x[c] - (y[c] * scale) * sg[c];
            }
        }
        float rn2 = 0.0f;
#pragma unroll
        for (int c = 0; c < 32; ++c) rn2 = __builtin_fmaf(y[c], y[c], rn2);
        // squares are non-negative: a finite sum clears every element
        bool resfinite = true;
        if (!isfinite_f(rn2)) {
#pragma unroll
            for (int c = 0; c < 32; ++c) resfinite &= isfinite_f(y[c]);
        }
        rn2 = rn2 + u2f(partner(f2u(rn2), h));
        const float rn = qjl_norm_bound(rn2);

        // QJL dots on the f16 matrix cores (v_mfma_f32_32x32x16_f16; bound at
        // qjl_scale): K step st covers dimensions 32h + 8st + j of lane (h, n)
        const float sc = qjl_scale(rn);
        const float xn = rn * sc;
        const uint32_t ptiles = proj / 32;
        v16f acc[2] = {};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            v4u xh, xl;
            qjl_split8(y, 8 * st, sc, xh, xl);
#pragma unroll
            for (uint32_t p = 0; p < 2; ++p) {
                if (p >= ptiles) break;
                const v4u* a = reinterpret_cast<const v4u*>(qa) + (p * 4 + st) * 2 * 64 + lane;
                const v4u ah = a[0], al = a[64];
                acc[p] = mfma16(ah, xh, acc[p]);
                acc[p] = mfma16(ah, xl, acc[p]);
                acc[p] = mfma16(al, xh, acc[p]);
            }
        }
        // accumulator register k of tile p: projection 32p + 8(k/4) + 4h + k%4
        // of vector n.  The sign bits shift in (v_alignbit) as negative flags,
        // register 15 first, so bit k of neg is register k; a dot is undecided
        // when |acc| <= a_j xn + b_j, collected wave-wide.
        uint32_t sbits[2] = {0u, 0u};
        uint64_t undecided = 0;
#pragma unroll
        for (uint32_t p = 0; p < 2; ++p) {
            if (p >= ptiles) break;
            const float2* ab = reinterpret_cast<const float2*>(qb) + p * 16 * 64 + lane;
            uint32_t neg = 0;
#pragma unroll
            for (int k = 15; k >= 0; --k) {
                const float2 c = ab[k * 64];
                const float bnd = __builtin_fmaf(c.x, xn, c.y);
                undecided |= __ballot(!(__builtin_fabsf(acc[p][k]) > bnd));
                neg = __builtin_amdgcn_alignbit(neg, f2u(acc[p][k]), 31);
                if constexpr (DIAG) {
                    if (active) {
                        const uint32_t j = static_cast<uint32_t>(8 * (k >> 2) + 4 * h + (k & 3));
                        float* dv = lc.diag + (static_cast<uint64_t>(t0 + static_cast<uint32_t>(n)) * proj + 32u * p + j) * 2u;
                        dv[0] = acc[p][k] / sc;
                        dv[1] = bnd / sc;
                    }
                }
            }
            // nibble m of neg -> bits 8m + 4h .. 8m + 4h + 3; a dot >= 0 (or -0,
            // always undecided) gives bit 1
            uint32_t sp = (neg | (neg << 8)) & 0x00ff00ffu;
            sp = (sp | (sp << 4)) & 0x0f0f0f0fu;
            const uint32_t sb = (sp ^ 0x0f0f0f0fu) << (4 * h);
            sbits[p] = sb | partner(sb, h);
        }
        // undecided signs: the reference's sequential dot, half 0's partial
        // sum continued by half 1
        if (undecided & __ballot(active)) {
            uint32_t unc[2] = {0u, 0u};
#pragma unroll
            for (uint32_t p = 0; p < 2; ++p) {
                if (p >= ptiles) break;
                const float2* ab = reinterpret_cast<const float2*>(qb) + p * 16 * 64 + lane;
                uint32_t un = 0;
#pragma unroll
                for (int k = 0; k < 16; ++k) {
                    const uint32_t j = static_cast<uint32_t>(8 * (k >> 2) + 4 * h + (k & 3));
                    const float2 c = ab[k * 64];
                    const float bnd = __builtin_fmaf(c.x, xn, c.y);
                    un |= (__builtin_fabsf(acc[p][k]) > bnd ? 0u : 1u) << j;
                }
                unc[p] = un | partner(un, h);
            }
#pragma unroll
            for (uint32_t p = 0; p < 2; ++p) {
                if (p >= ptiles) break;
                uint32_t m = active ? unc[p] : 0u;
                // the wave walks the union of its vectors' undecided projections
                uint32_t any = m;
                any |= partner(any, h);
                for (int sh2 = 1; sh2 < 32; sh2 <<= 1) any |= __shfl_xor(any, sh2);
                while (any) {
                    const uint32_t j = static_cast<uint32_t>(__ffs(any) - 1);
                    any &= any - 1u;
                    const float* g = qjl + static_cast<size_t>(32 * p + j) * DIM + 32 * h;
                    float dot = 0.0f;
#pragma unroll
                    for (int c = 0; c < 32; ++c) dot = dot + g[c] * y[c];   // half 0: dims 0..31 from 0
                    const float first = u2f(partner(f2u(dot), h));          // half 0's sum, seen by half 1
                    float d2 = first;
#pragma unroll
                    for (int c = 0; c < 32; ++c) d2 = d2 + g[c] * y[c];     // half 1: continues over 32..63
                    // every lane takes part in the swap (a cross-lane read under a
                    // lane-dependent condition would see the inactive half's
                    // lanes unchanged); half 0 then takes half 1's full sum
                    const uint32_t other = partner(f2u(d2), h);
                    const float full = u2f(h ? f2u(d2) : other);
                    if ((m >> j) & 1u) sbits[p] = (sbits[p] & ~(1u << j)) | (full >= 0.0f ? 1u << j : 0u);
                }
            }
        }

        // status (per vector, first failure in vector order) and the QJL words
        uint32_t bad = (finite ? 0u : 1u) | (rfinite ? 0u : 2u) | (resfinite ? 0u : 4u);
        bad |= partner(bad, h);
        if (active && h == 0) {
            const uint32_t vi = t0 + n;
            if (bad & 1u) status_fail(lc.status, sidx, 1, vi, KIND_NONFINITE_INPUT);
            else if (bad & 2u) status_fail(lc.status, sidx, 1, vi, KIND_NONFINITE_RADIUS);
            else if (bad & 4u) status_fail(lc.status, sidx, 1, vi, KIND_NONFINITE_RESIDUAL);
            pv[rwords + bwords] = sbits[0];
            if (proj > 32) pv[rwords + bwords + 1] = sbits[1];
        }
        wave_sync();
        if (!f32r) {   // close the gaps left by the f32 radii words
            // each half moves at most TMAX words: fixed trip count, predicated,
            // so tmp stays in registers
            constexpr uint32_t TMAX = (32 / 4 + 2) + 8 + 2;
            uint32_t tmp[TMAX];
            const uint32_t k0 = static_cast<uint32_t>(h) * (pwd / 2 + 1);
            const uint32_t k1 = h ? pwd : pwd / 2 + 1;
#pragma unroll
            for (uint32_t j = 0; j < TMAX; ++j) tmp[j] = (active && k0 + j < k1) ? pv[k0 + j] : 0u;
            wave_sync();
            if (active)
#pragma unroll
                for (uint32_t j = 0; j < TMAX; ++j)
                    if (k0 + j < k1) pay[n * pwd + k0 + j] = tmp[j];
            wave_sync();
        }
        lds_to_global(blob + 38 + static_cast<uint64_t>(t0) * plen, pay, nv * plen, lane);
    } while (false);
    if (tile == 0 && (blockIdx.x & 1u) == 0 && threadIdx.x < 38) {
        blob[threadIdx.x] = static_cast<uint8_t>(
            tqb1_byte(threadIdx.x, DIM, pbits, lc.radii, proj, seed, seg.n_vectors, plen));
    }
}

// Head_dim 128: four lanes per vector, lane (q, n) = (lane / 16, lane % 16)
// of a 16-vector group.  The encode reads elements 32q .. 32q + 31; FWHT
// stages 1..16 run in registers, stages 32 and 64 on v_permlane16_swap /
// v_permlane32_swap (same operands and rounding as fwht_normalized), and the
// transform stops in layout F: lane q holds 16-element blocks q and 4 + q
// (elements 16q + c in v[c], 64 + 16q + c in v[16 + c]) -- its pairs are
// 8q .. 8q + 7 and 32 + 8q .. 32 + 8q + 7.  The inverse transform runs on
// layout F (stages 1..8 in registers, 16, 32 and 64 across lanes) and stops in
// layout G: lane q holds blocks B(q) and 4 + B(q), B = (0, 2, 1, 3), where the
// residual and its QJL dots are formed.  The QJL dots come from
// v_mfma_f32_16x16x32_f16 on the f16 halves of the scaled residual (bound at
// qjl_scale): lane (q, n) gives the B operand's column n, and K step st
// covers its elements y[8st .. 8st + 7] (dimensions 16B(q) + 8st + j for st <
// 2, 64 + 16B(q) + 8(st - 2) + j after); a 16-projection tile accumulates in
// 4 registers per lane (projection 16p + 4q + r of vector n in register r).
// The undecided dots are recomputed in the reference's order, block by block,
// each block's holder continuing the previous block's sum.

// Value of lane l ^ 16 (the other quarter of the same half).
// fwht_normalized stages (turbo-quant/src/rotation.rs:379-398) on a 128-wide
// vector split over four lanes, 32 elements per lane.
template <int FIRST = 1>
__device__ __forceinline__ void fwht_quarter(float (&v)[32], int q) {
#pragma unroll
    for (int step = FIRST; step < 32; step *= 2) {
#pragma unroll
        for (int start = 0; start < 32; start += 2 * step) {
#pragma unroll
            for (int off = 0; off < step; ++off) {
                const float a = v[start + off], b = v[start + off + step];
                v[start + off] = a + b;
                v[start + off + step] = a - b;
            }
        }
    }
    // step 32: element c of quarter 2k with c of quarter 2k + 1: (a + b, a - b);
    // step 64: quarters 0, 1 with 2, 3.  On element pairs (c, c + 16): a
    // v_permlane16_swap of v[c], v[c + 16] leaves step 32's (a, b) of element
    // c in the even rows and of element c + 16 in the odd rows, and every lane
    // forms a + b, a - b; a v_permlane32_swap of those two then holds step 64's
    // (a, b) -- quarters 0 / 2 in rows 0, 1, quarters 1 / 3 in rows 2, 3 -- for
    // the same a + b, a - b; the two swaps in reverse order return every
    // result to its quarter and element.
    (void)q;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        auto p = __builtin_amdgcn_permlane16_swap(f2u(v[c]), f2u(v[c + 16]), false, false);
        float a = u2f(p[0]), b = u2f(p[1]);
        p = __builtin_amdgcn_permlane32_swap(f2u(a + b), f2u(a - b), false, false);
        a = u2f(p[0]);
        b = u2f(p[1]);
        p = __builtin_amdgcn_permlane32_swap(f2u(a + b), f2u(a - b), false, false);
        p = __builtin_amdgcn_permlane16_swap(p[0], p[1], false, false);
        v[c] = u2f(p[0]);
        v[c + 16] = u2f(p[1]);
    }
}

// Stages 2..64 of fwht_normalized on the standard layout (element 32q + c in
// v[c]; stage 1 already applied), ending in layout F.  Per c: a
// v_permlane16_swap of v[c], v[c + 16] gives each row the stage-32 pair
// (lower, upper) of one element -- row q: elements (c, 32 + c) + 16 (q & 1)
// + 64 (q >> 1) -- and a v_permlane32_swap of the sums and differences the
// stage-64 pair, (16q + c, 64 + 16q + c) in row q, which stays there.
__device__ __forceinline__ void fwht128_fwd(float (&v)[32]) {
#pragma unroll
    for (int step = 2; step < 32; step *= 2) {
#pragma unroll
        for (int start = 0; start < 32; start += 2 * step) {
#pragma unroll
            for (int off = 0; off < step; ++off) {
                const float a = v[start + off], b = v[start + off + step];
                v[start + off] = a + b;
                v[start + off + step] = a - b;
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        auto p = __builtin_amdgcn_permlane16_swap(f2u(v[c]), f2u(v[c + 16]), false, false);
        float a = u2f(p[0]), b = u2f(p[1]);
        p = __builtin_amdgcn_permlane32_swap(f2u(a + b), f2u(a - b), false, false);
        a = u2f(p[0]);
        b = u2f(p[1]);
        v[c] = a + b;
        v[c + 16] = a - b;
    }
}

// fwht_normalized on layout F, ending in layout G.  Stages 1..8 pair elements
// inside a 16-element block (registers); per c the three cross-lane stages:
// a v_permlane16_swap of v[c], v[c + 16] gives rows 0..3 the stage-16 pairs
// (c, 16 + c), (64 + c, 80 + c), (32 + c, 48 + c), (96 + c, 112 + c), a
// v_permlane32_swap of the sums and
// differences the stage-32 pairs (c, 32 + c), (64 + c, 96 + c), (16 + c,
// 48 + c), (80 + c, 112 + c), and a v_permlane16_swap of those results the
// stage-64 pairs (c, 64 + c), (32 + c, 96 + c), (16 + c, 80 + c),
// (48 + c, 112 + c): blocks B(q) and 4 + B(q), B = (0, 2, 1, 3).
__device__ __forceinline__ void fwht128_inv(float (&v)[32]) {
#pragma unroll
    for (int step = 1; step < 16; step *= 2) {
#pragma unroll
        for (int start = 0; start < 32; start += 2 * step) {
#pragma unroll
            for (int off = 0; off < step; ++off) {
                const float a = v[start + off], b = v[start + off + step];
                v[start + off] = a + b;
                v[start + off + step] = a - b;
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        auto p = __builtin_amdgcn_permlane16_swap(f2u(v[c]), f2u(v[c + 16]), false, false);
        float a = u2f(p[0]), b = u2f(p[1]);
        p = __builtin_amdgcn_permlane32_swap(f2u(a + b), f2u(a - b), false, false);
        a = u2f(p[0]);
        b = u2f(p[1]);
        p = __builtin_amdgcn_permlane16_swap(f2u(a + b), f2u(a - b), false, false);
        a = u2f(p[0]);
        b = u2f(p[1]);
        v[c] = a + b;
        v[c + 16] = a - b;
    }
}

// OR of a value over the four lanes of a vector.
__device__ __forceinline__ uint32_t or_quarters(uint32_t x, int q) {
    x |= partner16(x, q);
    return x | partner(x, q >> 1);
}

template <int PB, bool DIAG>
__global__ __launch_bounds__(TILE) void turbo_encode_qjl128_kernel(
    LaunchCommon lc, const void* __restrict__ in, uint8_t* __restrict__ wire, const float* __restrict__ signs,
    const float* __restrict__ qjl, const float* __restrict__ cs_tab, const uint32_t* __restrict__ qa,
    const float* __restrict__ qb, uint64_t seed, uint32_t pbits_rt, uint32_t proj) {
    constexpr int DIM = 128;
    constexpr int HP = 16;   // pairs per lane
    constexpr int GV = 16;   // vectors per wave
    extern __shared__ uint32_t smem_u[];   // per wave: 16 payloads
    __shared__ float cs_lds[512];
    __shared__ LogfEntry logf_lds[16];

    const uint32_t pbits = PB ? static_cast<uint32_t>(PB) : pbits_rt;
    const uint32_t levels = 1u << pbits;
    for (uint32_t t = threadIdx.x; t < 2 * levels; t += blockDim.x) cs_lds[t] = cs_tab[t];
    if (threadIdx.x < 16) logf_lds[threadIdx.x] = c_logf_tab[threadIdx.x];
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int q = lane >> 4, n = lane & 15;
    // four workgroups per TILE-vector tile, one 16-vector group per wave
    const uint32_t blk = blockIdx.x >> 2;
    const uint32_t sidx = segment_of(lc.tile_seg, lc.tile_start, lc.nseg, blk);
    const SegDev seg = lc.segs[sidx];
    const uint32_t tile = blk - lc.tile_start[sidx];
    const uint32_t plen = lc.plen, pwd = plen >> 2;
    const bool f32r = lc.radii == PKV_RADII_F32;
    uint32_t* pay = smem_u + wave * (GV * pwd + 4);
    uint8_t* blob = wire + seg.wire_offset;
    const bool bf16 = lc.in_bf16 != 0;
    const float scale = fwht_scale<DIM>();
    const uint32_t rwords = f32r ? 64u : 64u / 4 + 2;          // radii words in the payload
    const uint32_t bwords = (64u * pbits + 31) / 32;            // angle index words

    // this lane's 32 sign values, elements e0 + c (c < 16) and e1 + c - 16
    auto load_signs = [&](float (&sg)[32], uint32_t e0, uint32_t e1) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float4 v = reinterpret_cast<const float4*>(signs + (k < 4 ? e0 : e1))[k & 3];
            sg[4 * k] = v.x; sg[4 * k + 1] = v.y; sg[4 * k + 2] = v.z; sg[4 * k + 3] = v.w;
        }
    };
    // layout G: blocks B(q) and 4 + B(q), B = (0, 2, 1, 3)
    const uint32_t g0 = 16u * static_cast<uint32_t>(((q & 1) << 1) | (q >> 1)), g1 = 64u + g0;

    do {
        const uint32_t t0 = tile * TILE + (blockIdx.x & 3u) * (TILE / 4) + GV * static_cast<uint32_t>(wave);
        if (t0 >= seg.n_vectors) break;
        const uint32_t nv = min(static_cast<uint32_t>(GV), seg.n_vectors - t0);
        const bool active = static_cast<uint32_t>(n) < nv;   // other lanes repeat the last vector
        const uint64_t vbase = vec_elem_offset(seg, t0 + min(static_cast<uint32_t>(n), nv - 1));
        uint32_t* pv = pay + n * pwd;   // this vector's payload

        float y[32];
        // elements e0 + c (c < 16) and e1 + c - 16 of this lane's vector
        auto load_x = [&](float (&v)[32], uint32_t e0, uint32_t e1) {
            if (!bf16) {
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float4 w = reinterpret_cast<const float4*>(static_cast<const float*>(in) + vbase +
                                                                     (k < 4 ? e0 : e1))[k & 3];
                    v[4 * k] = w.x; v[4 * k + 1] = w.y; v[4 * k + 2] = w.z; v[4 * k + 3] = w.w;
                }
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint4 w = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(in) + vbase +
                                                                   (k < 2 ? e0 : e1))[k & 1];
                    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        v[8 * k + 2 * t] = u2f(ww[t] << 16);
                        v[8 * k + 2 * t + 1] = u2f(ww[t] & 0xffff0000u);
                    }
                }
            }
        };
        const uint32_t q0 = 32u * static_cast<uint32_t>(q);   // standard layout: elements 32q .. 32q + 31
        load_x(y, q0, q0 + 16);
        {
            float sg[32];
            load_signs(sg, q0, q0 + 16);
            signs_stage1(y, sg);
        }
        fwht128_fwd(y);   // -> layout F
#pragma unroll
        for (int c = 0; c < 32; ++c) y[c] *= scale;

        // zero this vector's angle index words: all quarters OR into them
        if (q == 0 && active)
            for (uint32_t k = 0; k < bwords; ++k) pv[rwords + k] = 0u;
        wave_sync();

        // radii and angle bins (polar.rs:246-266, 413-421) of pairs 8q + i
        // (i < 8) and 32 + 8q + i - 8 (layout F)
        float r[HP];
        float rsum;
        uint64_t pk;
        radii_bins<PB>(y, pbits, r, pk, rsum);
        // A non-finite input makes every FWHT output, so every radius,
        // non-finite; a finite sum of the (non-negative) radii therefore
        // clears both checks.  Otherwise (or on an overflowing sum) they run
        // element by element.
        bool finite = true, rfinite = true;
        if (!isfinite_f(rsum)) {
            float x[32];
            load_x(x, q0, q0 + 16);
#pragma unroll
            for (int c = 0; c < 32; ++c) finite &= isfinite_f(x[c]);
#pragma unroll
            for (int i = 0; i < HP; ++i) rfinite &= isfinite_f(r[i]);
        }
        // angle indices, pbits each, LSB-first (bitpack.rs:21-35): this
        // lane's two runs of 8 pairs, 8 * pbits <= 32 bits each, start at
        // bits 8 * pbits * q and 8 * pbits * (4 + q)
        if (active) {
            const uint32_t nb = 8u * pbits;
            const uint64_t lo = pk & ((1ull << nb) - 1u), hi = pk >> nb;
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const uint32_t bit0 = nb * (static_cast<uint32_t>(q) + 4u * half);
                const uint64_t run = (half ? hi : lo) << (bit0 & 31u);
                uint32_t* bwp = pv + rwords + (bit0 >> 5);
                atomicOr(bwp, static_cast<uint32_t>(run));
                if ((bit0 & 31u) + nb > 32) atomicOr(bwp + 1, static_cast<uint32_t>(run >> 32));
            }
        }
        if (f32r) {
            if (active)
#pragma unroll
                for (int i = 0; i < HP; ++i) pv[(i < 8 ? 8 * q : 24 + 8 * q) + i] = f2u(r[i]);
        } else {
            // CompressedRadiiV1 BlockLogU8 (turbo-quant/src/radius.rs:58-77)
            uint32_t code[4];
            float mn, mx;
            block_log_u8<4>(r, q, logf_lds, code, mn, mx);
            if (active) {
                // radius j in byte j: local codes 0..7 are radii 8q.., 8..15 are 32 + 8q..
#pragma unroll
                for (int w = 0; w < 4; ++w) pv[(w < 2 ? 2 * q : 6 + 2 * q) + w] = code[w];
                if (q == 0) {
                    pv[16] = f2u(mn);
                    pv[17] = f2u(mx);
                }
            }
        }

        // polar decode of the code just produced (polar.rs:272-278, 306-316)
#pragma unroll
        for (int i = 0; i < HP; ++i) {
            const uint32_t bin = static_cast<uint32_t>(pk >> (static_cast<uint32_t>(i) * pbits)) & (levels - 1u);
            y[2 * i] = r[i] * cs_lds[2 * bin];
            y[2 * i + 1] = r[i] * cs_lds[2 * bin + 1];
        }
        fwht128_inv(y);   // layout F -> layout G
        // residual against x read again (turbo.rs:269-273)
        asm volatile("" ::: "memory");
        {
            // x - (y * scale) * sign with sign = +-1: the product by the sign
            // is exact, so one fma with -sign rounds the same
            float x[32], sg[32];
            load_x(x, g0, g1);
            load_signs(sg, g0, g1);
#pragma unroll
            for (int c = 0; c < 32; ++c) y[c] = __builtin_fmaf(y[c] * scale, -sg[c], x[c]);
        }
        float rn2 = 0.0f;
#pragma unroll
        for (int c = 0; c < 32; ++c) rn2 = __builtin_fmaf(y[c], y[c], rn2);
        // squares are non-negative: a finite sum clears every element
        bool resfinite = true;
        if (!isfinite_f(rn2)) {
#pragma unroll
            for (int c = 0; c < 32; ++c) resfinite &= isfinite_f(y[c]);
        }
        rn2 = rn2 + u2f(partner16(f2u(rn2), q));
        rn2 = rn2 + u2f(partner(f2u(rn2), q >> 1));
        const float rn = qjl_norm_bound(rn2);

        // QJL dots on the f16 matrix cores (v_mfma_f32_16x16x32_f16; bound at
        // qjl_scale): K step st covers y[8st + j] of lane (q, n), dimensions
        // g0 + 8st + j (st < 2) and g1 + 8(st - 2) + j
        const float sc = qjl_scale(rn);
        const float xn = rn * sc;
        const uint32_t ptiles = proj / 16;
        v4f acc[4] = {};
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            v4u xh, xl;
            qjl_split8(y, 8 * st, sc, xh, xl);
#pragma unroll
            for (uint32_t p = 0; p < 4; ++p) {
                if (p >= ptiles) break;
                const v4u* a = reinterpret_cast<const v4u*>(qa) + (p * 4 + st) * 2 * 64 + lane;
                const v4u ah = a[0], al = a[64];
                acc[p] = mfma16x32(ah, xh, acc[p]);
                acc[p] = mfma16x32(ah, xl, acc[p]);
                acc[p] = mfma16x32(al, xh, acc[p]);
            }
        }
        // register r of tile p: projection j = 16p + 4q + r of vector n.  The
        // sign bits shift in (v_alignbit) as negative flags, tile 2w + 1 first,
        // so bit 4k + r of neg[w] is register r of tile 2w + k; a dot is
        // undecided when |acc| <= a_j xn + b_j, collected wave-wide.
        const float2* ab = reinterpret_cast<const float2*>(qb) + lane;
        uint32_t neg[2] = {0u, 0u};
        uint64_t undecided = 0;
#pragma unroll
        for (int p = 3; p >= 0; --p) {
            if (static_cast<uint32_t>(p) >= ptiles) continue;
#pragma unroll
            for (int rr = 3; rr >= 0; --rr) {
                const float2 c = ab[(p * 4 + rr) * 64];
                const float bnd = __builtin_fmaf(c.x, xn, c.y);
                undecided |= __ballot(!(__builtin_fabsf(acc[p][rr]) > bnd));
                neg[p >> 1] = __builtin_amdgcn_alignbit(neg[p >> 1], f2u(acc[p][rr]), 31);
                if constexpr (DIAG) {
                    if (active) {
                        const uint32_t j = 16u * p + 4u * static_cast<uint32_t>(q) + static_cast<uint32_t>(rr);
                        float* dv = lc.diag + (static_cast<uint64_t>(t0 + static_cast<uint32_t>(n)) * proj + j) * 2u;
                        dv[0] = acc[p][rr] / sc;
                        dv[1] = bnd / sc;
                    }
                }
            }
        }
        // word w: bits 4q + r (tile 2w) and 16 + 4q + r (tile 2w + 1); a dot
        // >= 0 (or -0, always undecided) gives bit 1
        uint32_t sbits[2];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            const uint32_t pos = ~neg[w] & 0xffu;
            sbits[w] = ((pos & 0xfu) | ((pos << 12) & 0xf0000u)) << (4 * q);
            sbits[w] = or_quarters(sbits[w], q);
        }
        // undecided signs: the reference's sequential dot, each quarter
        // continuing the previous quarter's partial sum
        if (undecided & __ballot(active)) {
            uint32_t unc[2] = {0u, 0u};
#pragma unroll
            for (uint32_t p = 0; p < 4; ++p) {
                if (p >= ptiles) break;
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const uint32_t j = 16u * p + 4u * static_cast<uint32_t>(q) + static_cast<uint32_t>(rr);
                    const float2 c = ab[(p * 4 + rr) * 64];
                    const float bnd = __builtin_fmaf(c.x, xn, c.y);
                    unc[j >> 5] |= (__builtin_fabsf(acc[p][rr]) > bnd ? 0u : 1u) << (j & 31u);
                }
            }
#pragma unroll
            for (uint32_t w = 0; w < 2; ++w) {
                if (32u * w >= proj) break;
                const uint32_t uq = or_quarters(unc[w], q);   // every lane swaps
                const uint32_t m = active ? uq : 0u;
                uint32_t any = m;
                for (int sh2 = 1; sh2 < 64; sh2 <<= 1) any |= __shfl_xor(any, sh2);
                while (any) {
                    const uint32_t j = static_cast<uint32_t>(__ffs(any) - 1);
                    any &= any - 1u;
                    const float* g = qjl + static_cast<size_t>(32 * w + j) * DIM;
                    // blocks 0..7 in order: block b sits in row B(b & 3), in
                    // y[0..15] (b < 4) or y[16..31]; its row continues the sum
                    // and every lane takes it
                    float run = 0.0f;
#pragma unroll
                    for (int b = 0; b < 8; ++b) {
                        const int hb = ((b & 1) << 1) | ((b >> 1) & 1);
                        if (q == hb) {
                            float d = run;
#pragma unroll
                            for (int c = 0; c < 16; ++c) d = d + g[16 * b + c] * y[(b < 4 ? 0 : 16) + c];
                            run = d;
                        }
                        run = __shfl(run, 16 * hb + n);
                    }
                    const float full = run;
                    if ((m >> j) & 1u) sbits[w] = (sbits[w] & ~(1u << j)) | (full >= 0.0f ? 1u << j : 0u);
                }
            }
        }

        // status (per vector, first failure in vector order) and the QJL words
        const uint32_t bad = or_quarters((finite ? 0u : 1u) | (rfinite ? 0u : 2u) | (resfinite ? 0u : 4u), q);
        if (active && q == 0) {
            const uint32_t vi = t0 + n;
            if (bad & 1u) status_fail(lc.status, sidx, 1, vi, KIND_NONFINITE_INPUT);
            else if (bad & 2u) status_fail(lc.status, sidx, 1, vi, KIND_NONFINITE_RADIUS);
            else if (bad & 4u) status_fail(lc.status, sidx, 1, vi, KIND_NONFINITE_RESIDUAL);
            pv[rwords + bwords] = sbits[0];
            if (proj > 32) pv[rwords + bwords + 1] = sbits[1];
        }
        wave_sync();
        lds_to_global(blob + 38 + static_cast<uint64_t>(t0) * plen, pay, nv * plen, lane);
    } while (false);
    if (tile == 0 && (blockIdx.x & 3u) == 0 && threadIdx.x < 38) {
        blob[threadIdx.x] = static_cast<uint8_t>(
            tqb1_byte(threadIdx.x, DIM, pbits, lc.radii, proj, seed, seg.n_vectors, plen));
    }
}

// ------------------------------------------------------------ turbo decode
template <int DIM, int PB>
__global__ __launch_bounds__(TILE) void turbo_decode_kernel(
    LaunchCommon lc, const uint8_t* __restrict__ wire, void* __restrict__ out,
    const float* __restrict__ signs, const float* __restrict__ cs_tab, uint64_t seed, uint32_t pbits_rt,
    uint32_t proj, uint32_t mode) {
    constexpr int PITCH = DIM + 4;
    constexpr int PAIRS = DIM / 2;
    constexpr int WAVE_FLOATS = WAVE * PITCH + 8;
    extern __shared__ float smem[];
    __shared__ float cs_lds[512];
    __shared__ uint64_t exp_lds[32];
    __shared__ float div255_lds[256];

    const uint32_t pbits = PB ? static_cast<uint32_t>(PB) : pbits_rt;
    const uint32_t levels = 1u << pbits;
    for (uint32_t t = threadIdx.x; t < 2 * levels; t += blockDim.x) cs_lds[t] = cs_tab[t];
    if (threadIdx.x < 32) exp_lds[threadIdx.x] = c_exp2f_tab[threadIdx.x];
    for (uint32_t t = threadIdx.x; t < 256; t += blockDim.x) div255_lds[t] = c_div255.v[t];
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float* stage = smem + wave * WAVE_FLOATS;
    const uint32_t blk = blockIdx.x;
    const uint32_t sidx = segment_of(lc.tile_seg, lc.tile_start, lc.nseg, blk);
    const SegDev seg = lc.segs[sidx];
    const uint32_t tile = blk - lc.tile_start[sidx];
    const uint32_t v0 = tile * TILE + wave * WAVE;
    const uint32_t plen = lc.plen;
    const uint8_t* blob = wire + seg.wire_offset;

    // header check (every wave; 38 bytes)
    uint32_t hb = lane < 38 ? blob[lane] : 0u;
    bool bad = lane < 38 && tqb1_checked(lane) &&
               hb != tqb1_byte(lane, DIM, pbits, lc.radii, proj, seed, seg.n_vectors, plen);
    if (__ballot(bad) != 0ull) {
        if (lane == 0) status_fail(lc.status, sidx, 0, 0u, KIND_HEADER);
        return;
    }
    if (v0 >= seg.n_vectors) return;
    const uint32_t nv = min(static_cast<uint32_t>(WAVE), seg.n_vectors - v0);
    uint32_t* sw = reinterpret_cast<uint32_t*>(stage);
    global_to_lds(sw, blob + 38 + static_cast<uint64_t>(v0) * plen, nv * plen, lane);
    wave_sync();

    const bool active = static_cast<uint32_t>(lane) < nv;
    const uint32_t* pw = sw + lane * (plen >> 2);
    float r[PAIRS];
    uint32_t bins[PAIRS];
    bool ok = true;
    uint32_t w = 0;
    if (active) {
        if (lc.radii == PKV_RADII_F32) {
#pragma unroll
            for (int i = 0; i < PAIRS; ++i) {
                r[i] = u2f(pw[w++]);
                ok &= isfinite_f(r[i]) && !(r[i] < 0.0f);   // radius.rs:88-104
            }
        } else {
            uint32_t q[PAIRS / 4];
#pragma unroll
            for (int i = 0; i < PAIRS / 4; ++i) q[i] = pw[w++];
            float mn = u2f(pw[w++]), mx = u2f(pw[w++]);
            ok &= isfinite_f(mn) && isfinite_f(mx) && !(mn > mx);   // radius.rs:171-177
            float span = mx - mn;
#pragma unroll
            for (int i = 0; i < PAIRS; ++i) {
                const uint32_t u = (q[i >> 2] >> (8 * (i & 3))) & 0xffu;
                r[i] = og_expf(mn + span * div255_lds[u], exp_lds);   // radius.rs:128-145
                ok &= isfinite_f(r[i]) && !(r[i] < 0.0f);     // polar.rs:127-133
            }
        }
        uint64_t acc = 0;
        uint32_t nb = 0;
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            if (nb < pbits) { acc |= static_cast<uint64_t>(pw[w++]) << nb; nb += 32; }
            bins[i] = static_cast<uint32_t>(acc) & (levels - 1u);
            acc >>= pbits;
            nb -= pbits;
        }
        // padding of the last angle word must be zero (bitpack.rs:88-109);
        // dword-multiple angle fields have none, the check stays for safety.
        if (acc != 0) ok = false;
        if (mode && (proj & 31u)) {
            uint32_t last = pw[w + ((proj - 1) >> 5)];
            if (last >> (proj & 31u)) ok = false;
        }
    }
    wave_sync();   // payload words are in registers now

    uint32_t skip_lo = 0, skip_hi = 0;
    if (active) {
        float y[DIM];
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            y[2 * i] = r[i] * cs_lds[2 * bins[i]];
            y[2 * i + 1] = r[i] * cs_lds[2 * bins[i] + 1];
        }
        fwht<DIM>(y);
        const float scale = fwht_scale<DIM>();
        float* orow = stage + lane * PITCH;
#pragma unroll
        for (int c = 0; c < DIM; ++c) orow[c] = (y[c] * scale) * signs[c];
        if (!ok) status_fail(lc.status, sidx, 1, v0 + lane, KIND_CORRUPT);
    }
    uint64_t badmask = __ballot(active && !ok);
    skip_lo = static_cast<uint32_t>(badmask);
    skip_hi = static_cast<uint32_t>(badmask >> 32);
    wave_sync();
    stage_rows_out<DIM>(out, lc, stage, seg, v0, nv, skip_lo, skip_hi, lane);
}

// LDS words per wave of turbo_decode_split_kernel: two buffers, each the
// aligned windows of two runs of 16 payloads (the decoded rows are staged
// over the buffer just consumed, 16 rows at a time).
__host__ __device__ constexpr uint32_t turbo_split_run_words(uint32_t pwd) { return 16 * pwd + 2; }
__host__ __device__ constexpr uint32_t turbo_split_buf_words(uint32_t pwd) {
    return (2 * turbo_split_run_words(pwd) > 16 * (64 + 4)) ? 2 * turbo_split_run_words(pwd) : 16 * (64 + 4);
}
__host__ __device__ constexpr uint32_t turbo_split_wave_words(uint32_t pwd) { return 2 * turbo_split_buf_words(pwd); }

// Turbo decode at head_dim 64 (TurboQuantizer::decode, turbo.rs:302-330:
// the polar part; the QJL words are validated, not used): two lanes per
// vector as in turbo_encode_qjl_kernel, 32 vectors per wave.  A resident grid
// walks the 128-vector half-tiles, each workgroup a contiguous share, and a
// wave's payloads for the next half-tile travel to LDS by direct loads
// (global_load_lds) while it decodes and stores the current one.  Wave w of a
// half-tile takes the two runs of 16 vectors starting at 64 (w / 2) +
// 16 (w % 2) and 32 later: when a blob holds 32 heads (vector = token * H +
// head) those are 16 heads at two consecutive tokens, so each store
// instruction writes two runs of two adjacent 256 B rows (tokens t, t + 1 of
// one head).  Any other layout is only another order of the same stores.
template <int PB>
__global__ __launch_bounds__(TILE) void turbo_decode_split_kernel(
    LaunchCommon lc, const uint8_t* __restrict__ wire, void* __restrict__ out,
    const float* __restrict__ signs, const float* __restrict__ cs_tab, uint64_t seed, uint32_t pbits_rt,
    uint32_t proj, uint32_t mode) {
    constexpr int DIM = 64;
    constexpr int HP = 16;
    constexpr int PITCH = DIM + 4;
    extern __shared__ uint32_t smem_u[];   // per wave: two buffers of turbo_split_buf_words
    __shared__ float cs_lds[32];           // levels <= 16
    __shared__ uint64_t exp_lds[32];
    __shared__ float div255_lds[256];

    const uint32_t pbits = PB ? static_cast<uint32_t>(PB) : pbits_rt;
    const uint32_t levels = 1u << pbits;
    for (uint32_t t = threadIdx.x; t < 2 * levels; t += blockDim.x) cs_lds[t] = cs_tab[t];
    if (threadIdx.x < 32) exp_lds[threadIdx.x] = c_exp2f_tab[threadIdx.x];
    for (uint32_t t = threadIdx.x; t < 256; t += blockDim.x) div255_lds[t] = c_div255.v[t];
    __syncthreads();

    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int h = lane >> 5, n = lane & 31;
    const uint32_t j = static_cast<uint32_t>(n) & 15u, run = static_cast<uint32_t>(n) >> 4;
    const uint32_t plen = lc.plen, pwd = plen >> 2, winw = turbo_split_run_words(pwd);
    const uint32_t bufw = turbo_split_buf_words(pwd);
    uint32_t* wbuf = smem_u + wave * turbo_split_wave_words(pwd);
    // half-tiles vb = 2 * tile + half, a contiguous share per workgroup (a
    // grid smaller than the count is a bounded share of the GPU, so another
    // kernel can run beside it); the next half-tile's segment is the current
    // one or a later one found by stepping on
    const uint32_t nvb = 2u * lc.tile_start[lc.nseg];
    const uint32_t per = (nvb + gridDim.x - 1) / gridDim.x;
    const uint32_t vb0 = blockIdx.x * per;
    if (vb0 >= nvb) return;
    const uint32_t vb_end = min(nvb, vb0 + per);
    uint32_t sidx = segment_of(lc.tile_seg, lc.tile_start, lc.nseg, vb0 >> 1);

    // One half-tile's share of this wave: segment, the two runs, and its
    // header bytes (lanes 0-37); fetch() also starts the payload copies of
    // both runs into `dst` (run q's aligned window at dst + q * winw).
    struct Item {
        uint32_t sidx, r0, r1, n0, n1;
        uint32_t hb;
    };
    auto fetch = [&](uint32_t vb, uint32_t* dst) -> Item {
        Item it;
        const uint32_t blk = vb >> 1;
        while (sidx + 1 < lc.nseg && lc.tile_start[sidx + 1] <= blk) ++sidx;
        it.sidx = sidx;
        const SegDev seg = lc.segs[sidx];
        const uint32_t tile = blk - lc.tile_start[sidx];
        it.r0 = tile * TILE + (vb & 1u) * (TILE / 2) + 64u * static_cast<uint32_t>(wave >> 1) +
                16u * static_cast<uint32_t>(wave & 1);
        it.r1 = it.r0 + 32u;
        it.n0 = it.r0 < seg.n_vectors ? min(16u, seg.n_vectors - it.r0) : 0u;
        it.n1 = it.r1 < seg.n_vectors ? min(16u, seg.n_vectors - it.r1) : 0u;
        const uint8_t* blob = wire + seg.wire_offset;
        it.hb = lane < 38 ? blob[lane] : 0u;
        // the aligned dwords holding each run's payload bytes (the segment's
        // extent was checked on the host, so they lie in the wire buffer)
#pragma unroll
        for (uint32_t q = 0; q < 2; ++q) {
            const uint32_t cnt = q ? it.n1 : it.n0;
            if (!cnt) continue;
            const uintptr_t a = reinterpret_cast<uintptr_t>(blob + 38 + static_cast<uint64_t>(q ? it.r1 : it.r0) * plen);
            const uintptr_t a0 = a & ~static_cast<uintptr_t>(3);
            const uint32_t ndw = static_cast<uint32_t>((((a + cnt * plen + 3u) & ~static_cast<uintptr_t>(3)) - a0) >> 2);
            for (uint32_t k0 = 0; k0 < ndw; k0 += WAVE)
                if (k0 + static_cast<uint32_t>(lane) < ndw)
                    __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(a0) + k0 + lane,
                                                     dst + q * winw + k0, 4, 0, 0);
        }
        return it;
    };

    Item cur = fetch(vb0, wbuf);
    uint32_t bsel = 0;
    for (uint32_t vb = vb0; vb < vb_end; ++vb) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this half-tile's payload copies have landed
        wave_sync();
        uint32_t* buf = wbuf + bsel * bufw;
        const Item it = cur;
        if (vb + 1 < vb_end) cur = fetch(vb + 1, wbuf + (bsel ^ 1u) * bufw);
        bsel ^= 1u;
        const SegDev seg = lc.segs[it.sidx];
        // header check (every wave; 38 bytes)
        const bool hbad = lane < 38 && tqb1_checked(lane) &&
                          it.hb != tqb1_byte(lane, DIM, pbits, lc.radii, proj, seed, seg.n_vectors, plen);
        if (__ballot(hbad) != 0ull) {
            if (lane == 0) status_fail(lc.status, it.sidx, 0, 0u, KIND_HEADER);
            continue;
        }
        if (!it.n0) continue;
        const uint32_t sh = static_cast<uint32_t>((seg.wire_offset + 38u) & 3u);   // payload lengths are whole words
        const uint32_t cnt = run ? it.n1 : it.n0;
        const bool active = j < cnt;
        // lanes past a run's end repeat its last vector (run 1 empty: run 0's first)
        const uint32_t* win = buf + (cnt ? run : 0u) * winw + (cnt ? min(j, cnt - 1u) : 0u) * pwd;
        auto pword = [&](uint32_t k) -> uint32_t {
            return sh ? __builtin_amdgcn_alignbyte(win[k + 1], win[k], sh) : win[k];
        };
        const uint32_t vi = (run ? it.r1 : it.r0) + j;
        // this lane's output row offset, computed once (one division by the
        // segment's group) and handed to the storing lanes by a shuffle
        const uint64_t my_off = vec_elem_offset(seg, vi);
        const bool f32r = lc.radii == PKV_RADII_F32;
        const uint32_t rwords = f32r ? 32u : 32u / 4 + 2;
        bool ok = true;
        float r[HP];
        if (f32r) {
#pragma unroll
            for (int i = 0; i < HP; ++i) {
                r[i] = u2f(pword(16 * h + i));
                ok &= isfinite_f(r[i]) && !(r[i] < 0.0f);   // radius.rs:88-104
            }
        } else {
            const float mn = u2f(pword(8)), mx = u2f(pword(9));
            ok &= isfinite_f(mn) && isfinite_f(mx) && !(mn > mx);   // radius.rs:171-177
            const float span = mx - mn;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t q = pword(4 * h + k);
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const uint32_t u = (q >> (8 * t)) & 0xffu;
                    const int i = 4 * k + t;
                    r[i] = og_expf(mn + span * div255_lds[u], exp_lds);   // radius.rs:128-145
                    ok &= isfinite_f(r[i]) && !(r[i] < 0.0f);             // polar.rs:127-133
                }
            }
        }
        // this half's 16 angle indices: bits 16 pbits h .. (pbits <= 4: <= 64 bits)
        const uint32_t bit0 = 16u * pbits * static_cast<uint32_t>(h);
        const uint32_t aw0 = rwords + (bit0 >> 5);
        const uint32_t ash = bit0 & 31u;
        const uint64_t lo64 = static_cast<uint64_t>(pword(aw0)) | static_cast<uint64_t>(pword(aw0 + 1)) << 32;
        uint64_t pk = lo64 >> ash;
        if (ash) pk |= static_cast<uint64_t>(pword(aw0 + 2)) << (64 - ash);
        // the angle field is 32 * pbits bits, a whole number of words: no padding
        // bits to check (bitpack.rs:88-109); nor in the 32/64-bit QJL field
        (void)mode;

        float y[32];
#pragma unroll
        for (int i = 0; i < HP; ++i) {
            const uint32_t bin = static_cast<uint32_t>(pk >> (static_cast<uint32_t>(i) * pbits)) & (levels - 1u);
            y[2 * i] = r[i] * cs_lds[2 * bin];
            y[2 * i + 1] = r[i] * cs_lds[2 * bin + 1];
        }
        fwht_split(y, h);
        const float scale = fwht_scale<DIM>();
        const bool vok = ok && partner(ok ? 1u : 0u, h);
        if (active && h == 0 && !vok) status_fail(lc.status, it.sidx, 1, vi, KIND_CORRUPT);
        // rows to write: the active, good vectors (lane n's vector: run n / 16, j)
        const uint32_t wmask = static_cast<uint32_t>(__ballot(active && h == 0 && vok));
        // Rows leave through LDS (staged over the consumed payload buffer), 16
        // at a time: pass p stages the vectors j = 8p .. 8p + 7 of both runs
        // (row (j % 8) + 8 run), and store k writes rows 2k, 2k + 8 (one head,
        // tokens t and t + 1: lanes 0-31) and 2k + 1, 2k + 9 (the next head:
        // lanes 32-63).
        float* stage = reinterpret_cast<float*>(buf);
        const uint32_t sel = static_cast<uint32_t>(lane) >> 4, c = static_cast<uint32_t>(lane) & 15u;
#pragma unroll
        for (uint32_t pass = 0; pass < 2; ++pass) {
            wave_sync();   // payload words / the previous pass's rows are no longer read
            if ((j >> 3) == pass) {
                float* srow = stage + ((j & 7u) + 8u * run) * PITCH + 32 * h;
                const float4* sp = reinterpret_cast<const float4*>(signs + 32 * h);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float4 sg = sp[k];
                    *reinterpret_cast<float4*>(srow + 4 * k) =
                        make_float4((y[4 * k] * scale) * sg.x, (y[4 * k + 1] * scale) * sg.y,
                                    (y[4 * k + 2] * scale) * sg.z, (y[4 * k + 3] * scale) * sg.w);
                }
            }
            wave_sync();
#pragma unroll
            for (uint32_t k = 0; k < 4; ++k) {
                const uint32_t row = 2u * k + (sel >> 1) + 8u * (sel & 1u);
                const uint32_t src = 8u * pass + (row & 7u) + 16u * (row >> 3);   // the lane of the row's vector
                const uint64_t off = shfl_u64(my_off, static_cast<int>(src));
                if ((wmask >> src) & 1u)   // whole rows per instruction: streaming stores (the L2 stays with
                                           // the pool encode that runs beside this decode in a rehydrate step)
                    store_out4<true>(out, lc, off + 4 * c,
                                     *reinterpret_cast<const float4*>(stage + row * PITCH + 4 * c));
            }
        }
    }
}

// Turbo decode at head_dim 128: four lanes per vector as in
// turbo_encode_qjl128_kernel, one 16-vector group per wave, four workgroups
// per tile; rows leave through LDS, 512 B contiguous per row.
__host__ __device__ constexpr uint32_t turbo_split128_wave_words(uint32_t pwd) {
    return (16 * pwd + 4 > 16 * (128 + 4) + 4) ? 16 * pwd + 4 : 16 * (128 + 4) + 4;
}

template <int PB>
__global__ __launch_bounds__(TILE) void turbo_decode_split128_kernel(
    LaunchCommon lc, const uint8_t* __restrict__ wire, void* __restrict__ out,
    const float* __restrict__ signs, const float* __restrict__ cs_tab, uint64_t seed, uint32_t pbits_rt,
    uint32_t proj) {
    constexpr int DIM = 128;
    constexpr int HP = 16;
    constexpr int GV = 16;
    extern __shared__ uint32_t smem_u[];   // per wave: 16 payloads, then 16 decoded rows
    __shared__ float cs_lds[512];
    __shared__ uint64_t exp_lds[32];
    __shared__ float div255_lds[256];

    const uint32_t pbits = PB ? static_cast<uint32_t>(PB) : pbits_rt;
    const uint32_t levels = 1u << pbits;
    for (uint32_t t = threadIdx.x; t < 2 * levels; t += blockDim.x) cs_lds[t] = cs_tab[t];
    if (threadIdx.x < 32) exp_lds[threadIdx.x] = c_exp2f_tab[threadIdx.x];
    for (uint32_t t = threadIdx.x; t < 256; t += blockDim.x) div255_lds[t] = c_div255.v[t];
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int q = lane >> 4, n = lane & 15;
    const uint32_t blk = blockIdx.x >> 2;
    const uint32_t sidx = segment_of(lc.tile_seg, lc.tile_start, lc.nseg, blk);
    const SegDev seg = lc.segs[sidx];
    const uint32_t tile = blk - lc.tile_start[sidx];
    const uint32_t plen = lc.plen, pwd = plen >> 2;
    const uint8_t* blob = wire + seg.wire_offset;

    // header check (every wave; 38 bytes)
    const uint32_t hb = lane < 38 ? blob[lane] : 0u;
    const bool hbad = lane < 38 && tqb1_checked(lane) &&
                      hb != tqb1_byte(lane, DIM, pbits, lc.radii, proj, seed, seg.n_vectors, plen);
    if (__ballot(hbad) != 0ull) {
        if (lane == 0) status_fail(lc.status, sidx, 0, 0u, KIND_HEADER);
        return;
    }
    const uint32_t t0 = tile * TILE + (blockIdx.x & 3u) * (TILE / 4) + GV * static_cast<uint32_t>(wave);
    if (t0 >= seg.n_vectors) return;
    const uint32_t nv = min(static_cast<uint32_t>(GV), seg.n_vectors - t0);
    uint32_t* sw = smem_u + wave * turbo_split128_wave_words(pwd);
    global_to_lds(sw, blob + 38 + static_cast<uint64_t>(t0) * plen, nv * plen, lane);
    wave_sync();

    const bool active = static_cast<uint32_t>(n) < nv;
    const uint32_t* pw = sw + min(static_cast<uint32_t>(n), nv - 1) * pwd;
    const bool f32r = lc.radii == PKV_RADII_F32;
    const uint32_t rwords = f32r ? 64u : 64u / 4 + 2;
    bool ok = true;
    float r[HP];
    if (f32r) {
#pragma unroll
        for (int i = 0; i < HP; ++i) {
            r[i] = u2f(pw[16 * q + i]);
            ok &= isfinite_f(r[i]) && !(r[i] < 0.0f);   // radius.rs:88-104
        }
    } else {
        const float mn = u2f(pw[16]), mx = u2f(pw[17]);
        ok &= isfinite_f(mn) && isfinite_f(mx) && !(mn > mx);   // radius.rs:171-177
        const float span = mx - mn;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t w = pw[4 * q + k];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint32_t u = (w >> (8 * t)) & 0xffu;
                const int i = 4 * k + t;
                r[i] = og_expf(mn + span * div255_lds[u], exp_lds);   // radius.rs:128-145
                ok &= isfinite_f(r[i]) && !(r[i] < 0.0f);             // polar.rs:127-133
            }
        }
    }
    // this quarter's 16 angle indices: bits 16 pbits q .. (pbits <= 4: <= 64 bits)
    const uint32_t bit0 = 16u * pbits * static_cast<uint32_t>(q);
    const uint32_t* aw = pw + rwords + (bit0 >> 5);
    const uint32_t sh = bit0 & 31u;
    const uint64_t lo64 = static_cast<uint64_t>(aw[0]) | static_cast<uint64_t>(aw[1]) << 32;
    uint64_t pk = lo64 >> sh;
    if (sh) pk |= static_cast<uint64_t>(aw[2]) << (64 - sh);
    // the angle field is 64 * pbits bits, a whole number of words: no padding
    // bits to check (bitpack.rs:88-109); nor in the 32/64-bit QJL field

    float y[32];
#pragma unroll
    for (int i = 0; i < HP; ++i) {
        const uint32_t bin = static_cast<uint32_t>(pk >> (static_cast<uint32_t>(i) * pbits)) & (levels - 1u);
        y[2 * i] = r[i] * cs_lds[2 * bin];
        y[2 * i + 1] = r[i] * cs_lds[2 * bin + 1];
    }
    fwht_quarter(y, q);
    const float scale = fwht_scale<DIM>();
    const bool vok = or_quarters(ok ? 0u : 1u, q) == 0u;
    if (active && q == 0 && !vok) status_fail(lc.status, sidx, 1, t0 + n, KIND_CORRUPT);
    // rows through LDS (over the consumed payloads) so they leave coalesced
    wave_sync();
    float* stage = reinterpret_cast<float*>(sw);
    {
        float* srow = stage + n * (DIM + 4) + 32 * q;
        const float4* sp = reinterpret_cast<const float4*>(signs + 32 * q);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float4 sg = sp[k];
            *reinterpret_cast<float4*>(srow + 4 * k) =
                make_float4((y[4 * k] * scale) * sg.x, (y[4 * k + 1] * scale) * sg.y, (y[4 * k + 2] * scale) * sg.z,
                            (y[4 * k + 3] * scale) * sg.w);
        }
    }
    const uint64_t badm = __ballot(active && q == 0 && !vok);
    wave_sync();
    stage_rows_out<DIM>(out, lc, stage, seg, t0, nv, static_cast<uint32_t>(badm), 0u, lane);
}

// ------------------------------------------------------------ scoring on codes
// TurboQuantizer::prepare_query (turbo-quant/src/turbo.rs:322-338) for nq
// queries, one wave per query: [R q (DIM)][G q (proj, QJL only)], with
//   R q = FastHadamardRotation::apply (rotation.rs:202-211): q * signs, the
//         in-place butterflies of fwht_normalized (rotation.rs:379-398) in
//         stage order, then * (1 / sqrt(DIM)); each butterfly is one f32 add
//         or subtract of the same two operands as the sequential loop, so
//         spreading a stage across lanes changes no bit;
//   G q = QjlQuantizer::project_query (qjl.rs:266-282): per projection j a
//         sequential f32 fold of G[j][c] * q[c] from -0.0, the neutral element
//         of Rust's f32 Sum (an all-zero sum keeps the sign of its terms).
// A query with a non-finite input, rotated or projected value marks status
// word 0 of segment 0 with its index (turbo.rs:330, polar.rs:341, qjl.rs:280).
template <int DIM>
__global__ __launch_bounds__(WAVE) void turbo_prepare_kernel(const float* __restrict__ q, uint32_t nq,
                                                             float* __restrict__ out, const float* __restrict__ signs,
                                                             const float* __restrict__ G, uint32_t proj,
                                                             uint32_t mode, float rscale, uint32_t* status) {
    __shared__ float v[DIM];
    __shared__ float raw[DIM];
    const uint32_t qi = blockIdx.x, lane = threadIdx.x;
    if (qi >= nq) return;
    const float* src = q + static_cast<uint64_t>(qi) * DIM;
    const uint32_t W = DIM + (mode ? proj : 0u);
    float* dst = out + static_cast<uint64_t>(qi) * W;
    bool bad = false;
#pragma unroll
    for (int c = lane; c < DIM; c += WAVE) {
        const float x = src[c];
        raw[c] = x;
        v[c] = x * signs[c];
        bad |= !isfinite_f(x);
    }
    wave_sync();
#pragma unroll
    for (int step = 1; step < DIM; step *= 2) {
#pragma unroll
        for (int bf = lane; bf < DIM / 2; bf += WAVE) {
            const int i = (bf / step) * 2 * step + bf % step, j = i + step;
            const float a = v[i], b = v[j];
            v[i] = a + b;
            v[j] = a - b;
        }
        wave_sync();
    }
#pragma unroll
    for (int c = lane; c < DIM; c += WAVE) {
        const float y = v[c] * rscale;
        dst[c] = y;
        bad |= !isfinite_f(y);
    }
    if (mode) {
        for (uint32_t j = lane; j < proj; j += WAVE) {
            const float* g = G + static_cast<uint64_t>(j) * DIM;
            float acc = -0.0f;
#pragma unroll 16
            for (int c = 0; c < DIM; ++c) acc = acc + g[c] * raw[c];
            dst[DIM + j] = acc;
            bad |= !isfinite_f(acc);
        }
    }
    if (__ballot(bad) != 0ull && lane == 0 && status) status_fail(status, 0, 0, qi, KIND_NONFINITE_INPUT);
}

// TurboQuantizer::inner_product_estimate_prepared (turbo.rs:341-369) of every
// code of every segment against nq prepared queries:
//   polar = sum over pairs i of r_i * (qa_i * cos(theta_i) + qb_i * sin(theta_i))
//           (PolarQuantizer::inner_product_estimate_with_projected_query,
//           polar.rs:346-370: a sequential f32 loop from +0.0)
//   qjl   = scale * sum_j s_j * (G q)_j, s_j = +1 for a set sign bit, -1
//           otherwise, a fold from -0.0, scale = sqrt(PI / 2) * 1 / m
//           (qjl.rs:294-330 with unit source norm)
//   score = polar + qjl, then * post (AttentionScale of
//           KvShadowCache::attention_scores_with_options, kv.rs:277-320:
//           applied after the finiteness check; post = 1 leaves it unchanged).
// One lane per code: its radii, its sign factors (+-1.0, folded in with an
// FMA whose product is exact, so each step rounds like the reference's add)
// and, at head_dim 64, the (cos, sin) of its angle bins stay in registers
// (head_dim 128 keeps the bins as LDS byte offsets into the (cos, sin) table)
// while the wave walks the queries, whose values are uniform across lanes
// and arrive as scalar loads.  A code the decoder rejects (header, radius
// checks, as decode_batch at wire.rs:401-568) marks status word 0 and gets no
// score; a non-finite score marks word 1 (polar.rs:364, qjl.rs:324,
// turbo.rs:362).  scores[q * ld + col], col = the segment's strided position
// of the code (elem_offset + (i / group) * stride_outer + (i % group) *
// stride_inner, in score units).  Segment s reads prepared rows
// s * qstride .. s * qstride + nq - 1 (qstride 0: every segment scores the
// same queries).  PROJ: 0 (PolarOnly), 32 or 64.
template <int DIM, int PROJ, bool LOSSY, bool NARROW>
__global__ __launch_bounds__(TILE) void turbo_score_kernel(
    LaunchCommon lc, const uint8_t* __restrict__ wire, const float* __restrict__ prepared, uint32_t nq,
    uint64_t qstride, float* __restrict__ scores, uint64_t ld, const float* __restrict__ cs_tab, uint64_t seed,
    uint32_t pbits, uint32_t hproj, float qscale, float post) {
    constexpr int PAIRS = DIM / 2;
    constexpr bool HOIST = DIM == 64;     // (cos, sin) per pair in registers
    constexpr int OB = NARROW ? 8 : 16;   // bits per LDS byte offset (8 when 8 * (levels - 1) < 256)
    constexpr int OPW = 32 / OB;
    constexpr int W = DIM + PROJ;
    extern __shared__ uint32_t smem_u[];  // per wave: 64 payloads
    __shared__ float2 cs_lds[256];
    __shared__ uint64_t exp_lds[32];
    __shared__ float div255_lds[256];

    const uint32_t levels = 1u << pbits;
    for (uint32_t t = threadIdx.x; t < levels; t += blockDim.x)
        cs_lds[t] = make_float2(cs_tab[2 * t], cs_tab[2 * t + 1]);
    if (threadIdx.x < 32) exp_lds[threadIdx.x] = c_exp2f_tab[threadIdx.x];
    for (uint32_t t = threadIdx.x; t < 256; t += blockDim.x) div255_lds[t] = c_div255.v[t];
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t blk = blockIdx.x;
    const uint32_t sidx = segment_of(lc.tile_seg, lc.tile_start, lc.nseg, blk);
    const SegDev seg = lc.segs[sidx];
    const uint32_t tile = blk - lc.tile_start[sidx];
    const uint32_t plen = lc.plen, pwd = plen >> 2;
    const uint8_t* blob = wire + seg.wire_offset;
    const uint32_t hb = lane < 38 ? blob[lane] : 0u;
    const bool hbad = lane < 38 && tqb1_checked(lane) &&
                      hb != tqb1_byte(lane, DIM, pbits, lc.radii, hproj, seed, seg.n_vectors, plen);
    if (__ballot(hbad) != 0ull) {
        if (lane == 0) status_fail(lc.status, sidx, 0, 0u, KIND_HEADER);
        return;
    }
    const uint32_t v0 = tile * TILE + static_cast<uint32_t>(wave) * WAVE;
    if (v0 >= seg.n_vectors) return;
    const uint32_t nv = min(static_cast<uint32_t>(WAVE), seg.n_vectors - v0);
    uint32_t* sw = smem_u + wave * (WAVE * pwd + 4);
    global_to_lds(sw, blob + 38 + static_cast<uint64_t>(v0) * plen, nv * plen, lane);
    wave_sync();
    const bool active = static_cast<uint32_t>(lane) < nv;
    const uint32_t* pw = sw + min(static_cast<uint32_t>(lane), nv - 1) * pwd;

    // radii: f32 or BlockLogU8 through expf, with the decoder's checks
    // (radius.rs:88-104, 128-145, 171-177; polar.rs:127-133)
    float r[PAIRS];
    bool ok = true;
    uint32_t w = 0;
    if constexpr (!LOSSY) {
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            r[i] = u2f(pw[w++]);
            ok &= isfinite_f(r[i]) && !(r[i] < 0.0f);
        }
    } else {
        constexpr int QW = PAIRS / 4;
        const float mn = u2f(pw[QW]), mx = u2f(pw[QW + 1]);
        ok &= isfinite_f(mn) && isfinite_f(mx) && !(mn > mx);
        const float span = mx - mn;
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            const uint32_t u = (pw[i >> 2] >> (8 * (i & 3))) & 0xffu;
            r[i] = og_expf(mn + span * div255_lds[u], exp_lds);
            ok &= isfinite_f(r[i]) && !(r[i] < 0.0f);
        }
        w = QW + 2;
    }
    // angle bins, pbits each, LSB-first; PAIRS * pbits is a whole number of
    // words for every accepted profile, so there is no padding to check
    const uint32_t* aw = pw + w;
    float cs[HOIST ? DIM : 1];
    uint32_t boff[HOIST ? 1 : PAIRS / OPW];   // byte offsets into cs_lds, OB bits each
    {
        uint64_t acc = 0;
        uint32_t nb = 0, k = 0;
#pragma unroll
        for (int i = 0; i < (HOIST ? 1 : PAIRS / OPW); ++i) boff[i] = 0u;
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            if (nb < pbits) { acc |= static_cast<uint64_t>(aw[k++]) << nb; nb += 32; }
            const uint32_t b = static_cast<uint32_t>(acc) & (levels - 1u);
            acc >>= pbits;
            nb -= pbits;
            if constexpr (HOIST) {
                const float2 c = cs_lds[b];
                cs[2 * i] = c.x;
                cs[2 * i + 1] = c.y;
            } else {
                boff[i / OPW] |= (b * 8u) << (OB * (i % OPW));
            }
        }
    }
    const uint32_t* sgw = aw + (PAIRS * pbits + 31) / 32;
    float sg[PROJ ? PROJ : 1];
#pragma unroll
    for (int j = 0; j < PROJ; ++j) sg[j] = ((sgw[j >> 5] >> (j & 31)) & 1u) ? 1.0f : -1.0f;
    if (active && !ok) status_fail(lc.status, sidx, 0, v0 + lane, KIND_CORRUPT);
    const uint64_t col = vec_elem_offset(seg, v0 + min(static_cast<uint32_t>(lane), nv - 1));
    const bool store = active && ok;
    const char* csb = reinterpret_cast<const char*>(cs_lds);
    bool fin = true;
    const float* pseg = prepared + static_cast<uint64_t>(sidx) * qstride * W;
    for (uint32_t q = 0; q < nq; ++q) {
        const float* pq = pseg + static_cast<uint64_t>(q) * W;
        float est = 0.0f;
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            float c, sn;
            if constexpr (HOIST) {
                c = cs[2 * i];
                sn = cs[2 * i + 1];
            } else {
                const float2 t =
                    *reinterpret_cast<const float2*>(csb + ((boff[i / OPW] >> (OB * (i % OPW))) & ((1u << OB) - 1u)));
                c = t.x;
                sn = t.y;
            }
            est = est + r[i] * (pq[2 * i] * c + pq[2 * i + 1] * sn);
        }
        bool f = isfinite_f(est);
        float total = est;
        if constexpr (PROJ != 0) {
            float e2 = -0.0f;
#pragma unroll
            for (int j = 0; j < PROJ; ++j) e2 = __builtin_fmaf(sg[j], pq[DIM + j], e2);
            const float qj = qscale * e2;
            f &= isfinite_f(qj);
            total = est + qj;
        }
        f &= isfinite_f(total);
        fin &= f;
        if (store) scores[static_cast<uint64_t>(q) * ld + col] = total * post;
    }
    if (store && !fin) status_fail(lc.status, sidx, 1, v0 + lane, KIND_SCORE_NONFINITE);
}

// The same scores for profiles with at most 16 angle bins (pbits <= 4), with
// the per-pair term looked up instead of recomputed: for a chunk of up to
// four queries the block first tabulates, in LDS,
//   T[q][i][b] = qa_i * cos(theta_b) + qb_i * sin(theta_b)
// -- the parenthesised sum of polar.rs:361, the same two products and add --
// so each (code, query, pair) costs one LDS read, a multiply by r_i and the
// sequential add: est = est + r_i * T[q][i][bin_i], bit for bit the
// reference's expression.  Payloads are staged through LDS 32 lanes at a
// time (raw words into registers), and the staging space is then reused for
// the table, which keeps four workgroups per CU at head_dim 128.
template <int DIM, int PROJ, bool LOSSY, int PB>
__global__ __launch_bounds__(TILE) __attribute__((amdgpu_waves_per_eu(DIM == 128 && PROJ ? 3 : 4))) void
turbo_score_lut_kernel(
    LaunchCommon lc, const uint8_t* __restrict__ wire, const float* __restrict__ prepared, uint32_t nq,
    uint64_t qstride, float* __restrict__ scores, uint64_t ld, const float* __restrict__ cs_tab, uint64_t seed,
    uint32_t hproj, float qscale, float post) {
    constexpr uint32_t pbits = PB;
    constexpr int PAIRS = DIM / 2;
    constexpr int LUTQ = PAIRS * 16;             // floats per query: [pair][bin]
    constexpr int W = DIM + PROJ;
    constexpr int RW = LOSSY ? PAIRS / 4 + 2 : PAIRS;   // radii words
    constexpr int AWMAX = (PAIRS * PB + 31) / 32;       // angle words
    constexpr int SW = PROJ / 32;                       // sign words
    extern __shared__ uint32_t smem_u[];
    __shared__ float2 cs_lds[16];
    __shared__ uint64_t exp_lds[32];
    __shared__ float div255_lds[256];

    constexpr uint32_t levels = 1u << pbits;
    if (threadIdx.x < 16)
        cs_lds[threadIdx.x] = threadIdx.x < levels ? make_float2(cs_tab[2 * threadIdx.x], cs_tab[2 * threadIdx.x + 1])
                                                   : make_float2(0.0f, 0.0f);
    if (threadIdx.x < 32) exp_lds[threadIdx.x] = c_exp2f_tab[threadIdx.x];
    if (LOSSY)
        for (uint32_t t = threadIdx.x; t < 256; t += blockDim.x) div255_lds[t] = c_div255.v[t];
    __syncthreads();   // the tables are read by every wave (radii below, the (cos, sin) terms later)

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t blk = blockIdx.x;
    const uint32_t sidx = segment_of(lc.tile_seg, lc.tile_start, lc.nseg, blk);
    const SegDev seg = lc.segs[sidx];
    const uint32_t tile = blk - lc.tile_start[sidx];
    const uint32_t plen = lc.plen, pwd = plen >> 2;
    const uint8_t* blob = wire + seg.wire_offset;
    const uint32_t hb = lane < 38 ? blob[lane] : 0u;   // checked once the payloads are staged
    const uint32_t v0 = tile * TILE + static_cast<uint32_t>(wave) * WAVE;
    const uint32_t nv = v0 < seg.n_vectors ? min(static_cast<uint32_t>(WAVE), seg.n_vectors - v0) : 0u;
    const bool active = static_cast<uint32_t>(lane) < nv;

    // raw payload words, 32 lanes per round through this wave's staging area
    uint32_t rw[RW], aw[AWMAX], sgw[SW ? SW : 1];
    {
        uint32_t* sw = smem_u + wave * (32 * pwd + 4);
        constexpr uint32_t nwa = AWMAX;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const uint32_t h0 = 32u * half;
            const uint32_t hn = nv > h0 ? min(32u, nv - h0) : 0u;
            if (hn) global_to_lds<16>(sw, blob + 38 + static_cast<uint64_t>(v0 + h0) * plen, hn * plen, lane);
            wave_sync();
            if ((lane >> 5) == half) {
                const uint32_t* pw = sw + min(static_cast<uint32_t>(lane & 31), hn ? hn - 1 : 0u) * pwd;
#pragma unroll
                for (int k = 0; k < RW; ++k) rw[k] = pw[k];
#pragma unroll
                for (int k = 0; k < AWMAX; ++k) aw[k] = pw[RW + k];
#pragma unroll
                for (int k = 0; k < SW; ++k) sgw[k] = pw[RW + nwa + k];
            }
            wave_sync();
        }
    }
    const bool hbad = lane < 38 && tqb1_checked(lane) &&
                      hb != tqb1_byte(lane, DIM, pbits, lc.radii, hproj, seed, seg.n_vectors, plen);
    if (__ballot(hbad) != 0ull) {   // the same header for every wave of the block: all leave
        if (lane == 0 && wave == 0) status_fail(lc.status, sidx, 0, 0u, KIND_HEADER);
        return;
    }
    // radii with the decoder's checks (radius.rs:88-104, 128-145, 171-177; polar.rs:127-133)
    float r[PAIRS];
    bool ok = true;
    if constexpr (!LOSSY) {
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            r[i] = u2f(rw[i]);
            ok &= isfinite_f(r[i]) && !(r[i] < 0.0f);
        }
    } else {
        const float mn = u2f(rw[PAIRS / 4]), mx = u2f(rw[PAIRS / 4 + 1]);
        ok &= isfinite_f(mn) && isfinite_f(mx) && !(mn > mx);
        const float span = mx - mn;
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            const uint32_t u = (rw[i >> 2] >> (8 * (i & 3))) & 0xffu;
            r[i] = og_expf(mn + span * div255_lds[u], exp_lds);
            ok &= isfinite_f(r[i]) && !(r[i] < 0.0f);
        }
    }
    // byte offsets bin * 4 of every pair, four per word
    uint32_t boff[PAIRS / 4];
#pragma unroll
    for (int i = 0; i < PAIRS / 4; ++i) boff[i] = 0u;
#pragma unroll
    for (int i = 0; i < PAIRS; ++i) {
        constexpr uint32_t M = levels - 1u;
        const int bit = i * PB, wd = bit >> 5, sh = bit & 31;
        uint32_t b = aw[wd] >> sh;
        if (sh + PB > 32) b |= aw[wd + 1] << (32 - sh);
        boff[i >> 2] |= ((b & M) * 4u) << (8 * (i & 3));
    }
    // sketch signs as f16 +-1.0, two per register, folded in by a mixed FMA
    // whose product (+-1 times p) is exact: e2 + s_j * p_j rounds once, as the
    // reference's add of sign as f32 * p (qjl.rs:316-321)
    uint32_t sgh[PROJ ? PROJ / 2 : 1];
#pragma unroll
    for (int j2 = 0; j2 < PROJ / 2; ++j2) {
        const uint32_t w = sgw[(2 * j2) >> 5] >> ((2 * j2) & 31);
        sgh[j2] = ((w & 1u) ? 0x3c00u : 0xbc00u) | (((w & 2u) ? 0x3c00u : 0xbc00u) << 16);
    }
    if (active && !ok) status_fail(lc.status, sidx, 0, v0 + lane, KIND_CORRUPT);
    const uint64_t col = vec_elem_offset(seg, v0 + min(static_cast<uint32_t>(lane), nv ? nv - 1 : 0u));
    const bool store = active && ok;
    const float* pseg = prepared + static_cast<uint64_t>(sidx) * qstride * W;
    float* lut = reinterpret_cast<float*>(smem_u);
    constexpr int PER = LUTQ / TILE;   // table entries per thread and query
    static_assert(LUTQ % TILE == 0, "table fill");
    float qa[PER], qb[PER];           // the next query's rotated pairs this thread tabulates
    auto fetch = [&](uint32_t q) {
        const float* pq = pseg + static_cast<uint64_t>(q) * W;
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const uint32_t i = (threadIdx.x + k * TILE) / 16;
            qa[k] = pq[2 * i];
            qb[k] = pq[2 * i + 1];
        }
    };
    if (nq) fetch(0);
    bool fin = true;
    for (uint32_t q = 0; q < nq; ++q) {
        __syncthreads();   // staging / the previous query's table is no longer read
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const uint32_t e = threadIdx.x + k * TILE;
            const float2 c = cs_lds[e % 16];
            lut[e] = qa[k] * c.x + qb[k] * c.y;
        }
        __syncthreads();
        if (q + 1 < nq) fetch(q + 1);   // in flight while this query is scored
        // keep the per-pair offsets and the signs packed: unpacked per query, not hoisted
        // out of the loop into one register each
#pragma unroll
        for (int k = 0; k < PAIRS / 4; ++k) asm volatile("" : "+v"(boff[k]));
#pragma unroll
        for (int k = 0; k < (PROJ ? PROJ / 2 : 1); ++k) asm volatile("" : "+v"(sgh[k]));
        const char* lb = reinterpret_cast<const char*>(lut);
        auto tab = [&](int i) {
            const uint32_t off = (boff[i >> 2] >> (8 * (i & 3))) & 0xffu;
            return *reinterpret_cast<const float*>(lb + off + 4 * (i * 16));
        };
        constexpr int DEPTH = 4;   // table reads in flight ahead of the sequential sum
        float ring[DEPTH];
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) ring[k] = tab(k);
        float est = 0.0f;
#pragma unroll
        for (int i = 0; i < PAIRS; ++i) {
            const float t = ring[i % DEPTH];
            if (i + DEPTH < PAIRS) ring[i % DEPTH] = tab(i + DEPTH);
            est = est + r[i] * t;
        }
        bool f = isfinite_f(est);
        float total = est;
        if constexpr (PROJ != 0) {
            const float* pq = pseg + static_cast<uint64_t>(q) * W;
            float e2 = -0.0f;
#pragma unroll
            for (int j = 0; j < PROJ; ++j) {
                const _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(sgh[j >> 1] >> (16 * (j & 1))));
                e2 = __builtin_fmaf(static_cast<float>(h), pq[DIM + j], e2);
            }
            const float qj = qscale * e2;
            f &= isfinite_f(qj);
            total = est + qj;
        }
        f &= isfinite_f(total);
        fin &= f;
        if (store) scores[static_cast<uint64_t>(q) * ld + col] = total * post;
    }
    if (store && !fin) status_fail(lc.status, sidx, 1, v0 + lane, KIND_SCORE_NONFINITE);
}

// ------------------------------------------------------------ fib encode
// FibQuantizer::encode_batch (fib-quant/src/codec.rs:578-729; n < 4 takes
// FibQuantizer::encode, 471-516) + FibCodeV1::encode_batch (FB2, 225-320).
//
// The reference computes rho = f32(Pi x_hat) with sequential f64 rows and
// then, per 4-block, an exact f32 argmin over 32 codewords.  Only the argmin
// reaches the wire, so the main kernel decides it on the matrix cores from
// approximations and proves every decision:
//   rho'  = Pi x_hat' by v_mfma_f32_32x32x16_f16 on f16 hi/lo halves
//           (hi*hi + hi*lo + lo*hi, f32 accumulation): per wave 64 rows x 32
//           vectors.  The rows of Pi are permuted (fib_mfma_row) so that the
//           accumulator layout is already what the scoring step needs: lane
//           (h, n) holds rho'[4b + 2m + h] of vector n in register
//           2(b % 8) + m of row tile b / 8.
//   key_w = bits(|c_w|^2 + off - 2 c_w . rho') for the 32 codewords of one
//           block: one more 32x32x16 f16 MFMA whose K holds the split
//           products and |c_w|^2 + off (times 1.0); codeword index in the 5
//           low bits; each half-wave keeps its two smallest keys and the
//           halves meet through v_permlane32_swap.
// If the second smallest key exceeds the smallest by more than `thr` (twice
// the host-derived worst-case error of a key against the reference's f32
// distance, rounded up), the smallest key's codeword is the reference's
// strict argmin.  Otherwise the vector goes to its wave's LDS list with the
// mask of its undecided blocks (a few % of vectors), and the wave redoes
// those blocks exactly once it has encoded its units (fib_redo_list): f64
// sequential rows of the exact x_hat and the AVX2-order f32 distances.  Segments of fewer than 4
// vectors and per-vector encodes (the reference's single-vector path with an
// f64 x_hat) take the same test; their undecided blocks are redone under the
// per-vector semantics.


// f16 halves of a, b by round-toward-zero: hi = (a_hi, b_hi), lo = the
// rounded remainders; a - a_hi is exact in f32 (one v_fma_mix_f32 each).
__device__ __forceinline__ uint2 split2(float a, float b) {
    const uint32_t h = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
    return make_uint2(h, __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(sub_f16<0>(a, h), sub_f16<1>(b, h))));
}

__device__ __forceinline__ uint32_t umed3(uint32_t a, uint32_t b, uint32_t c) {
    uint32_t r;
    asm("v_med3_u32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

// Elements 32h .. 32h + 31 of vector vi as 8 float4 (f32, or bf16 widened);
// all loads are issued before any use.  Returns the vector's first element.
__device__ __forceinline__ uint64_t load_half_row(float4 (&v)[8], const void* __restrict__ in, bool bf16,
                                                  const SegDev& s, uint32_t vi, int h) {
    const uint64_t row = vec_elem_offset(s, vi);
    const uint64_t off = row + 32u * static_cast<uint32_t>(h);
    if (!bf16) {
        const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(in) + off);
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = p[k];
    } else {
        const uint4* p = reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(in) + off);
        uint4 w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = p[k];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            v[2 * k] = make_float4(u2f(w[k].x << 16), u2f(w[k].x & 0xffff0000u), u2f(w[k].y << 16),
                                   u2f(w[k].y & 0xffff0000u));
            v[2 * k + 1] = make_float4(u2f(w[k].z << 16), u2f(w[k].z & 0xffff0000u), u2f(w[k].w << 16),
                                       u2f(w[k].w & 0xffff0000u));
        }
    }
    return row;
}

// Value of `x` in lane (l % 32) + 32 * from_h, for every lane l.
__device__ __forceinline__ uint32_t half_lane(uint32_t x, int from_h) {
    const auto p = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return from_h ? p[1] : p[0];
}
__device__ __forceinline__ double half_lane(double x, int from_h) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = half_lane(static_cast<uint32_t>(b), from_h);
    const uint32_t hi = half_lane(static_cast<uint32_t>(b >> 32), from_h);
    return __builtin_bit_cast(double, static_cast<uint64_t>(hi) << 32 | lo);
}

// Phase 1 of one 32-vector MFMA tile of fib_encode_kernel: norm and rotated
// components.  Lane (h, n) = (lane / 32, lane % 32) holds elements
// 32h .. 32h + 31 of vector v0 + n in x.
struct FibTileRot {
    v16f acc0, acc1;   // rho' rows, accumulator layout of row tiles 0 and 1
    double nrm;
    bool finite_all, zero;
};

__device__ __forceinline__ void fib_encode_rotate(FibTileRot& t, const float4 (&x)[8], const uint32_t* rot_lds,
                                                  int lane) {
    // l2_norm (codec.rs:1049-1057): sequential f64 sum of squares.  A square
    // of an f32 is exact in f64, so fma(d, d, s) rounds like s + d * d.
    // Half 0 sums elements 0..31, hands the partial to half 1, which adds
    // 32..63; a non-finite element makes the sum non-finite (check_finite).
    double ss = 0.0;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float e[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const double d = static_cast<double>(e[j]);
            ss = __builtin_fma(d, d, ss);
        }
    }
    ss = half_lane(ss, 0);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float e[4] = {x[k].x, x[k].y, x[k].z, x[k].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const double d = static_cast<double>(e[j]);
            ss = __builtin_fma(d, d, ss);
        }
    }
    ss = half_lane(ss, 1);
    t.nrm = __builtin_sqrt(ss);
    t.finite_all = ss == ss && ss < __builtin_inf();
    t.zero = t.finite_all && t.nrm == 0.0;
    const double safe_nrm = (t.finite_all && !t.zero) ? t.nrm : 1.0;
    const float r32 = static_cast<float>(1.0 / safe_nrm);

    // B operands: f16 halves of x_hat' elements 32h + 8q .. 32h + 8q + 7
    v4u xh[4], xl[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 u = x[2 * q], v = x[2 * q + 1];
        const uint2 s0 = split2(u.x * r32, u.y * r32), s1 = split2(u.z * r32, u.w * r32);
        const uint2 s2 = split2(v.x * r32, v.y * r32), s3 = split2(v.z * r32, v.w * r32);
        xh[q] = v4u{s0.x, s1.x, s2.x, s3.x};
        xl[q] = v4u{s0.y, s1.y, s2.y, s3.y};
    }
    const v4u* rl = reinterpret_cast<const v4u*>(rot_lds);   // [t][q][part][lane]
    v16f acc0 = {}, acc1 = {};
#pragma unroll
    for (int q = 0; q < 4; ++q) {   // small cross products first
        acc0 = mfma16(rl[((0 * 4 + q) * 2 + 0) * 64 + lane], xl[q], acc0);
        acc1 = mfma16(rl[((1 * 4 + q) * 2 + 0) * 64 + lane], xl[q], acc1);
        acc0 = mfma16(rl[((0 * 4 + q) * 2 + 1) * 64 + lane], xh[q], acc0);
        acc1 = mfma16(rl[((1 * 4 + q) * 2 + 1) * 64 + lane], xh[q], acc1);
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        acc0 = mfma16(rl[((0 * 4 + q) * 2 + 0) * 64 + lane], xh[q], acc0);
        acc1 = mfma16(rl[((1 * 4 + q) * 2 + 0) * 64 + lane], xh[q], acc1);
    }
    t.acc0 = acc0;
    t.acc1 = acc1;
}

// Phase 2 of a 32-vector tile: approximate argmin per block, norm status and
// the payload words (into LDS).  Returns the blocks of this lane's vector that
// the exact redo must decide (gap to the second key within thr), or 0 for an
// inactive lane or a rejected input.  The same test serves FibQuantizer::
// encode semantics (segments of fewer than 4 vectors, per-vector calls): thr
// bounds the keys against the exact rho = Pi (x / |x|) plus the reference's
// own roundings, and those are smaller there (x / |x| stays f64; only rho's
// cast to f32 remains), so only the undecided blocks go to the redo, which
// follows the per-vector semantics.
// DIAG: also write every block's 32 approximate keys (before the index bits
// replace their low 5 bits) to lc.diag[(vector * 16 + block) * 32 + w].
template <int DIM, bool DIAG>
__device__ __forceinline__ uint32_t fib_encode_score(const LaunchCommon& lc, const SegDev& seg, uint32_t sidx,
                                                     uint32_t v0, const FibTileRot& t, uint32_t* pay, const v4u& sa,
                                                     float thr, int lane) {
    const int h = lane >> 5, n = lane & 31;
    const uint32_t nv = min(32u, seg.n_vectors - v0);
    const bool active = static_cast<uint32_t>(n) < nv;   // other lanes repeat the last vector
    const v16f& acc0 = t.acc0;
    const v16f& acc1 = t.acc1;
    const double nrm = t.nrm;
    const bool finite_all = t.finite_all, zero = t.zero;

    // Both decisions are shifted in by v_alignbit, one instruction per block:
    // the 5-bit indices from the top (blocks 0..5 in ra, 6..7 in ra2, 8..13 in
    // rb, 14..15 in rb2; the newest block highest) and the acceptance bits from
    // the bottom (da, db: bit 0 the newest block, set when thr - gap < 0, which
    // is gap > thr exactly: a difference's sign is never lost to rounding)
    uint32_t ra = 0, ra2 = 0, rb = 0, rb2 = 0, da = 0, db = 0;
    const v16f zero16 = {};
#pragma unroll
    for (int i = 0; i < 8; ++i) {   // blocks i (row tile 0) and i + 8 (row tile 1)
        // B: (p0 hi, p1 hi), (p0 lo, p1 lo), (p0 hi, p1 hi), (1, 1) with
        // p0 = rho'[4b + h], p1 = rho'[4b + 2 + h]
        const uint2 qa = split2(acc0[2 * i], acc0[2 * i + 1]), qb = split2(acc1[2 * i], acc1[2 * i + 1]);
        // (built by a shuffle: the tuples then take the split results in place, one copy each)
        const v2u one2 = {0x3C003C00u, 0x3C003C00u};
        const v4u ba = __builtin_shufflevector(v2u{qa.x, qa.y}, one2, 0, 1, 0, 2);
        const v4u bb = __builtin_shufflevector(v2u{qb.x, qb.y}, one2, 0, 1, 0, 2);
        const v16f d0 = mfma16(sa, ba, zero16);
        const v16f d1 = mfma16(sa, bb, zero16);
        if constexpr (DIAG) {
            if (active) {
                float* dv = lc.diag + static_cast<uint64_t>(v0 + static_cast<uint32_t>(n)) * 512u;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int w = 8 * (r >> 2) + 4 * h + (r & 3);
                    dv[32 * i + w] = d0[r];
                    dv[32 * (i + 8) + w] = d1[r];
                }
            }
        }
        // keys of accumulator rows w = 8(r/4) + 4h + r%4; two smallest per
        // half-wave, two keys per step: m2 = min(m2, med3(m1, k, k')),
        // m1 = min3(m1, k, k') (m1 <= m2 throughout)
        uint32_t a1 = 0xFFFFFFFFu, a2 = 0xFFFFFFFFu, b1 = 0xFFFFFFFFu, b2 = 0xFFFFFFFFu;
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            const uint32_t w0 = static_cast<uint32_t>(8 * (r >> 2) + (r & 3)), w1 = w0 + 1;
            const uint32_t ka = (f2u(d0[r]) & ~31u) | w0, kA = (f2u(d0[r + 1]) & ~31u) | w1;
            const uint32_t kb = (f2u(d1[r]) & ~31u) | w0, kB = (f2u(d1[r + 1]) & ~31u) | w1;
            a2 = min(a2, umed3(a1, ka, kA));
            a1 = min(a1, min(ka, kA));
            b2 = min(b2, umed3(b1, kb, kB));
            b1 = min(b1, min(kb, kB));
        }
        // merge the halves for the owner lanes (h = 0), whose results are the
        // only ones used: with (a, b) = this block's two smallest keys in half
        // 0 and (c, d) in half 1, the smallest is min(a, c) and the second
        // min(max(a, c), min(b, d)).  Swapping (a1, a2) gives lanes 0-31 the
        // pair (a, c) and lanes 32-63 (b, d); one more swap brings the upper
        // lanes' min(b, d) down.  Only the smallest keys need the half bit
        // (index bit 2) of their codeword; the gap test compares keys with
        // their index bits in place, which the bound E already covers (31 ulp
        // per key).
        const uint32_t hb = static_cast<uint32_t>(h) << 2;
        a1 |= hb;
        b1 |= hb;
        const auto pa = __builtin_amdgcn_permlane32_swap(a1, a2, false, false);
        const auto pb = __builtin_amdgcn_permlane32_swap(b1, b2, false, false);
        const uint32_t ma = min(pa[0], pa[1]), Ma = max(pa[0], pa[1]);
        const uint32_t mb = min(pb[0], pb[1]), Mb = max(pb[0], pb[1]);
        const auto qa2 = __builtin_amdgcn_permlane32_swap(ma, pa[0], false, false);
        const auto qb2 = __builtin_amdgcn_permlane32_swap(mb, pb[0], false, false);
        const uint32_t ka1 = qa2[0], ka2 = min(Ma, qa2[1]);
        const uint32_t kb1 = qb2[0], kb2 = min(Mb, qb2[1]);
        const float ta = thr - (u2f(ka2) - u2f(ka1)), tb = thr - (u2f(kb2) - u2f(kb1));
        da = __builtin_amdgcn_alignbit(da, f2u(ta), 31);   // (da << 1) | sign(ta)
        db = __builtin_amdgcn_alignbit(db, f2u(tb), 31);
        if (i < 6) {
            ra = __builtin_amdgcn_alignbit(ka1, ra, 5);     // (ra >> 5) | (ka1 << 27)
            rb = __builtin_amdgcn_alignbit(kb1, rb, 5);
        } else {
            ra2 = __builtin_amdgcn_alignbit(ka1, ra2, 5);
            rb2 = __builtin_amdgcn_alignbit(kb1, rb2, 5);
        }
        // materialise this pair's decisions now: the optimiser would otherwise
        // sink every pair's tests and index packing past the loop and keep all
        // eight pairs' candidate keys live at once
        asm volatile("" : "+v"(da), "+v"(db), "+v"(ra), "+v"(ra2), "+v"(rb), "+v"(rb2));
        __builtin_amdgcn_sched_barrier(0);   // keep one block pair's results live at a time
    }
    // the 80-bit index field: blocks 0..5 = ra >> 2, 6..7 = x, 8..13 = rb >> 2,
    // 14..15 = y at bits 0, 30, 40, 70
    const uint32_t x = ra2 >> 22, y = rb2 >> 22;
    const uint32_t iw[3] = {__builtin_amdgcn_alignbit(x, ra, 2), (x >> 2) | (rb << 6), (rb >> 26) | (y << 6)};
    // undecided blocks: bit j of the bit-reversed da / db is block j's (j + 8's) acceptance
    const uint32_t redo = (~(__builtin_bitreverse32(da) >> 24) & 0xFFu) |
                          ((~(__builtin_bitreverse32(db) >> 24) & 0xFFu) << 8);

    // encode_norm Fp16Paper (codec.rs:994-1020)
    const uint16_t h16 = f32_to_f16(static_cast<float>(nrm));
    const bool h_ok = (h16 & 0x7c00u) != 0x7c00u && (h16 & 0x7fffu) != 0 && !(h16 & 0x8000u);
    const bool owner = active && h == 0;
    const uint32_t vi = v0 + static_cast<uint32_t>(n);
    if (owner) {
        if (!finite_all) status_fail(lc.status, sidx, 0, vi, KIND_NONFINITE_INPUT);
        else if (zero) status_fail(lc.status, sidx, 0, vi, KIND_ZERO_NORM);
        else if (!h_ok) status_fail(lc.status, sidx, 1, vi, KIND_NORM16);
    }
    // payload [f16 norm][16 x 5-bit indices] = 12 bytes, kept in LDS: the
    // exact redo patches it there and the wave's 32 payloads then leave as
    // one byte range
    if (owner) {
        pay[3 * n + 0] = static_cast<uint32_t>(h16) | (iw[0] << 16);
        pay[3 * n + 1] = (iw[0] >> 16) | (iw[1] << 16);
        pay[3 * n + 2] = (iw[1] >> 16) | (iw[2] << 16);
    }
    return (active && finite_all && !zero) ? redo : 0u;
}

// True when every value within err of v rounds to the same f32 as v: no f32
// rounding boundary (the midpoint of two adjacent f32 values, ties included)
// lies within err of v.  v finite.
__device__ __forceinline__ bool f32_rounding_stable(double v, double err) {
    const double a = __builtin_fabs(v);
    const float y = static_cast<float>(a);   // nearest, ties to even
    const uint32_t b = f2u(y);
    if (b == 0u) return a + err < 0x1p-150;   // rounds to zero: below half the smallest subnormal
    const double yd = static_cast<double>(y);
    // y and its neighbours are f32: their sums are exact in f64, and so are the halves
    const double m_hi = (yd + static_cast<double>(u2f(b + 1u))) * 0.5;
    const double m_lo = (yd + static_cast<double>(u2f(b - 1u))) * 0.5;
    return m_hi - a > err && a - m_lo > err;
}

constexpr uint32_t FIB_UNIT = 32;                          // vectors per wave iteration (one MFMA tile)
constexpr uint32_t FIB_UNITS_PER_TILE = TILE / FIB_UNIT;   // a segment tile of 256 vectors is 8 units
constexpr int FIB_PAY_WORDS = 32 * 3 + 4;                  // one unit's payloads + lds_to_global padding
constexpr uint32_t FIB_LCAP = 96;                          // a wave's list of undecided vectors (LDS)

// Lane permutations inside each row of 16 lanes (DPP, no LDS round trip):
// quad xor 1, quad xor 2, i <-> 7 - i within 8, i <-> 15 - i within 16.
constexpr int DPP_QUAD_XOR1 = 0xB1, DPP_QUAD_XOR2 = 0x4E, DPP_HALF_MIRROR = 0x141, DPP_MIRROR = 0x140;
constexpr int DPP_ROW_ROR4 = 0x124, DPP_ROW_ROR8 = 0x128;   // rotate by 4 / 8 lanes within the 16
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ double dpp_f64(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = dpp_u32<CTRL>(static_cast<uint32_t>(b)), hi = dpp_u32<CTRL>(static_cast<uint32_t>(b >> 32));
    return __builtin_bit_cast(double, static_cast<uint64_t>(hi) << 32 | lo);
}
// (d, w) := the smaller of (d, w) and the pair from the permuted lane (ties: the lower index)
template <int CTRL>
__device__ __forceinline__ void argmin_step(float& d, uint32_t& w) {
    const float od = u2f(dpp_u32<CTRL>(f2u(d)));
    const uint32_t ow = dpp_u32<CTRL>(w);
    if (od < d || (od == d && ow < w)) { d = od; w = ow; }
}

// A vector with undecided argmin blocks, in its encode wave's LDS list.
struct FibRedoEntry {
    uint64_t in_off;      // the vector's first input element
    uint64_t field_off;   // wire byte of its payload's index field (payload byte 2)
    double nrm;           // |x| (the reference's sequential f64 l2_norm)
    uint32_t flags;       // undecided blocks (bits 0..15) | FibQuantizer::encode semantics << 16
    uint32_t field[3];    // the index field as encoded (bits 0..31, 32..63, 64..79), patched by the redo
};

// Exact decisions for the nq (<= FIB_LCAP) listed vectors of one wave, then
// their index fields back to the wire.  The wave's four groups of 16 lanes
// take one entry each per round; with PREFETCH (after the wave's last unit,
// when nothing else is live) the next round's x and Pi rows load while the
// current one is redone, without it (a full list in the middle of the unit
// loop, rare) each round loads its own.  Per undecided block b, the
// reference's exact path: x_hat = f32(x / |x|) (codec.rs:608; f64 x / |x|
// under FibQuantizer::encode semantics, codec.rs:481), rho_r = f32(sequential
// f64 sum of f64 products over row 4b + r of Pi) (rotation.rs:107-113), the
// AVX2 argmin over the 32 codewords (simd_nearest.rs:44-104).  Lane g of a
// group converts elements 4g .. 4g + 3 and holds codewords 2g, 2g + 1; rows
// 4b .. 4b + 3 of Pi are 2 KB in a row, which the group loads as 16-byte
// pieces g + 16c (c = 0 .. 7, 256 contiguous bytes per load), so lane g holds
// columns 2g, 2g + 1, 2g + 32, 2g + 33 of every one of the four rows.
//
// Both roundings are taken from faster forms that provably round the same:
//  * x_hat: q = x * fl64(1 / |x|) is within 2^-50 |q| of fl64(x / |x|)
//    (three roundings of at most 2^-53 relative and the reciprocal's
//    2^-52), so if no f32 rounding boundary lies within that distance of q
//    (tested on q's bits, f32_rounding_stable_rel50), f32(q) =
//    f32(fl64(x / |x|)); otherwise the division is done.
//  * rho_r: each lane's FMA chain over its four columns, then four levels of
//    adds over the 16 lanes (two that halve the rows a lane keeps, then two
//    rotations, after which lane 2 (r % 2) + r / 2 of the group holds row r),
//    rounds every term at most 8 times, so it is within gamma_8 A of the
//    exact sum, and the reference's sequential sum is within gamma_64 A,
//    A = sum |Pi_rc x_hat_c| <= |Pi_r| |x_hat| < 1.01: the two differ by less
//    than 96 * 2^-53; if no f32 rounding boundary lies within 2^-46 of the
//    fast result, f32 of it is the reference's rho_r; otherwise that lane
//    sums the row in the reference's order.
// A vector is listed once, so every wave writes only its own vectors' index
// fields (after the encode wrote their payloads: the same wave's stores to the
// same bytes, in order).
template <int DIM, bool PREFETCH>
__device__ __forceinline__ void fib_redo_list(const LaunchCommon& lc, const void* __restrict__ in,
                                              uint8_t* __restrict__ wire, const double* __restrict__ rot64,
                                              const float* __restrict__ cb, FibRedoEntry* list, double* xh_wave,
                                              uint32_t nq, int lane) {
    static_assert(DIM == 64, "16 lanes x 4 columns of 4 rows per 4-dimensional block");
    const uint32_t grp = static_cast<uint32_t>(lane) >> 4, g = static_cast<uint32_t>(lane) & 15u;
    const bool b0 = (g & 1u) != 0, b1 = (g & 2u) != 0;
    const uint32_t my_row = (b0 ? 2u : 0u) + (b1 ? 1u : 0u);   // the row whose sum this lane ends with (g < 4)
    const int gb = lane & ~15;   // the group's first lane
    double* xh = xh_wave + grp * DIM;
    const bool bf16 = lc.in_bf16 != 0;
    const float4 cw0 = reinterpret_cast<const float4*>(cb)[2 * g], cw1 = reinterpret_cast<const float4*>(cb)[2 * g + 1];
    // p[4r + 0..3] = Pi[4b + r][2g], [2g + 1], [2g + 32], [2g + 33]
    auto load_rows = [&](uint32_t b, double (&p)[16]) {
        const double2* base = reinterpret_cast<const double2*>(rot64 + static_cast<size_t>(4u * b) * DIM) + g;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const double2 v2 = base[16 * c];
            p[2 * c] = v2.x;
            p[2 * c + 1] = v2.y;
        }
    };
    // round j: group grp redoes entry 4j + grp; its x elements 4g .. 4g + 3
    // and its first undecided block's rows (every round loads: past the end,
    // the last entry again)
    struct In {
        float x[4];
        double p[16];
    };
    auto fetch = [&](uint32_t j, In& d) {
        const FibRedoEntry& e = list[min(4u * j + grp, nq - 1u)];
        const uint64_t off = e.in_off + 4u * g;
        if (!bf16) {
            const float4 q4 = *reinterpret_cast<const float4*>(static_cast<const float*>(in) + off);
            d.x[0] = q4.x; d.x[1] = q4.y; d.x[2] = q4.z; d.x[3] = q4.w;
        } else {
            const uint2 w2 = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(in) + off);
            d.x[0] = u2f(w2.x << 16); d.x[1] = u2f(w2.x & 0xffff0000u);
            d.x[2] = u2f(w2.y << 16); d.x[3] = u2f(w2.y & 0xffff0000u);
        }
        if constexpr (PREFETCH) load_rows(static_cast<uint32_t>(__ffs((e.flags & 0xFFFFu) | 0x10000u) - 1) & 15u, d.p);
    };
    auto redo = [&](uint32_t j, const In& d) {
        const uint32_t idx = 4u * j + grp;
        if (idx >= nq) return;   // group-uniform
        FibRedoEntry& e = list[idx];
        const uint32_t flags = e.flags;
        const bool small = (flags >> 16) & 1u;
        const double nv = e.nrm;
        {   // x_hat[4g .. 4g + 3]
            const double rinv = 1.0 / nv;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const double xd = static_cast<double>(d.x[q]);
                double x1;
                if (small) {
                    x1 = xd / nv;
                } else {
                    const double qq = xd * rinv;
                    float y = static_cast<float>(qq);
                    if (!f32_rounding_stable_rel50(qq)) y = static_cast<float>(xd / nv);   // |qq| <= 1 + 2^-50
                    x1 = static_cast<double>(y);
                }
                xh[4 * g + q] = x1;
            }
        }
        uint64_t ilo = e.field[0] | static_cast<uint64_t>(e.field[1]) << 32;   // field bits 0..63
        uint32_t ihi = e.field[2];                                               // and 64..79
        wave_sync();
        const double2 xa = *reinterpret_cast<const double2*>(xh + 2 * g);
        const double2 xb = *reinterpret_cast<const double2*>(xh + 2 * g + 32);
        bool first = true;
        for (uint32_t m = flags & 0xFFFFu; m != 0u; m &= m - 1u) {
            const uint32_t b = static_cast<uint32_t>(__ffs(m) - 1);
            double p[16];
            if (PREFETCH && first) {
#pragma unroll
                for (int c = 0; c < 16; ++c) p[c] = d.p[c];
            } else {
                load_rows(b, p);
            }
            first = false;
            double sr[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                double t = __builtin_fma(p[4 * r], xa.x, 0.0);
                t = __builtin_fma(p[4 * r + 1], xa.y, t);
                t = __builtin_fma(p[4 * r + 2], xb.x, t);
                sr[r] = __builtin_fma(p[4 * r + 3], xb.y, t);
            }
            // lanes g, g ^ 1: even lanes keep rows 0, 1, odd lanes rows 2, 3
            const double ka = b0 ? sr[2] : sr[0], kb = b0 ? sr[3] : sr[1];
            const double ra = ka + dpp_f64<DPP_QUAD_XOR1>(b0 ? sr[0] : sr[2]);
            const double rb = kb + dpp_f64<DPP_QUAD_XOR1>(b0 ? sr[1] : sr[3]);
            // lanes g, g ^ 2: row 2 (g % 2) + (g / 2) % 2
            double t = (b1 ? rb : ra) + dpp_f64<DPP_QUAD_XOR2>(b1 ? ra : rb);
            // lanes g, g + 4, g + 8, g + 12 hold the same row
            t += dpp_f64<DPP_ROW_ROR4>(t);
            t += dpp_f64<DPP_ROW_ROR8>(t);
            float rho_l = static_cast<float>(t);
            if (!f32_rounding_stable(t, 0x1p-46)) {   // the reference's order: fl64 products, sequential fl64 sum
                const double* prow = rot64 + static_cast<size_t>(4u * b + my_row) * DIM;
                double a = 0.0;
                for (int c = 0; c < DIM; ++c) {
                    const double prod = prow[c] * xh[c];
                    a = a + prod;
                }
                rho_l = static_cast<float>(a);
            }
            const float rho[4] = {__shfl(rho_l, gb), __shfl(rho_l, gb + 2), __shfl(rho_l, gb + 1),
                                  __shfl(rho_l, gb + 3)};
            // AVX2 distances (cw - s, (d0^2 + d1^2) + (d2^2 + d3^2)) to codewords 2g, 2g + 1
            float bd = 0.0f;
            uint32_t bw = 0;
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const float4 cw = w ? cw1 : cw0;
                const float e0 = cw.x - rho[0], e1 = cw.y - rho[1], e2 = cw.z - rho[2], e3 = cw.w - rho[3];
                const float dd = (e0 * e0 + e1 * e1) + (e2 * e2 + e3 * e3);
                if (w == 0 || dd < bd) { bd = dd; bw = 2 * g + w; }
            }
            // the first codeword with the smallest distance over the 16 lanes
            argmin_step<DPP_QUAD_XOR1>(bd, bw);
            argmin_step<DPP_QUAD_XOR2>(bd, bw);
            argmin_step<DPP_HALF_MIRROR>(bd, bw);
            argmin_step<DPP_MIRROR>(bd, bw);
            const uint32_t pos = 5u * b;   // field bits pos .. pos + 4
            if (pos + 5u <= 64u) {
                ilo = (ilo & ~(31ull << pos)) | (static_cast<uint64_t>(bw) << pos);
            } else if (pos >= 64u) {
                ihi = (ihi & ~(31u << (pos - 64u))) | (bw << (pos - 64u));
            } else {   // bits pos .. 63 in ilo, the rest in ihi
                ilo = (ilo & ~(~0ull << pos)) | (static_cast<uint64_t>(bw) << pos);
                ihi = (ihi & ~(31u >> (64u - pos))) | (bw >> (64u - pos));
            }
        }
        if (g == 0) {
            e.field[0] = static_cast<uint32_t>(ilo);
            e.field[1] = static_cast<uint32_t>(ilo >> 32);
            e.field[2] = ihi;
        }
        wave_sync();   // xh is rewritten in the group's next round
    };
    const uint32_t rounds = (nq + 3u) / 4u;
    if constexpr (PREFETCH) {
        In da, db;
        fetch(0, da);
        for (uint32_t j = 0; j < rounds; j += 2) {   // two rounds per pass: no register copies of loads in flight
            fetch(j + 1, db);
            redo(j, da);
            fetch(j + 2, da);
            redo(j + 1, db);
        }
    } else {
        for (uint32_t j = 0; j < rounds; ++j) {
            In d;
            fetch(j, d);
            redo(j, d);
        }
    }
    wave_sync();
    if (static_cast<uint32_t>(lane) < nq) {   // lane i writes entry i's index field
        const FibRedoEntry& e = list[lane];
        const uint64_t lo = e.field[0] | static_cast<uint64_t>(e.field[1]) << 32;
        const uint16_t hi = static_cast<uint16_t>(e.field[2]);
        __builtin_memcpy(wire + e.field_off, &lo, 8);
        __builtin_memcpy(wire + e.field_off + 8, &hi, 2);
    }
    wave_sync();   // the list is refilled
}

// FibQuantizer::encode_batch (codec.rs:578-668) + finish_batch_encode
// (670-729) + FibCodeV1::encode_batch (225-320) for every segment.  Each wave
// walks 32-vector units (unit u: 256-vector tile u / 8 of the segment table,
// eighth u % 8) with a stride of the whole grid; the next unit's rows are
// loaded while the current one is scored, and each unit's payloads leave as
// one byte range.  A vector with undecided blocks goes to the wave's LDS list
// with a copy of its index field; the wave redoes its list after its last
// unit, or earlier when the next unit could overflow it.  No workgroup
// barrier after the rotation operands are in LDS: the waves never wait for
// each other.
template <int DIM, bool DIAG>
__global__ __launch_bounds__(TILE) __attribute__((amdgpu_waves_per_eu(3))) void fib_encode_kernel(LaunchCommon lc,
    const void* __restrict__ in, uint8_t* __restrict__ wire, const uint32_t* __restrict__ mf, float thr,
    const double* __restrict__ rot64, const float* __restrict__ cb, uint32_t nunits,
    const SegDev* __restrict__ segs, const uint32_t* __restrict__ tile_start, const uint32_t* __restrict__ tile_seg) {
    // (the segment tables come as restrict arguments, not through lc: the
    // compiler then reads them with scalar loads, which wait on their own
    // counter; vector loads share vmcnt with the prefetched rows and the
    // payload stores, whose in-order count would make each segment read wait
    // for them)
    static_assert(DIM == 64, "the MFMA layout is built for head_dim 64");
    extern __shared__ uint32_t smem_u[];
    uint32_t* rot_lds = smem_u;   // MF_ROT block (MF_SCA words)
    // wave index as a wave-uniform value: the unit loop, its segment lookups
    // and offsets then stay scalar
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int lane = threadIdx.x & 63;
    const int h = lane >> 5, n = lane & 31;
    uint32_t* pay = smem_u + MF_SCA + wave * FIB_PAY_WORDS;
    FibRedoEntry* list = reinterpret_cast<FibRedoEntry*>(smem_u + MF_SCA + WAVES * FIB_PAY_WORDS) + wave * FIB_LCAP;
    double* xh = reinterpret_cast<double*>(reinterpret_cast<FibRedoEntry*>(smem_u + MF_SCA + WAVES * FIB_PAY_WORDS) +
                                           WAVES * FIB_LCAP) + wave * 4 * DIM;
    const bool bf16 = lc.in_bf16 != 0;
    {
        const uint4* src = reinterpret_cast<const uint4*>(mf + MF_ROT);
        uint4* dst = reinterpret_cast<uint4*>(rot_lds);
        uint4 t[MF_SCA / 4 / TILE];
#pragma unroll
        for (int q = 0; q < MF_SCA / 4 / TILE; ++q) t[q] = src[threadIdx.x + q * TILE];
#pragma unroll
        for (int q = 0; q < MF_SCA / 4 / TILE; ++q) dst[threadIdx.x + q * TILE] = t[q];
    }
    const uint4 sa4 = reinterpret_cast<const uint4*>(mf + MF_SCA)[lane];
    const v4u sa = {sa4.x, sa4.y, sa4.z, sa4.w};
    __syncthreads();   // the only barrier: the rotation operands are in LDS

    const uint32_t stride = gridDim.x * WAVES;
    // first unit >= u (step stride) with vectors -> its segment and first vector; nunits when none.
    // A wave visits units in increasing order, so after a binary search for its
    // first unit the segment search continues forward from the previous unit's
    // segment (sidx on entry).
    auto next_unit = [&](uint32_t u, uint32_t& sidx, uint32_t& v0) -> uint32_t {
        if (u < nunits && sidx == 0xFFFFFFFFu) sidx = segment_of(tile_seg, tile_start, lc.nseg, u / FIB_UNITS_PER_TILE);
        for (; u < nunits; u += stride) {
            const uint32_t tile = u / FIB_UNITS_PER_TILE;
            while (sidx + 1 < lc.nseg && tile_start[sidx + 1] <= tile) ++sidx;
            v0 = (tile - tile_start[sidx]) * TILE + (u % FIB_UNITS_PER_TILE) * FIB_UNIT;
            if (v0 < segs[sidx].n_vectors) return u;
        }
        return nunits;
    };
    uint32_t sidx = 0xFFFFFFFFu, v0 = 0;
    uint32_t u = next_unit(blockIdx.x * WAVES + static_cast<uint32_t>(wave), sidx, v0);
    float4 x[8];
    uint64_t xrow = 0;   // first element of the vector whose rows x holds
    if (u < nunits) {
        const SegDev s = segs[sidx];
        xrow = load_half_row(x, in, bf16, s, min(v0 + static_cast<uint32_t>(n), s.n_vectors - 1), h);
    }
    uint32_t nq = 0;   // listed vectors
    while (u < nunits) {   // wave-uniform
        {   // a wave near its last units steps down so the ones with more left issue
            // first (the arbiter otherwise favours the oldest waves, which then
            // finish early and leave the late ones at low occupancy)
            const uint32_t rem = (nunits - u + stride - 1) / stride;
            if (rem >= 4) __builtin_amdgcn_s_setprio(3);
            else if (rem == 3) __builtin_amdgcn_s_setprio(2);
            else if (rem == 2) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
        }
        const SegDev seg = segs[sidx];
        const uint64_t row = xrow;
        FibTileRot t;
        fib_encode_rotate(t, x, rot_lds, lane);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t sidx2 = sidx, v02 = 0;
        const uint32_t u2 = next_unit(u + stride, sidx2, v02);
        if (u2 < nunits) {   // the next unit's rows land while this one is scored
            const SegDev s2 = segs[sidx2];
            xrow = load_half_row(x, in, bf16, s2, min(v02 + static_cast<uint32_t>(n), s2.n_vectors - 1), h);
        }
        const uint32_t mask = fib_encode_score<DIM, DIAG>(lc, seg, sidx, v0, t, pay, sa, thr, lane);
        wave_sync();   // the unit's payloads are in LDS
        // list this unit's undecided vectors, with their index fields
        const bool small = seg.n_vectors < 4 || lc.per_vector != 0;
        const bool queued = h == 0 && mask != 0u;
        const uint64_t bal = __ballot(queued);
        if (queued) {
            const uint32_t vi = v0 + static_cast<uint32_t>(n);
            const uint32_t w0 = pay[3 * n], w1 = pay[3 * n + 1], w2 = pay[3 * n + 2];
            FibRedoEntry& en = list[nq + static_cast<uint32_t>(__popcll(bal & ((1ull << lane) - 1ull)))];
            en.in_off = row;   // (a listed lane is active: its vector's own offset)
            en.field_off = seg.wire_offset + 19u + 12ull * vi + 2u;   // payload bytes 2 .. 11
            en.nrm = t.nrm;
            en.flags = mask | (small ? 1u << 16 : 0u);
            en.field[0] = (w0 >> 16) | (w1 << 16);
            en.field[1] = (w1 >> 16) | (w2 << 16);
            en.field[2] = w2 >> 16;
        }
        nq += static_cast<uint32_t>(__popcll(bal));
        uint8_t* blob = wire + seg.wire_offset;
        lds_to_global(blob + 19 + static_cast<uint64_t>(v0) * 12u, pay, min(FIB_UNIT, seg.n_vectors - v0) * 12u, lane);
        if (v0 == 0 && lane < 19)
            blob[lane] = static_cast<uint8_t>(fb2_byte(static_cast<uint32_t>(lane), 5u, DIM / 4, seg.n_vectors, 10u));
        wave_sync();   // the payload words are rewritten by the next unit
        if (nq > FIB_LCAP - FIB_UNIT) {   // the next unit could overflow the list
            fib_redo_list<DIM, false>(lc, in, wire, rot64, cb, list, xh, nq, lane);
            nq = 0;
        }
        u = u2;
        sidx = sidx2;
        v0 = v02;
    }
    if (nq) {   // the list's rounds are latency-bound and short: issued ahead of the other waves' units
        __builtin_amdgcn_s_setprio(3);
        fib_redo_list<DIM, true>(lc, in, wire, rot64, cb, list, xh, nq, lane);
    }
}

// ------------------------------------------------------------ fib decode
// FibCodeV1::decode_batch (codec.rs:323-424) + decode_batch_fast (797-844).
//
// One lane per output column: lane `col` keeps column col of f32(Pi) (row
// `row` at f32(Pi)[row][col]) in 64 VGPRs and rebuilds
//   x[col] = (((0 + P[0][col] c_0) + P[1][col] c_1) + ...) * norm
// with every product and sum rounded (the reference's sequential f32 loop),
// where c_row = codebook[w_{row/4}][row % 4] is the same for every lane:
// the indices are decoded once per vector and the codeword components are
// scalar loads, so each term costs one v_mul_f32 and one v_add_f32 with an
// SGPR operand.  A wave walks its 64 vectors one by one and stores each
// decoded row as one coalesced 256-byte write.
template <int DIM>
__global__ __launch_bounds__(TILE) void fib_decode_kernel(LaunchCommon lc, const uint8_t* __restrict__ wire,
                                                          void* __restrict__ out,
                                                          const float* __restrict__ rot32t,
                                                          const float* __restrict__ cb) {
    static_assert(DIM == 64, "one lane per column of a 64-wide vector");
    constexpr int BLOCKS = DIM / 4;
    constexpr uint32_t PLEN = 2 + (BLOCKS * 5 + 7) / 8;   // 12
    constexpr int PAY_WORDS = WAVE * PLEN / 4 + 4;
    __shared__ uint32_t pay_s[WAVES][PAY_WORDS];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const uint32_t blk = blockIdx.x;
    const uint32_t sidx = segment_of(lc.tile_seg, lc.tile_start, lc.nseg, blk);
    const SegDev seg = lc.segs[sidx];
    const uint32_t tile = blk - lc.tile_start[sidx];
    const uint32_t v0 = tile * TILE + wave * WAVE;
    const uint8_t* blob = wire + seg.wire_offset;

    uint32_t hb = lane < 19 ? blob[lane] : 0u;
    bool bad = lane < 19 && fb2_checked(lane, seg.n_vectors) &&
               hb != fb2_byte(lane, 5u, BLOCKS, seg.n_vectors, PLEN - 2);
    if (lane == 14 && hb != 0u) bad = true;   // norm format must be Fp16Paper
    if (__ballot(bad) != 0ull) {
        if (lane == 0) status_fail(lc.status, sidx, 0, 0u, KIND_HEADER);
        return;
    }
    if (v0 >= seg.n_vectors) return;
    const uint32_t nv = min(static_cast<uint32_t>(WAVE), seg.n_vectors - v0);

    // column `lane` of f32(Pi): rot32t is [col][row]
    float pc[DIM];
    {
        const float4* src = reinterpret_cast<const float4*>(rot32t + lane * DIM);
#pragma unroll
        for (int k = 0; k < DIM / 4; ++k) {
            const float4 v = src[k];
            pc[4 * k] = v.x; pc[4 * k + 1] = v.y; pc[4 * k + 2] = v.z; pc[4 * k + 3] = v.w;
        }
    }
    // the wave's payloads into LDS (coalesced), then lane v keeps vector v's
    // three payload words and output offset for the walk below
    uint32_t* sw = pay_s[wave];
    global_to_lds(sw, blob + 19 + static_cast<uint64_t>(v0) * PLEN, nv * PLEN, lane);
    wave_sync();
    // lane v decodes vector v: norm bits, output offset and the byte offsets
    // of its 16 codewords in the codebook; the walk below reads them with
    // v_readlane, so the scalar unit only issues the loads
    const uint32_t mine = min(static_cast<uint32_t>(lane), nv - 1);
    const uint32_t q0 = sw[3 * mine], q1 = sw[3 * mine + 1], q2 = sw[3 * mine + 2];
    const uint64_t my_off = vec_elem_offset(seg, v0 + mine);
    uint32_t cofs[BLOCKS];
    {
        // 16 x 5-bit indices, LSB-first, starting at payload byte 2
        const uint64_t lo = (static_cast<uint64_t>(q0) >> 16) | (static_cast<uint64_t>(q1) << 16) |
                            (static_cast<uint64_t>(q2) << 48);
        const uint32_t hi = q2 >> 16;
#pragma unroll
        for (int b = 0; b < BLOCKS; ++b) {
            const int bit = 5 * b;
            uint32_t w;
            if (bit + 5 <= 64) w = static_cast<uint32_t>(lo >> bit) & 31u;
            else if (bit >= 64) w = (hi >> (bit - 64)) & 31u;
            else w = (static_cast<uint32_t>(lo >> bit) | (hi << (64 - bit))) & 31u;
            cofs[b] = w * 16u;
        }
    }
    const char* cbb = reinterpret_cast<const char*>(cb);
    for (uint32_t v = 0; v < nv; ++v) {
        float4 c[BLOCKS];
#pragma unroll
        for (int b = 0; b < BLOCKS; ++b)
            c[b] = *reinterpret_cast<const float4*>(
                cbb + static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(cofs[b], v))));
        float s = 0.0f;
#pragma unroll
        for (int b = 0; b < BLOCKS; ++b) {
            s = s + pc[4 * b + 0] * c[b].x;
            s = s + pc[4 * b + 1] * c[b].y;
            s = s + pc[4 * b + 2] * c[b].z;
            s = s + pc[4 * b + 3] * c[b].w;
        }
        const uint32_t olo = __builtin_amdgcn_readlane(static_cast<uint32_t>(my_off), v);
        const uint32_t ohi = __builtin_amdgcn_readlane(static_cast<uint32_t>(my_off >> 32), v);
        const uint64_t off = static_cast<uint64_t>(ohi) << 32 | olo;
        const float nrm = f16_to_f32(static_cast<uint16_t>(__builtin_amdgcn_readlane(q0, v) & 0xffffu));
        const bool ok = isfinite_f(nrm) && nrm > 0.0f;
        const float o = s * nrm;
        const bool ofinite = __ballot(!isfinite_f(o)) == 0ull;
        const uint32_t vi = v0 + v;
        if (!ok) {
            if (lane == 0) status_fail(lc.status, sidx, 1, vi, KIND_CORRUPT);
        } else if (!ofinite) {
            if (lane == 0) status_fail(lc.status, sidx, 1, vi, KIND_DECODE_NONFINITE);
        } else {
            store_out1(out, lc, off + lane, o);
        }
    }
}

// Decode with the products on the matrix cores.  For one rotation row r the
// products of all columns and vectors form the rank-1 matrix
// f32(Pi)[r][:] x c_r[:], so v_mfma_f32_32x32x1_2b_f32 with a zero
// accumulator yields them (2 x 32 columns x 32 vectors per instruction); the
// VALU keeps only the sequential f32 additions, in the reference's order.
// A product from the matrix core must equal f32 multiplication bit for bit:
// fib_product_check_kernel checks every product this kernel can form
// (64 rows x 64 columns x 32 codewords) when a profile is created, and the
// profile falls back to fib_decode_kernel on any difference.
typedef float v32f __attribute__((ext_vector_type(32)));

template <int DIM, bool STAGED>
__global__ __launch_bounds__(TILE) void fib_decode_mfma_kernel(LaunchCommon lc, const uint8_t* __restrict__ wire,
                                                               void* __restrict__ out,
                                                               const float* __restrict__ rot32,
                                                               const float* __restrict__ cb,
                                                               const SegDev* __restrict__ segs,
                                                               const uint32_t* __restrict__ tile_start,
                                                               const uint32_t* __restrict__ tile_seg) {
    // (segment tables as restrict arguments: scalar loads, so a tile's segment
    // lookup does not wait for the previous tile's stores to drain)
    static_assert(DIM == 64, "two 32-column MFMA blocks");
    constexpr int BLOCKS = DIM / 4;
    constexpr uint32_t PLEN = 2 + (BLOCKS * 5 + 7) / 8;   // 12
    constexpr int PAY_WORDS = WAVE * PLEN / 4 + 4;
    constexpr int RPITCH = DIM + 4;      // one staged row per vector, padded
    __shared__ float rot_s[DIM * DIM];   // f32(Pi), row-major
    __shared__ float4 cb_s[32];
    __shared__ uint32_t pay_s[WAVES][PAY_WORDS];
    __shared__ float half_s[STAGED ? WAVES : 1][STAGED ? 16 * RPITCH : 4];   // output staging: 16 rows
    {
        const float4* src = reinterpret_cast<const float4*>(rot32);
        float4* dst = reinterpret_cast<float4*>(rot_s);
        float4 t[DIM * DIM / 4 / TILE];
#pragma unroll
        for (int k = 0; k < DIM * DIM / 4 / TILE; ++k) t[k] = src[threadIdx.x + k * TILE];
#pragma unroll
        for (int k = 0; k < DIM * DIM / 4 / TILE; ++k) dst[threadIdx.x + k * TILE] = t[k];
        if (threadIdx.x < 32) cb_s[threadIdx.x] = reinterpret_cast<const float4*>(cb)[threadIdx.x];
    }
    __syncthreads();

    const int wave = threadIdx.x >> 6;
    // one tile per workgroup, or (grid capped) a workgroup walks the tiles
    // blockIdx.x, blockIdx.x + gridDim.x, ... with the tables loaded once
    const uint32_t nblk = tile_start[lc.nseg];
    for (uint32_t blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    wave_sync();   // the previous tile's LDS reads are done
    // opaque per tile: the loop must not keep lane-derived addresses or table
    // reads live across tiles (register pressure)
    int zoff = 0, lane = threadIdx.x & 63;
    asm volatile("" : "+s"(zoff), "+v"(lane));
    const int h = lane >> 5, n = lane & 31;
    const uint32_t sidx = segment_of(tile_seg, tile_start, lc.nseg, blk);
    const SegDev seg = segs[sidx];
    const uint32_t tile = blk - tile_start[sidx];
    const uint32_t v0 = tile * TILE + wave * WAVE;
    const uint8_t* blob = wire + seg.wire_offset;

    uint32_t hb = lane < 19 ? blob[lane] : 0u;
    bool bad = lane < 19 && fb2_checked(lane, seg.n_vectors) &&
               hb != fb2_byte(lane, 5u, BLOCKS, seg.n_vectors, PLEN - 2);
    if (lane == 14 && hb != 0u) bad = true;   // norm format must be Fp16Paper
    if (__ballot(bad) != 0ull) {
        if (lane == 0) status_fail(lc.status, sidx, 0, 0u, KIND_HEADER);
        continue;
    }
    if (v0 >= seg.n_vectors) continue;
    const uint32_t nv = min(static_cast<uint32_t>(WAVE), seg.n_vectors - v0);
    uint32_t* sw = pay_s[wave];
    global_to_lds(sw, blob + 19 + static_cast<uint64_t>(v0) * PLEN, nv * PLEN, lane);
    wave_sync();

    // Sub-tile s, lane n: wave vector w = (n % 16) + 16 s + 32 (n / 16) -- vectors
    // w and w + 32 are the same head at consecutive tokens when a blob holds
    // 32 heads (vector = token * H + head), so the staged stores below write
    // two adjacent rows per run.  Any other layout is just another order.
    for (uint32_t sub = 0; sub < 2; ++sub) {
        if (sub == 1 && nv <= 16) break;
        const uint32_t w = (static_cast<uint32_t>(n) & 15u) + 16u * sub + 32u * (static_cast<uint32_t>(n) >> 4);
        const uint32_t my = min(w, nv - 1);   // lanes past the end repeat the last
        const uint32_t q0 = sw[3 * my], q1 = sw[3 * my + 1], q2 = sw[3 * my + 2];
        const uint64_t lo = (static_cast<uint64_t>(q0) >> 16) | (static_cast<uint64_t>(q1) << 16) |
                            (static_cast<uint64_t>(q2) << 48);
        const uint32_t hi = q2 >> 16;
        const v32f zero = {};
        v32f acc = {};
#pragma unroll 2
        for (int b = 0; b < BLOCKS; ++b) {
            const int bit = 5 * b;
            // 5-bit index b, LSB-first from payload byte 2 (bit may straddle the 64-bit word)
            const uint32_t w = static_cast<uint32_t>(bit < 64 ? (lo >> bit) | (bit > 59 ? static_cast<uint64_t>(hi) << (64 - bit) : 0ull)
                                                             : static_cast<uint64_t>(hi >> (bit - 64))) & 31u;
            const float4 c = cb_s[w];
            const float cr[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(rot_s[(4 * b + t) * DIM + lane + zoff], cr[t], zero, 0, 0, 0);
#pragma unroll
                for (int q = 0; q < 32; ++q) acc[q] = acc[q] + p[q];
            }
        }
        const float nrm = f16_to_f32(static_cast<uint16_t>(q0 & 0xffffu));
        const bool ok = isfinite_f(nrm) && nrm > 0.0f;
        bool fin = true;
#pragma unroll
        for (int q = 0; q < 32; ++q) {
            acc[q] = acc[q] * nrm;
            fin &= isfinite_f(acc[q]);
        }
        // a vector is bad if either half-wave saw a bad value
        const uint64_t badm = __ballot(!(ok && fin));
        const bool vbad = ((badm >> n) | (badm >> (n + 32))) & 1ull;
        const bool active = w < nv;
        const uint32_t vi = v0 + w;
        if (active && h == 0 && vbad) status_fail(lc.status, sidx, 1, vi, ok ? KIND_DECODE_NONFINITE : KIND_CORRUPT);
        if constexpr (!STAGED) {
            if (active && !vbad) {
                const uint64_t orow = vec_elem_offset(seg, vi);
#pragma unroll
                for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {   // registers q .. q + 3: columns 32bb + 8g + 4h .. + 3
                        const int q = 16 * bb + 4 * g;
                        store_out4(out, lc, orow + 32 * bb + 8 * g + 4 * h,
                                   make_float4(acc[q], acc[q + 1], acc[q + 2], acc[q + 3]));
                    }
            }
            continue;
        }
        // vectors (of the 32) to write: active and good; each lane's row
        // offset is computed once and handed to the storing lanes by a shuffle
        const uint32_t wmask = static_cast<uint32_t>(__ballot(active && !vbad && h == 0));
        const uint64_t my_off = vec_elem_offset(seg, min(vi, seg.n_vectors - 1));
        // Fan-out: rows go through LDS, 16 whole rows (8 heads x 2 tokens) per
        // pass, so each store instruction writes 4 whole 256 B rows -- two
        // runs of two adjacent rows -- instead of 32 B into each of 32 rows
        // (direct stores: 1.4 TB/s at 8 copies).  Row p of a pass holds lane
        // n = (p % 8) + 8 pass + 16 (p / 8); one copy keeps the direct stores.
        float* hs = half_s[wave];
#pragma unroll
        for (uint32_t pass = 0; pass < 2; ++pass) {
            if (((static_cast<uint32_t>(n) >> 3) & 1u) == pass) {
                const uint32_t row = (static_cast<uint32_t>(n) & 7u) + 8u * (static_cast<uint32_t>(n) >> 4);
#pragma unroll
                for (int bb = 0; bb < 2; ++bb)
#pragma unroll
                    for (int g = 0; g < 4; ++g) {   // registers q .. q + 3: columns 32bb + 8g + 4h .. + 3
                        const int q = 16 * bb + 4 * g;
                        *reinterpret_cast<float4*>(hs + row * RPITCH + 32 * bb + 8 * g + 4 * h) =
                            make_float4(acc[q], acc[q + 1], acc[q + 2], acc[q + 3]);
                    }
            }
            wave_sync();
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                // lanes 0-15: row 2kk (token t), 16-31: row 2kk + 8 (token t + 1), then the next head
                const uint32_t sel = static_cast<uint32_t>(lane) >> 4, c = lane & 15;
                const uint32_t row = 2u * kk + (sel >> 1) + 8u * (sel & 1u);
                const uint32_t ln = (row & 7u) + 8u * pass + 16u * (row >> 3);
                const uint64_t off = shfl_u64(my_off, static_cast<int>(ln));
                if ((wmask >> ln) & 1u)
                    store_out4(out, lc, off + 4 * c, *reinterpret_cast<const float4*>(hs + row * RPITCH + 4 * c));
            }
            wave_sync();   // the next pass overwrites the staging rows
        }
    }
    }
}

// Counts the products of (f32(Pi)[r][col], codeword component c[j][r % 4])
// whose matrix-core result differs from f32 multiplication, over every row,
// column and codeword, with the operand placement of fib_decode_mfma_kernel.
__global__ __launch_bounds__(64) void fib_product_check_kernel(const float* __restrict__ rot32,
                                                               const float* __restrict__ cb, uint32_t* bad) {
    const int lane = threadIdx.x, h = lane >> 5, j = lane & 31;
    const v32f zero = {};
    uint32_t cnt = 0;
    for (int r = 0; r < 64; ++r) {
        const float a = rot32[r * 64 + lane], b = cb[j * 4 + (r & 3)];
        const v32f p = __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, zero, 0, 0, 0);
#pragma unroll
        for (int q = 0; q < 32; ++q) {
            const int col = 32 * (q >> 4) + 8 * ((q & 15) >> 2) + 4 * h + (q & 3);
            const float e = rot32[r * 64 + col] * b;
            cnt += f2u(p[q]) != f2u(e) ? 1u : 0u;
        }
    }
    if (cnt) atomicAdd(bad, cnt);
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t value, uint64_t n) {
    uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
    if (i < n) p[i] = value;
}

// g_logb measurement: every normal positive float v in [2^-126, 2^128), a
// contiguous run of `per` per thread.  The running maximum of
// |cheap_logf(v) - logf(v)| (exact in f64, rounded up to f32) goes to
// g_logb_raw[biased exponent of |logf(v)|] whenever that exponent changes.
constexpr uint32_t kLogbLo = 0x00800000u, kLogbHi = 0x7f800000u;
constexpr uint32_t kLogbBlocks = 2048;

__global__ __launch_bounds__(256) void logf_bound_kernel(uint32_t per) {
    __shared__ LogfEntry tab[16];
    if (threadIdx.x < 16) tab[threadIdx.x] = c_logf_tab[threadIdx.x];
    __syncthreads();
    const uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
    const uint64_t b0 = kLogbLo + t * per;
    const uint32_t u0 = static_cast<uint32_t>(b0 < kLogbHi ? b0 : kLogbHi);
    const uint32_t u1 = static_cast<uint32_t>(b0 + per < kLogbHi ? b0 + per : kLogbHi);
    uint32_t cur = 0xffffffffu, best = 0;
    for (uint32_t u = u0; u < u1; ++u) {
        const float v = u2f(u);
        const float l = og_logf_normal(v, tab);
        const double err = __builtin_fabs(static_cast<double>(cheap_logf(v)) - static_cast<double>(l));
        float e = static_cast<float>(err);
        if (static_cast<double>(e) < err) e = u2f(f2u(e) + 1u);
        const uint32_t b = f2u(__builtin_fabsf(l)) >> 23;
        if (b != cur) {
            if (cur != 0xffffffffu) atomicMax(&g_logb_raw[cur], best);
            cur = b;
            best = 0;
        }
        best = f2u(e) > best ? f2u(e) : best;
    }
    if (cur != 0xffffffffu) atomicMax(&g_logb_raw[cur], best);
}

// g_logb[e] = max of g_logb_raw[0..e] (non-negative floats order as their bits).
__global__ void logf_bound_finish_kernel() {
    if (threadIdx.x == 0) {
        uint32_t m = 0;
        for (int e = 0; e < 256; ++e) {
            m = g_logb_raw[e] > m ? g_logb_raw[e] : m;
            g_logb[e] = u2f(m);
        }
    }
}

// Subnormal f16 operands on the matrix cores (the QJL acceptance bound needs
// them kept): out[0] = one 16x16x32 product sum 2^-20 * 1024 + 1024 * 2^-24,
// out[1] = one 32x32x16 product 2^-20 * 1024.
__global__ void f16_subnormal_probe_kernel(float* out) {
    const int lane = threadIdx.x;
    v8h a = {}, b = {};
    if (lane == 0) {
        a[0] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(0x0010));   // 2^-20
        b[0] = static_cast<_Float16>(1024.0f);
        a[1] = static_cast<_Float16>(1024.0f);
        b[1] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(0x0001));   // 2^-24
    }
    const v4f c16 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, v4f{}, 0, 0, 0);
    v8h a2 = {}, b2 = {};
    if (lane == 0) {
        a2[0] = __builtin_bit_cast(_Float16, static_cast<uint16_t>(0x0010));
        b2[0] = static_cast<_Float16>(1024.0f);
    }
    const v16f c32 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a2, b2, v16f{}, 0, 0, 0);
    if (lane == 0) {
        out[0] = c16[0];
        out[1] = c32[0];
    }
}

// sqrt_normal against __builtin_sqrtf on every float it is used on (2^-96 ..
// +inf) and on +0 and NaN; *bad counts the disagreements.
constexpr uint32_t kSqrtLo = 0x0f800000u, kSqrtHi = 0x7f800001u;

__global__ __launch_bounds__(256) void sqrt_check_kernel(uint32_t per, uint32_t* bad) {
    const uint64_t t = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
    const uint64_t b0 = kSqrtLo + t * per;
    const uint32_t u0 = static_cast<uint32_t>(b0 < kSqrtHi ? b0 : kSqrtHi);
    const uint32_t u1 = static_cast<uint32_t>(b0 + per < kSqrtHi ? b0 + per : kSqrtHi);
    uint32_t n = 0;
    for (uint32_t u = u0; u < u1; ++u) n += f2u(sqrt_normal(u2f(u))) != f2u(__builtin_sqrtf(u2f(u))) ? 1u : 0u;
    if (t == 0) {
        n += f2u(sqrt_normal(0.0f)) != 0u ? 1u : 0u;
        n += isfinite_f(sqrt_normal(u2f(0x7fc00000u))) || (f2u(sqrt_normal(u2f(0x7fc00000u))) & 0x7fffffu) == 0u ? 1u : 0u;
    }
    if (n) atomicAdd(bad, n);
}

__global__ void logf_bound_read_kernel(float* out) {
    if (threadIdx.x < 256) out[threadIdx.x] = g_logb[threadIdx.x];
}

template <int DIM>
constexpr size_t stage_bytes() {
    return static_cast<size_t>(WAVES) * (WAVE * (DIM + 4) + 8) * sizeof(float);
}

// Dynamic LDS above 64 KiB must be allowed per kernel before launch.
template <typename K>
hipError_t allow_lds(K kernel, size_t bytes) {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(bytes));
}

}  // namespace

int launch_logf_bound(void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    constexpr uint64_t threads = static_cast<uint64_t>(kLogbBlocks) * 256;
    const uint32_t per = static_cast<uint32_t>((static_cast<uint64_t>(kLogbHi - kLogbLo) + threads - 1) / threads);
    hipLaunchKernelGGL(logf_bound_kernel, dim3(kLogbBlocks), dim3(256), 0, st, per);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(logf_bound_finish_kernel, dim3(1), dim3(64), 0, st);
    return hipGetLastError();
}

int launch_f16_subnormal_probe(float* out, void* stream) {
    hipLaunchKernelGGL(f16_subnormal_probe_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), out);
    return hipGetLastError();
}

int launch_sqrt_check(uint32_t* bad, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    constexpr uint64_t threads = static_cast<uint64_t>(kLogbBlocks) * 256;
    const uint32_t per = static_cast<uint32_t>((static_cast<uint64_t>(kSqrtHi - kSqrtLo) + threads - 1) / threads);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(1), dim3(64), 0, st, bad, 0u, static_cast<uint64_t>(1));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(sqrt_check_kernel, dim3(kLogbBlocks), dim3(256), 0, st, per, bad);
    return hipGetLastError();
}

int launch_logf_bound_read(float* out, void* stream) {
    hipLaunchKernelGGL(logf_bound_read_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), out);
    return hipGetLastError();
}

int launch_fill_u32(uint32_t* p, uint32_t value, uint64_t n, void* stream) {
    if (n == 0) return hipSuccess;
    uint32_t blocks = static_cast<uint32_t>((n + 255) / 256);
    hipLaunchKernelGGL(fill_u32_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), p, value, n);
    return hipGetLastError();
}

template <typename K, typename... Args>
hipError_t launch_big_lds(K kernel, uint32_t nblocks, size_t lds, hipStream_t st, Args... args) {
    hipError_t e = allow_lds(kernel, lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kernel, dim3(nblocks), dim3(TILE), lds, st, args...);
    return hipGetLastError();
}

int launch_turbo_encode(const LaunchCommon& lc, const TurboDev& td, const void* in, uint8_t* wire,
                        uint32_t nblocks, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (td.dim == 64 && td.mode && td.qa && td.pbits <= 4) {
        if (nblocks > (1u << 30)) return hipErrorInvalidValue;   // 2 workgroups per tile
        const size_t vec_words = (lc.plen >> 2) + (lc.radii == PKV_RADII_F32 ? 0u : 32u);
        const size_t lds = static_cast<size_t>(WAVES) * (32 * vec_words + 4) * sizeof(uint32_t);
#define PKV_QJL64(PB, DG)                                                                                      \
    launch_big_lds(turbo_encode_qjl_kernel<PB, DG>, 2 * nblocks, lds, st, lc, in, wire, td.signs, td.qjl, td.cs, \
                   td.qa, td.qb, td.seed, td.pbits, td.proj)
        if (lc.diag) return td.pbits == 3 ? PKV_QJL64(3, true) : PKV_QJL64(0, true);
        return td.pbits == 3 ? PKV_QJL64(3, false) : PKV_QJL64(0, false);
#undef PKV_QJL64
    }
    if (td.dim == 128 && td.mode && td.qa && td.pbits <= 4) {
        if (nblocks > (1u << 29)) return hipErrorInvalidValue;   // 4 workgroups per tile
        const size_t lds = static_cast<size_t>(WAVES) * (16 * (lc.plen >> 2) + 4) * sizeof(uint32_t);
#define PKV_QJL128(PB, DG)                                                                                      \
    launch_big_lds(turbo_encode_qjl128_kernel<PB, DG>, 4 * nblocks, lds, st, lc, in, wire, td.signs, td.qjl,   \
                   td.cs, td.qa, td.qb, td.seed, td.pbits, td.proj)
        if (lc.diag) return td.pbits == 3 ? PKV_QJL128(3, true) : PKV_QJL128(0, true);
        return td.pbits == 3 ? PKV_QJL128(3, false) : PKV_QJL128(0, false);
#undef PKV_QJL128
    }
    if (lc.diag) return hipErrorInvalidValue;   // diagnostics exist for the matrix-core paths only
    if (td.dim == 64)
        return td.pbits == 3
                   ? launch_big_lds(turbo_encode_kernel<64, 3>, nblocks, stage_bytes<64>(), st, lc, in, wire, td.signs,
                                    td.qjl, td.cs, td.seed, td.pbits, td.proj, td.mode)
                   : launch_big_lds(turbo_encode_kernel<64, 0>, nblocks, stage_bytes<64>(), st, lc, in, wire, td.signs,
                                    td.qjl, td.cs, td.seed, td.pbits, td.proj, td.mode);
    return td.pbits == 3
               ? launch_big_lds(turbo_encode_kernel<128, 3>, nblocks, stage_bytes<128>(), st, lc, in, wire, td.signs,
                                td.qjl, td.cs, td.seed, td.pbits, td.proj, td.mode)
               : launch_big_lds(turbo_encode_kernel<128, 0>, nblocks, stage_bytes<128>(), st, lc, in, wire, td.signs,
                                td.qjl, td.cs, td.seed, td.pbits, td.proj, td.mode);
}

int launch_turbo_decode(const LaunchCommon& lc, const TurboDev& td, const uint8_t* wire, void* out,
                        uint32_t nblocks, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (td.dim == 64 && td.pbits <= 4) {
        const size_t lds = static_cast<size_t>(WAVES) * turbo_split_wave_words(lc.plen >> 2) * sizeof(uint32_t);
        if (nblocks > (1u << 30)) return hipErrorInvalidValue;   // 2 workgroups per tile
        // a resident grid (four workgroups per CU) walking contiguous shares
        const uint32_t grid = std::min(2 * nblocks, lc.grid_cap ? lc.grid_cap : 1024u);
        return td.pbits == 3 ? launch_big_lds(turbo_decode_split_kernel<3>, grid, lds, st, lc, wire, out,
                                              td.signs, td.cs, td.seed, td.pbits, td.proj, td.mode)
                             : launch_big_lds(turbo_decode_split_kernel<0>, grid, lds, st, lc, wire, out,
                                              td.signs, td.cs, td.seed, td.pbits, td.proj, td.mode);
    }
    if (td.dim == 128 && td.pbits <= 4) {
        if (nblocks > (1u << 29)) return hipErrorInvalidValue;   // 4 workgroups per tile
        const size_t lds = static_cast<size_t>(WAVES) * turbo_split128_wave_words(lc.plen >> 2) * sizeof(uint32_t);
        return td.pbits == 3 ? launch_big_lds(turbo_decode_split128_kernel<3>, 4 * nblocks, lds, st, lc, wire, out,
                                              td.signs, td.cs, td.seed, td.pbits, td.proj)
                             : launch_big_lds(turbo_decode_split128_kernel<0>, 4 * nblocks, lds, st, lc, wire, out,
                                              td.signs, td.cs, td.seed, td.pbits, td.proj);
    }
    if (td.dim == 64)
        return td.pbits == 3
                   ? launch_big_lds(turbo_decode_kernel<64, 3>, nblocks, stage_bytes<64>(), st, lc, wire, out, td.signs,
                                    td.cs, td.seed, td.pbits, td.proj, td.mode)
                   : launch_big_lds(turbo_decode_kernel<64, 0>, nblocks, stage_bytes<64>(), st, lc, wire, out, td.signs,
                                    td.cs, td.seed, td.pbits, td.proj, td.mode);
    return td.pbits == 3
               ? launch_big_lds(turbo_decode_kernel<128, 3>, nblocks, stage_bytes<128>(), st, lc, wire, out, td.signs,
                                td.cs, td.seed, td.pbits, td.proj, td.mode)
               : launch_big_lds(turbo_decode_kernel<128, 0>, nblocks, stage_bytes<128>(), st, lc, wire, out, td.signs,
                                td.cs, td.seed, td.pbits, td.proj, td.mode);
}

int launch_turbo_prepare(const TurboDev& td, const float* q, uint32_t nq, float* out, float rscale,
                         uint32_t* status, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (nq == 0) return hipSuccess;
    if (td.dim == 64)
        hipLaunchKernelGGL(turbo_prepare_kernel<64>, dim3(nq), dim3(WAVE), 0, st, q, nq, out, td.signs, td.qjl,
                           td.proj, td.mode, rscale, status);
    else if (td.dim == 128)
        hipLaunchKernelGGL(turbo_prepare_kernel<128>, dim3(nq), dim3(WAVE), 0, st, q, nq, out, td.signs, td.qjl,
                           td.proj, td.mode, rscale, status);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

int launch_turbo_score(const LaunchCommon& lc, const TurboDev& td, const uint8_t* wire, const float* prepared,
                       uint32_t nq, uint64_t qstride, float* scores, uint64_t ld, float qscale, float post,
                       uint32_t nblocks, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t lds = static_cast<size_t>(WAVES) * (WAVE * (lc.plen >> 2) + 4) * sizeof(uint32_t);
    if (td.pbits < 1 || td.pbits > 8) return hipErrorInvalidValue;
    const uint32_t proj = td.mode ? td.proj : 0u;
#define PKV_SCORE(D, P, LO, NA)                                                                                \
    launch_big_lds(turbo_score_kernel<D, P, LO, NA>, nblocks, lds, st, lc, wire, prepared, nq, qstride, scores, \
                   ld, td.cs, td.seed, td.pbits, td.proj, qscale, post)
#define PKV_SCORE_R(D, P)                                                                                      \
    (lc.radii == PKV_RADII_F32 ? (narrow ? PKV_SCORE(D, P, false, true) : PKV_SCORE(D, P, false, false))        \
                               : (narrow ? PKV_SCORE(D, P, true, true) : PKV_SCORE(D, P, true, false)))
    if ((td.pbits == 3 || td.pbits == 4) && proj <= 32) {   // table path: [pair][bin] terms in LDS
        const size_t stage = static_cast<size_t>(WAVES) * (32 * (lc.plen >> 2) + 4) * sizeof(uint32_t);
        const size_t table = static_cast<size_t>(td.dim / 2) * 16 * sizeof(float);
        const size_t llds = std::max(stage, table);
#define PKV_LUT(D, P, PB)                                                                                      \
    (lc.radii == PKV_RADII_F32                                                                                 \
         ? launch_big_lds(turbo_score_lut_kernel<D, P, false, PB>, nblocks, llds, st, lc, wire, prepared, nq,   \
                          qstride, scores, ld, td.cs, td.seed, td.proj, qscale, post)                           \
         : launch_big_lds(turbo_score_lut_kernel<D, P, true, PB>, nblocks, llds, st, lc, wire, prepared, nq,    \
                          qstride, scores, ld, td.cs, td.seed, td.proj, qscale, post))
        if (td.dim == 64)
            return td.pbits == 3 ? (proj ? PKV_LUT(64, 32, 3) : PKV_LUT(64, 0, 3))
                                 : (proj ? PKV_LUT(64, 32, 4) : PKV_LUT(64, 0, 4));
        if (td.dim == 128)
            return td.pbits == 3 ? (proj ? PKV_LUT(128, 32, 3) : PKV_LUT(128, 0, 3))
                                 : (proj ? PKV_LUT(128, 32, 4) : PKV_LUT(128, 0, 4));
#undef PKV_LUT
        return hipErrorInvalidValue;
    }
    const bool narrow = td.dim == 128 && td.pbits <= 5;
    if (td.dim == 64) {
        if (proj == 0) return lc.radii == PKV_RADII_F32 ? PKV_SCORE(64, 0, false, false) : PKV_SCORE(64, 0, true, false);
        if (proj == 32) return lc.radii == PKV_RADII_F32 ? PKV_SCORE(64, 32, false, false) : PKV_SCORE(64, 32, true, false);
        if (proj == 64) return lc.radii == PKV_RADII_F32 ? PKV_SCORE(64, 64, false, false) : PKV_SCORE(64, 64, true, false);
    } else if (td.dim == 128) {
        if (proj == 0) return PKV_SCORE_R(128, 0);
        if (proj == 32) return PKV_SCORE_R(128, 32);
        if (proj == 64) return PKV_SCORE_R(128, 64);
    }
#undef PKV_SCORE_R
#undef PKV_SCORE
    return hipErrorInvalidValue;
}

// Workgroups of a persistent launch: every workgroup slot of the device
// (compute units x resident workgroups of `kernel`), at most `want`.
template <typename K>
uint32_t persistent_grid(K kernel, size_t dyn_lds, uint32_t want) {
    static std::mutex mu;
    static std::map<std::pair<int, const void*>, uint32_t> slots;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return want;
    const auto key = std::make_pair(dev, reinterpret_cast<const void*>(kernel));
    uint32_t n = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        auto it = slots.find(key);
        if (it != slots.end()) n = it->second;
    }
    if (n == 0) {
        int cus = 0, per_cu = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0 ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(kernel), TILE,
                                                         dyn_lds) != hipSuccess || per_cu <= 0)
            return want;
        n = static_cast<uint32_t>(cus) * static_cast<uint32_t>(per_cu);
        std::lock_guard<std::mutex> lock(mu);
        slots[key] = n;
    }
    return std::max(1u, std::min(n, want));
}

int launch_fib_encode(const LaunchCommon& lc, const FibDev& fd, const void* in, uint8_t* wire, uint32_t nblocks,
                      void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    constexpr size_t lds = (MF_SCA + WAVES * FIB_PAY_WORDS) * sizeof(uint32_t) +
                           WAVES * (FIB_LCAP * sizeof(FibRedoEntry) + 4 * 64 * sizeof(double));
    const uint64_t units = static_cast<uint64_t>(nblocks) * FIB_UNITS_PER_TILE;
    if (units > 0xFFFFFFFFull) return hipErrorInvalidValue;
    const uint32_t want = static_cast<uint32_t>((units + WAVES - 1) / WAVES);
    auto kern = lc.diag ? fib_encode_kernel<64, true> : fib_encode_kernel<64, false>;
    uint32_t grid = persistent_grid(kern, lds, want);
    if (lc.grid_cap) grid = std::min(grid, lc.grid_cap);   // a bounded share of the GPU
    return launch_big_lds(kern, grid, lds, st, lc, in, wire, fd.mf, fd.thr, fd.rot64, fd.codebook,
                          static_cast<uint32_t>(units), lc.segs, lc.tile_start, lc.tile_seg);
}

int launch_fib_decode(const LaunchCommon& lc, const FibDev& fd, const uint8_t* wire, void* out, uint32_t nblocks,
                      void* stream) {
    const uint32_t grid = lc.grid_cap ? std::min(nblocks, lc.grid_cap) : nblocks;
    if (fd.mfma_decode && lc.fanout > 1)
        hipLaunchKernelGGL((fib_decode_mfma_kernel<64, true>), dim3(grid), dim3(TILE), 0,
                           static_cast<hipStream_t>(stream), lc, wire, out, fd.rot32, fd.codebook, lc.segs,
                           lc.tile_start, lc.tile_seg);
    else if (fd.mfma_decode)
        hipLaunchKernelGGL((fib_decode_mfma_kernel<64, false>), dim3(grid), dim3(TILE), 0,
                           static_cast<hipStream_t>(stream), lc, wire, out, fd.rot32, fd.codebook, lc.segs,
                           lc.tile_start, lc.tile_seg);
    else
        hipLaunchKernelGGL(fib_decode_kernel<64>, dim3(nblocks), dim3(TILE), 0, static_cast<hipStream_t>(stream), lc,
                           wire, out, fd.rot32t, fd.codebook);
    return hipGetLastError();
}

int launch_fib_product_check(const float* rot32, const float* cb, uint32_t* bad, void* stream) {
    hipLaunchKernelGGL(fib_product_check_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), rot32, cb, bad);
    return hipGetLastError();
}

}  // namespace pkv
