// pkv_records.hip -- gfx950 kernels for the legacy per-vector wire records
// behind KVecCodec::encode / decode and their batch forms
// (proveKV/src/codec.rs:8-66, 339-413, 582-668): TQW1
// (turbo-quant/src/wire.rs:44-256) and compact FB1
// (fib-quant/src/codec.rs:81-176), plus the f64 inverse rotation of
// FibQuantizer::decode (codec.rs:506-537, rotation.rs:117-128).
//
// A batch of n records is one byte buffer plus n + 1 offsets.  Records are
// reshaped to and from the batched blob layout (TQB1 / FB2: one header, then
// n fixed-size payloads) by byte-shuffle kernels, so the batched encode and
// decode kernels do the codec arithmetic unchanged.  The shuffles move only
// header and payload bytes (23 B per FB1 record, 46 + 144 B per TQW1 record
// at head_dim 64), a few percent of the f32 traffic of the same vectors.
#include <hip/hip_runtime.h>

#include "pkv_internal.h"
#include "pkv_math.h"

namespace pkv {
namespace {

constexpr uint32_t RB_THREADS = 256;
constexpr uint32_t RB_MAX_BLOCKS = 16384;

__device__ __forceinline__ uint32_t hdr_byte(const HdrBytes& h, uint32_t i) {
    return (h.w[i >> 2] >> (8 * (i & 3))) & 0xffu;
}

__device__ __forceinline__ uint64_t grid_threads() {
    return static_cast<uint64_t>(gridDim.x) * blockDim.x;
}

__device__ __forceinline__ uint64_t thread_id() {
    return static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
}

// Blob (header + n payloads) -> n records of rec_hdr constant header bytes
// followed by the payload.  One thread per output dword; the last dword of
// the buffer is written bytewise.
__global__ __launch_bounds__(RB_THREADS) void records_pack_kernel(const uint8_t* __restrict__ pay,
                                                                 uint8_t* __restrict__ out, uint64_t n,
                                                                 uint32_t plen, uint32_t rec_hdr, HdrBytes hdr) {
    const uint64_t rec_len = static_cast<uint64_t>(rec_hdr) + plen;
    const uint64_t total = n * rec_len;
    const uint64_t words = (total + 3) >> 2;
    for (uint64_t w = thread_id(); w < words; w += grid_threads()) {
        uint32_t b[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint64_t p = 4 * w + t;
            b[t] = 0;
            if (p < total) {
                const uint64_t i = p / rec_len;
                const uint32_t j = static_cast<uint32_t>(p - i * rec_len);
                b[t] = j < rec_hdr ? hdr_byte(hdr, j) : pay[i * plen + (j - rec_hdr)];
            }
        }
        if (4 * w + 4 <= total) {
            reinterpret_cast<uint32_t*>(out)[w] = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
        } else {
            for (int t = 0; t < 4; ++t)
                if (4 * w + t < total) out[4 * w + t] = static_cast<uint8_t>(b[t]);
        }
    }
}

__device__ __forceinline__ uint32_t rd_u16(const uint8_t* p) { return p[0] | (p[1] << 8); }
__device__ __forceinline__ uint32_t rd_u32(const uint8_t* p) {
    return p[0] | (p[1] << 8) | (p[2] << 16) | (static_cast<uint32_t>(p[3]) << 24);
}

// Which status word a rejected record goes to.  fb1 != 0 splits failures as
// FibCodeV1::from_compact_bytes (codec.rs:100-176: length, magic, version,
// norm length, index length) -> word 0, from the later checks
// (validate_code_header, decode_norm) -> word 1; TQW1 failures all go to
// word 1 (every check of TurboCodeWireV1::decode sits in one per-record pass).
__device__ __forceinline__ int reject_word(const uint8_t* r, uint64_t len, uint32_t fb1) {
    if (!fb1) return 1;
    bool parse = len >= 11 && r[0] == 'F' && r[1] == 'B' && r[2] == '1' && r[3] == 1;
    if (parse) {
        const uint64_t nlen = rd_u16(r + 9);
        const uint64_t want = (static_cast<uint64_t>(rd_u32(r + 5)) * r[4] + 7) / 8;
        parse = len >= 11 + nlen && len - 11 - nlen == want;
    }
    return parse ? 1 : 0;
}

// One thread per record.  A record is valid iff its length is rec_len and
// its header equals the profile's (every TQW1 / FB1 header field is fixed by
// the profile).
__global__ __launch_bounds__(RB_THREADS) void records_check_kernel(const uint8_t* __restrict__ rec,
                                                                  const uint64_t* __restrict__ off, uint64_t n,
                                                                  uint32_t rec_len, uint32_t rec_hdr, uint32_t fb1,
                                                                  HdrBytes hdr, uint32_t* __restrict__ status) {
    for (uint64_t i = thread_id(); i < n; i += grid_threads()) {
        const uint64_t a = off[i], len = off[i + 1] - a;
        const uint8_t* r = rec + a;
        bool ok = len == rec_len;
        for (uint32_t j = 0; ok && j < rec_hdr; ++j) ok = r[j] == hdr_byte(hdr, j);
        if (!ok) atomicMin(status + reject_word(r, len, fb1), (static_cast<uint32_t>(i) << 4) | KIND_CORRUPT);
    }
}

// The same check when record i sits at i * rec_len (every record the right
// length): one thread per dword of the 4-byte-aligned record buffer compares
// the header bytes it holds; a thread that sees a difference classifies that
// record.
__global__ __launch_bounds__(RB_THREADS) void records_check_packed_kernel(const uint8_t* __restrict__ rec, uint64_t n,
                                                                         uint32_t rec_len, uint32_t rec_hdr,
                                                                         uint32_t fb1, HdrBytes hdr,
                                                                         uint32_t* __restrict__ status) {
    const uint64_t total = n * rec_len;
    const uint64_t words = (total + 3) >> 2;
    const uint32_t* r32 = reinterpret_cast<const uint32_t*>(rec);
    for (uint64_t w = thread_id(); w < words; w += grid_threads()) {
        const uint64_t p0 = 4 * w;
        const uint64_t i0 = p0 / rec_len;
        const uint32_t j0 = static_cast<uint32_t>(p0 - i0 * rec_len);
        // skip dwords that hold no header byte
        if (j0 >= rec_hdr && j0 + 4 <= rec_len) continue;
        const uint32_t v = p0 + 4 <= total ? r32[w] : 0u;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint64_t p = p0 + t;
            if (p >= total) break;
            const uint64_t i = p / rec_len;
            const uint32_t j = static_cast<uint32_t>(p - i * rec_len);
            const uint32_t b = p0 + 4 <= total ? (v >> (8 * t)) & 0xffu : rec[p];
            if (j < rec_hdr && b != hdr_byte(hdr, j))
                atomicMin(status + reject_word(rec + i * rec_len, rec_len, fb1),
                          (static_cast<uint32_t>(i) << 4) | KIND_CORRUPT);
        }
    }
}

// Records -> blob: the blob header bytes, then each record's payload; a
// record of the wrong length contributes zeros (it is already flagged).
// packed != 0: record i sits at i * rec_len (no offset loads).
__global__ __launch_bounds__(RB_THREADS) void records_gather_kernel(const uint8_t* __restrict__ rec,
                                                                   const uint64_t* __restrict__ off, uint64_t n,
                                                                   uint32_t rec_len, uint32_t rec_hdr,
                                                                   uint8_t* __restrict__ blob, uint32_t blob_hdr,
                                                                   HdrBytes bhdr, uint32_t plen, uint32_t packed) {
    const uint64_t total = blob_hdr + n * static_cast<uint64_t>(plen);
    const uint64_t words = (total + 3) >> 2;
    for (uint64_t w = thread_id(); w < words; w += grid_threads()) {
        uint32_t v = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint64_t p = 4 * w + t;
            uint32_t b = 0;
            if (p < blob_hdr) {
                b = hdr_byte(bhdr, static_cast<uint32_t>(p));
            } else if (p < total) {
                const uint64_t i = (p - blob_hdr) / plen;
                const uint32_t j = static_cast<uint32_t>(p - blob_hdr - i * plen);
                if (packed) {
                    b = rec[i * rec_len + rec_hdr + j];
                } else {
                    const uint64_t a = off[i];
                    if (off[i + 1] - a == rec_len) b = rec[a + rec_hdr + j];
                }
            }
            v |= b << (8 * t);
        }
        reinterpret_cast<uint32_t*>(blob)[w] = v;
    }
}

// FibQuantizer::decode (fib-quant/src/codec.rs:506-537), one wave per
// vector: gather the codewords as f64 (codebook.rs:118-131), then
//   out[col] = f32((sum_row M[row][col] * c[row]) * norm)
// with the sum sequential in f64 from 0.0 (StoredRotation::apply_inverse,
// rotation.rs:117-128) and every product and sum rounded separately.  Lane l
// owns column l and keeps it in registers (64 doubles); the vector's 16
// codeword offsets are read back with v_readlane, so the codewords arrive
// through scalar loads and each row step is one v_mul_f64 + one v_add_f64
// with an SGPR operand: no LDS traffic (an LDS-staged M and c moved 1 KiB per
// row step and was bound by the LDS return path).  Checks (index < n, f16
// norm finite and > 0, finite output) flag the vector in status[0].  The
// payload is [f16 norm][16 x bits indices]; 16 * bits is a multiple of 8, so
// there are no padding bits.
__global__ __launch_bounds__(RB_THREADS) void fib_decode_f64_kernel(const uint8_t* __restrict__ pay, uint64_t n,
                                                                   uint32_t plen, const double* __restrict__ rot_t,
                                                                   const double* __restrict__ cb64, uint32_t ncw,
                                                                   uint32_t bits, float* __restrict__ out,
                                                                   uint32_t* __restrict__ status) {
    constexpr int DIM = 64, BLOCKS = 16;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    double m[DIM];   // column `lane` of M; rot_t is [col][row]
    {
        const double2* src = reinterpret_cast<const double2*>(rot_t + lane * DIM);
#pragma unroll
        for (int k = 0; k < DIM / 2; ++k) {
            const double2 v = src[k];
            m[2 * k] = v.x;
            m[2 * k + 1] = v.y;
        }
    }
    const uint64_t nw = static_cast<uint64_t>(gridDim.x) * (RB_THREADS / 64);
    const uint32_t ilen = plen - 2;
    const uint32_t mask = (1u << bits) - 1u;
    for (uint64_t v = static_cast<uint64_t>(blockIdx.x) * (RB_THREADS / 64) + wave; v < n; v += nw) {
        const uint8_t* p = pay + v * plen;
        // lane b < 16: index of block b -> double offset of its codeword
        uint32_t idx = 0;
        if (lane < BLOCKS) {
            const uint32_t bit = bits * static_cast<uint32_t>(lane);
            uint32_t w = p[2 + (bit >> 3)];
            if ((bit >> 3) + 1 < ilen) w |= static_cast<uint32_t>(p[3 + (bit >> 3)]) << 8;
            idx = (w >> (bit & 7)) & mask;
        }
        bool bad = idx >= ncw;
        const uint32_t coff = min(idx, ncw - 1) * 4;
        const float nv = f16_to_f32(static_cast<uint16_t>(__builtin_amdgcn_readfirstlane(rd_u16(p))));
        bad |= !(nv > 0.0f) || (__float_as_uint(nv) & 0x7f800000u) == 0x7f800000u;
        double s = 0.0;
#pragma unroll
        for (int b = 0; b < BLOCKS; ++b) {
            const double* c = cb64 + static_cast<uint64_t>(static_cast<uint32_t>(__builtin_amdgcn_readlane(coff, b)));
#pragma unroll
            for (int t = 0; t < 4; ++t) s = s + m[4 * b + t] * c[t];
        }
        const float o = static_cast<float>(s * static_cast<double>(nv));
        bad |= (__float_as_uint(o) & 0x7f800000u) == 0x7f800000u;
        out[v * DIM + lane] = o;
        if (__ballot(bad) != 0 && lane == 0) atomicMin(status, (static_cast<uint32_t>(v) << 4) | KIND_CORRUPT);
    }
}

uint32_t rb_blocks(uint64_t work) {
    const uint64_t b = (work + RB_THREADS - 1) / RB_THREADS;
    return static_cast<uint32_t>(b < 1 ? 1 : (b > RB_MAX_BLOCKS ? RB_MAX_BLOCKS : b));
}

}  // namespace

int launch_records_pack(const uint8_t* pay, uint8_t* out, uint64_t n, uint32_t plen, uint32_t rec_hdr,
                        const HdrBytes& hdr, void* stream) {
    if (n == 0) return hipSuccess;
    const uint64_t words = (n * (static_cast<uint64_t>(rec_hdr) + plen) + 3) / 4;
    hipLaunchKernelGGL(records_pack_kernel, dim3(rb_blocks(words)), dim3(RB_THREADS), 0,
                       static_cast<hipStream_t>(stream), pay, out, n, plen, rec_hdr, hdr);
    return hipGetLastError();
}

int launch_records_check(const uint8_t* rec, const uint64_t* off, uint64_t n, uint32_t rec_len, uint32_t rec_hdr,
                         uint32_t fb1, bool packed, const HdrBytes& hdr, uint32_t* status, void* stream) {
    if (n == 0) return hipSuccess;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (packed) {
        const uint64_t words = (n * rec_len + 3) / 4;
        hipLaunchKernelGGL(records_check_packed_kernel, dim3(rb_blocks(words)), dim3(RB_THREADS), 0, st, rec, n,
                           rec_len, rec_hdr, fb1, hdr, status);
    } else {
        hipLaunchKernelGGL(records_check_kernel, dim3(rb_blocks(n)), dim3(RB_THREADS), 0, st, rec, off, n, rec_len,
                           rec_hdr, fb1, hdr, status);
    }
    return hipGetLastError();
}

int launch_records_gather(const uint8_t* rec, const uint64_t* off, uint64_t n, uint32_t rec_len, uint32_t rec_hdr,
                          bool packed, uint8_t* blob, uint32_t blob_hdr, const HdrBytes& bhdr, uint32_t plen,
                          void* stream) {
    const uint64_t words = (blob_hdr + n * static_cast<uint64_t>(plen) + 3) / 4;
    hipLaunchKernelGGL(records_gather_kernel, dim3(rb_blocks(words)), dim3(RB_THREADS), 0,
                       static_cast<hipStream_t>(stream), rec, off, n, rec_len, rec_hdr, blob, blob_hdr, bhdr, plen,
                       packed ? 1u : 0u);
    return hipGetLastError();
}

int launch_fib_decode_f64(const FibDev& fd, const uint8_t* pay, uint64_t n, uint32_t plen, float* out,
                          uint32_t* status, void* stream) {
    if (n == 0) return hipSuccess;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (fd.dim != 64) return hipErrorInvalidValue;   // fib profiles are fib_k4_n32 at head_dim 64
    const uint32_t blocks = static_cast<uint32_t>(std::min<uint64_t>((n + 3) / 4, 2048));
    hipLaunchKernelGGL(fib_decode_f64_kernel, dim3(blocks), dim3(RB_THREADS), 0, st, pay, n, plen, fd.rot_t,
                       fd.codebook64, fd.n, fd.bits, out, status);
    return hipGetLastError();
}

}  // namespace pkv
