// pkv_blake3.hip -- BLAKE3 digests of device-resident byte ranges (the TQB1 /
// FB2 payloads of a pool or of shells, where the encode wrote them) and the
// pool / shell layer digests built from them.
//
// Reference call sites (blake3 1.8.5, lower-case hex of the 32-byte hash):
//   CompressedBlock::new       proveKV/src/codec.rs:85-95   blake3(payload)
//   PoolLayer::compute_digest  proveKV/src/pool.rs:83-103   blake3(layer JSON)
//   ShellLayer::compute_digest proveKV/src/shell.rs:48-66   (same JSON)
// The reference hashes each payload on one host core after copying it back;
// here the payloads never leave HBM.
//
// Tree (the BLAKE3 specification, §2.3-2.4): a range is cut into 1024-byte
// chunks, each chained through its 64-byte blocks into a chaining value; the
// chaining values are merged by parent nodes into the left-complete binary
// tree, which is what merging neighbours pairwise level by level gives when an
// unpaired last element is carried up unchanged.  Any aligned run of 64
// elements of one level therefore reduces to one element of the level six
// above, independently of the rest, and one launch does that for every range:
//   pass 0     lane = chunk (64 chunks per wave, one range per wave): chain the
//              chunk's blocks, then merge the wave's 64 chaining values over
//              six levels with cross-lane shuffles;
//   pass p>0   lane = chaining value of pass p-1, merged the same way.
// A range whose elements of a pass fit one wave ends in that pass: its last
// merge (or, for a one-chunk range, its last block) carries the ROOT flag and
// lane 0 writes the hash.  Ranges of up to 64 KiB take one launch, up to
// 4 MiB two.  Roofline: VALU -- 7 rounds x 8 G x 12 operations per 64-byte
// block, about 680 lane operations, ~10.6 per byte, against 8 bytes per
// operation that HBM would need to be the bound.
#include <hip/hip_runtime.h>

#include "pkv_blake3.h"
#include "pkv_internal.h"

namespace pkv {

namespace {

// 16 message dwords (plus one when the base is misaligned) of a block of
// blen bytes at dword-aligned p: each dword read holds at least one byte of
// the range, so no load touches a page the range does not.
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ void load_block(const uint32_t* p, uint32_t blen, uint32_t sh, uint32_t dw[17]) {
    if (blen == 64u) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const u32x4_a4 v = *reinterpret_cast<const u32x4_a4*>(p + 4 * q);
            dw[4 * q] = v.x;
            dw[4 * q + 1] = v.y;
            dw[4 * q + 2] = v.z;
            dw[4 * q + 3] = v.w;
        }
        dw[16] = sh ? p[16] : 0u;   // holds the block's last bytes when misaligned
    } else {
        const uint32_t nd = blen ? (sh + blen + 3u) >> 2 : 0u;
#pragma unroll
        for (int k = 0; k < 17; ++k) dw[k] = static_cast<uint32_t>(k) < nd ? p[k] : 0u;
    }
}

// Chaining value (or, with root, the hash) of chunk `chunk` of the range
// [base, base + len).  v_alignbyte shifts the dwords into place for a
// misaligned base; the next block's loads are issued before this block's
// compression, so one wave per SIMD still overlaps memory with the rounds.
__device__ __forceinline__ void chunk_cv(const uint8_t* base, uint64_t len, uint64_t chunk, bool root,
                                         uint32_t cv[8]) {
    const uint64_t start = chunk * b3::CHUNK_BYTES;
    const uint64_t left = len - start;
    const uint32_t clen = left < b3::CHUNK_BYTES ? static_cast<uint32_t>(left) : b3::CHUNK_BYTES;
    const uint32_t nblk = clen == 0 ? 1u : (clen + 63u) / 64u;
    const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(base + start) & 3u);
    const uint32_t* p = reinterpret_cast<const uint32_t*>(base + start - sh);   // pointer arithmetic: global loads
    b3::set_iv(cv);
    uint32_t nxt[17];
    load_block(p, clen < 64u ? clen : 64u, sh, nxt);
    for (uint32_t b = 0; b < nblk; ++b) {
        const uint32_t blen = clen - 64u * b < 64u ? clen - 64u * b : 64u;
        uint32_t dw[17];
#pragma unroll
        for (int k = 0; k < 17; ++k) dw[k] = nxt[k];
        if (b + 1 < nblk) {
            const uint32_t rest = clen - 64u * (b + 1);
            load_block(p + 16 * (b + 1), rest < 64u ? rest : 64u, sh, nxt);
        }
        uint32_t m[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) m[i] = __builtin_amdgcn_alignbyte(dw[i + 1], dw[i], sh);
        if (blen < 64u) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int rem = static_cast<int>(blen) - 4 * i;
                m[i] = rem >= 4 ? m[i] : rem <= 0 ? 0u : (m[i] & ((1u << (8 * rem)) - 1u));
            }
        }
        uint32_t flags = b == 0 ? b3::CHUNK_START : 0u;
        if (b == nblk - 1) flags |= b3::CHUNK_END | (root ? b3::ROOT : 0u);
        b3::compress(cv, m, chunk, blen, flags);
    }
}

}  // namespace

// One wave per tile of 64 elements of one range (pass table: B3Pass per range
// plus a sentinel whose tile_start is the pass's tile count).
__global__ __launch_bounds__(256) void blake3_tree_kernel(const uint8_t* __restrict__ buf,
                                                          const B3Range* __restrict__ ranges,
                                                          const B3Pass* __restrict__ pass, uint32_t nr,
                                                          const uint32_t* __restrict__ cv_in,
                                                          uint32_t* __restrict__ cv_out, uint32_t* __restrict__ out,
                                                          uint32_t leaf) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t tile = __builtin_amdgcn_readfirstlane(blockIdx.x * 4u + (threadIdx.x >> 6));
    if (tile >= pass[nr].tile_start) return;
    uint32_t lo = 0, hi = nr;   // pass[lo].tile_start <= tile < pass[hi].tile_start
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (pass[mid].tile_start <= tile) lo = mid;
        else hi = mid;
    }
    const uint32_t r = lo;
    const B3Pass ps = pass[r];
    const uint32_t g = tile - ps.tile_start;
    const uint32_t first = g * 64u;
    const uint32_t nw = ps.count - first < 64u ? ps.count - first : 64u;
    const bool root_group = ps.count <= 64u;
    uint32_t cv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (lane < nw) {
        if (leaf) {
            const B3Range rg = ranges[r];
            chunk_cv(buf + rg.offset, rg.len, first + lane, ps.count == 1u, cv);
        } else {
            const uint4* src = reinterpret_cast<const uint4*>(cv_in + 8ull * (ps.in_base + first + lane));
            const uint4 x = src[0], y = src[1];
            cv[0] = x.x; cv[1] = x.y; cv[2] = x.z; cv[3] = x.w;
            cv[4] = y.x; cv[5] = y.y; cv[6] = y.z; cv[7] = y.w;
        }
    }
    // level s: elements are the lanes that are multiples of s, ceil(nw / s) of
    // them; even element e absorbs element e + 1 when it exists
    for (uint32_t s = 1; s < nw; s <<= 1) {
        uint32_t o[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = __shfl_down(cv[i], s, 64);
        const uint32_t c = (nw + s - 1u) / s;
        if ((lane & (2u * s - 1u)) == 0u && lane / s + 1u < c)
            b3::parent(cv, o, root_group && c == 2u ? b3::ROOT : 0u);
    }
    if (lane == 0) {   // out is only 4-byte aligned
        uint32_t* dst = root_group ? out + 8ull * r : cv_out + 8ull * (ps.out_base + g);
#pragma unroll
        for (int i = 0; i < 8; ++i) dst[i] = cv[i];
    }
}

// Layer digests: entry i holds the payload digests of layer i % layers, key
// then value (16 words); out[i] = blake3 of serde_json's compact text of
// json!({"layer_index", "key_digests": [k], "value_digests": [v]}) -- a
// BTreeMap (serde_json without preserve_order), so the keys print sorted:
//   {"key_digests":["<64 hex>"],"layer_index":<decimal>,"value_digests":["<64 hex>"]}
// At most 194 bytes: one chunk of four blocks, hashed by one lane.
__global__ __launch_bounds__(64) void blake3_layer_kernel(const uint32_t* __restrict__ kv, uint32_t n,
                                                          uint32_t layers, uint32_t* __restrict__ out) {
    __shared__ uint32_t text[64][65];   // one 256-byte row per lane (+1 word: no bank conflicts)
    const uint32_t i = blockIdx.x * 64u + threadIdx.x;
    if (i >= n) return;
    uint32_t* row = text[threadIdx.x];
    for (int w = 0; w < 64; ++w) row[w] = 0u;
    uint32_t pos = 0;
    auto put = [&](uint32_t byte) {
        row[pos >> 2] |= byte << (8u * (pos & 3u));
        ++pos;
    };
    auto put_str = [&](const char* s) {
        for (; *s; ++s) put(static_cast<uint8_t>(*s));
    };
    auto put_hex = [&](const uint32_t* d) {
        for (int j = 0; j < 32; ++j) {
            const uint32_t byte = (d[j >> 2] >> (8 * (j & 3))) & 255u;
            const uint32_t hi = byte >> 4, lo = byte & 15u;
            put(hi < 10u ? '0' + hi : 'a' + hi - 10u);
            put(lo < 10u ? '0' + lo : 'a' + lo - 10u);
        }
    };
    uint32_t d[16];
#pragma unroll
    for (int w = 0; w < 16; ++w) d[w] = kv[16ull * i + w];
    put_str("{\"key_digests\":[\"");
    put_hex(d);
    put_str("\"],\"layer_index\":");
    uint32_t li = i % layers, digits[10], nd = 0;
    do {
        digits[nd++] = li % 10u;
        li /= 10u;
    } while (li);
    while (nd) put('0' + digits[--nd]);
    put_str(",\"value_digests\":[\"");
    put_hex(d + 8);
    put_str("\"]}");
    const uint32_t len = pos, nblk = (len + 63u) / 64u;
    uint32_t cv[8];
    b3::set_iv(cv);
    for (uint32_t b = 0; b < nblk; ++b) {
        uint32_t m[16];
#pragma unroll
        for (int w = 0; w < 16; ++w) m[w] = row[16 * b + w];
        uint32_t flags = b == 0 ? b3::CHUNK_START : 0u;
        if (b == nblk - 1) flags |= b3::CHUNK_END | b3::ROOT;
        b3::compress(cv, m, 0, b == nblk - 1 ? len - 64u * b : 64u, flags);
    }
    uint32_t* dst = out + 8ull * i;
#pragma unroll
    for (int w = 0; w < 8; ++w) dst[w] = cv[w];
}

int launch_blake3_pass(const uint8_t* buf, const B3Range* ranges, const B3Pass* pass, uint32_t nr, uint32_t tiles,
                       const uint32_t* cv_in, uint32_t* cv_out, uint32_t* out, bool leaf, void* stream) {
    if (tiles == 0) return hipSuccess;
    const uint32_t grid = (tiles + 3u) / 4u;
    hipLaunchKernelGGL(blake3_tree_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), buf, ranges, pass, nr, cv_in, cv_out,
                       out, leaf ? 1u : 0u);
    return hipGetLastError();
}

int launch_blake3_layers(const uint32_t* kv, uint32_t n, uint32_t layers, uint32_t* out, void* stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(blake3_layer_kernel, dim3((n + 63u) / 64u), dim3(64), 0, static_cast<hipStream_t>(stream), kv,
                       n, layers, out);
    return hipGetLastError();
}

}  // namespace pkv
