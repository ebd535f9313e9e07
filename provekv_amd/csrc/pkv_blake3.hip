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

// ---- four lanes per chunk (wires with too few chunks to fill the GPU one
// lane per chunk)
//
// Lane i of a quad holds column i of the compression state: a = v[i],
// b = v[4 + i], c = v[8 + i], d = v[12 + i].  The column step is the quad's
// four G at once; for the diagonal step lane i needs b, c, d of lanes i + 1,
// i + 2, i + 3 (mod 4), brought by DPP quad rotations and sent back after.
// The chaining value stays split the same way (lane i: words i and 4 + i),
// so blocks chain without moving data between lanes.  Message words come from
// the quad's 64-byte block in LDS; lane i's four words of round r are
// m[s_r(2i)], m[s_r(2i + 1)], m[s_r(8 + 2i)], m[s_r(9 + 2i)], whose LDS
// addresses are computed once per kernel.

__device__ __forceinline__ void wave_sync_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// DPP quad rotations: lane i reads lane i + 1, i + 2, i + 3 (mod 4)
__device__ __forceinline__ uint32_t qrot1(uint32_t x) { return __builtin_amdgcn_mov_dpp(x, 0x39, 0xf, 0xf, false); }
__device__ __forceinline__ uint32_t qrot2(uint32_t x) { return __builtin_amdgcn_mov_dpp(x, 0x4e, 0xf, 0xf, false); }
__device__ __forceinline__ uint32_t qrot3(uint32_t x) { return __builtin_amdgcn_mov_dpp(x, 0x93, 0xf, 0xf, false); }

__device__ __forceinline__ void g1(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d, uint32_t mx, uint32_t my) {
    b3::g(a, b, c, d, mx, my);
}

// Word indices (0..15) of lane i's four message words in each round.
struct QuadMsgIdx {
    uint32_t w[7][4];
};
__device__ __forceinline__ QuadMsgIdx quad_msg_idx(uint32_t i) {
    QuadMsgIdx q;
#pragma unroll
    for (int r = 0; r < 7; ++r) {
        const uint8_t* s = b3::SCHED.s[r];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            q.w[r][k] = i == 0 ? s[k] : i == 1 ? s[2 + k] : i == 2 ? s[4 + k] : s[6 + k];
            q.w[r][2 + k] = i == 0 ? s[8 + k] : i == 1 ? s[10 + k] : i == 2 ? s[12 + k] : s[14 + k];
        }
    }
    return q;
}

// One compression on the quad.  (cv_lo, cv_hi) = chaining value words
// (i, 4 + i) in and out; message word k is word(k), read from LDS.
template <typename Word>
__device__ __forceinline__ void quad_compress(uint32_t& cv_lo, uint32_t& cv_hi, uint32_t i, const QuadMsgIdx& q,
                                              Word word, uint64_t counter, uint32_t block_len, uint32_t flags) {
    uint32_t a = cv_lo, b = cv_hi;
    uint32_t c = i == 0 ? PKV_B3_IV0 : i == 1 ? PKV_B3_IV1 : i == 2 ? PKV_B3_IV2 : PKV_B3_IV3;
    uint32_t d = i == 0 ? static_cast<uint32_t>(counter)
               : i == 1 ? static_cast<uint32_t>(counter >> 32)
               : i == 2 ? block_len
                        : flags;
#pragma unroll
    for (int r = 0; r < 7; ++r) {
        const uint32_t mx = word(q.w[r][0]), my = word(q.w[r][1]);
        const uint32_t nx = word(q.w[r][2]), ny = word(q.w[r][3]);
        g1(a, b, c, d, mx, my);
        b = qrot1(b);
        c = qrot2(c);
        d = qrot3(d);
        g1(a, b, c, d, nx, ny);
        b = qrot3(b);
        c = qrot2(c);
        d = qrot1(d);
    }
    cv_lo = a ^ c;
    cv_hi = b ^ d;
}

}  // namespace

// The first pass with one lane per chunk: one wave per tile of 64 chunks of
// one range (pass table: B3Pass per range plus a sentinel whose tile_start
// is the pass's tile count); the wave merges its 64 chaining values.
__global__ __launch_bounds__(256) void blake3_tree_kernel(const uint8_t* __restrict__ buf,
                                                          const B3Range* __restrict__ ranges,
                                                          const B3Pass* __restrict__ pass, uint32_t nr,
                                                          uint32_t* __restrict__ cv_out, uint32_t* __restrict__ out) {
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
        const B3Range rg = ranges[r];
        chunk_cv(buf + rg.offset, rg.len, first + lane, ps.count == 1u, cv);
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

// Pass 0 with four lanes per chunk: 16 chunks per wave (one per quad), then
// the wave merges its 16 chaining values over four levels, one parent per
// active quad.  Tiles are 16 chunks; a range of at most 16 chunks ends here.
__global__ __launch_bounds__(256) void blake3_quad_kernel(const uint8_t* __restrict__ buf,
                                                          const B3Range* __restrict__ ranges,
                                                          const B3Pass* __restrict__ pass, uint32_t nr,
                                                          uint32_t* __restrict__ cv_out, uint32_t* __restrict__ out) {
    __shared__ uint32_t blk_s[4][16][16];   // per wave, per quad: the current 64-byte block
    __shared__ uint32_t cv_s[4][16][8];     // per wave, per quad: its chaining value
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t quad = lane >> 2, i = lane & 3u;
    const uint32_t tile = __builtin_amdgcn_readfirstlane(blockIdx.x * 4u + wave);
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
    const uint32_t first = g * 16u;
    const uint32_t nq = ps.count - first < 16u ? ps.count - first : 16u;   // quads with a chunk
    const bool root_group = ps.count <= 16u;
    const QuadMsgIdx qi = quad_msg_idx(i);
    const uint32_t* my_blk = blk_s[wave][quad];

    uint32_t cv_lo = i == 0 ? PKV_B3_IV0 : i == 1 ? PKV_B3_IV1 : i == 2 ? PKV_B3_IV2 : PKV_B3_IV3;
    uint32_t cv_hi = i == 0 ? PKV_B3_IV4 : i == 1 ? PKV_B3_IV5 : i == 2 ? PKV_B3_IV6 : PKV_B3_IV7;
    {
        const B3Range rg = ranges[r];
        const uint64_t chunk = first + (quad < nq ? quad : 0u);
        const uint64_t start = chunk * b3::CHUNK_BYTES;
        const uint64_t left = rg.len - start;
        const uint32_t clen = left < b3::CHUNK_BYTES ? static_cast<uint32_t>(left) : b3::CHUNK_BYTES;
        // the wave runs as many blocks as its longest chunk (every chunk but
        // a range's last is whole: 16 blocks); quads past nq and a shorter
        // last chunk idle through the rest
        const uint32_t nblk = clen == 0 ? 1u : (clen + 63u) / 64u;
        const uint32_t wblk = nq > 1u ? 16u : __builtin_amdgcn_readfirstlane(nblk);
        const uint8_t* base = buf + rg.offset + start;
        const uint32_t sh = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(base) & 3u);
        const uint32_t* p = reinterpret_cast<const uint32_t*>(base - sh);
        const bool root = ps.count == 1u;
        for (uint32_t b = 0; b < wblk; ++b) {
            const bool live = quad < nq && b < nblk;
            const uint32_t blen = clen - 64u * b < 64u ? clen - 64u * b : 64u;
            // lane i: message words 4i .. 4i + 3 from dwords 4i .. 4i + 4 of the block
            uint32_t dw[5] = {0u, 0u, 0u, 0u, 0u};
            if (live) {
                const uint32_t nd = blen ? (sh + blen + 3u) >> 2 : 0u;
#pragma unroll
                for (uint32_t k = 0; k < 5; ++k)
                    if (4u * i + k < nd) dw[k] = p[16u * b + 4u * i + k];
            }
            uint32_t w[4];
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                w[j] = __builtin_amdgcn_alignbyte(dw[j + 1], dw[j], sh);
                const int rem = static_cast<int>(blen) - static_cast<int>(4u * (4u * i + j));
                w[j] = rem >= 4 ? w[j] : rem <= 0 ? 0u : (w[j] & ((1u << (8 * rem)) - 1u));
            }
            *reinterpret_cast<uint4*>(&blk_s[wave][quad][4u * i]) = make_uint4(w[0], w[1], w[2], w[3]);
            wave_sync_lds();
            uint32_t flags = b == 0 ? b3::CHUNK_START : 0u;
            if (b == nblk - 1) flags |= b3::CHUNK_END | (root ? b3::ROOT : 0u);
            uint32_t nlo = cv_lo, nhi = cv_hi;
            quad_compress(nlo, nhi, i, qi, [&](uint32_t k) { return my_blk[k]; }, chunk, blen, flags);
            if (live) {
                cv_lo = nlo;
                cv_hi = nhi;
            }
            wave_sync_lds();   // every quad has read its block before the next one lands
        }
    }
    // merge the quads' chaining values: level s pairs quads q, q + s
    cv_s[wave][quad][i] = cv_lo;
    cv_s[wave][quad][4u + i] = cv_hi;
    wave_sync_lds();
    for (uint32_t s = 1; s < nq; s <<= 1) {
        const uint32_t c = (nq + s - 1u) / s;
        const bool act = (quad & (2u * s - 1u)) == 0u && quad / s + 1u < c;
        const uint32_t partner = act ? quad + s : quad;
        uint32_t plo = i == 0 ? PKV_B3_IV0 : i == 1 ? PKV_B3_IV1 : i == 2 ? PKV_B3_IV2 : PKV_B3_IV3;
        uint32_t phi = i == 0 ? PKV_B3_IV4 : i == 1 ? PKV_B3_IV5 : i == 2 ? PKV_B3_IV6 : PKV_B3_IV7;
        const uint32_t* left = cv_s[wave][quad];
        const uint32_t* right = cv_s[wave][partner];
        quad_compress(plo, phi, i, qi, [&](uint32_t k) { return k < 8u ? left[k] : right[k - 8u]; }, 0,
                      b3::BLOCK_BYTES, b3::PARENT | (root_group && c == 2u ? b3::ROOT : 0u));
        wave_sync_lds();   // all reads of this level done
        if (act) {
            cv_s[wave][quad][i] = plo;
            cv_s[wave][quad][4u + i] = phi;
        }
        wave_sync_lds();
    }
    if (quad == 0) {   // out is only 4-byte aligned
        uint32_t* dst = root_group ? out + 8ull * r : cv_out + 8ull * (ps.out_base + g);
        dst[i] = cv_s[wave][0][i];
        dst[4u + i] = cv_s[wave][0][4u + i];
    }
}

// A merge pass (after the leaf pass) with four lanes per compression: one
// workgroup per tile of 64 values of one range.  Wave w merges values
// 16w .. 16w + 15 of the tile on its quads, level by level as
// blake3_quad_kernel does, then wave 0 merges the waves' results the same
// way -- together the pairwise level-by-level order over the 64 values (an
// aligned 16-value group is the first four levels).  A single lane per
// compression leaves one wave per range chaining whole compressions, which is
// most of a small wire's digest time.
__global__ __launch_bounds__(256) void blake3_merge4_kernel(const B3Pass* __restrict__ pass, uint32_t nr,
                                                            const uint32_t* __restrict__ cv_in,
                                                            uint32_t* __restrict__ cv_out, uint32_t* __restrict__ out) {
    __shared__ uint32_t cv_s[4][16][8];   // per wave, per quad: a chaining value
    const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63u;
    const uint32_t quad = lane >> 2, i = lane & 3u;
    const uint32_t tile = blockIdx.x;
    if (tile >= pass[nr].tile_start) return;   // the whole workgroup leaves
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
    const uint32_t nw = ps.count - first < 64u ? ps.count - first : 64u;   // values of this tile (>= 1)
    const bool root_group = ps.count <= 64u;
    const QuadMsgIdx qi = quad_msg_idx(i);
    // level-by-level merge of the n chaining values in cv_s[wv][0 .. n) on
    // wave wv's quads; `last` when these n values are the whole range
    auto merge = [&](uint32_t wv, uint32_t n, bool last) {
        for (uint32_t s = 1; s < n; s <<= 1) {
            const uint32_t c = (n + s - 1u) / s;
            const bool act = (quad & (2u * s - 1u)) == 0u && quad / s + 1u < c;
            const uint32_t partner = act ? quad + s : quad;
            uint32_t plo = i == 0 ? PKV_B3_IV0 : i == 1 ? PKV_B3_IV1 : i == 2 ? PKV_B3_IV2 : PKV_B3_IV3;
            uint32_t phi = i == 0 ? PKV_B3_IV4 : i == 1 ? PKV_B3_IV5 : i == 2 ? PKV_B3_IV6 : PKV_B3_IV7;
            const uint32_t* left = cv_s[wv][quad];
            const uint32_t* right = cv_s[wv][partner];
            quad_compress(plo, phi, i, qi, [&](uint32_t k) { return k < 8u ? left[k] : right[k - 8u]; }, 0,
                          b3::BLOCK_BYTES, b3::PARENT | (last && c == 2u ? b3::ROOT : 0u));
            wave_sync_lds();   // all reads of this level done
            if (act) {
                cv_s[wv][quad][i] = plo;
                cv_s[wv][quad][4u + i] = phi;
            }
            wave_sync_lds();
        }
    };
    const uint32_t base = 16u * wave;
    const uint32_t nq = nw > base ? (nw - base < 16u ? nw - base : 16u) : 0u;   // this wave's values
    if (quad < nq) {
        const uint32_t* src = cv_in + 8ull * (ps.in_base + first + base + quad);
        cv_s[wave][quad][i] = src[i];
        cv_s[wave][quad][4u + i] = src[4u + i];
    }
    wave_sync_lds();
    if (nq > 1) merge(wave, nq, root_group && nw <= 16u);
    __syncthreads();
    const uint32_t ng = (nw + 15u) / 16u;   // waves that held values
    if (wave == 0) {
        if (ng > 1) {
            // the waves' results become quads 0 .. ng - 1 of wave 0
            uint32_t wlo = 0, whi = 0;
            if (quad < ng) {
                wlo = cv_s[quad][0][i];
                whi = cv_s[quad][0][4u + i];
            }
            wave_sync_lds();
            if (quad < ng) {
                cv_s[0][quad][i] = wlo;
                cv_s[0][quad][4u + i] = whi;
            }
            wave_sync_lds();
            merge(0, ng, root_group);
        }
        if (quad == 0) {   // out is only 4-byte aligned
            uint32_t* dst = root_group ? out + 8ull * r : cv_out + 8ull * (ps.out_base + g);
            dst[i] = cv_s[0][0][i];
            dst[4u + i] = cv_s[0][0][4u + i];
        }
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
                       uint32_t* cv_out, uint32_t* out, void* stream) {
    if (tiles == 0) return hipSuccess;
    const uint32_t grid = (tiles + 3u) / 4u;
    hipLaunchKernelGGL(blake3_tree_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream), buf, ranges,
                       pass, nr, cv_out, out);
    return hipGetLastError();
}

int launch_blake3_quad(const uint8_t* buf, const B3Range* ranges, const B3Pass* pass, uint32_t nr, uint32_t tiles,
                       uint32_t* cv_out, uint32_t* out, void* stream) {
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(blake3_quad_kernel, dim3((tiles + 3u) / 4u), dim3(256), 0, static_cast<hipStream_t>(stream), buf,
                       ranges, pass, nr, cv_out, out);
    return hipGetLastError();
}

int launch_blake3_merge4(const B3Pass* pass, uint32_t nr, uint32_t tiles, const uint32_t* cv_in, uint32_t* cv_out,
                         uint32_t* out, void* stream) {
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(blake3_merge4_kernel, dim3(tiles), dim3(256), 0, static_cast<hipStream_t>(stream), pass, nr,
                       cv_in, cv_out, out);
    return hipGetLastError();
}

int launch_blake3_layers(const uint32_t* kv, uint32_t n, uint32_t layers, uint32_t* out, void* stream) {
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(blake3_layer_kernel, dim3((n + 63u) / 64u), dim3(64), 0, static_cast<hipStream_t>(stream), kv,
                       n, layers, out);
    return hipGetLastError();
}

}  // namespace pkv
