// pkv_blake3.h -- the BLAKE3 compression function of the digest kernels.
//
// BLAKE3 is the `blake3` crate 1.8.5 that the reference links (its payload and
// layer digests: proveKV/src/codec.rs:85-95, pool.rs:83-103, shell.rs:48-66;
// profile digests: quant-codec-core/src/digest.rs:14-58).  This restates the
// published specification (O'Connor, Aumasson, Neves, Wilcox-O'Hearn, 2020):
// 32-bit words, 7 rounds of the column-then-diagonal G mix, the message
// re-indexed between rounds by a fixed permutation.  Only the unkeyed hash
// with a 32-byte output is used, so only the first 8 output words are formed.
// The compression is host and device code: the host hashes the small JSON
// texts behind the fib profile / codebook / rotation digests with it.
#pragma once
#include <stdint.h>

#include <hip/hip_runtime.h>

namespace pkv {
namespace b3 {

constexpr uint32_t CHUNK_START = 1u, CHUNK_END = 2u, PARENT = 4u, ROOT = 8u;
constexpr uint32_t CHUNK_BYTES = 1024u, BLOCK_BYTES = 64u;

// the SHA-256 initial hash value
#define PKV_B3_IV0 0x6A09E667u
#define PKV_B3_IV1 0xBB67AE85u
#define PKV_B3_IV2 0x3C6EF372u
#define PKV_B3_IV3 0xA54FF53Au
#define PKV_B3_IV4 0x510E527Fu
#define PKV_B3_IV5 0x9B05688Cu
#define PKV_B3_IV6 0x1F83D9ABu
#define PKV_B3_IV7 0x5BE0CD19u

// Message word read at position i of round r: the permutation
// {2,6,3,10,7,0,4,13,1,11,12,5,9,14,15,8} applied r times.  Unrolled code
// indexes the message registers with these constants, so the permutation
// costs nothing on the device.
struct Schedule {
    uint8_t s[7][16];
};
constexpr Schedule make_schedule() {
    constexpr uint8_t perm[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};
    Schedule t{};
    for (int i = 0; i < 16; ++i) t.s[0][i] = static_cast<uint8_t>(i);
    for (int r = 1; r < 7; ++r)
        for (int i = 0; i < 16; ++i) t.s[r][i] = t.s[r - 1][perm[i]];
    return t;
}
constexpr Schedule SCHED = make_schedule();

__host__ __device__ __forceinline__ uint32_t rotr(uint32_t w, uint32_t c) { return (w >> c) | (w << (32u - c)); }

__host__ __device__ __forceinline__ void g(uint32_t& a, uint32_t& b, uint32_t& c, uint32_t& d, uint32_t mx, uint32_t my) {
    a = a + b + mx;
    d = rotr(d ^ a, 16);
    c = c + d;
    b = rotr(b ^ c, 12);
    a = a + b + my;
    d = rotr(d ^ a, 8);
    c = c + d;
    b = rotr(b ^ c, 7);
}

// cv <- first 8 words of compress(cv, m, counter, block_len, flags).
__host__ __device__ __forceinline__ void compress(uint32_t cv[8], const uint32_t m[16], uint64_t counter, uint32_t block_len,
                                         uint32_t flags) {
    uint32_t v0 = cv[0], v1 = cv[1], v2 = cv[2], v3 = cv[3], v4 = cv[4], v5 = cv[5], v6 = cv[6], v7 = cv[7];
    uint32_t v8 = PKV_B3_IV0, v9 = PKV_B3_IV1, v10 = PKV_B3_IV2, v11 = PKV_B3_IV3;
    uint32_t v12 = static_cast<uint32_t>(counter), v13 = static_cast<uint32_t>(counter >> 32);
    uint32_t v14 = block_len, v15 = flags;
#define PKV_B3_ROUND(R)                                                          \
    g(v0, v4, v8, v12, m[SCHED.s[R][0]], m[SCHED.s[R][1]]);                      \
    g(v1, v5, v9, v13, m[SCHED.s[R][2]], m[SCHED.s[R][3]]);                      \
    g(v2, v6, v10, v14, m[SCHED.s[R][4]], m[SCHED.s[R][5]]);                     \
    g(v3, v7, v11, v15, m[SCHED.s[R][6]], m[SCHED.s[R][7]]);                     \
    g(v0, v5, v10, v15, m[SCHED.s[R][8]], m[SCHED.s[R][9]]);                     \
    g(v1, v6, v11, v12, m[SCHED.s[R][10]], m[SCHED.s[R][11]]);                   \
    g(v2, v7, v8, v13, m[SCHED.s[R][12]], m[SCHED.s[R][13]]);                    \
    g(v3, v4, v9, v14, m[SCHED.s[R][14]], m[SCHED.s[R][15]]);
    PKV_B3_ROUND(0)
    PKV_B3_ROUND(1)
    PKV_B3_ROUND(2)
    PKV_B3_ROUND(3)
    PKV_B3_ROUND(4)
    PKV_B3_ROUND(5)
    PKV_B3_ROUND(6)
#undef PKV_B3_ROUND
    cv[0] = v0 ^ v8;
    cv[1] = v1 ^ v9;
    cv[2] = v2 ^ v10;
    cv[3] = v3 ^ v11;
    cv[4] = v4 ^ v12;
    cv[5] = v5 ^ v13;
    cv[6] = v6 ^ v14;
    cv[7] = v7 ^ v15;
}

__host__ __device__ __forceinline__ void set_iv(uint32_t cv[8]) {
    cv[0] = PKV_B3_IV0; cv[1] = PKV_B3_IV1; cv[2] = PKV_B3_IV2; cv[3] = PKV_B3_IV3;
    cv[4] = PKV_B3_IV4; cv[5] = PKV_B3_IV5; cv[6] = PKV_B3_IV6; cv[7] = PKV_B3_IV7;
}

// Parent node: key = IV, message = left cv || right cv, counter 0, 64 bytes.
__host__ __device__ __forceinline__ void parent(uint32_t l[8], const uint32_t r[8], uint32_t extra_flags) {
    uint32_t m[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        m[i] = l[i];
        m[8 + i] = r[i];
    }
    set_iv(l);
    compress(l, m, 0, BLOCK_BYTES, PARENT | extra_flags);
}

// Chunks a range of `len` bytes splits into (an empty range is one empty chunk).
__host__ __device__ __forceinline__ uint64_t chunks_of(uint64_t len) {
    return len == 0 ? 1 : (len + CHUNK_BYTES - 1) / CHUNK_BYTES;
}

}  // namespace b3
}  // namespace pkv
