/* CPU restatement of BLAKE3 (unkeyed hash, 32-byte output) and of the proveKV
 * digests built on it.  TEST INFRASTRUCTURE ONLY: tests/ and bench.py's
 * cpu_baseline leg use it as the checker; the product never links it.
 *
 * BLAKE3 is the `blake3` crate, version 1.8.5 (the reference's Cargo.lock
 * pins it; the crate is not vendored under the reference).  This file
 * restates its published algorithm (the BLAKE3 specification, O'Connor,
 * Aumasson, Neves, Wilcox-O'Hearn, 2020: compression function §2.2, chunk
 * chaining §2.3, tree §2.4) in the style of the specification's incremental
 * hasher: chunk states fed byte by byte, and a stack of chaining values merged
 * whenever a completed subtree is known to be complete (the count of chunks
 * finished so far has a trailing zero bit).  The device kernels build the
 * same tree level by level instead, and the tests also hold a third,
 * recursive form (left subtree = the largest power-of-two number of chunks
 * that leaves at least one for the right).
 *
 * Call sites restated (all hash with blake3::hash and print lower-case hex):
 *   CompressedBlock::new          proveKV/src/codec.rs:85-95   (payload digest)
 *   PoolLayer::compute_digest     proveKV/src/pool.rs:83-103   (layer digest)
 *   ShellLayer::compute_digest    proveKV/src/shell.rs:48-66   (same JSON)
 *   CodecProfileDigest::from_parts quant-codec-core/src/digest.rs:20-27
 * The layer digest hashes serde_json::to_string of json!({layer_index,
 * key_digests, value_digests}).  serde_json 1.0.150 is built without its
 * preserve_order feature (the lock file gives it no indexmap dependency), so
 * the object is a BTreeMap and prints its keys sorted, compactly:
 *   {"key_digests":["<hex>",...],"layer_index":N,"value_digests":["<hex>",...]}
 */
#include <stddef.h>
#include <stdint.h>
#include <string.h>
#include <stdio.h>

#define B3_CHUNK_START 1u
#define B3_CHUNK_END 2u
#define B3_PARENT 4u
#define B3_ROOT 8u

/* the SHA-256 initial hash value, BLAKE3's IV (spec Table 1) */
static const uint32_t B3_IV[8] = {0x6A09E667u, 0xBB67AE85u, 0x3C6EF372u, 0xA54FF53Au,
                                  0x510E527Fu, 0x9B05688Cu, 0x1F83D9ABu, 0x5BE0CD19u};
/* message word permutation applied between rounds (spec Table 2) */
static const uint8_t B3_PERM[16] = {2, 6, 3, 10, 7, 0, 4, 13, 1, 11, 12, 5, 9, 14, 15, 8};

static uint32_t rotr32(uint32_t w, unsigned c) { return (w >> c) | (w << (32 - c)); }

static void b3_g(uint32_t v[16], int a, int b, int c, int d, uint32_t mx, uint32_t my) {
    v[a] = v[a] + v[b] + mx;
    v[d] = rotr32(v[d] ^ v[a], 16);
    v[c] = v[c] + v[d];
    v[b] = rotr32(v[b] ^ v[c], 12);
    v[a] = v[a] + v[b] + my;
    v[d] = rotr32(v[d] ^ v[a], 8);
    v[c] = v[c] + v[d];
    v[b] = rotr32(v[b] ^ v[c], 7);
}

/* The compression function: 7 rounds of column then diagonal G over the
 * state (cv, IV[0..4], counter lo/hi, block_len, flags), the message permuted
 * between rounds; output word i = v[i] ^ v[i+8] (the first 8 words are all a
 * chaining value or a 32-byte hash needs). */
static void b3_compress(const uint32_t cv[8], const uint32_t block[16], uint64_t counter, uint32_t block_len,
                        uint32_t flags, uint32_t out[8]) {
    uint32_t v[16], m[16], t[16];
    for (int i = 0; i < 8; i++) v[i] = cv[i];
    for (int i = 0; i < 4; i++) v[8 + i] = B3_IV[i];
    v[12] = (uint32_t)counter;
    v[13] = (uint32_t)(counter >> 32);
    v[14] = block_len;
    v[15] = flags;
    memcpy(m, block, sizeof m);
    for (int r = 0; r < 7; r++) {
        b3_g(v, 0, 4, 8, 12, m[0], m[1]);
        b3_g(v, 1, 5, 9, 13, m[2], m[3]);
        b3_g(v, 2, 6, 10, 14, m[4], m[5]);
        b3_g(v, 3, 7, 11, 15, m[6], m[7]);
        b3_g(v, 0, 5, 10, 15, m[8], m[9]);
        b3_g(v, 1, 6, 11, 12, m[10], m[11]);
        b3_g(v, 2, 7, 8, 13, m[12], m[13]);
        b3_g(v, 3, 4, 9, 14, m[14], m[15]);
        for (int i = 0; i < 16; i++) t[i] = m[B3_PERM[i]];
        memcpy(m, t, sizeof m);
    }
    for (int i = 0; i < 8; i++) out[i] = v[i] ^ v[i + 8];
}

static void b3_words(const uint8_t b[64], uint32_t w[16]) {
    for (int i = 0; i < 16; i++)
        w[i] = (uint32_t)b[4 * i] | (uint32_t)b[4 * i + 1] << 8 | (uint32_t)b[4 * i + 2] << 16 |
               (uint32_t)b[4 * i + 3] << 24;
}

/* chunk state: up to 1024 bytes as 16 blocks of 64 */
typedef struct {
    uint32_t cv[8];
    uint64_t counter;
    uint8_t buf[64];
    uint32_t buf_len;
    uint32_t blocks_done;
} b3_chunk;

static void b3_chunk_init(b3_chunk* c, uint64_t counter) {
    memcpy(c->cv, B3_IV, sizeof c->cv);
    c->counter = counter;
    c->buf_len = 0;
    c->blocks_done = 0;
    memset(c->buf, 0, sizeof c->buf);
}

static uint32_t b3_chunk_len(const b3_chunk* c) { return 64u * c->blocks_done + c->buf_len; }

static void b3_chunk_update(b3_chunk* c, const uint8_t* in, size_t n) {
    while (n) {
        if (c->buf_len == 64) {   /* a full block that is not the chunk's last */
            uint32_t w[16];
            b3_words(c->buf, w);
            b3_compress(c->cv, w, c->counter, 64, c->blocks_done == 0 ? B3_CHUNK_START : 0, c->cv);
            c->blocks_done++;
            c->buf_len = 0;
            memset(c->buf, 0, sizeof c->buf);
        }
        size_t take = 64 - c->buf_len;
        if (take > n) take = n;
        memcpy(c->buf + c->buf_len, in, take);
        c->buf_len += (uint32_t)take;
        in += take;
        n -= take;
    }
}

/* the chunk's last block: its output (chaining value, or the hash with ROOT) */
static void b3_chunk_output(const b3_chunk* c, uint32_t extra_flags, uint32_t out[8]) {
    uint32_t w[16];
    b3_words(c->buf, w);
    uint32_t flags = B3_CHUNK_END | (c->blocks_done == 0 ? B3_CHUNK_START : 0) | extra_flags;
    b3_compress(c->cv, w, c->counter, c->buf_len, flags, out);
}

static void b3_parent(const uint32_t l[8], const uint32_t r[8], uint32_t flags, uint32_t out[8]) {
    uint32_t w[16];
    memcpy(w, l, 32);
    memcpy(w + 8, r, 32);
    b3_compress(B3_IV, w, 0, 64, B3_PARENT | flags, out);
}

/* blake3::hash(data) -> 32 bytes */
void ora_blake3(const uint8_t* data, uint64_t len, uint8_t out[32]) {
    uint32_t stack[64][8];
    int depth = 0;
    b3_chunk c;
    b3_chunk_init(&c, 0);
    while (len) {
        if (b3_chunk_len(&c) == 1024) {
            /* the chunk is complete and more input follows: push its chaining
             * value, merging the subtrees this chunk completes */
            uint32_t cv[8];
            b3_chunk_output(&c, 0, cv);
            uint64_t total = c.counter + 1;
            while ((total & 1) == 0) {
                b3_parent(stack[--depth], cv, 0, cv);
                total >>= 1;
            }
            memcpy(stack[depth++], cv, 32);
            b3_chunk_init(&c, c.counter + 1);
        }
        size_t take = 1024 - b3_chunk_len(&c);
        if (take > len) take = (size_t)len;
        b3_chunk_update(&c, data, take);
        data += take;
        len -= take;
    }
    uint32_t h[8];
    if (depth == 0) {
        b3_chunk_output(&c, B3_ROOT, h);
    } else {
        b3_chunk_output(&c, 0, h);
        while (depth > 1) b3_parent(stack[--depth], h, 0, h);
        b3_parent(stack[0], h, B3_ROOT, h);
    }
    for (int i = 0; i < 8; i++)
        for (int b = 0; b < 4; b++) out[4 * i + b] = (uint8_t)(h[i] >> (8 * b));
}

static void hex32(const uint8_t d[32], char* s) {
    static const char X[] = "0123456789abcdef";
    for (int i = 0; i < 32; i++) {
        s[2 * i] = X[d[i] >> 4];
        s[2 * i + 1] = X[d[i] & 15];
    }
}

/* PoolLayer::compute_digest / ShellLayer::compute_digest for the batched
 * layers (one key block and one value block): blake3 of
 * {"key_digests":["<hex k>"],"layer_index":N,"value_digests":["<hex v>"]}. */
void ora_layer_digest(uint32_t layer_index, const uint8_t kd[32], const uint8_t vd[32], uint8_t out[32]) {
    char json[256];
    char kh[65], vh[65];
    hex32(kd, kh);
    hex32(vd, vh);
    kh[64] = vh[64] = 0;
    int n = snprintf(json, sizeof json, "{\"key_digests\":[\"%s\"],\"layer_index\":%u,\"value_digests\":[\"%s\"]}",
                     kh, layer_index, vh);
    ora_blake3((const uint8_t*)json, (uint64_t)n, out);
}

/* many ranges of one buffer, one after the other (the CPU baseline of the
 * device digest) */
void ora_blake3_ranges(const uint8_t* buf, const uint64_t* offsets, const uint64_t* lens, uint32_t n, uint8_t* out) {
    for (uint32_t i = 0; i < n; i++) ora_blake3(buf + offsets[i], lens[i], out + 32ull * i);
}
