// pkv_internal.h -- declarations shared by the host and device halves of
// libpkv_hip.so (not part of the C ABI).
#pragma once
#include <stdint.h>
#include <vector>

#include "../../include/pkv_codec.h"

namespace pkv {

// Status-word kinds (low 4 bits of a per-segment status word; the vector
// index sits above them).
enum Kind : uint32_t {
    KIND_NONFINITE_INPUT = 0,
    KIND_ZERO_NORM = 1,
    KIND_NORM16 = 2,
    KIND_NONFINITE_RADIUS = 3,
    KIND_NONFINITE_RESIDUAL = 4,
    KIND_CORRUPT = 5,
    KIND_HEADER = 6,
    KIND_DECODE_NONFINITE = 7,
    KIND_SCORE_NONFINITE = 8,
};
constexpr uint32_t STATUS_NONE = 0xFFFFFFFFu;
constexpr uint32_t MAX_SEG_VECTORS = (1u << 28) - 1;

// Segment record as the kernels read it (same layout as pkv_seg).
struct SegDev {
    uint64_t elem_offset;
    uint64_t stride_outer;
    uint64_t stride_inner;
    uint64_t wire_offset;
    uint32_t n_vectors;
    uint32_t group;
};
static_assert(sizeof(SegDev) == sizeof(pkv_seg), "segment layout");

// Vectors handled by one workgroup (4 waves x 64 lanes, one vector per lane).
constexpr uint32_t TILE = 256;

struct TurboDev {
    const float* signs;     // dim
    const float* qjl;       // proj * dim, row-major
    const float* cs;        // 2 * levels: cos, sin of each dequantized angle
    // QJL sketch on the f16 matrix cores (head_dim 64 / 128 with QJL): G's f16
    // halves as MFMA A operands (qa) and per-projection acceptance-bound
    // coefficients (qb); layouts at turbo_qjl_mfma_constants (pkv_capi.cpp)
    const uint32_t* qa;
    const float* qb;
    uint64_t seed;
    uint32_t dim, pbits, proj, mode;
};

// Per-profile constants of the fib encode MFMA path (32-bit words, each two
// f16, built on the host, read by fib_encode_kernel):
//   MF_ROT  [t 2][q 4][part 2][lane 64][4]: A operand of the rotation MFMAs:
//           f16 hi (part 0) / lo (part 1) halves of
//           Pi[fib_mfma_row(t, lane % 32)][32 (lane / 32) + 8q + j], j = 0..7
//   MF_SCA  [lane 64][4]: A operand of the scoring MFMA for codeword
//           w = lane % 32, h = lane / 32: f16 halves j = 0..7 of
//           (-2c[w][h])hi, (-2c[w][2+h])hi, same, same, (-2c[w][h])lo,
//           (-2c[w][2+h])lo, then (|c_w|^2 + off) hi, lo (h = 0) or 0, 0
constexpr int MF_ROT = 0;
constexpr int MF_SCA = 4096;
constexpr int MF_WORDS = MF_SCA + 256;

// Logical rotation row held by physical row m (0..31) of MFMA row tile t:
// the 32x32 accumulator keeps rows 8(r/4) + 4h + r%4 in register r of lane
// half h, and the scoring step wants rho[4b + 2s + h] of block b = 8t + r/2,
// K-step s = r % 2, in that register.
constexpr uint32_t fib_mfma_row(uint32_t t, uint32_t m) {
    return 4 * (8 * t + (4 * (m >> 3) + (m & 3)) / 2) + 2 * ((4 * (m >> 3) + (m & 3)) % 2) + ((m >> 2) & 1);
}

struct FibDev {
    const float* codebook;  // n * k
    const double* codebook64;  // n * k, the same values widened (per-vector f64 decode)
    const double* rot_t;    // dim * dim, transposed: [col][row] (per-vector f64 decode)
    const double* rot64;    // dim * dim, row-major (the encode's exact redo)
    const float* rot32t;    // dim * dim, f32(rot) transposed: [col][row] (VALU decode)
    const float* rot32;     // dim * dim, f32(rot) row-major (MFMA decode)
    int mfma_decode;        // matrix-core products verified bit-exact for this profile
    const uint32_t* mf;     // MF_WORDS (encode MFMA operands)
    float thr;              // argmin acceptance margin for the approximate keys
    uint32_t dim, k, n, bits;
};

struct LaunchCommon {
    const SegDev* segs;
    const uint32_t* tile_start;   // nseg + 1 prefix of workgroups per segment
    const uint32_t* tile_seg = nullptr;   // segment of every tile (tile_start[nseg] entries), or null
    uint32_t nseg;
    uint32_t* status;             // 2 * nseg words, or a dummy
    uint32_t radii;               // turbo radii codec
    uint32_t plen;                // payload bytes per vector
    uint32_t in_bf16;             // encode input dtype
    uint32_t per_vector;          // fib encode: FibQuantizer::encode semantics for every vector
    uint32_t out_dtype;           // decode output: PKV_F32, PKV_BF16 or PKV_F16 (RNE from the f32 decode)
    uint32_t fanout;              // decode: copies of every output vector (>= 1) ...
    uint64_t fanout_stride;       // ... this many elements apart
    uint32_t grid_cap = 0;        // at most this many workgroups, each walking tiles (0: one per tile);
                                  // d64 turbo decode and the fib MFMA decode
    float* diag = nullptr;        // encode diagnostics (pkv_encode_diagnostics): the matrix-core values
                                  // the kernel decided from, per vector of the (single) segment;
                                  // non-null selects the kernels' diagnostic instantiations
};

// Up to 48 constant header bytes (TQW1 / FB1 record headers, TQB1 / FB2 blob
// headers), little-endian packed, passed to kernels by value.
struct HdrBytes {
    uint32_t w[12];
};

// Host-side profile construction (pkv_profile.cpp).
int make_turbo_constants(uint32_t dim, uint32_t proj, uint64_t seed, std::vector<float>& signs,
                         std::vector<float>& G);
int make_fib_rotation(uint32_t dim, uint64_t seed, std::vector<double>& rot);
// Runs the Lloyd iterations of every restart of a codebook build on a device
// (pkv_capi.cpp implements it over a context, with the kernel of
// pkv_lloyd.hip).  samples [ns][k], starts [restarts][n][k]; out [restarts][n][k],
// mse [restarts], init_mse = MSE of starts[0].  Returns a pkv status.
struct LloydDevice {
    virtual ~LloydDevice() = default;
    virtual int refine(const std::vector<double>& samples, uint32_t ns, uint32_t k, uint32_t n,
                       const std::vector<double>& starts, uint32_t restarts, uint32_t iterations,
                       std::vector<double>& out, std::vector<double>& mse, double* init_mse) const = 0;
};
int make_fib_codebook(uint32_t dim, uint32_t k, uint32_t n, uint64_t seed, uint32_t training,
                      uint32_t restarts, uint32_t iterations, std::vector<float>& codebook,
                      double* init_mse, double* train_mse,
                      const LloydDevice* dev = nullptr);
// LloydReportV1 and LloydRepairEventV1 (fib-quant/src/lloyd.rs:17-59): the
// refinement receipt FibCodebookV1's digest covers.
struct LloydRepairEvent {
    uint32_t restart, iteration, empty_cell, donor_cell, donor_count_before;
    double donor_distortion, residual_norm;   // split_epsilon is the constant 1e-6
};
struct LloydReport {
    uint32_t restarts = 0, iterations = 0, training_samples = 0;
    double init_mse = 0.0, best_mse = 0.0;
    uint32_t best_restart = 0, repairs = 0;
    std::vector<LloydRepairEvent> events;
    uint64_t seed = 0;
};
// The codebook build of make_fib_codebook run on the host with its report
// (not memoised; same codewords).
int fib_codebook_report(uint32_t dim, uint32_t k, uint32_t n, uint64_t seed, uint32_t training, uint32_t restarts,
                        uint32_t iterations, std::vector<float>& codebook, LloydReport& report);
// The make_* builders above memoise per process (one build per distinct profile).
// A JSON-serialised TurboCode / FibCodeV1 -> the payload of the equivalent
// TQW1 / FB1 record (pkv_json.cpp; pkv_code_from_json's contract: stage 1 =
// does not deserialize, 2 = does not fit the profile, 0 with an error = not
// a payload fault).
int code_from_json(const pkv_codec_params& p, const uint8_t* json, uint64_t len, std::vector<uint8_t>* payload,
                   int* stage);
void constants_cache_stats(uint64_t* hits, uint64_t* misses, uint64_t* entries);
void constants_cache_clear();

// Kernel launchers (pkv_kernels.hip).  Return a hipError_t as int.
int launch_turbo_encode(const LaunchCommon& lc, const TurboDev& td, const void* in, uint8_t* wire,
                        uint32_t nblocks, void* stream);
int launch_turbo_decode(const LaunchCommon& lc, const TurboDev& td, const uint8_t* wire, void* out,
                        uint32_t nblocks, void* stream);
int launch_turbo_prepare(const TurboDev& td, const float* q, uint32_t nq, float* out, float rscale,
                         uint32_t* status, void* stream);
int launch_turbo_score(const LaunchCommon& lc, const TurboDev& td, const uint8_t* wire, const float* prepared,
                       uint32_t nq, uint64_t qstride, float* scores, uint64_t ld, float qscale, float post,
                       uint32_t nblocks, void* stream);
int launch_fib_encode(const LaunchCommon& lc, const FibDev& fd, const void* in, uint8_t* wire, uint32_t nblocks,
                      void* stream);
int launch_fib_decode(const LaunchCommon& lc, const FibDev& fd, const uint8_t* wire, void* out,
                      uint32_t nblocks, void* stream);
int launch_fill_u32(uint32_t* p, uint32_t value, uint64_t n, void* stream);
// Measure the cheap-log bound table the BlockLogU8 encodes read (once per
// device, before any encode there); copy it (256 floats) to device memory.
int launch_logf_bound(void* stream);
// 2 floats: matrix-core products with subnormal f16 operands (expected 2^-10 + 2^-14, 2^-10).
int launch_f16_subnormal_probe(float* out, void* stream);
int launch_logf_bound_read(float* out, void* stream);
int launch_sqrt_check(uint32_t* bad, void* stream);
int launch_fib_product_check(const float* rot32, const float* cb, uint32_t* bad, void* stream);

// Legacy per-vector records (pkv_records.hip).  Records are rec_hdr header
// bytes + one payload; a batch is a byte buffer plus n + 1 offsets.
int launch_records_pack(const uint8_t* pay, uint8_t* out, uint64_t n, uint32_t plen, uint32_t rec_hdr,
                        const HdrBytes& hdr, void* stream);
// packed: record i starts at i * rec_len (no offset table reads); the record
// buffer is then 4-byte aligned.  Rejections go to status[0] / status[1].
int launch_records_check(const uint8_t* rec, const uint64_t* off, uint64_t n, uint32_t rec_len, uint32_t rec_hdr,
                         uint32_t fb1, bool packed, const HdrBytes& hdr, uint32_t* status, void* stream);
int launch_records_gather(const uint8_t* rec, const uint64_t* off, uint64_t n, uint32_t rec_len, uint32_t rec_hdr,
                          bool packed, uint8_t* blob, uint32_t blob_hdr, const HdrBytes& bhdr, uint32_t plen,
                          void* stream);
int launch_fib_decode_f64(const FibDev& fd, const uint8_t* pay, uint64_t n, uint32_t plen, float* out,
                          uint32_t* status, void* stream);

// Lloyd-Max refinement on the device (pkv_lloyd.hip): one workgroup per
// restart over host-drawn samples [ns][k] and starts [restarts][n][k] (f64).
// Outputs: refined codebooks [restarts][n][k], each restart's final MSE, the
// MSE of restart 0's start, status[r] = 1 when an empty cell had no donor.
// Scratch: ns f64 distances and ns u8 assignments per restart.
constexpr uint32_t LLOYD_MAX_N = 256, LLOYD_MAX_K = 16, LLOYD_MAX_NK = 2048;
int launch_lloyd(const double* samples, uint32_t ns, uint32_t k, uint32_t n, const double* starts, uint32_t restarts,
                 uint32_t iterations, double* out_cb, double* out_mse, double* init_mse, uint32_t* status,
                 double* bd_scratch, uint8_t* asg_scratch, void* stream);

// BLAKE3 digests (pkv_blake3.hip).  A range as the kernels read it (same
// layout as pkv_range) and one pass's record per range: the pass's first
// tile (64 elements) of the range, its element count (chunks in pass 0,
// chaining values after), where its input chaining values start (pass > 0) and
// where its outputs go when it does not finish the range (units of 8 words).
// A pass table has nr + 1 records; the last one's tile_start is the tile count.
struct B3Range {
    uint64_t offset;
    uint64_t len;
};
static_assert(sizeof(B3Range) == sizeof(pkv_range), "range layout");
struct B3Pass {
    uint32_t tile_start, count, in_base, out_base;
};
// Pass 0 with one lane per chunk (tiles of 64 chunks).
int launch_blake3_pass(const uint8_t* buf, const B3Range* ranges, const B3Pass* pass, uint32_t nr, uint32_t tiles,
                       uint32_t* cv_out, uint32_t* out, void* stream);
// Pass 0 with four lanes per chunk (tiles of 16 chunks; pass records as for
// launch_blake3_pass).
int launch_blake3_quad(const uint8_t* buf, const B3Range* ranges, const B3Pass* pass, uint32_t nr, uint32_t tiles,
                       uint32_t* cv_out, uint32_t* out, void* stream);
// A merge pass (tiles of 64 chaining values) with four lanes per
// compression, one workgroup per tile.
int launch_blake3_merge4(const B3Pass* pass, uint32_t nr, uint32_t tiles, const uint32_t* cv_in, uint32_t* cv_out,
                         uint32_t* out, void* stream);
int launch_blake3_layers(const uint32_t* kv, uint32_t n, uint32_t layers, uint32_t* out, void* stream);

}  // namespace pkv
