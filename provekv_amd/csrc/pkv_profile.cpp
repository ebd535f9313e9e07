// pkv_profile.cpp -- host-side construction of the codec profile constants.
//
// The reference rebuilds these on the CPU every time a quantizer is made
// (proveKV/src/codec.rs:249-250, 296-297, 471-499); the MI355X path builds them
// once per profile, uploads them, and keeps them resident next to the kernels.
//
//   turbo: FastHadamardRotation signs (turbo-quant/src/rotation.rs:143-157) and
//          the QJL projection matrix (turbo-quant/src/qjl.rs:341-352; seed
//          derivation turbo.rs:166-167).
//   fib:   StoredRotation (fib-quant/src/rotation.rs:24-58) and the refined
//          codebook (fib-quant/src/codebook.rs:40-60, 161-184; lloyd.rs:106-337;
//          spherical_beta.rs; directions.rs).
//
// Randomness follows the crates pinned in the reference Cargo.lock:
// rand_core 0.6.4 seed_from_u64 (PCG32 key expansion), rand_chacha 0.3.1
// ChaCha8 (8 rounds, 64-bit block counter, stream 0, a 4-block output buffer
// that behaves as one continuous word stream), rand 0.8 Standard/Open01,
// rand_distr 0.4.3 StandardNormal (ZIGNOR ziggurat, tables regenerated from
// the published recipe) and Gamma (Marsaglia-Tsang).
//
// Compiled with -ffp-contract=off (Rust never fuses multiply-add).
#include "pkv_internal.h"
#include "pkv_math.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <tuple>
#include <type_traits>
#include <vector>

namespace pkv {
namespace {

// ------------------------------------------------------------ ChaCha8 stream
class ChaCha8 {
public:
    explicit ChaCha8(uint64_t seed) {
        // rand_core::SeedableRng::seed_from_u64
        constexpr uint64_t kMul = 6364136223846793005ull;
        constexpr uint64_t kInc = 11634580027462260723ull;
        uint64_t st = seed;
        for (uint32_t& w : key_) {
            st = st * kMul + kInc;
            uint32_t xs = static_cast<uint32_t>(((st >> 18) ^ st) >> 27);
            uint32_t rot = static_cast<uint32_t>(st >> 59);
            w = (xs >> rot) | (xs << ((32u - rot) & 31u));
        }
    }

    uint32_t next_u32() {
        if (pos_ == kWords) refill();
        return buf_[pos_++];
    }
    uint64_t next_u64() {
        uint64_t lo = next_u32();
        uint64_t hi = next_u32();
        return (hi << 32) | lo;
    }
    bool gen_bool() { return static_cast<int32_t>(next_u32()) < 0; }
    double gen_f64() { return static_cast<double>(next_u64() >> 11) * 0x1.0p-53; }
    double open01() {
        uint64_t frac = next_u64() >> 12;
        return u2d(frac | 0x3FF0000000000000ull) - (1.0 - 0x1.0p-53);
    }

private:
    static constexpr int kWords = 64;   // four 16-word blocks per refill
    static uint32_t rotl(uint32_t v, int c) { return (v << c) | (v >> (32 - c)); }

    void refill() {
        for (int b = 0; b < 4; ++b) {
            uint32_t in[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
            for (int i = 0; i < 8; ++i) in[4 + i] = key_[i];
            in[12] = static_cast<uint32_t>(counter_);
            in[13] = static_cast<uint32_t>(counter_ >> 32);
            in[14] = in[15] = 0;
            uint32_t x[16];
            std::memcpy(x, in, sizeof x);
            for (int dr = 0; dr < 4; ++dr) {
                quarter(x, 0, 4, 8, 12); quarter(x, 1, 5, 9, 13);
                quarter(x, 2, 6, 10, 14); quarter(x, 3, 7, 11, 15);
                quarter(x, 0, 5, 10, 15); quarter(x, 1, 6, 11, 12);
                quarter(x, 2, 7, 8, 13); quarter(x, 3, 4, 9, 14);
            }
            for (int i = 0; i < 16; ++i) buf_[b * 16 + i] = x[i] + in[i];
            ++counter_;
        }
        pos_ = 0;
    }
    static void quarter(uint32_t* x, int a, int b, int c, int d) {
        x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 16);
        x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 12);
        x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 8);
        x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 7);
    }

    uint32_t key_[8];
    uint64_t counter_ = 0;
    uint32_t buf_[kWords];
    int pos_ = kWords;
};

// ------------------------------------------------------------ ziggurat normal
struct ZigTables {
    double x[257], f[257], r;
    ZigTables() {
        // rand's ziggurat_tables.py recipe, printed with "%.18f" into the
        // Rust source; the literals are reproduced by formatting the same way.
        // exp / log correctly rounded (x87 extended precision rounded to
        // double; every call of this recursion sits far enough from a
        // rounding midpoint): the table of any correctly rounded libm.
        auto fdens = [](double v) {
            const double t = -v * v / 2.0;
            return static_cast<double>(std::exp(static_cast<long double>(t)));
        };
        auto finv = [](double y) {
            return std::sqrt(-2.0 * static_cast<double>(std::log(static_cast<long double>(y))));
        };
        auto lit = [](double v) {
            char buf[64];
            std::snprintf(buf, sizeof buf, "%.18f", v);
            return std::strtod(buf, nullptr);
        };
        const double R = 3.6541528853610088, V = 0.00492867323399;
        double raw[257];
        raw[0] = V / fdens(R);
        raw[1] = R;
        for (int i = 2; i < 256; ++i) raw[i] = finv(V / raw[i - 1] + fdens(raw[i - 1]));
        raw[256] = 0.0;
        for (int i = 0; i < 257; ++i) { x[i] = lit(raw[i]); f[i] = lit(fdens(raw[i])); }
        r = lit(R);
    }
};

const ZigTables& zig() {
    static const ZigTables t;
    return t;
}

double standard_normal(ChaCha8& rng) {
    const ZigTables& z = zig();
    for (;;) {
        uint64_t bits = rng.next_u64();
        int i = static_cast<int>(bits & 0xff);
        double u = u2d((bits >> 12) | 0x4000000000000000ull) - 3.0;   // [2,4) - 3
        double x = u * z.x[i];
        if (std::fabs(x) < z.x[i + 1]) return x;
        if (i == 0) {
            double tx = 1.0, ty = 0.0;
            while (-2.0 * ty < tx * tx) {
                double a = rng.open01();
                double b = rng.open01();
                tx = std::log(a) / z.r;
                ty = std::log(b);
            }
            return u < 0.0 ? tx - z.r : z.r - tx;
        }
        if (z.f[i + 1] + (z.f[i] - z.f[i + 1]) * rng.gen_f64() < std::exp(-x * x / 2.0)) return x;
    }
}

// Gamma(shape > 1, scale 1), Marsaglia-Tsang as in rand_distr 0.4.3.
double gamma_large(ChaCha8& rng, double shape) {
    const double d = shape - 1.0 / 3.0;
    const double c = 1.0 / std::sqrt(9.0 * d);
    for (;;) {
        double x = standard_normal(rng);
        double vc = 1.0 + c * x;
        if (vc <= 0.0) continue;
        double v = vc * vc * vc;
        double u = rng.open01();
        double x2 = x * x;
        if (u < 1.0 - 0.0331 * x2 * x2 || std::log(u) < 0.5 * x2 + d * (1.0 - v + std::log(v)))
            return d * v * 1.0;
    }
}

// ------------------------------------------------------------ QR rotation
// nalgebra 0.33 Householder QR (clear_column_unchecked + QR::q); its dot
// product folds eight partial sums.  R's diagonal is |diag| >= 0, so the
// reference's column sign fix is a no-op and Q is the unique orthogonal
// factor with a non-negative R diagonal.
double nalgebra_dot(const double* a, const double* b, int len) {
    double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i = 0;
    for (; len - i >= 8; i += 8)
        for (int t = 0; t < 8; ++t) acc[t] += a[i + t] * b[i + t];
    double res = 0.0;
    res += acc[0] + acc[4];
    res += acc[1] + acc[5];
    res += acc[2] + acc[6];
    res += acc[3] + acc[7];
    for (; i < len; ++i) res += a[i] * b[i];
    return res;
}

void reflect_columns(const double* axis, int len, double sign, double* cols, int ncols, int ld) {
    for (int j = 0; j < ncols; ++j) {
        double* c = cols + static_cast<size_t>(j) * ld;
        double factor = nalgebra_dot(axis, c, len) * (sign * -2.0);
        for (int t = 0; t < len; ++t) c[t] = factor * axis[t] + sign * c[t];
    }
}

// Orthogonal factor of a dim x dim Gaussian (ChaCha8(seed), column-major
// fill), returned row-major.
std::vector<double> stored_rotation(int dim, uint64_t seed) {
    ChaCha8 rng(seed);
    const size_t nn = static_cast<size_t>(dim) * dim;
    std::vector<double> a(nn), q(nn, 0.0), diag(dim);
    for (double& v : a) v = standard_normal(rng);
    for (int i = 0; i < dim; ++i) {
        double* col = a.data() + static_cast<size_t>(i) * dim + i;
        const int len = dim - i;
        double sq = nalgebra_dot(col, col, len);
        double nrm = std::sqrt(sq);
        double sgn = col[0] < 0.0 ? -1.0 : 1.0;
        double signed_norm = sgn * nrm;
        double factor = (sq + std::fabs(col[0]) * nrm) * 2.0;
        col[0] += signed_norm;
        if (factor != 0.0) {
            double s = std::sqrt(factor);
            for (int t = 0; t < len; ++t) col[t] /= s;
            diag[i] = -signed_norm;
            reflect_columns(col, len, diag[i] < 0.0 ? -1.0 : 1.0,
                            a.data() + static_cast<size_t>(i + 1) * dim + i, dim - i - 1, dim);
        } else {
            diag[i] = signed_norm;
        }
    }
    for (int j = 0; j < dim; ++j) q[static_cast<size_t>(j) * dim + j] = 1.0;
    for (int i = dim - 1; i >= 0; --i) {
        const double* axis = a.data() + static_cast<size_t>(i) * dim + i;
        reflect_columns(axis, dim - i, diag[i] < 0.0 ? -1.0 : 1.0,
                        q.data() + static_cast<size_t>(i) * dim + i, dim - i, dim);
    }
    std::vector<double> rowmajor(nn);
    for (int r = 0; r < dim; ++r)
        for (int c = 0; c < dim; ++c) rowmajor[static_cast<size_t>(r) * dim + c] = q[static_cast<size_t>(c) * dim + r];
    return rowmajor;
}

// ------------------------------------------------------------ special functions
// Normal and Beta inverse CDFs, solved in x87 long double and rounded once to
// the nearest double (the exact quantiles statrs approximates; the Lloyd
// refinement replaces every codeword by a sample mean, so the codebook does
// not depend on their last bits, but the initial MSE in the codebook's
// Lloyd report, and so its digest, does).
long double normal_cdf(long double x) { return 0.5L * std::erfc(-x / std::sqrt(2.0L)); }

double normal_quantile(double p) {
    // Lower half by bisection on erfc plus a Newton polish; the upper half by
    // symmetry (1 - p is exact for p >= 0.5), where erfc keeps full relative
    // accuracy in the tail.
    if (p > 0.5) return -normal_quantile(1.0 - p);
    long double lo = -40.0L, hi = 0.0L;
    for (int it = 0; it < 200 && hi - lo > 1e-18L * (1.0L + std::fabs(lo)); ++it) {
        long double mid = 0.5L * (lo + hi);
        if (normal_cdf(mid) < p) lo = mid; else hi = mid;
    }
    long double x = 0.5L * (lo + hi);
    for (int it = 0; it < 3; ++it) {
        long double pdf = std::exp(-0.5L * x * x) / std::sqrt(2.0L * 3.14159265358979323846264338327950288L);
        if (!(pdf > 0.0L)) break;
        long double nx = x - (normal_cdf(x) - p) / pdf;
        if (!(std::fabs(nx - x) < 1e-6L)) break;
        x = nx;
    }
    return static_cast<double>(x);
}

long double incomplete_beta_cf(long double a, long double b, long double x) {
    const long double tiny = 1e-300L;
    long double c = 1.0L, d = 1.0L - (a + b) * x / (a + 1.0L);
    if (std::fabs(d) < tiny) d = tiny;
    d = 1.0L / d;
    long double h = d;
    for (int m = 1; m <= 20000; ++m) {
        long double m2 = 2.0L * m;
        long double num = m * (b - m) * x / ((a - 1.0L + m2) * (a + m2));
        d = 1.0L + num * d; if (std::fabs(d) < tiny) d = tiny;
        c = 1.0L + num / c; if (std::fabs(c) < tiny) c = tiny;
        d = 1.0L / d; h *= d * c;
        num = -(a + m) * (a + b + m) * x / ((a + m2) * (a + 1.0L + m2));
        d = 1.0L + num * d; if (std::fabs(d) < tiny) d = tiny;
        c = 1.0L + num / c; if (std::fabs(c) < tiny) c = tiny;
        d = 1.0L / d;
        long double del = d * c;
        h *= del;
        if (std::fabs(del - 1.0L) < 1e-20L) break;
    }
    return h;
}

long double beta_cdf(long double a, long double b, long double x) {
    if (x <= 0.0L) return 0.0L;
    if (x >= 1.0L) return 1.0L;
    long double lbt = std::lgamma(a + b) - std::lgamma(a) - std::lgamma(b) + a * std::log(x) + b * std::log1p(-x);
    long double bt = std::exp(lbt);
    if (x < (a + 1.0L) / (a + b + 2.0L)) return bt * incomplete_beta_cf(a, b, x) / a;
    return 1.0L - bt * incomplete_beta_cf(b, a, 1.0L - x) / b;
}

double beta_quantile(double q, double a, double b) {
    if (q <= 0.0) return 0.0;
    if (q >= 1.0) return 1.0;
    long double lo = 0.0L, hi = 1.0L;
    for (int it = 0; it < 72; ++it) {
        long double mid = 0.5L * (lo + hi);
        if (beta_cdf(a, b, mid) < q) lo = mid; else hi = mid;
    }
    long double x = 0.5L * (lo + hi);
    const long double la = a, lb = b;
    for (int it = 0; it < 6; ++it) {
        long double pdf = std::exp(std::lgamma(la + lb) - std::lgamma(la) - std::lgamma(lb) +
                                   (la - 1.0L) * std::log(x) + (lb - 1.0L) * std::log1p(-x));
        if (!(pdf > 0.0L)) break;
        long double nx = x - (beta_cdf(la, lb, x) - q) / pdf;
        if (!(nx > lo && nx < hi) || nx == x) break;
        x = nx;
    }
    return static_cast<double>(x < 0.0L ? 0.0L : (x > 1.0L ? 1.0L : x));
}

// compiler-rt __powidf2 (f64::powi with a run-time exponent).
double powi(double a, int b) {
    bool recip = b < 0;
    double r = 1.0;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1.0 / r : r;
}

// ------------------------------------------------------------ fib codebook
struct Lloyd {
    int k, n;
    const std::vector<double>& samples;   // ns * k

    int nearest(const double* s, const double* cb, double* best_dist) const {
        int best = 0;
        double bd = INFINITY;
        for (int w = 0; w < n; ++w) {
            double dist = 0.0;
            for (int t = 0; t < k; ++t) { double dl = s[t] - cb[w * k + t]; dist += dl * dl; }
            if (dist < bd) { bd = dist; best = w; }
        }
        if (best_dist) *best_dist = bd;
        return best;
    }
    double mse(const std::vector<double>& cb) const {
        const int ns = static_cast<int>(samples.size()) / k;
        double sum = 0.0;
        for (int i = 0; i < ns; ++i) { double bd; nearest(&samples[static_cast<size_t>(i) * k], cb.data(), &bd); sum += bd; }
        return sum / static_cast<double>(ns);
    }
    // One assign_samples + update_centroids round (lloyd.rs:215-317); each
    // empty-cell repair is appended to `events` (when given) as the
    // reference's RepairRecorder does.
    bool iterate(std::vector<double>& cb, std::vector<LloydRepairEvent>* events = nullptr, uint32_t restart = 0,
                 uint32_t iteration = 0) const {
        const int ns = static_cast<int>(samples.size()) / k;
        std::vector<double> sums(cb.size(), 0.0), dist(n, 0.0), far(cb.size(), 0.0), fard(n, -1.0);
        std::vector<int> counts(n, 0), asg(ns);
        for (int i = 0; i < ns; ++i) asg[i] = nearest(&samples[static_cast<size_t>(i) * k], cb.data(), nullptr);
        for (int i = 0; i < ns; ++i) {
            const double* s = &samples[static_cast<size_t>(i) * k];
            int a = asg[i];
            counts[a] += 1;
            double sd = 0.0;
            for (int t = 0; t < k; ++t) {
                sums[a * k + t] += s[t];
                double dl = s[t] - cb[a * k + t];
                sd += dl * dl;
            }
            dist[a] += sd;
            if (sd > fard[a]) { fard[a] = sd; std::memcpy(&far[a * k], s, sizeof(double) * k); }
        }
        for (int w = 0; w < n; ++w)
            if (counts[w] > 0)
                for (int t = 0; t < k; ++t) cb[w * k + t] = sums[w * k + t] / static_cast<double>(counts[w]);
        for (int e = 0; e < n; ++e) {
            if (counts[e] != 0) continue;
            int donor = -1;   // last maximum of distortion among cells with > 1 sample
            for (int w = 0; w < n; ++w)
                if (counts[w] > 1 && (donor < 0 || !(dist[w] < dist[donor]))) donor = w;
            if (donor < 0) return false;
            double res[32], rn2 = 0.0;
            for (int t = 0; t < k; ++t) { res[t] = far[donor * k + t] - cb[donor * k + t]; rn2 += res[t] * res[t]; }
            double rn = std::sqrt(rn2);
            if (!std::isfinite(rn) || rn <= 2.220446049250313e-16) return false;
            for (int t = 0; t < k; ++t) {
                double dir = res[t] / rn, cen = cb[donor * k + t];
                cb[donor * k + t] = cen - 1.0e-6 * dir;
                cb[e * k + t] = cen + 1.0e-6 * dir;
            }
            if (events)
                events->push_back({restart, iteration, static_cast<uint32_t>(e), static_cast<uint32_t>(donor),
                                   static_cast<uint32_t>(counts[donor]), dist[donor], rn});
            counts[donor] -= 1;
            counts[e] = 1;
            dist[donor] = 0.0;
            dist[e] = 0.0;
        }
        return true;
    }
};

}  // namespace

// -------------------------------------------------------------- builders
namespace {

int build_turbo_constants(uint32_t dim, uint32_t proj, uint64_t seed, std::vector<float>& signs,
                          std::vector<float>& G) {
    signs.assign(dim, 0.0f);
    ChaCha8 srng(seed + 0xA11CE55ED5A5EED5ull);
    for (uint32_t i = 0; i < dim; ++i) signs[i] = srng.gen_bool() ? 1.0f : -1.0f;
    G.assign(static_cast<size_t>(proj) * dim, 0.0f);
    if (proj) {
        ChaCha8 grng((seed + 0xCAFEBABE00000001ull) + 0xDEADBEEF12345678ull);
        for (float& g : G) g = static_cast<float>(standard_normal(grng));
    }
    return PKV_OK;
}

int build_fib_rotation(uint32_t dim, uint64_t seed, std::vector<double>& rot) {
    if (dim == 0 || dim > 4096) return PKV_ERR_INVALID_ARG;
    rot = stored_rotation(static_cast<int>(dim), seed);
    return PKV_OK;
}

int build_fib_codebook(uint32_t dim, uint32_t k, uint32_t n, uint64_t seed, uint32_t training,
                       uint32_t restarts, uint32_t iterations, std::vector<float>& codebook,
                       double* init_mse, double* train_mse, const LloydDevice* dev,
                       LloydReport* report = nullptr) {
    if (k < 4 || k > 32 || dim % k != 0 || n < 2 || dim <= k) return PKV_ERR_UNSUPPORTED;
    const uint64_t cseed = seed + 0x9e3779b97f4a7c15ull;
    const int K = static_cast<int>(k), N = static_cast<int>(n), D = static_cast<int>(dim);
    // Roberts-Kronecker directions (directions.rs:38-71)
    double lo = 1.0, hi = 2.0;
    for (int it = 0; it < 128; ++it) {
        double mid = (lo + hi) / 2.0;
        if (powi(mid, K + 1) - mid - 1.0 > 0.0) hi = mid; else lo = mid;
    }
    const double phi = (lo + hi) / 2.0;
    std::vector<double> init(static_cast<size_t>(N) * K);
    const double alpha = K / 2.0;
    const double beta = (static_cast<double>(K) / (K + 2.0)) * ((D - static_cast<double>(K) - 2.0) / 2.0) + 1.0;
    for (int idx = 0; idx < N; ++idx) {
        double dir[32], norm_sq = 0.0;
        for (int j = 1; j <= K; ++j) {
            double t = (idx + 0.5) * powi(phi, -j);
            double frac = t - std::trunc(t);
            frac = frac < 1.0e-12 ? 1.0e-12 : (frac > 1.0 - 1.0e-12 ? 1.0 - 1.0e-12 : frac);
            dir[j - 1] = normal_quantile(frac);
            norm_sq += dir[j - 1] * dir[j - 1];
        }
        if (!(norm_sq > 0.0) || !std::isfinite(norm_sq)) return PKV_ERR_INVALID_ARG;
        double nrm = std::sqrt(norm_sq);
        double q = (idx + 1 - 0.5) / static_cast<double>(N);
        double radius = std::sqrt(beta_quantile(q, alpha, beta));
        for (int t = 0; t < K; ++t) init[static_cast<size_t>(idx) * K + t] = radius * (dir[t] / nrm);
    }
    // spherical-Beta training samples (lloyd.rs:184-195, spherical_beta.rs:58-126)
    const int ns = static_cast<int>(training > n ? training : n);
    std::vector<double> samples(static_cast<size_t>(ns) * K);
    ChaCha8 rng(cseed ^ 0x465155414e54ull);
    for (int i = 0; i < ns; ++i) {
        double a = gamma_large(rng, K / 2.0);
        double b = gamma_large(rng, (D - K) / 2.0);
        double sum = a + b;
        if (sum <= 0.0 || !std::isfinite(sum)) return PKV_ERR_INVALID_ARG;
        double r2 = a / sum;
        double dir[32];
        for (;;) {
            double nsq = 0.0;
            for (int t = 0; t < K; ++t) { dir[t] = standard_normal(rng); nsq += dir[t] * dir[t]; }
            if (nsq > 0.0 && std::isfinite(nsq)) {
                double nn = std::sqrt(nsq);
                for (int t = 0; t < K; ++t) dir[t] = dir[t] / nn;
                break;
            }
        }
        double rr = std::sqrt(r2);
        for (int t = 0; t < K; ++t) samples[static_cast<size_t>(i) * K + t] = rr * dir[t];
    }
    // each restart's start: the initial codebook, then its codewords turned by
    // a seeded k x k rotation (lloyd.rs:196-213)
    const uint32_t nr = restarts ? restarts : 1;
    const size_t nk = init.size();
    std::vector<double> starts(nr * nk);
    for (uint32_t rs = 0; rs < nr; ++rs) {
        double* cb = &starts[rs * nk];
        if (rs == 0) {
            std::copy(init.begin(), init.end(), cb);
            continue;
        }
        std::vector<double> rot = stored_rotation(K, cseed + static_cast<uint64_t>(rs) * 0x9e3779b9ull);
        for (int w = 0; w < N; ++w)
            for (int r = 0; r < K; ++r) {
                double s = 0.0;
                for (int c = 0; c < K; ++c) s += rot[r * K + c] * init[static_cast<size_t>(w) * K + c];
                cb[static_cast<size_t>(w) * K + r] = s;
            }
    }
    // the restarts' refined codebooks and MSEs: on the device when one is
    // given (and the shape fits its kernel), else here
    // given (and the shape fits its kernel), else here; the repair events of
    // a report are recorded by the host iterations only
    std::vector<double> refined, mses(nr);
    std::vector<LloydRepairEvent> events;
    double imse;
    if (dev && !report && N <= static_cast<int>(LLOYD_MAX_N) && K <= static_cast<int>(LLOYD_MAX_K) &&
        nk <= LLOYD_MAX_NK) {
        int rc = dev->refine(samples, static_cast<uint32_t>(ns), k, n, starts, nr, iterations, refined, mses, &imse);
        if (rc) return rc;
    } else {
        Lloyd lloyd{K, N, samples};
        imse = lloyd.mse(init);
        refined = starts;
        for (uint32_t rs = 0; rs < nr; ++rs) {
            std::vector<double> cb(starts.begin() + rs * nk, starts.begin() + (rs + 1) * nk);
            for (uint32_t it = 0; it < iterations; ++it)
                if (!lloyd.iterate(cb, report ? &events : nullptr, rs, it)) return PKV_ERR_INVALID_ARG;
            mses[rs] = lloyd.mse(cb);
            std::copy(cb.begin(), cb.end(), refined.begin() + rs * nk);
        }
    }
    // refine_codebook's choice (lloyd.rs:148-163): a restart replaces the best
    // so far only when strictly better; none better than the start keeps it
    // (best_restart u32::MAX)
    double best_mse = imse;
    uint32_t best_restart = 0;
    std::vector<double> best = init;
    for (uint32_t rs = 0; rs < nr; ++rs) {
        const double m = mses[rs];
        if (m < best_mse || (rs == 0 && std::isinf(imse))) {
            best_mse = m;
            best_restart = rs;
            best.assign(refined.begin() + rs * nk, refined.begin() + (rs + 1) * nk);
        }
    }
    if (best_mse > imse) { best = init; best_mse = imse; best_restart = 0xFFFFFFFFu; }
    codebook.resize(best.size());
    for (size_t t = 0; t < best.size(); ++t) codebook[t] = static_cast<float>(best[t]);
    if (init_mse) *init_mse = imse;
    if (train_mse) *train_mse = best_mse;
    if (report) {   // LloydReportV1 (lloyd.rs:165-176)
        report->restarts = nr;
        report->iterations = iterations;
        report->training_samples = static_cast<uint32_t>(ns);
        report->init_mse = imse;
        report->best_mse = best_mse;
        report->best_restart = best_restart;
        report->repairs = static_cast<uint32_t>(std::min<size_t>(events.size(), 0xFFFFFFFFu));
        report->events = std::move(events);
        report->seed = cseed;
    }
    return PKV_OK;
}

// ---- profile-constant service
// The reference rebuilds a quantizer's constants on every adapter call: the
// Lloyd codebook and the QR rotation 2x per layer in a pool build and again
// per decompress (proveKV/src/codec.rs:471-499, pool.rs:225, 265-266,
// 517-519), the Hadamard signs and QJL matrix per turbo call (codec.rs:249,
// 296).  Here every distinct profile is built once per process and shared:
// the key is the full parameter set the constants (and the reference's
// profile digest) are a function of.
struct FibCodebook {
    std::vector<float> cb;
    double init_mse, train_mse;
};
struct TurboConsts {
    std::vector<float> signs, G;
};
using FibKey = std::tuple<uint32_t, uint32_t, uint32_t, uint64_t, uint32_t, uint32_t, uint32_t>;
using RotKey = std::tuple<uint32_t, uint64_t>;
using TurboKey = std::tuple<uint32_t, uint32_t, uint64_t>;

struct ConstCache {
    std::mutex mu;
    std::map<FibKey, std::shared_ptr<const FibCodebook>> cb;
    std::map<RotKey, std::shared_ptr<const std::vector<double>>> rot;
    std::map<TurboKey, std::shared_ptr<const TurboConsts>> turbo;
    uint64_t hits = 0, misses = 0;
};
ConstCache& cache() {
    static ConstCache c;
    return c;
}

// Look `key` up in `m`; on a miss build outside the lock (two threads may
// both build a new key; the first insert wins and both results are equal).
template <typename M, typename K, typename Build>
int cached(M& m, const K& key, std::shared_ptr<const typename M::mapped_type::element_type>& out, Build build) {
    ConstCache& c = cache();
    {
        std::lock_guard<std::mutex> lock(c.mu);
        auto it = m.find(key);
        if (it != m.end()) {
            ++c.hits;
            out = it->second;
            return PKV_OK;
        }
        ++c.misses;
    }
    auto v = std::make_shared<std::remove_const_t<typename M::mapped_type::element_type>>();
    int rc = build(*v);
    if (rc) return rc;
    std::lock_guard<std::mutex> lock(c.mu);
    out = m.emplace(key, std::move(v)).first->second;
    return PKV_OK;
}

}  // namespace

// -------------------------------------------------------------- public helpers
int make_turbo_constants(uint32_t dim, uint32_t proj, uint64_t seed, std::vector<float>& signs,
                         std::vector<float>& G) {
    std::shared_ptr<const TurboConsts> t;
    int rc = cached(cache().turbo, TurboKey(dim, proj, seed), t,
                    [&](TurboConsts& v) { return build_turbo_constants(dim, proj, seed, v.signs, v.G); });
    if (rc) return rc;
    signs = t->signs;
    G = t->G;
    return PKV_OK;
}

int make_fib_rotation(uint32_t dim, uint64_t seed, std::vector<double>& rot) {
    std::shared_ptr<const std::vector<double>> r;
    int rc = cached(cache().rot, RotKey(dim, seed), r,
                    [&](std::vector<double>& v) { return build_fib_rotation(dim, seed, v); });
    if (rc) return rc;
    rot = *r;
    return PKV_OK;
}

int make_fib_codebook(uint32_t dim, uint32_t k, uint32_t n, uint64_t seed, uint32_t training,
                      uint32_t restarts, uint32_t iterations, std::vector<float>& codebook,
                      double* init_mse, double* train_mse, const LloydDevice* dev) {
    std::shared_ptr<const FibCodebook> f;
    int rc = cached(cache().cb, FibKey(dim, k, n, seed, training, restarts, iterations), f, [&](FibCodebook& v) {
        return build_fib_codebook(dim, k, n, seed, training, restarts, iterations, v.cb, &v.init_mse, &v.train_mse,
                                  dev);
    });
    if (rc) return rc;
    codebook = f->cb;
    if (init_mse) *init_mse = f->init_mse;
    if (train_mse) *train_mse = f->train_mse;
    return PKV_OK;
}

int fib_codebook_report(uint32_t dim, uint32_t k, uint32_t n, uint64_t seed, uint32_t training, uint32_t restarts,
                        uint32_t iterations, std::vector<float>& codebook, LloydReport& report) {
    return build_fib_codebook(dim, k, n, seed, training, restarts, iterations, codebook, nullptr, nullptr, nullptr,
                              &report);
}

void constants_cache_stats(uint64_t* hits, uint64_t* misses, uint64_t* entries) {
    ConstCache& c = cache();
    std::lock_guard<std::mutex> lock(c.mu);
    if (hits) *hits = c.hits;
    if (misses) *misses = c.misses;
    if (entries) *entries = c.cb.size() + c.rot.size() + c.turbo.size();
}

void constants_cache_clear() {
    ConstCache& c = cache();
    std::lock_guard<std::mutex> lock(c.mu);
    c.cb.clear();
    c.rot.clear();
    c.turbo.clear();
    c.hits = c.misses = 0;
}

}  // namespace pkv
