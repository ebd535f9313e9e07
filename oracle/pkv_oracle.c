/*
 * pkv_oracle.c -- CPU restatement of proveKV's codec hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the provekv_amd product links, loads
 * or calls this file; only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py use it, and only as the checker (or as the
 * timed CPU baseline).  Plain C, compiled with -O3 -ffp-contract=off so that
 * every `a*b + c` rounds twice exactly like the Rust reference (Rust never
 * contracts floating-point expressions).  Transcendentals come from the host
 * glibc, which is what Rust's f32/f64 methods lower to on linux-gnu.
 *
 * Every function cites the reference file:line it restates (paths are
 * relative to the reference repository root).  Pieces whose arithmetic lives
 * in third-party crates absent from the reference tree restate the published
 * algorithm of the pinned crate version (Cargo.lock):
 *   rand_core 0.6.4   SeedableRng::seed_from_u64 (PCG32 key expansion)
 *   rand_chacha 0.3.1 ChaCha8Rng (64-bit block counter, zero stream id)
 *   rand 0.8.x        Standard<bool>, Standard<f64>, Open01<f64>
 *   rand_distr 0.4.3  StandardNormal (ZIGNOR ziggurat), Gamma (Marsaglia-Tsang)
 *   statrs 0.17.1     Normal / Beta inverse CDF (restated to full double
 *                     accuracy; see the notes at each function)
 *   nalgebra 0.33.3   Householder QR (restated; Q is unique given R_jj >= 0)
 *   half 2.7.1        f16::from_f32 (IEEE binary16, round-to-nearest-even)
 *
 * Parity status of each part is stated in the header comment of that part.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <float.h>

#define ORA_OK 0
#define ORA_ERR_INVALID_ARG -1      /* bad profile / dims */
#define ORA_ERR_NONFINITE_INPUT -2  /* NonFiniteInput */
#define ORA_ERR_ZERO_NORM -3        /* FibQuantError::ZeroNorm */
#define ORA_ERR_NORM_UNREPRESENTABLE -4 /* encode_norm: not finite positive fp16 */
#define ORA_ERR_MALFORMED -5        /* MalformedCode / CorruptPayload on decode */
#define ORA_ERR_RADIUS -6           /* PolarCode validate: radius not finite >= 0 */
#define ORA_ERR_RESIDUAL -7         /* QJL sketch: residual not finite */
#define ORA_ERR_CAPACITY -8         /* caller buffer too small */
#define ORA_ERR_EMPTY -9            /* empty batch */
#define ORA_ERR_NUMERICAL -10       /* profile construction failure */

/* ======================================================================
 * 1. ChaCha8Rng stream  (rand_chacha 0.3.1; rand_core 0.6.4 seed_from_u64)
 *    Call sites: turbo-quant/src/rotation.rs:152, qjl.rs:346,
 *    fib-quant/src/rotation.rs:36, lloyd.rs:188.
 *    The BlockRng buffer of four blocks is a continuous keystream of u32
 *    words (next_u64 = lo word then hi word, also across refills), so the
 *    stream is modelled one 16-word block at a time.
 * ====================================================================== */
typedef struct {
    uint32_t key[8];
    uint64_t block;     /* next block counter */
    uint32_t buf[16];
    int pos;            /* 16 = empty */
    int rounds;
    /* test hook, not part of the restatement: when set, the stream is
     * rand_pcg 0.3's Pcg32 (Lcg64Xsh32) instead of ChaCha, the generator the
     * value-stability tests of rand 0.8 and rand_distr 0.4 draw from, so the
     * conversions below can be checked against those tests' known answers */
    int pcg;
    uint64_t pcg_state, pcg_inc;
} ora_rng;

static uint32_t rotl32(uint32_t v, int c) { return (v << c) | (v >> (32 - c)); }

static void chacha_block(const uint32_t key[8], uint64_t counter, int rounds, uint32_t out[16]) {
    uint32_t s[16], x[16];
    s[0] = 0x61707865u; s[1] = 0x3320646eu; s[2] = 0x79622d32u; s[3] = 0x6b206574u;
    for (int i = 0; i < 8; ++i) s[4 + i] = key[i];
    s[12] = (uint32_t)counter; s[13] = (uint32_t)(counter >> 32);
    s[14] = 0; s[15] = 0;   /* stream id 0 */
    memcpy(x, s, sizeof s);
#define QR(a, b, c, d) \
    x[a] += x[b]; x[d] = rotl32(x[d] ^ x[a], 16); \
    x[c] += x[d]; x[b] = rotl32(x[b] ^ x[c], 12); \
    x[a] += x[b]; x[d] = rotl32(x[d] ^ x[a], 8);  \
    x[c] += x[d]; x[b] = rotl32(x[b] ^ x[c], 7);
    for (int r = 0; r < rounds; r += 2) {
        QR(0, 4, 8, 12) QR(1, 5, 9, 13) QR(2, 6, 10, 14) QR(3, 7, 11, 15)
        QR(0, 5, 10, 15) QR(1, 6, 11, 12) QR(2, 7, 8, 13) QR(3, 4, 9, 14)
    }
#undef QR
    for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
}

static void rng_from_key(ora_rng* r, const uint32_t key[8], int rounds) {
    memcpy(r->key, key, 32);
    r->block = 0; r->pos = 16; r->rounds = rounds;
    r->pcg = 0;
}

/* rand_pcg 0.3 Pcg32::new(state, stream): increment = stream * 2 + 1, state
 * moved off its initial value by adding the increment and one LCG step
 * (Lcg64Xsh32::from_state_incr), as pcg32_srandom_r of the PCG reference. */
static void rng_pcg32(ora_rng* r, uint64_t state, uint64_t stream) {
    memset(r, 0, sizeof *r);
    r->pcg = 1;
    r->pcg_inc = (stream << 1) | 1u;
    r->pcg_state = (state + r->pcg_inc) * 6364136223846793005ull + r->pcg_inc;
}

/* Lcg64Xsh32::next_u32: XSH RR output of the old state, then one LCG step. */
static uint32_t pcg_u32(ora_rng* r) {
    const uint64_t old = r->pcg_state;
    r->pcg_state = old * 6364136223846793005ull + r->pcg_inc;
    const uint32_t xsh = (uint32_t)(((old >> 18) ^ old) >> 27);
    const uint32_t rot = (uint32_t)(old >> 59);
    return (xsh >> rot) | (xsh << ((32 - rot) & 31));
}

/* rand_core 0.6.4 SeedableRng::seed_from_u64: PCG32 fills the 32-byte seed. */
static void rng_seed_from_u64(ora_rng* r, uint64_t state) {
    uint32_t key[8];
    const uint64_t MUL = 6364136223846793005ull, INC = 11634580027462260723ull;
    for (int i = 0; i < 8; ++i) {
        state = state * MUL + INC;
        uint32_t xorshifted = (uint32_t)(((state >> 18) ^ state) >> 27);
        uint32_t rot = (uint32_t)(state >> 59);
        key[i] = (xorshifted >> rot) | (xorshifted << ((32 - rot) & 31));
    }
    rng_from_key(r, key, 8);
}

static uint32_t rng_u32(ora_rng* r) {
    if (r->pcg) return pcg_u32(r);
    if (r->pos >= 16) {
        chacha_block(r->key, r->block, r->rounds, r->buf);
        r->block++;
        r->pos = 0;
    }
    return r->buf[r->pos++];
}

static uint64_t rng_u64(ora_rng* r) {
    uint64_t lo = rng_u32(r);
    uint64_t hi = rng_u32(r);
    return (hi << 32) | lo;
}

/* rand 0.8 Standard for bool: most significant bit of a u32. */
static int rng_bool(ora_rng* r) { return (int32_t)rng_u32(r) < 0; }

/* rand 0.8 Standard for f64: 53 high bits * 2^-53, in [0,1). */
static double rng_f64(ora_rng* r) {
    return (double)(rng_u64(r) >> 11) * (1.0 / 9007199254740992.0);
}

static double bits_to_f64(uint64_t b) { double d; memcpy(&d, &b, 8); return d; }

/* rand 0.8 Open01 for f64: 52-bit fraction in [1,2) minus (1 - eps/2). */
static double rng_open01(ora_rng* r) {
    uint64_t frac = rng_u64(r) >> 12;
    return bits_to_f64(frac | 0x3FF0000000000000ull) - (1.0 - DBL_EPSILON / 2.0);
}

/* ======================================================================
 * 2. StandardNormal (rand_distr 0.4.3, ZIGNOR ziggurat) and Gamma.
 *    Call sites: turbo-quant/src/qjl.rs:349-351, rotation.rs:340;
 *    fib-quant/src/rotation.rs:37-39, spherical_beta.rs:96-104,121-122.
 *    The 257-entry tables are regenerated with the procedure of rand's
 *    ziggurat_tables.py (R = 3.6541528853610088, V = 0.00492867323399,
 *    x0 = V/f(R), x_i = f^-1(V/x_{i-1} + f(x_{i-1})), x_256 = 0), then
 *    round-tripped through "%.18f" exactly as the generated Rust literals
 *    were written.  Pinned against remembered literals of ziggurat_tables.rs
 *    (tests/test_oracle_rng.py) and, entry by entry, against the correctly
 *    rounded recursion (tests/test_oracle_pins.py).
 * ====================================================================== */
static double ZX[257], ZF[257];
static double ZIG_R;
static int zig_ready = 0;

/* Test hooks (not part of the restatement): how far the draws are from
 * depending on the last bit of a libm result.  While g_track is set,
 * track() keeps the smallest relative gap between the two sides of every
 * accept / reject comparison that involves exp or log, and the tail branch
 * records the arguments and results of its log calls (the drawn value is
 * built from them directly). */
static int g_track = 0;
static double g_margin = INFINITY;
/* branch counts while g_track is set: ziggurat iterations, wedge tests,
 * wedge acceptances, base-strip tail entries; gamma proposals (v > 0),
 * squeeze acceptances, log acceptances */
static uint64_t g_cnt[7];
#define ORA_TAIL_LOGS 4096
static double g_tail_arg[ORA_TAIL_LOGS], g_tail_val[ORA_TAIL_LOGS];
static uint64_t g_tail_n = 0;

static void track(double lhs, double rhs) {
    if (!g_track) return;
    const double den = fabs(lhs) > fabs(rhs) ? fabs(lhs) : fabs(rhs);
    const double m = den > 0.0 ? fabs(lhs - rhs) / den : INFINITY;
    if (m < g_margin) g_margin = m;
}

static double tail_log(double v) {
    const double l = log(v);
    if (g_track) {
        if (g_tail_n < ORA_TAIL_LOGS) { g_tail_arg[g_tail_n] = v; g_tail_val[g_tail_n] = l; }
        g_tail_n++;
    }
    return l;
}

static double zig_f(double x) { return exp(-x * x / 2.0); }
/* The table takes the correctly rounded exp / log (x87 expl / logl rounded
 * to double: every call of the recursion lands far enough from a midpoint
 * for that, which tests/test_oracle_pins.py checks against mpmath), so it is
 * the table any correctly rounded libm gives -- glibc before 2.28 among
 * them.  glibc 2.35's exp differs at one call (F[94], 1 ulp);
 * ora_set_zig_glibc(1) rebuilds the table with it, for that comparison. */
static int g_zig_glibc = 0;
static double zig_f_tab(double x) {
    const double t = -x * x / 2.0;
    return g_zig_glibc ? exp(t) : (double)expl((long double)t);
}
static double zig_finv_tab(double y) { return sqrt(-2.0 * (g_zig_glibc ? log(y) : (double)logl((long double)y))); }
void ora_set_zig_glibc(int on) { g_zig_glibc = on; zig_ready = 0; }

static double round18(double v) {
    char buf[64];
    snprintf(buf, sizeof buf, "%.18f", v);
    return strtod(buf, NULL);
}

static void zig_init(void) {
    if (zig_ready) return;
    const double R = 3.6541528853610088, V = 0.00492867323399;
    double x[257];
    x[0] = V / zig_f_tab(R);
    x[1] = R;
    for (int i = 2; i < 256; ++i) x[i] = zig_finv_tab(V / x[i - 1] + zig_f_tab(x[i - 1]));
    x[256] = 0.0;
    for (int i = 0; i < 257; ++i) {
        ZF[i] = round18(zig_f_tab(x[i]));
        ZX[i] = round18(x[i]);
    }
    ZIG_R = round18(R);
    zig_ready = 1;
}

static double rng_normal(ora_rng* r) {
    zig_init();
    for (;;) {
        uint64_t bits = rng_u64(r);
        int i = (int)(bits & 0xff);
        double u = bits_to_f64((bits >> 12) | ((uint64_t)(1023 + 1) << 52)) - 3.0;
        double x = u * ZX[i];
        if (g_track) g_cnt[0]++;
        if (fabs(x) < ZX[i + 1]) return x;
        if (i == 0) {
            if (g_track) g_cnt[3]++;
            double xx = 1.0, yy = 0.0;
            while (-2.0 * yy < xx * xx) {
                double x_ = rng_open01(r);
                double y_ = rng_open01(r);
                xx = tail_log(x_) / ZIG_R;
                yy = tail_log(y_);
                track(-2.0 * yy, xx * xx);
            }
            return (u < 0.0) ? xx - ZIG_R : ZIG_R - xx;
        }
        const double lhs = ZF[i + 1] + (ZF[i] - ZF[i + 1]) * rng_f64(r), rhs = zig_f(x);
        track(lhs, rhs);
        if (g_track) g_cnt[1]++;
        if (lhs < rhs) {
            if (g_track) g_cnt[2]++;
            return x;
        }
    }
}

/* rand_distr 0.4.3 Gamma(shape > 1, scale): Marsaglia & Tsang (2000).
 * Called by fib-quant/src/spherical_beta.rs:116-121 with shapes k/2 and
 * (d-k)/2 (2 and 30 for d=64, k=4), both on the large-shape branch. */
typedef struct { double d, c, scale; } ora_gamma;

static void gamma_init(ora_gamma* g, double shape, double scale) {
    g->d = shape - 1.0 / 3.0;
    g->c = 1.0 / sqrt(9.0 * g->d);
    g->scale = scale;
}

static double rng_gamma(ora_rng* r, const ora_gamma* g) {
    for (;;) {
        double x = rng_normal(r);
        double v_cbrt = 1.0 + g->c * x;
        if (v_cbrt <= 0.0) continue;
        double v = v_cbrt * v_cbrt * v_cbrt;
        double u = rng_open01(r);
        double x_sqr = x * x;
        if (g_track) g_cnt[4]++;
        if (u < 1.0 - 0.0331 * x_sqr * x_sqr) {
            if (g_track) g_cnt[5]++;
            return g->d * v * g->scale;
        }
        const double lhs = log(u), rhs = 0.5 * x_sqr + g->d * (1.0 - v + log(v));
        track(lhs, rhs);
        if (lhs < rhs) {
            if (g_track) g_cnt[6]++;
            return g->d * v * g->scale;
        }
    }
}

/* ======================================================================
 * 3. Householder QR and the stored rotations.
 *    fib-quant/src/rotation.rs:24-58 (StoredRotation::new): d*d f64 normals
 *    fill a COLUMN-major matrix, Q of its QR with R_jj >= 0 (the column
 *    sign fix at :44-49), stored row-major.  turbo-quant's StoredQr
 *    (rotation.rs:334-370) is the same construction in f32 and is not on
 *    the power-of-two path.
 *    Parity: the Q with a non-negative R diagonal is unique, so any backward
 *    stable QR agrees with nalgebra's to ~1e-15; bit-identity with nalgebra
 *    is unpinned.  The reflector sequence below follows nalgebra's
 *    clear_column_unchecked / Reflection::reflect_with_sign / QR::q order.
 * ====================================================================== */
/* nalgebra Matrix::dotx: eight partial sums over chunks of 8, folded as
 * (a0+a4),(a1+a5),(a2+a6),(a3+a7), then a sequential tail. */
static double nal_dot(const double* a, const double* b, int len) {
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

/* A: n*n column-major, overwritten; Q: n*n column-major output. */
static int qr_q(int n, double* A, double* Q) {
    double* diag = (double*)malloc(sizeof(double) * n);
    if (!diag) return ORA_ERR_NUMERICAL;
    for (int i = 0; i < n; ++i) {
        double* col = A + (size_t)i * n;        /* column i, rows i..n-1 */
        int len = n - i;
        double sq = nal_dot(col + i, col + i, len);
        double nrm = sqrt(sq);
        double x0 = col[i];
        double modulus = fabs(x0);
        double sgn = (x0 < 0.0) ? -1.0 : 1.0;   /* signum of a real; +1 for +0 */
        double signed_norm = sgn * nrm;
        double factor = (sq + modulus * nrm) * 2.0;
        col[i] += signed_norm;
        if (factor != 0.0) {
            double s = sqrt(factor);
            for (int t = 0; t < len; ++t) col[i + t] /= s;
            diag[i] = -signed_norm;
            double rsign = (diag[i] < 0.0) ? -1.0 : 1.0;
            /* reflect the trailing columns with sign = signum(diag) */
            for (int j = i + 1; j < n; ++j) {
                double* cj = A + (size_t)j * n;
                double dot = nal_dot(col + i, cj + i, len);
                double f = dot * (rsign * -2.0);
                for (int t = 0; t < len; ++t) cj[i + t] = f * col[i + t] + rsign * cj[i + t];
            }
        } else {
            diag[i] = signed_norm;
        }
    }
    /* Q = H_0 ... H_{n-1} applied to the identity, last reflector first. */
    for (int j = 0; j < n; ++j)
        for (int r = 0; r < n; ++r) Q[(size_t)j * n + r] = (r == j) ? 1.0 : 0.0;
    for (int i = n - 1; i >= 0; --i) {
        const double* axis = A + (size_t)i * n;   /* rows i..n-1 */
        int len = n - i;
        double rsign = (diag[i] < 0.0) ? -1.0 : 1.0;
        for (int j = i; j < n; ++j) {
            double* cj = Q + (size_t)j * n;
            double dot = nal_dot(axis + i, cj + i, len);
            double f = dot * (rsign * -2.0);
            for (int t = 0; t < len; ++t) cj[i + t] = f * axis[i + t] + rsign * cj[i + t];
        }
    }
    /* R_jj = |diag_j| >= 0 always, so the reference's sign fix
     * (fib-quant/src/rotation.rs:44-49) leaves Q unchanged. */
    free(diag);
    return ORA_OK;
}

/* StoredRotation::new -> row-major f64 matrix (fib-quant/src/rotation.rs:24-58). */
static int stored_rotation(int d, uint64_t seed, double* out_rowmajor) {
    ora_rng r;
    rng_seed_from_u64(&r, seed);
    size_t nn = (size_t)d * d;
    double* A = (double*)malloc(sizeof(double) * nn);
    double* Q = (double*)malloc(sizeof(double) * nn);
    if (!A || !Q) { free(A); free(Q); return ORA_ERR_NUMERICAL; }
    for (size_t t = 0; t < nn; ++t) A[t] = rng_normal(&r);   /* column-major fill */
    int rc = qr_q(d, A, Q);
    if (rc == ORA_OK)
        for (int row = 0; row < d; ++row)
            for (int col = 0; col < d; ++col)
                out_rowmajor[(size_t)row * d + col] = Q[(size_t)col * d + row];
    free(A); free(Q);
    return rc;
}

/* StoredRotation::apply (fib-quant/src/rotation.rs:104-115): y = Pi x, f64,
 * each row a sequential sum. */
static void rot_apply_f64(int d, const double* M, const double* x, double* y) {
    for (int row = 0; row < d; ++row) {
        double s = 0.0;
        for (int c = 0; c < d; ++c) s += M[(size_t)row * d + c] * x[c];
        y[row] = s;
    }
}

/* ======================================================================
 * 4. Special functions for the fib codebook initialisation.
 *    Normal::inverse_cdf is used by directions.rs:49-58; Beta::inverse_cdf
 *    by beta_inv.rs:17-19 via spherical_beta.rs:24-39.  Both are restated
 *    to full double accuracy (initial guess + safeguarded Newton), not as
 *    the statrs code path: the Lloyd-Max refinement that follows replaces
 *    every codeword by the mean of its assigned training samples, so an
 *    initial codeword that differs by ~1e-15 yields a bit-identical final
 *    codebook unless a training sample sits within ~1e-15 of a Voronoi
 *    boundary.  Parity of these two functions is pinned by closed forms
 *    (tests/test_oracle_profile.py), not by reference values.
 * ====================================================================== */

static double inv_norm_cdf_lower(double p);

/* Upper half by symmetry: 1 - p is exact for p in [0.5, 1] (Sterbenz), and
 * the lower-tail refinement keeps full relative accuracy there (statrs
 * evaluates -sqrt2 * erfc_inv(2p), which is the same quantity). */
static double inv_norm_cdf(double p) {
    if (p > 0.5) return -inv_norm_cdf_lower(1.0 - p);
    return inv_norm_cdf_lower(p);
}

static long double norm_cdf_l(long double x) { return 0.5L * erfcl(-x / sqrtl(2.0L)); }

static double inv_norm_cdf_lower(double p) {
    /* Acklam's rational approximation, then Halley steps on erfc carried in
     * x87 long double and rounded once: the correctly rounded quantile (the
     * exact value statrs approximates; checked against mpmath for the
     * profiles tested, tests/test_oracle_pins.py). */
    static const double a[] = {-3.969683028665376e+01, 2.209460984245205e+02,
        -2.759285104469687e+02, 1.383577518672690e+02, -3.066479806614716e+01, 2.506628277459239e+00};
    static const double b[] = {-5.447609879822406e+01, 1.615858368580409e+02,
        -1.556989798598866e+02, 6.680131188771972e+01, -1.328068155288572e+01};
    static const double c[] = {-7.784894002430293e-03, -3.223964580411365e-01,
        -2.400758277161838e+00, -2.549732539343734e+00, 4.374664141464968e+00, 2.938163982698783e+00};
    static const double dd[] = {7.784695709041462e-03, 3.224671290700398e-01,
        2.445134137142996e+00, 3.754408661907416e+00};
    double q, x;
    if (p < 0.02425) {
        q = sqrt(-2 * log(p));
        x = (((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5]) /
            ((((dd[0] * q + dd[1]) * q + dd[2]) * q + dd[3]) * q + 1);
    } else if (p > 1 - 0.02425) {
        q = sqrt(-2 * log(1 - p));
        x = -(((((c[0] * q + c[1]) * q + c[2]) * q + c[3]) * q + c[4]) * q + c[5]) /
            ((((dd[0] * q + dd[1]) * q + dd[2]) * q + dd[3]) * q + 1);
    } else {
        q = p - 0.5;
        double rr = q * q;
        x = (((((a[0] * rr + a[1]) * rr + a[2]) * rr + a[3]) * rr + a[4]) * rr + a[5]) * q /
            (((((b[0] * rr + b[1]) * rr + b[2]) * rr + b[3]) * rr + b[4]) * rr + 1);
    }
    long double xl = x;
    for (int it = 0; it < 4; ++it) {
        long double e = norm_cdf_l(xl) - (long double)p;
        long double u = e * sqrtl(2.0L * 3.14159265358979323846264338327950288L) * expl(xl * xl / 2.0L);
        xl = xl - u / (1.0L + xl * u / 2.0L);
    }
    return (double)xl;
}

/* Regularized incomplete beta I_x(a,b) by Lentz's continued fraction, in
 * long double. */
static long double betacf(long double a, long double b, long double x) {
    const long double TINY = 1e-300L;
    long double qab = a + b, qap = a + 1, qam = a - 1;
    long double c = 1, d = 1 - qab * x / qap;
    if (fabsl(d) < TINY) d = TINY;
    d = 1 / d;
    long double h = d;
    for (int m = 1; m <= 10000; ++m) {
        int m2 = 2 * m;
        long double aa = m * (b - m) * x / ((qam + m2) * (a + m2));
        d = 1 + aa * d; if (fabsl(d) < TINY) d = TINY;
        c = 1 + aa / c; if (fabsl(c) < TINY) c = TINY;
        d = 1 / d; h *= d * c;
        aa = -(a + m) * (qab + m) * x / ((a + m2) * (qap + m2));
        d = 1 + aa * d; if (fabsl(d) < TINY) d = TINY;
        c = 1 + aa / c; if (fabsl(c) < TINY) c = TINY;
        d = 1 / d;
        long double del = d * c;
        h *= del;
        if (fabsl(del - 1) < 1e-20L) break;
    }
    return h;
}

static long double beta_reg(long double a, long double b, long double x) {
    if (x <= 0) return 0;
    if (x >= 1) return 1;
    long double lbt = lgammal(a + b) - lgammal(a) - lgammal(b) + a * logl(x) + b * log1pl(-x);
    long double bt = expl(lbt);
    if (x < (a + 1) / (a + b + 2)) return bt * betacf(a, b, x) / a;
    return 1 - bt * betacf(b, a, 1 - x) / b;
}

static long double beta_pdf(long double a, long double b, long double x) {
    return expl(lgammal(a + b) - lgammal(a) - lgammal(b) + (a - 1) * logl(x) + (b - 1) * log1pl(-x));
}

/* Beta(a,b) inverse CDF: bisection to a bracket, then safeguarded Newton,
 * in long double, rounded once (the correctly rounded quantile; see
 * inv_norm_cdf_lower). */
static double beta_inv(double q, double a, double b) {
    if (q <= 0) return 0;
    if (q >= 1) return 1;
    long double lo = 0, hi = 1, x = 0.5L;
    for (int it = 0; it < 70; ++it) {
        x = 0.5L * (lo + hi);
        if (beta_reg(a, b, x) < (long double)q) lo = x; else hi = x;
    }
    for (int it = 0; it < 8; ++it) {
        long double f = beta_reg(a, b, x) - (long double)q;
        long double p = beta_pdf(a, b, x);
        if (!(p > 0)) break;
        long double nx = x - f / p;
        if (!(nx > lo && nx < hi)) break;
        if (nx == x) break;
        x = nx;
    }
    if (x < 0) x = 0;
    if (x > 1) x = 1;
    return (double)x;
}

/* compiler-rt __powidf2: what Rust's f64::powi lowers to for a runtime
 * exponent (directions.rs:50, 105). */
static double powi_rt(double a, int b) {
    int recip = b < 0;
    double r = 1;
    for (;;) {
        if (b & 1) r *= a;
        b /= 2;
        if (b == 0) break;
        a *= a;
    }
    return recip ? 1 / r : r;
}

/* fib-quant/src/directions.rs:96-114 */
static double roberts_phi(int k) {
    double lo = 1.0, hi = 2.0;
    for (int it = 0; it < 128; ++it) {
        double mid = (lo + hi) / 2.0;
        double v = powi_rt(mid, k + 1) - mid - 1.0;
        if (v > 0.0) hi = mid; else lo = mid;
    }
    return (lo + hi) / 2.0;
}

/* fib-quant/src/directions.rs:38-71 (n directions of dimension k, row-major). */
static int roberts_kronecker(int k, int n, double* out) {
    if (k < 4 || n <= 0) return ORA_ERR_INVALID_ARG;
    double phi = roberts_phi(k);
    for (int idx = 0; idx < n; ++idx) {
        double norm_sq = 0.0;
        for (int j = 1; j <= k; ++j) {
            double step = powi_rt(phi, -j);
            double t = ((double)idx + 0.5) * step;
            double frac = t - trunc(t);
            if (frac < 1.0e-12) frac = 1.0e-12;
            if (frac > 1.0 - 1.0e-12) frac = 1.0 - 1.0e-12;
            double v = inv_norm_cdf(frac);
            norm_sq += v * v;
            out[(size_t)idx * k + (j - 1)] = v;
        }
        if (!(norm_sq > 0.0) || !isfinite(norm_sq)) return ORA_ERR_NUMERICAL;
        double nrm = sqrt(norm_sq);
        for (int j = 0; j < k; ++j) out[(size_t)idx * k + j] /= nrm;
    }
    return ORA_OK;
}

/* fib-quant/src/spherical_beta.rs:6-21 */
static double beta_d_k(int d, int k) {
    if (k == d) return 1.0;
    double dk = ((double)d - (double)k - 2.0) / 2.0;
    return ((double)k / ((double)k + 2.0)) * dk + 1.0;
}

/* fib-quant/src/spherical_beta.rs:24-39 */
static double radius_quantile(int d, int k, int n, int n_total) {
    if (k == d) return 1.0;
    double q = ((double)n - 0.5) / (double)n_total;
    double alpha = (double)k / 2.0;
    double beta = beta_d_k(d, k);
    double x = beta_inv(q, alpha, beta);
    if (x < 0) x = 0;
    if (x > 1) x = 1;
    return sqrt(x);
}

/* ======================================================================
 * 5. FibCodebookV1::build  (codebook.rs:40-60, 161-184; lloyd.rs:106-337;
 *    spherical_beta.rs:58-126).  Profile: proveKV overrides
 *    (proveKV/src/codec.rs:475-491, policy.rs:137-145) of paper_default
 *    (profile.rs:132-173): codebook_seed = seed + 0x9e3779b97f4a7c15.
 *    Parity: exact given the RNG chain; the RNG chain is pinned by known
 *    answers, the end result (the codebook values) is unpinned against the
 *    reference (no reference codebook is committed anywhere).
 * ====================================================================== */
static void sample_unit_sphere(ora_rng* r, int k, double* out) {
    for (;;) {
        double norm_sq = 0.0;
        for (int t = 0; t < k; ++t) { out[t] = rng_normal(r); norm_sq += out[t] * out[t]; }
        if (norm_sq > 0.0 && isfinite(norm_sq)) {
            double nrm = sqrt(norm_sq);
            for (int t = 0; t < k; ++t) out[t] = out[t] / nrm;
            return;
        }
    }
}

static int sample_spherical_beta(ora_rng* r, int d, int k, double* out) {
    if (k == d) { sample_unit_sphere(r, k, out); return ORA_OK; }
    ora_gamma ga, gb;
    gamma_init(&ga, (double)k / 2.0, 1.0);
    gamma_init(&gb, (double)(d - k) / 2.0, 1.0);
    /* both shapes > 1 for the in-scope profiles (k=4; d=64 or 128) */
    if ((double)k / 2.0 <= 1.0 || (double)(d - k) / 2.0 <= 1.0) return ORA_ERR_INVALID_ARG;
    double a = rng_gamma(r, &ga);
    double b = rng_gamma(r, &gb);
    double sum = a + b;
    if (sum <= 0.0 || !isfinite(sum)) return ORA_ERR_NUMERICAL;
    double r2 = a / sum;
    double dir[16];
    sample_unit_sphere(r, k, dir);
    double rad = sqrt(r2);
    for (int t = 0; t < k; ++t) out[t] = rad * dir[t];
    return ORA_OK;
}

/* lloyd.rs:319-337 */
static int nearest_index_f64(const double* s, const double* cb, int k, int n, double* best_out) {
    int best = 0;
    double bd = INFINITY;
    for (int w = 0; w < n; ++w) {
        double dist = 0.0;
        for (int t = 0; t < k; ++t) { double dl = s[t] - cb[(size_t)w * k + t]; dist += dl * dl; }
        if (dist < bd) { bd = dist; best = w; }
    }
    if (best_out) *best_out = bd;
    return best;
}

static double mse_for_codebook(const double* cb, int k, int n, const double* samples, int ns) {
    double sum = 0.0;
    for (int i = 0; i < ns; ++i) {
        double bd;
        nearest_index_f64(samples + (size_t)i * k, cb, k, n, &bd);
        sum += bd;
    }
    return sum / (double)ns;
}

/* LloydRepairEventV1 rows of a refinement (lloyd.rs:17-34, pushed at
 * 297-306): restart, iteration, empty_cell, donor_cell, donor_count_before,
 * donor_distortion, residual_norm; split_epsilon is the constant 1e-6. */
typedef struct {
    double* rows;   /* 7 per event */
    int n, cap;
    int restart, iteration;
} ora_events;

static void events_push(ora_events* ev, int empty, int donor, int count, double distortion, double rnorm) {
    if (!ev) return;
    if (ev->n == ev->cap) {
        ev->cap = ev->cap ? 2 * ev->cap : 16;
        ev->rows = (double*)realloc(ev->rows, sizeof(double) * 7 * (size_t)ev->cap);
    }
    double* r = ev->rows + 7 * (size_t)ev->n++;
    r[0] = ev->restart; r[1] = ev->iteration; r[2] = empty; r[3] = donor; r[4] = count;
    r[5] = distortion; r[6] = rnorm;
}

/* lloyd.rs:222-317 (SplitHighestDistortion policy) */
static int update_centroids(double* cb, int k, int n, const double* samples, int ns, const int* asg,
                            ora_events* ev) {
    double* sums = (double*)calloc((size_t)n * k, sizeof(double));
    int* counts = (int*)calloc(n, sizeof(int));
    double* distortion = (double*)calloc(n, sizeof(double));
    double* far = (double*)calloc((size_t)n * k, sizeof(double));
    double* fard = (double*)malloc(sizeof(double) * n);
    int rc = ORA_OK;
    for (int w = 0; w < n; ++w) fard[w] = -1.0;
    for (int i = 0; i < ns; ++i) {
        int a = asg[i];
        const double* s = samples + (size_t)i * k;
        counts[a] += 1;
        double sd = 0.0;
        for (int t = 0; t < k; ++t) {
            sums[(size_t)a * k + t] += s[t];
            double dl = s[t] - cb[(size_t)a * k + t];
            sd += dl * dl;
        }
        distortion[a] += sd;
        if (sd > fard[a]) { fard[a] = sd; memcpy(far + (size_t)a * k, s, sizeof(double) * k); }
    }
    for (int w = 0; w < n; ++w)
        if (counts[w] > 0)
            for (int t = 0; t < k; ++t) cb[(size_t)w * k + t] = sums[(size_t)w * k + t] / (double)counts[w];
    for (int e = 0; e < n; ++e) {
        if (counts[e] != 0) continue;
        /* Iterator::max_by keeps the LAST maximum; total_cmp ordering. */
        int donor = -1;
        for (int w = 0; w < n; ++w) {
            if (counts[w] <= 1) continue;
            if (donor < 0 || !(distortion[w] < distortion[donor])) donor = w;
        }
        if (donor < 0) { rc = ORA_ERR_NUMERICAL; break; }
        double res[16], rn2 = 0.0;
        for (int t = 0; t < k; ++t) {
            res[t] = far[(size_t)donor * k + t] - cb[(size_t)donor * k + t];
            rn2 += res[t] * res[t];
        }
        double rn = sqrt(rn2);
        if (!isfinite(rn) || rn <= DBL_EPSILON) { rc = ORA_ERR_NUMERICAL; break; }
        for (int t = 0; t < k; ++t) {
            double dir = res[t] / rn;
            double cen = cb[(size_t)donor * k + t];
            cb[(size_t)donor * k + t] = cen - 1.0e-6 * dir;
            cb[(size_t)e * k + t] = cen + 1.0e-6 * dir;
        }
        events_push(ev, e, donor, counts[donor], distortion[donor], rn);
        counts[donor] -= 1;
        counts[e] = 1;
        distortion[donor] = 0.0;
        distortion[e] = 0.0;
    }
    free(sums); free(counts); free(distortion); free(far); free(fard);
    return rc;
}

/* refine_codebook's restart loop (lloyd.rs:128-147) over given samples
 * [ns][k] and starts [restarts][n][k]: each restart iterates assign_samples +
 * update_centroids `iterations` times, then mse_for_codebook; init_mse is the
 * MSE of starts[0].  Returns ORA_ERR_NUMERICAL when a repair finds no donor. */
int ora_lloyd_refine(const double* samples, int ns, int k, int n, const double* starts, int restarts,
                     int iterations, double* out_cb, double* out_mse, double* init_mse) {
    if (ns <= 0 || k <= 0 || k > 16 || n < 2 || restarts <= 0) return ORA_ERR_INVALID_ARG;
    size_t nk = (size_t)n * k;
    int* asg = (int*)malloc(sizeof(int) * (size_t)ns);
    int rc = ORA_OK;
    *init_mse = mse_for_codebook(starts, k, n, samples, ns);
    for (int r = 0; r < restarts && rc == ORA_OK; ++r) {
        double* cb = out_cb + (size_t)r * nk;
        memcpy(cb, starts + (size_t)r * nk, sizeof(double) * nk);
        for (int it = 0; it < iterations && rc == ORA_OK; ++it) {
            for (int i = 0; i < ns; ++i) asg[i] = nearest_index_f64(samples + (size_t)i * k, cb, k, n, NULL);
            rc = update_centroids(cb, k, n, samples, ns, asg, NULL);
        }
        out_mse[r] = mse_for_codebook(cb, k, n, samples, ns);
    }
    free(asg);
    return rc;
}

/* Test hook (not part of the restatement): every initial codeword
 * coordinate and every restart's rotated start is multiplied by
 * 1 +- g_perturb (sign from a fixed pseudo-random pattern), standing in for
 * last-bit differences of the inverse CDFs (statrs) and of the k x k QR
 * (nalgebra) behind them. */
static double g_perturb = 0.0;
static void perturb(double* v, size_t n, uint64_t salt) {
    if (g_perturb == 0.0) return;
    for (size_t t = 0; t < n; ++t) {
        uint64_t h = (t + 1) * 0x9e3779b97f4a7c15ull ^ salt;
        h ^= h >> 29;
        h *= 0xbf58476d1ce4e5b9ull;
        h ^= h >> 32;
        v[t] *= (h & 1) ? 1.0 + g_perturb : 1.0 - g_perturb;
    }
}

/* Build the (N x k) f32 codebook; returns init/training mse, the best
 * restart (UINT32_MAX when the start is kept, lloyd.rs:158-162) and, when
 * `ev` is given, the repair events of every restart. */
static int fib_codebook(int d, int k, int n, uint64_t seed, int training, int restarts, int iterations,
                        float* out, double* init_mse_out, double* train_mse_out, uint32_t* best_restart_out,
                        ora_events* ev) {
    if (k < 4 || k > 16 || d % k != 0 || n < 2) return ORA_ERR_INVALID_ARG;
    uint64_t cseed = seed + 0x9e3779b97f4a7c15ull;
    size_t nk = (size_t)n * k;
    double* init = (double*)malloc(sizeof(double) * nk);
    double* dirs = (double*)malloc(sizeof(double) * nk);
    int ns = training > n ? training : n;
    double* samples = (double*)malloc(sizeof(double) * (size_t)ns * k);
    double* best = (double*)malloc(sizeof(double) * nk);
    double* cbk = (double*)malloc(sizeof(double) * nk);
    int* asg = (int*)malloc(sizeof(int) * ns);
    int rc = roberts_kronecker(k, n, dirs);
    if (rc != ORA_OK) goto done;
    for (int idx = 0; idx < n; ++idx) {
        double rad = radius_quantile(d, k, idx + 1, n);
        for (int t = 0; t < k; ++t) init[(size_t)idx * k + t] = rad * dirs[(size_t)idx * k + t];
    }
    perturb(init, nk, 0);
    {
        ora_rng r;
        rng_seed_from_u64(&r, cseed ^ 0x465155414e54ull);
        for (int i = 0; i < ns; ++i) {
            rc = sample_spherical_beta(&r, d, k, samples + (size_t)i * k);
            if (rc != ORA_OK) goto done;
        }
    }
    double init_mse = mse_for_codebook(init, k, n, samples, ns);
    double best_mse = init_mse;
    uint32_t best_restart = 0;
    memcpy(best, init, sizeof(double) * nk);
    if (restarts < 1) restarts = 1;
    for (int rs = 0; rs < restarts; ++rs) {
        if (rs == 0) {
            memcpy(cbk, init, sizeof(double) * nk);
        } else {
            double rot[16 * 16];
            rc = stored_rotation(k, cseed + (uint64_t)rs * 0x9e3779b9ull, rot);
            if (rc != ORA_OK) goto done;
            for (int w = 0; w < n; ++w) rot_apply_f64(k, rot, init + (size_t)w * k, cbk + (size_t)w * k);
            perturb(cbk, nk, (uint64_t)rs);
        }
        for (int it = 0; it < iterations; ++it) {
            for (int i = 0; i < ns; ++i) asg[i] = nearest_index_f64(samples + (size_t)i * k, cbk, k, n, NULL);
            if (ev) { ev->restart = rs; ev->iteration = it; }
            rc = update_centroids(cbk, k, n, samples, ns, asg, ev);
            if (rc != ORA_OK) goto done;
        }
        double mse = mse_for_codebook(cbk, k, n, samples, ns);
        if (mse < best_mse || (rs == 0 && isinf(init_mse))) {
            best_mse = mse;
            best_restart = (uint32_t)rs;
            memcpy(best, cbk, sizeof(double) * nk);
        }
    }
    if (best_mse > init_mse) {
        memcpy(best, init, sizeof(double) * nk);
        best_mse = init_mse;
        best_restart = UINT32_MAX;
    }
    for (size_t t = 0; t < nk; ++t) out[t] = (float)best[t];
    if (init_mse_out) *init_mse_out = init_mse;
    if (train_mse_out) *train_mse_out = best_mse;
    if (best_restart_out) *best_restart_out = best_restart;
done:
    free(init); free(dirs); free(samples); free(best); free(cbk); free(asg);
    return rc;
}

/* ======================================================================
 * 6. turbo-quant codec: TurboQuantizer(dim, bits, projections, seed),
 *    PolarWithQjl (turbo.rs:124-188) or PolarOnly; FastHadamard rotation
 *    (power-of-two dims); TQB1 batch wire (wire.rs:260-568).
 * ====================================================================== */
#define ORA_PI_F 3.14159265358979323846f   /* std::f32::consts::PI */

/* FastHadamardRotation::new (rotation.rs:143-157) and
 * generate_projection_matrix (qjl.rs:341-352, seeds turbo.rs:166-167). */
int ora_turbo_constants(uint32_t dim, uint32_t proj, uint64_t seed, float* signs, float* G) {
    if (dim == 0 || (dim & (dim - 1)) != 0) return ORA_ERR_INVALID_ARG;
    ora_rng r;
    rng_seed_from_u64(&r, seed + 0xA11CE55ED5A5EED5ull);
    for (uint32_t i = 0; i < dim; ++i) signs[i] = rng_bool(&r) ? 1.0f : -1.0f;
    if (G && proj > 0) {
        uint64_t qseed = (seed + 0xCAFEBABE00000001ull) + 0xDEADBEEF12345678ull;
        rng_seed_from_u64(&r, qseed);
        for (size_t t = 0; t < (size_t)proj * dim; ++t) G[t] = (float)rng_normal(&r);
    }
    return ORA_OK;
}

/* fwht_normalized (rotation.rs:379-398) */
static void fwht_normalized(float* v, int n) {
    for (int step = 1; step < n; step *= 2) {
        int block = step * 2;
        for (int start = 0; start < n; start += block)
            for (int off = 0; off < step; ++off) {
                float a = v[start + off], b = v[start + off + step];
                v[start + off] = a + b;
                v[start + off + step] = a - b;
            }
    }
    float scale = 1.0f / sqrtf((float)n);
    for (int i = 0; i < n; ++i) v[i] *= scale;
}

/* FastHadamardRotation::apply (rotation.rs:202-211) */
void ora_turbo_rotate(uint32_t dim, const float* signs, const float* x, float* y) {
    for (uint32_t i = 0; i < dim; ++i) y[i] = x[i] * signs[i];
    fwht_normalized(y, (int)dim);
}

/* apply_inverse (rotation.rs:212-222) */
void ora_turbo_rotate_inverse(uint32_t dim, const float* signs, const float* y, float* x) {
    for (uint32_t i = 0; i < dim; ++i) x[i] = y[i];
    fwht_normalized(x, (int)dim);
    for (uint32_t i = 0; i < dim; ++i) x[i] *= signs[i];
}

/* encode_pair (polar.rs:413-421) */
static void encode_pair(float a, float b, int bits, float* r, uint16_t* idx) {
    float aa = a * a, bb = b * b;
    *r = sqrtf(aa + bb);
    float theta = atan2f(b, a);
    uint32_t levels = 1u << bits;
    float normalized = (theta + ORA_PI_F) / (2.0f * ORA_PI_F);
    float f = floorf(normalized * (float)levels);
    uint32_t u;
    if (!(f > 0.0f)) u = 0;                     /* `as u32` saturates; NaN -> 0 */
    else if (f >= 4294967296.0f) u = 0xFFFFFFFFu;
    else u = (uint32_t)f;
    *idx = (uint16_t)(u % levels);
}

/* dequantize_angle (polar.rs:91-95) */
static float dequant_angle(uint16_t idx, int bits) {
    uint32_t levels = 1u << bits;
    return ((float)idx / (float)levels) * (2.0f * ORA_PI_F) - ORA_PI_F;
}

/* decode_to_rotated + apply_inverse (polar.rs:272-278, 306-316) */
static void polar_decode(uint32_t dim, const float* signs, const float* radii, const uint16_t* idx,
                         int bits, float* out) {
    float rot[256];
    for (uint32_t i = 0; i < dim / 2; ++i) {
        float th = dequant_angle(idx[i], bits);
        rot[2 * i] = radii[i] * cosf(th);
        rot[2 * i + 1] = radii[i] * sinf(th);
    }
    ora_turbo_rotate_inverse(dim, signs, rot, out);
}

/* TurboQuantizer::encode (turbo.rs:256-288) for one vector.  Returns an
 * ORA_ERR code; radii/idx/signbits filled on success.  mode 1 =
 * PolarWithQjl, 0 = PolarOnly. */
int ora_turbo_encode_vector(uint32_t dim, uint32_t bits, uint32_t proj, int mode, const float* signs,
                            const float* G, const float* x, float* radii, uint16_t* idx,
                            uint8_t* signbits) {
    int pbits = mode ? (int)bits - 1 : (int)bits;
    for (uint32_t i = 0; i < dim; ++i) if (!isfinite(x[i])) return ORA_ERR_NONFINITE_INPUT;
    float y[256];
    ora_turbo_rotate(dim, signs, x, y);
    for (uint32_t i = 0; i < dim / 2; ++i) encode_pair(y[2 * i], y[2 * i + 1], pbits, &radii[i], &idx[i]);
    for (uint32_t i = 0; i < dim / 2; ++i)
        if (!isfinite(radii[i]) || radii[i] < 0.0f) return ORA_ERR_RADIUS;
    if (!mode) return ORA_OK;
    float rec[256], res[256];
    polar_decode(dim, signs, radii, idx, pbits, rec);
    for (uint32_t i = 0; i < dim; ++i) res[i] = x[i] - rec[i];
    for (uint32_t i = 0; i < dim; ++i) if (!isfinite(res[i])) return ORA_ERR_RESIDUAL;
    memset(signbits, 0, (proj + 7) / 8);
    for (uint32_t j = 0; j < proj; ++j) {
        float dot = 0.0f;
        for (uint32_t c = 0; c < dim; ++c) dot = dot + G[(size_t)j * dim + c] * res[c];
        if (dot >= 0.0f) signbits[j / 8] |= (uint8_t)(1u << (j % 8));
    }
    return ORA_OK;
}

/* LSB-first bit writer (turbo bitpack.rs:135-143, fib bitpack.rs:4-45) */
static void write_bits(uint8_t* bytes, size_t bit_off, int bits, uint32_t v) {
    for (int b = 0; b < bits; ++b) {
        if (v & 1u) { size_t a = bit_off + b; bytes[a / 8] |= (uint8_t)(1u << (a % 8)); }
        v >>= 1;
    }
}
static uint32_t read_bits(const uint8_t* bytes, size_t bit_off, int bits) {
    uint32_t v = 0;
    for (int b = 0; b < bits; ++b) {
        size_t a = bit_off + b;
        v |= (uint32_t)((bytes[a / 8] >> (a % 8)) & 1u) << b;
    }
    return v;
}
static int padding_zero(const uint8_t* bytes, size_t used_bits, size_t nbytes) {
    for (size_t p = used_bits; p < nbytes * 8; ++p)
        if ((bytes[p / 8] >> (p % 8)) & 1u) return 0;
    return 1;
}

static void put_u16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }
static void put_u32(uint8_t* p, uint32_t v) { for (int i = 0; i < 4; ++i) p[i] = (uint8_t)(v >> (8 * i)); }
static void put_u64(uint8_t* p, uint64_t v) { for (int i = 0; i < 8; ++i) p[i] = (uint8_t)(v >> (8 * i)); }
static uint16_t get_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t get_u32(const uint8_t* p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}
static uint64_t get_u64(const uint8_t* p) { return (uint64_t)get_u32(p) | ((uint64_t)get_u32(p + 4) << 32); }
static float get_f32(const uint8_t* p) { uint32_t u = get_u32(p); float f; memcpy(&f, &u, 4); return f; }
static void put_f32(uint8_t* p, float f) { uint32_t u; memcpy(&u, &f, 4); put_u32(p, u); }

/* Rust f32::round: half away from zero. */
static float round_half_away(float v) { return roundf(v); }

/* CompressedRadiiV1::compress, BlockLogU8 branch (radius.rs:58-77). */
static void radii_log_u8(const float* radii, int count, uint8_t* q, float* mn_out, float* mx_out) {
    float logged[128];
    float mn = INFINITY, mx = -INFINITY;
    for (int i = 0; i < count; ++i) {
        float v = radii[i] < FLT_MIN ? FLT_MIN : radii[i];    /* f32::max(MIN_POSITIVE) */
        logged[i] = logf(v);
    }
    for (int i = 0; i < count; ++i) { mn = fminf(mn, logged[i]); mx = fmaxf(mx, logged[i]); }
    float span = fmaxf(mx - mn, FLT_EPSILON);
    for (int i = 0; i < count; ++i) {
        float nrm = (logged[i] - mn) / span;
        if (nrm < 0.0f) nrm = 0.0f;
        if (nrm > 1.0f) nrm = 1.0f;
        float v = round_half_away(nrm * 255.0f);
        q[i] = (uint8_t)(v >= 255.0f ? 255 : (v <= 0.0f ? 0 : (int)v));
    }
    *mn_out = mn; *mx_out = mx;
}

static uint32_t turbo_payload_len(uint32_t dim, int pbits, uint32_t proj, int mode, int radii_codec) {
    uint32_t pairs = dim / 2;
    uint32_t angle = (pairs * (uint32_t)pbits + 7) / 8;
    uint32_t sig = mode ? (proj + 7) / 8 : 0;
    uint32_t rad = radii_codec ? pairs + 8 : pairs * 4;
    return rad + angle + sig;
}

uint32_t ora_turbo_payload_len(uint32_t dim, uint32_t bits, uint32_t proj, int mode, int radii_codec) {
    return turbo_payload_len(dim, mode ? (int)bits - 1 : (int)bits, proj, mode, radii_codec);
}

static int turbo_check_profile(uint32_t dim, uint32_t bits, uint32_t proj, int mode) {
    if (dim == 0 || dim % 2 != 0 || dim > 256 || (dim & (dim - 1)) != 0) return 0;
    if (mode) { if (bits < 2 || bits > 16 || proj == 0 || proj > 1024) return 0; }
    else if (bits < 1 || bits > 16) return 0;
    return 1;
}

/* One vector's payload: [radii (f32, or BlockLogU8 u8s + min + max)]
 * [packed angle indices][packed QJL signs] (wire.rs:63-95, 350-390). */
static int turbo_encode_payload(uint32_t dim, uint32_t bits, uint32_t proj, int mode, int radii_codec,
                                const float* signs, const float* G, const float* xv, uint8_t* p) {
    int pbits = mode ? (int)bits - 1 : (int)bits;
    uint32_t pairs = dim / 2;
    uint32_t plen = turbo_payload_len(dim, pbits, proj, mode, radii_codec);
    uint32_t angle_bytes = (pairs * (uint32_t)pbits + 7) / 8;
    float radii[128];
    uint16_t idx[128];
    uint8_t sb[128];
    int rc = ora_turbo_encode_vector(dim, bits, proj, mode, signs, G, xv, radii, idx, sb);
    if (rc != ORA_OK) return rc;
    memset(p, 0, plen);
    if (radii_codec) {
        float mn, mx;
        radii_log_u8(radii, (int)pairs, p, &mn, &mx);
        put_f32(p + pairs, mn);
        put_f32(p + pairs + 4, mx);
        p += pairs + 8;
    } else {
        for (uint32_t i = 0; i < pairs; ++i) put_f32(p + 4 * i, radii[i]);
        p += 4 * pairs;
    }
    for (uint32_t i = 0; i < pairs; ++i) write_bits(p, (size_t)i * pbits, pbits, idx[i]);
    p += angle_bytes;
    if (mode) memcpy(p, sb, (proj + 7) / 8);
    return ORA_OK;
}

/* TurboQuantAdapter::encode_batch_compact (proveKV/src/codec.rs:248-291) =
 * per-vector TurboQuantizer::encode + TurboCodeWireV1::encode_batch_with_radii
 * (wire.rs:291-398).  x: n*dim row-major.  radii_codec: 0 F32, 1 BlockLogU8. */
int ora_turbo_encode_batch(uint32_t dim, uint32_t bits, uint32_t proj, uint64_t seed, int mode,
                           int radii_codec, const float* signs, const float* G, const float* x,
                           uint64_t n, uint8_t* out, uint64_t cap, uint64_t* out_len,
                           uint64_t* fail_index) {
    if (!turbo_check_profile(dim, bits, proj, mode)) return ORA_ERR_INVALID_ARG;
    int pbits = mode ? (int)bits - 1 : (int)bits;
    uint32_t plen = turbo_payload_len(dim, pbits, proj, mode, radii_codec);
    uint64_t total = 38 + n * (uint64_t)plen;
    if (out_len) *out_len = total;
    if (n == 0) return ORA_ERR_EMPTY;
    if (cap < total) return ORA_ERR_CAPACITY;
    memcpy(out, "TQB1", 4);
    put_u16(out + 4, 1);
    put_u16(out + 6, 1);       /* resolved FastHadamard for power-of-two dims */
    out[8] = 2; out[9] = 0;
    put_u32(out + 10, dim);
    out[14] = (uint8_t)pbits;
    out[15] = radii_codec ? 1 : 0;
    out[16] = 0; out[17] = 0;
    put_u32(out + 18, proj);
    put_u64(out + 22, seed);
    put_u32(out + 30, (uint32_t)n);
    put_u32(out + 34, plen);
    for (uint64_t v = 0; v < n; ++v) {
        int rc = turbo_encode_payload(dim, bits, proj, mode, radii_codec, signs, G, x + v * dim,
                                      out + 38 + v * plen);
        if (rc != ORA_OK) { if (fail_index) *fail_index = v; return rc; }
    }
    return ORA_OK;
}

/* TurboQuantAdapter::decode_batch_compact (proveKV/src/codec.rs:295-326) =
 * TurboCodeWireV1::decode_batch (wire.rs:401-568) + decode_approximate_batch
 * (turbo.rs:414-420). */
int ora_turbo_decode_batch(uint32_t dim, uint32_t bits, uint32_t proj, uint64_t seed, int mode,
                           const float* signs, const uint8_t* in, uint64_t len, float* out,
                           uint64_t cap_vectors, uint64_t* n_out, uint64_t* fail_index) {
    if (!turbo_check_profile(dim, bits, proj, mode)) return ORA_ERR_INVALID_ARG;
    if (len < 38) return ORA_ERR_MALFORMED;
    if (memcmp(in, "TQB1", 4) != 0) return ORA_ERR_MALFORMED;
    if (get_u16(in + 4) != 1) return ORA_ERR_MALFORMED;
    if (get_u16(in + 6) != 1) return ORA_ERR_MALFORMED;   /* rotation flag vs profile */
    if (in[8] != 2) return ORA_ERR_MALFORMED;
    uint32_t wdim = get_u32(in + 10);
    int pbits_w = in[14];
    int rc_byte = in[15];
    if (rc_byte > 1) return ORA_ERR_MALFORMED;
    uint32_t wproj = get_u32(in + 18);
    uint64_t wseed = get_u64(in + 22);
    uint64_t n = get_u32(in + 30);
    uint32_t plen = get_u32(in + 34);
    if (wdim != dim || wproj != proj || wseed != seed) return ORA_ERR_MALFORMED;
    int pbits = mode ? (int)bits - 1 : (int)bits;
    if (pbits_w != pbits) return ORA_ERR_MALFORMED;
    uint32_t pairs = dim / 2;
    if (plen != turbo_payload_len(dim, pbits, proj, mode, rc_byte)) return ORA_ERR_MALFORMED;
    if (len < 38 + n * (uint64_t)plen) return ORA_ERR_MALFORMED;   /* wire.rs:489-498 */
    if (n_out) *n_out = n;
    if (cap_vectors < n) return ORA_ERR_CAPACITY;
    uint32_t angle_bytes = (pairs * (uint32_t)pbits + 7) / 8;
    uint32_t sign_bytes = mode ? (proj + 7) / 8 : 0;
    float radii[128];
    uint16_t idx[128];
    for (uint64_t v = 0; v < n; ++v) {
        const uint8_t* p = in + 38 + v * plen;
        if (rc_byte) {
            float mn = get_f32(p + pairs), mx = get_f32(p + pairs + 4);
            if (!isfinite(mn) || !isfinite(mx) || mn > mx) { if (fail_index) *fail_index = v; return ORA_ERR_MALFORMED; }
            float span = mx - mn;
            for (uint32_t i = 0; i < pairs; ++i) radii[i] = expf(mn + span * ((float)p[i] / 255.0f));
            p += pairs + 8;
        } else {
            for (uint32_t i = 0; i < pairs; ++i) {
                radii[i] = get_f32(p + 4 * i);
                if (!isfinite(radii[i]) || radii[i] < 0.0f) { if (fail_index) *fail_index = v; return ORA_ERR_MALFORMED; }
            }
            p += 4 * pairs;
        }
        if (!padding_zero(p, (size_t)pairs * pbits, angle_bytes)) { if (fail_index) *fail_index = v; return ORA_ERR_MALFORMED; }
        for (uint32_t i = 0; i < pairs; ++i) idx[i] = (uint16_t)read_bits(p, (size_t)i * pbits, pbits);
        p += angle_bytes;
        if (mode && !padding_zero(p, proj, sign_bytes)) { if (fail_index) *fail_index = v; return ORA_ERR_MALFORMED; }
        /* PolarCode::validate_for (polar.rs:104-153): radii finite, >= 0 */
        for (uint32_t i = 0; i < pairs; ++i)
            if (!isfinite(radii[i]) || radii[i] < 0.0f) { if (fail_index) *fail_index = v; return ORA_ERR_MALFORMED; }
    }
    /* cursor.finish() (wire.rs:566): trailing bytes are rejected only after
     * every vector has been read and validated */
    if (len != 38 + n * (uint64_t)plen) return ORA_ERR_MALFORMED;
    if (!out) return ORA_OK;   /* validation only */
    for (uint64_t v = 0; v < n; ++v) {
        const uint8_t* p = in + 38 + v * plen;
        if (rc_byte) {
            float mn = get_f32(p + pairs), mx = get_f32(p + pairs + 4);
            float span = mx - mn;
            for (uint32_t i = 0; i < pairs; ++i) radii[i] = expf(mn + span * ((float)p[i] / 255.0f));
            p += pairs + 8;
        } else {
            for (uint32_t i = 0; i < pairs; ++i) radii[i] = get_f32(p + 4 * i);
            p += 4 * pairs;
        }
        for (uint32_t i = 0; i < pairs; ++i) idx[i] = (uint16_t)read_bits(p, (size_t)i * pbits, pbits);
        polar_decode(dim, signs, radii, idx, pbits, out + v * dim);
    }
    return ORA_OK;
}

/* ======================================================================
 * 7. fib-quant codec (fib_k4_n32): FibQuantizer::encode_batch / encode,
 *    finish_batch_encode, decode_batch_fast, FB2 (fib-quant/src/codec.rs).
 * ====================================================================== */

/* half 2.7.1 f16::from_f32: IEEE binary16, round to nearest even. */
uint16_t ora_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xff) {
        if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int e = (int)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;          /* 24-bit significand -> subnormal field */
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t q = m >> shift;
        if (rem > half || (rem == half && (q & 1u))) q += 1;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1;  /* may carry into inf: correct */
    return (uint16_t)(sign | q);
}

float ora_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t out;
    if (e == 0) {
        if (m == 0) out = sign;
        else {
            int sh = 0;
            while (!(m & 0x400u)) { m <<= 1; ++sh; }
            m &= 0x3ffu;
            out = sign | ((uint32_t)(127 - 15 + 1 - sh) << 23) | (m << 13);
        }
    } else if (e == 0x1f) {
        out = sign | 0x7f800000u | (m << 13);
    } else {
        out = sign | ((e - 15 + 127) << 23) | (m << 13);
    }
    float f; memcpy(&f, &out, 4); return f;
}

/* gpu-backend/src/simd_nearest.rs:44-104: AVX2 k=4 argmin,
 * dist = (d0^2 + d1^2) + (d2^2 + d3^2) with d = cw - s, strict <, lowest
 * index wins ties.  The GPU box host is x86-64 with AVX2+FMA, so this is the
 * order the reference takes there. */
int ora_nearest_codeword_k4(const float* s, const float* cb, int n) {
    int best = 0;
    float bd = INFINITY;
    int i = 0;
    for (; i + 2 <= n; i += 2) {
        for (int h = 0; h < 2; ++h) {
            const float* c = cb + (size_t)(i + h) * 4;
            float e0 = c[0] - s[0], e1 = c[1] - s[1], e2 = c[2] - s[2], e3 = c[3] - s[3];
            float q0 = e0 * e0, q1 = e1 * e1, q2 = e2 * e2, q3 = e3 * e3;
            float dd = (q0 + q1) + (q2 + q3);
            if (dd < bd) { bd = dd; best = i + h; }
        }
    }
    if (i < n) {   /* odd tail: scalar sequential order (simd_nearest.rs:79-89) */
        float dist = 0.0f;
        for (int j = 0; j < 4; ++j) { float dl = s[j] - cb[(size_t)i * 4 + j]; dist += dl * dl; }
        if (dist < bd) best = i;
    }
    return best;
}

/* simd_nearest.rs:24-38 scalar oracle (any k). */
int ora_nearest_codeword_scalar(const float* s, const float* cb, int k, int n) {
    int best = 0;
    float bd = INFINITY;
    for (int w = 0; w < n; ++w) {
        float dist = 0.0f;
        for (int j = 0; j < k; ++j) { float dl = s[j] - cb[(size_t)w * k + j]; dist += dl * dl; }
        if (dist < bd) { bd = dist; best = w; }
    }
    return best;
}

/* nearest_codeword_f32_avx2_k4 (simd_nearest.rs:44-92) with the same vector
 * instructions: two codewords per _mm256_sub_ps / _mm256_mul_ps against the
 * broadcast sample, each half summed by two _mm_hadd_ps, i.e. (q0 + q1) +
 * (q2 + q3); strict < in codeword order; scalar sequential tail.  Results
 * equal ora_nearest_codeword_k4 (the same IEEE operations); this is the CPU
 * baseline's hot loop, as the reference runs it on an AVX2 host. */
#if defined(__x86_64__)
#include <immintrin.h>
__attribute__((target("avx2,fma"))) int ora_nearest_codeword_k4_avx2(const float* s, const float* cb, int n) {
    const __m256 sv = _mm256_setr_ps(s[0], s[1], s[2], s[3], s[0], s[1], s[2], s[3]);
    int best = 0, i = 0;
    float bd = INFINITY;
    for (; i + 2 <= n; i += 2) {
        const __m256 cw = _mm256_loadu_ps(cb + (size_t)i * 4);
        const __m256 dl = _mm256_sub_ps(cw, sv);
        const __m256 sq = _mm256_mul_ps(dl, dl);
        __m128 lo = _mm256_castps256_ps128(sq), hi = _mm256_extractf128_ps(sq, 1);
        lo = _mm_hadd_ps(lo, lo);
        hi = _mm_hadd_ps(hi, hi);
        const float d0 = _mm_cvtss_f32(_mm_hadd_ps(lo, lo)), d1 = _mm_cvtss_f32(_mm_hadd_ps(hi, hi));
        if (d0 < bd) { bd = d0; best = i; }
        if (d1 < bd) { bd = d1; best = i + 1; }
    }
    if (i < n) {
        float dist = 0.0f;
        for (int j = 0; j < 4; ++j) { float dl = s[j] - cb[(size_t)i * 4 + j]; dist += dl * dl; }
        if (dist < bd) best = i;
    }
    return best;
}
static int have_avx2(void) {
    static int cached = -1;   /* benign race: every thread stores the same value */
    if (cached < 0) cached = __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
    return cached;
}
#else
int ora_nearest_codeword_k4_avx2(const float* s, const float* cb, int n) { return ora_nearest_codeword_k4(s, cb, n); }
static int have_avx2(void) { return 0; }
#endif

/* nearest_codeword_f32 (simd_nearest.rs:13-21) on an AVX2 + FMA host: the
 * AVX2 routine for k = 4 (its pairwise order also without AVX2 here, through
 * the scalar restatement, so results never depend on the host running the
 * oracle).  The reference itself, on a host without AVX2, would take the
 * sequential sum of nearest_codeword_f32_scalar (simd_nearest.rs:24-38);
 * this build, like the reference on every AVX2 server, uses the pairwise one. */
static int nearest_dispatch(const float* s, const float* cb, int k, int n) {
    if (k == 4) return have_avx2() ? ora_nearest_codeword_k4_avx2(s, cb, n) : ora_nearest_codeword_k4(s, cb, n);
    return ora_nearest_codeword_scalar(s, cb, k, n);
}

/* l2_norm (codec.rs:1049-1057) */
static double l2_norm_f64(const float* x, int d) {
    double s = 0.0;
    for (int i = 0; i < d; ++i) { double v = (double)x[i]; s += v * v; }
    return sqrt(s);
}

/* encode_norm Fp16Paper (codec.rs:994-1020): f64 -> f32 -> f16 RNE. */
static int encode_norm16(double nrm, uint16_t* out) {
    if (!isfinite(nrm) || nrm <= 0.0) return ORA_ERR_NORM_UNREPRESENTABLE;
    uint16_t h = ora_f32_to_f16((float)nrm);
    if ((h & 0x7c00u) == 0x7c00u || (h & 0x7fffu) == 0 || (h & 0x8000u)) return ORA_ERR_NORM_UNREPRESENTABLE;
    *out = h;
    return ORA_OK;
}

static uint32_t fib_wire_bits(int n) {
    uint32_t bits = 0;
    uint32_t v = (uint32_t)(n - 1);
    while (v) { bits++; v >>= 1; }
    return bits;
}

/* Payloads [f16 norm][16 x 5-bit indices] of n vectors (plen bytes each).
 * per_vector = 0: FibQuantizer::encode_batch (codec.rs:578-668): a validation
 * pass over the whole batch first (592-610), x^ = f32(x / |x|) (608).
 * per_vector = 1: FibQuantizer::encode on each vector (codec.rs:471-516):
 * checks vector by vector, x^ = x / |x| kept in f64 (481-483).
 * Both: rho = f32(Pi x^) row by row in f64 (rotation.rs:104-115), norm f64 ->
 * f32 -> f16 (994-1020), AVX2 argmin per k-block, indices LSB-first. */
static int fib_encode_payloads(uint32_t d, uint32_t k, uint32_t N, const float* cb, const double* rot,
                               const float* x, uint64_t n, int per_vector, uint8_t* pay, uint32_t plen,
                               uint64_t* fail_index) {
    uint32_t bits = fib_wire_bits((int)N);
    uint32_t blocks = d / k;
    double xn[256], yr[256];
    float xh[256], rho[256];
    if (!per_vector) {
        for (uint64_t v = 0; v < n; ++v) {
            const float* xv = x + v * d;
            for (uint32_t i = 0; i < d; ++i)
                if (!isfinite(xv[i])) { if (fail_index) *fail_index = v; return ORA_ERR_NONFINITE_INPUT; }
            if (l2_norm_f64(xv, (int)d) == 0.0) { if (fail_index) *fail_index = v; return ORA_ERR_ZERO_NORM; }
        }
    }
    for (uint64_t v = 0; v < n; ++v) {
        const float* xv = x + v * d;
        double nrm;
        if (per_vector) {
            for (uint32_t i = 0; i < d; ++i)
                if (!isfinite(xv[i])) { if (fail_index) *fail_index = v; return ORA_ERR_NONFINITE_INPUT; }
            nrm = l2_norm_f64(xv, (int)d);
            if (nrm == 0.0) { if (fail_index) *fail_index = v; return ORA_ERR_ZERO_NORM; }
            for (uint32_t i = 0; i < d; ++i) xn[i] = (double)xv[i] / nrm;          /* codec.rs:481 */
        } else {
            nrm = l2_norm_f64(xv, (int)d);
            for (uint32_t i = 0; i < d; ++i) { xh[i] = (float)((double)xv[i] / nrm); xn[i] = (double)xh[i]; }
        }
        rot_apply_f64((int)d, rot, xn, yr);
        for (uint32_t i = 0; i < d; ++i) rho[i] = (float)yr[i];
        uint16_t h;
        int rc = encode_norm16(nrm, &h);
        if (rc != ORA_OK) { if (fail_index) *fail_index = v; return rc; }
        uint8_t* p = pay + v * plen;
        memset(p, 0, plen);
        put_u16(p, h);
        for (uint32_t b = 0; b < blocks; ++b) {
            int w = nearest_dispatch(rho + (size_t)b * k, cb, (int)k, (int)N);
            write_bits(p + 2, (size_t)b * bits, (int)bits, (uint32_t)w);
        }
    }
    return ORA_OK;
}

/* FibQuantAdapter::encode_batch_compact (proveKV/src/codec.rs:513-525) =
 * FibQuantizer::encode_batch (codec.rs:578-668; n < 4 takes encode,
 * codec.rs:471-516) + finish_batch_encode (670-729) + FibCodeV1::encode_batch
 * FB2 (225-320).  cb: N*k f32 row-major; rot: d*d f64 row-major. */
int ora_fib_encode_batch(uint32_t d, uint32_t k, uint32_t N, const float* cb, const double* rot,
                         const float* x, uint64_t n, uint8_t* out, uint64_t cap, uint64_t* out_len,
                         uint64_t* fail_index) {
    if (d == 0 || k == 0 || d % k != 0 || d > 256 || N < 2) return ORA_ERR_INVALID_ARG;
    uint32_t bits = fib_wire_bits((int)N);
    uint32_t blocks = d / k;
    uint32_t ilen = (blocks * bits + 7) / 8;
    uint32_t plen = 2 + ilen;
    uint64_t total = 19 + n * (uint64_t)plen;
    if (out_len) *out_len = total;
    if (n == 0) return ORA_ERR_EMPTY;
    if (cap < total) return ORA_ERR_CAPACITY;
    memcpy(out, "FB2", 3);
    out[3] = 1;
    out[4] = (uint8_t)bits;
    out[5] = 0;
    put_u32(out + 6, blocks);
    put_u32(out + 10, (uint32_t)n);
    out[14] = 0;                 /* Fp16Paper */
    put_u16(out + 15, 2);
    put_u16(out + 17, (uint16_t)ilen);
    return fib_encode_payloads(d, k, N, cb, rot, x, n, n < 4, out + 19, plen, fail_index);
}

/* One payload [norm (nlen bytes)][indices (ilen bytes)] -> d floats.
 * f64_path = 0: decode_batch_fast (codec.rs:797-844): gather f32 codewords,
 *   out[col] = (sum_row f32(M)[row][col] * c[row], sequential f32 from 0)
 *   * f32(norm) with StoredRotation::apply_inverse_f32 (rotation.rs:136-149).
 * f64_path = 1: FibQuantizer::decode (codec.rs:506-537): f64 codewords
 *   (codebook.rs:118-131), out[col] = f32((sum_row M[row][col] * c[row],
 *   sequential f64 from 0) * norm_f64) with apply_inverse (rotation.rs:117-128).
 * Checks in the reference's order: index padding (bitpack.rs:47-90), index <
 * N, decode_norm (codec.rs:1022-1047: exactly 2 bytes, finite > 0), finite
 * output (check_finite).  m32: f32(M) row-major. */
static int fib_decode_payload(uint32_t d, uint32_t k, uint32_t N, const float* cb, const double* rot,
                              const float* m32, const uint8_t* p, uint32_t nlen, uint32_t ilen, int f64_path,
                              float* o) {
    uint32_t bits = fib_wire_bits((int)N);
    uint32_t blocks = d / k;
    const uint8_t* ip = p + nlen;
    if (!padding_zero(ip, (size_t)blocks * bits, ilen)) return ORA_ERR_MALFORMED;
    float c[256];
    for (uint32_t b = 0; b < blocks; ++b) {
        uint32_t w = read_bits(ip, (size_t)b * bits, (int)bits);
        if (w >= N) return ORA_ERR_MALFORMED;
        for (uint32_t t = 0; t < k; ++t) c[b * k + t] = cb[(size_t)w * k + t];
    }
    if (nlen != 2) return ORA_ERR_MALFORMED;
    float nv = ora_f16_to_f32(get_u16(p));
    if (!isfinite(nv) || !(nv > 0.0f)) return ORA_ERR_MALFORMED;
    for (uint32_t col = 0; col < d; ++col) {
        if (f64_path) {
            double s = 0.0;
            for (uint32_t row = 0; row < d; ++row) s += rot[(size_t)row * d + col] * (double)c[row];
            o[col] = (float)(s * (double)nv);
        } else {
            float s = 0.0f;
            for (uint32_t row = 0; row < d; ++row) s += m32[(size_t)row * d + col] * c[row];
            o[col] = s * nv;
        }
    }
    for (uint32_t col = 0; col < d; ++col)
        if (!isfinite(o[col])) return ORA_ERR_MALFORMED;
    return ORA_OK;
}

/* FibQuantAdapter::decode_batch_compact (proveKV/src/codec.rs:530-569) =
 * FibCodeV1::decode_batch FB2 (codec.rs:323-424) + decode_batch_fast
 * (797-844) with StoredRotation::apply_inverse_f32 (rotation.rs:136-149). */
int ora_fib_decode_batch(uint32_t d, uint32_t k, uint32_t N, const float* cb, const double* rot,
                         const uint8_t* in, uint64_t len, float* out, uint64_t cap_vectors,
                         uint64_t* n_out, uint64_t* fail_index) {
    if (d == 0 || k == 0 || d % k != 0 || d > 256 || N < 2) return ORA_ERR_INVALID_ARG;
    if (len < 19) return ORA_ERR_MALFORMED;
    if (memcmp(in, "FB2", 3) != 0 || in[3] != 1) return ORA_ERR_MALFORMED;
    uint32_t bits = fib_wire_bits((int)N);
    uint32_t blocks = d / k;
    if (in[4] != bits) return ORA_ERR_MALFORMED;
    if (get_u32(in + 6) != blocks) return ORA_ERR_MALFORMED;
    uint64_t n = get_u32(in + 10);
    if (in[14] > 1) return ORA_ERR_MALFORMED;
    if (in[14] != 0) return ORA_ERR_MALFORMED;       /* profile is Fp16Paper */
    uint32_t nlen = get_u16(in + 15), ilen = get_u16(in + 17);
    uint64_t plen = (uint64_t)nlen + ilen;
    if (len < 19 + n * plen) return ORA_ERR_MALFORMED;   /* trailing bytes allowed */
    if (ilen != (blocks * bits + 7) / 8) return ORA_ERR_MALFORMED;
    if (n_out) *n_out = n;
    if (cap_vectors < n) return ORA_ERR_CAPACITY;
    float* m32 = (float*)malloc(sizeof(float) * d * d);
    if (!m32) return ORA_ERR_CAPACITY;
    for (size_t t = 0; t < (size_t)d * d; ++t) m32[t] = (float)rot[t];
    int rc = ORA_OK;
    for (uint64_t v = 0; v < n && rc == ORA_OK; ++v) {
        rc = fib_decode_payload(d, k, N, cb, rot, m32, in + 19 + v * plen, nlen, ilen, 0, out + v * d);
        if (rc != ORA_OK && fail_index) *fail_index = v;
    }
    free(m32);
    return rc;
}

/* ======================================================================
 * 9. Legacy per-vector formats behind KVecCodec::encode / decode and their
 *    batch forms (proveKV/src/codec.rs:8-66, 339-413, 582-668):
 *    TQW1 (turbo-quant/src/wire.rs:44-256) and compact FB1
 *    (fib-quant/src/codec.rs:81-176).  A batch of records is given as one
 *    byte buffer plus n + 1 offsets (record i = in[off[i] .. off[i+1])).
 *    Parity: header layouts are pinned by the reference's own tests
 *    (turbo-quant/tests/wire_format.rs offsets 9/15/22/38/46,
 *    fib-quant/tests/compact_bytes_roundtrip.rs header literals) and the
 *    payloads by the TQB1/FB2 paths; the f64 fib decode is pinned against an
 *    exact rational evaluation (tests/test_oracle_codecs.py).
 * ====================================================================== */

/* TurboCodeWireV1::encode header (wire.rs:44-90): 46 bytes. */
static void tqw1_header(uint8_t* h, uint32_t dim, int pbits, uint32_t proj, uint64_t seed, int mode,
                        uint32_t plen) {
    memcpy(h, "TQW1", 4);
    put_u16(h + 4, 1);
    put_u16(h + 6, 1);            /* FastHadamard (power-of-two dims) */
    h[8] = 1;                     /* VARIANT_TURBO_CODE */
    h[9] = 0;
    put_u32(h + 10, dim);
    h[14] = (uint8_t)pbits;
    h[15] = h[16] = h[17] = 0;
    put_u32(h + 18, proj);
    put_u64(h + 22, seed);
    put_u32(h + 30, dim / 2);
    put_u32(h + 34, mode ? proj : 0);
    put_u64(h + 38, plen);
}

uint32_t ora_tqw1_record_len(uint32_t dim, uint32_t bits, uint32_t proj, int mode) {
    return 46 + ora_turbo_payload_len(dim, bits, proj, mode, 0);
}

/* TurboQuantAdapter::encode (proveKV/src/codec.rs:339-365) on each vector --
 * KVecCodec::encode_batch is the trait's default loop (codec.rs:28-30).
 * out: n records of ora_tqw1_record_len bytes; TQW1 always carries f32 radii. */
int ora_turbo_encode_tqw1(uint32_t dim, uint32_t bits, uint32_t proj, uint64_t seed, int mode,
                          const float* signs, const float* G, const float* x, uint64_t n, uint8_t* out,
                          uint64_t cap, uint64_t* out_len, uint64_t* fail_index) {
    if (!turbo_check_profile(dim, bits, proj, mode)) return ORA_ERR_INVALID_ARG;
    int pbits = mode ? (int)bits - 1 : (int)bits;
    uint32_t plen = turbo_payload_len(dim, pbits, proj, mode, 0);
    uint64_t rec = 46 + (uint64_t)plen;
    if (out_len) *out_len = n * rec;
    if (cap < n * rec) return ORA_ERR_CAPACITY;
    for (uint64_t v = 0; v < n; ++v) {
        uint8_t* r = out + v * rec;
        int rc = turbo_encode_payload(dim, bits, proj, mode, 0, signs, G, x + v * dim, r + 46);
        if (rc != ORA_OK) { if (fail_index) *fail_index = v; return rc; }
        tqw1_header(r, dim, pbits, proj, seed, mode, plen);
    }
    return ORA_OK;
}

/* TurboCodeWireV1::decode (wire.rs:100-256) + PolarQuantizer::decode
 * (polar.rs:272-278) on each record, as TurboQuantAdapter::decode
 * (proveKV/src/codec.rs:367-405) looped by KVecCodec::decode_batch.  Any
 * rejection returns ORA_ERR_MALFORMED with the record's index. */
int ora_turbo_decode_tqw1(uint32_t dim, uint32_t bits, uint32_t proj, uint64_t seed, int mode,
                          const float* signs, const uint8_t* in, const uint64_t* off, uint64_t n, float* out,
                          uint64_t* fail_index) {
    if (!turbo_check_profile(dim, bits, proj, mode)) return ORA_ERR_INVALID_ARG;
    int pbits = mode ? (int)bits - 1 : (int)bits;
    uint32_t pairs = dim / 2;
    uint32_t plen = turbo_payload_len(dim, pbits, proj, mode, 0);
    uint32_t angle_bytes = (pairs * (uint32_t)pbits + 7) / 8;
    uint32_t sign_bytes = mode ? (proj + 7) / 8 : 0;
    float radii[128];
    uint16_t idx[128];
    for (uint64_t v = 0; v < n; ++v) {
        if (fail_index) *fail_index = v;
        if (off[v + 1] < off[v]) return ORA_ERR_MALFORMED;
        const uint8_t* r = in + off[v];
        uint64_t len = off[v + 1] - off[v];
        if (len < 46) return ORA_ERR_MALFORMED;                         /* cursor reads */
        if (memcmp(r, "TQW1", 4) != 0 || get_u16(r + 4) != 1) return ORA_ERR_MALFORMED;
        if (get_u16(r + 6) != 1 || r[8] != 1 || r[9] != 0) return ORA_ERR_MALFORMED;
        if (get_u32(r + 10) != dim || r[14] != pbits || get_u32(r + 18) != proj) return ORA_ERR_MALFORMED;
        if (r[15] || r[16] || r[17]) return ORA_ERR_MALFORMED;
        if (get_u64(r + 22) != seed) return ORA_ERR_MALFORMED;
        if (get_u32(r + 30) != pairs || get_u32(r + 34) != (mode ? proj : 0)) return ORA_ERR_MALFORMED;
        if (get_u64(r + 38) != plen || len != 46 + (uint64_t)plen) return ORA_ERR_MALFORMED;   /* + finish() */
        const uint8_t* p = r + 46;
        for (uint32_t i = 0; i < pairs; ++i) radii[i] = get_f32(p + 4 * i);
        p += 4 * pairs;
        if (!padding_zero(p, (size_t)pairs * pbits, angle_bytes)) return ORA_ERR_MALFORMED;
        for (uint32_t i = 0; i < pairs; ++i) idx[i] = (uint16_t)read_bits(p, (size_t)i * pbits, pbits);
        p += angle_bytes;
        if (mode && !padding_zero(p, proj, sign_bytes)) return ORA_ERR_MALFORMED;
        for (uint32_t i = 0; i < pairs; ++i)                            /* validate_for */
            if (!isfinite(radii[i]) || radii[i] < 0.0f) return ORA_ERR_MALFORMED;
        polar_decode(dim, signs, radii, idx, pbits, out + v * dim);
    }
    if (fail_index) *fail_index = 0;
    return ORA_OK;
}

uint32_t ora_fb1_record_len(uint32_t d, uint32_t k, uint32_t N) {
    return 11 + 2 + ((d / k) * fib_wire_bits((int)N) + 7) / 8;
}

/* FibQuantAdapter::encode (proveKV/src/codec.rs:582-594; each = 1) or
 * encode_batch (596-610; each = 0, FibQuantizer::encode_batch semantics),
 * then FibCodeV1::to_compact_bytes (fib-quant/src/codec.rs:81-92) per code:
 * "FB1", version 1, wire_index_bits, block_count u32, norm_len u16, norm,
 * indices. */
int ora_fib_encode_fb1(uint32_t d, uint32_t k, uint32_t N, const float* cb, const double* rot, const float* x,
                       uint64_t n, int each, uint8_t* out, uint64_t cap, uint64_t* out_len, uint64_t* fail_index) {
    if (d == 0 || k == 0 || d % k != 0 || d > 256 || N < 2) return ORA_ERR_INVALID_ARG;
    uint32_t bits = fib_wire_bits((int)N);
    uint32_t plen = 2 + ((d / k) * bits + 7) / 8;
    uint64_t rec = 11 + (uint64_t)plen;
    if (out_len) *out_len = n * rec;
    if (cap < n * rec) return ORA_ERR_CAPACITY;
    if (n == 0) return ORA_OK;
    uint8_t* pay = (uint8_t*)malloc(n * plen);
    if (!pay) return ORA_ERR_CAPACITY;
    int rc = fib_encode_payloads(d, k, N, cb, rot, x, n, each || n < 4, pay, plen, fail_index);
    if (rc == ORA_OK) {
        for (uint64_t v = 0; v < n; ++v) {
            uint8_t* r = out + v * rec;
            memcpy(r, "FB1", 3);
            r[3] = 1;
            r[4] = (uint8_t)bits;
            put_u32(r + 5, d / k);
            put_u16(r + 9, 2);
            memcpy(r + 11, pay + v * plen, plen);
        }
    }
    free(pay);
    return rc;
}

/* FibCodeV1::from_compact_bytes (fib-quant/src/codec.rs:100-176): 1 if the
 * record parses; fills the header fields. */
static int fb1_parse(const uint8_t* r, uint64_t len, uint32_t* bits, uint32_t* blocks, uint32_t* nlen) {
    if (len < 11) return 0;
    if (memcmp(r, "FB1", 3) != 0 || r[3] != 1) return 0;
    *bits = r[4];
    *blocks = get_u32(r + 5);
    *nlen = get_u16(r + 9);
    if (len < 11 + (uint64_t)*nlen) return 0;
    uint64_t ilen = len - 11 - *nlen;
    if (ilen != ((uint64_t)*blocks * *bits + 7) / 8) return 0;
    return 1;
}

/* FibQuantAdapter::decode (proveKV/src/codec.rs:612-637; each = 1): per
 * record parse, FibQuantizer::decode (f64 path), first failure wins.
 * FibQuantAdapter::decode_batch (639-665; each = 0): every record parsed
 * first (a parse failure anywhere wins), then decode_batch_fast (f32 path)
 * with validate_code_header (codec.rs:926-975) per code. */
int ora_fib_decode_fb1(uint32_t d, uint32_t k, uint32_t N, const float* cb, const double* rot,
                       const uint8_t* in, const uint64_t* off, uint64_t n, int each, float* out,
                       uint64_t* fail_index) {
    if (d == 0 || k == 0 || d % k != 0 || d > 256 || N < 2) return ORA_ERR_INVALID_ARG;
    uint32_t bits_p = fib_wire_bits((int)N);
    uint32_t blocks_p = d / k;
    uint32_t bits, blocks, nlen;
    if (!each) {
        for (uint64_t v = 0; v < n; ++v) {
            if (off[v + 1] < off[v] || !fb1_parse(in + off[v], off[v + 1] - off[v], &bits, &blocks, &nlen)) {
                if (fail_index) *fail_index = v;
                return ORA_ERR_MALFORMED;
            }
        }
    }
    float* m32 = (float*)malloc(sizeof(float) * d * d);
    if (!m32) return ORA_ERR_CAPACITY;
    for (size_t t = 0; t < (size_t)d * d; ++t) m32[t] = (float)rot[t];
    int rc = ORA_OK;
    for (uint64_t v = 0; v < n && rc == ORA_OK; ++v) {
        const uint8_t* r = in + off[v];
        if (off[v + 1] < off[v] || !fb1_parse(r, off[v + 1] - off[v], &bits, &blocks, &nlen))
            rc = ORA_ERR_MALFORMED;
        else if (bits != bits_p || blocks != blocks_p)                         /* validate_code_header */
            rc = ORA_ERR_MALFORMED;
        else if (fib_decode_payload(d, k, N, cb, rot, m32, r + 11, nlen, (blocks * bits + 7) / 8, each,
                                    out + v * d) != ORA_OK)
            rc = ORA_ERR_MALFORMED;
        if (rc != ORA_OK && fail_index) *fail_index = v;
    }
    free(m32);
    return rc;
}

/* ======================================================================
 * 10. Scoring on compressed codes: TurboQuantizer::prepare_query and
 *     inner_product_estimate_prepared (turbo-quant/src/turbo.rs:316-381),
 *     PolarQuantizer::project_query / inner_product_estimate_with_projected_query
 *     (polar.rs:330-370), QjlQuantizer::project_query /
 *     inner_product_estimate_with_projected_query(_and_source_norm)
 *     (qjl.rs:265-330).  Parity: pinned by the estimator's own identities
 *     (tests/test_oracle_score.py): unbiasedness against the exact inner
 *     product, the l2 identity, and exact reconstruction cases.
 * ====================================================================== */

/* prepared = [R q (dim)][G q (proj, QJL only)]; R q is the forward
 * FastHadamard rotation (sign, FWHT, scale), G q sequential f32 dots. */
int ora_turbo_prepare_query(uint32_t dim, uint32_t proj, int mode, const float* signs, const float* G,
                            const float* q, float* out) {
    for (uint32_t c = 0; c < dim; ++c)
        if (!isfinite(q[c])) return ORA_ERR_NONFINITE_INPUT;           /* prepare_query, turbo.rs:330 */
    ora_turbo_rotate(dim, signs, q, out);
    for (uint32_t c = 0; c < dim; ++c)
        if (!isfinite(out[c])) return ORA_ERR_NONFINITE_INPUT;         /* polar.rs:341 */
    if (mode) {
        for (uint32_t j = 0; j < proj; ++j) {
            float s = -0.0f;   /* Rust's f32 Sum folds from -0.0 */
            for (uint32_t c = 0; c < dim; ++c) s += G[(size_t)j * dim + c] * q[c];
            out[dim + j] = s;
            if (!isfinite(s)) return ORA_ERR_NONFINITE_INPUT;          /* qjl.rs:279 */
        }
    }
    return ORA_OK;
}

/* Scores of every code of a TQB1 blob against nq prepared queries:
 * scores[q * n + i] = polar(i, q) + qjl(i, q), with
 *   polar = sum_pairs r * (qa * cos(theta) + qb * sin(theta))   (sequential f32)
 *   qjl   = (sqrt(PI / 2) * 1 / m) * sum_j sign_j * (G q)_j       (unit source norm)
 * The blob is validated as decode_batch does (wire.rs:401-568) before any
 * score; a non-finite polar / qjl / total score fails (polar.rs:362-366,
 * qjl.rs:322-327, turbo.rs:362-367).  fail_index: the lowest failing code. */
int ora_turbo_score(uint32_t dim, uint32_t bits, uint32_t proj, uint64_t seed, int mode, const float* signs,
                    const uint8_t* in, uint64_t len, const float* prepared, uint32_t nq, float* scores,
                    uint64_t* n_out, uint64_t* fail_index) {
    uint64_t n = 0;
    /* the batch decoder's header and payload validation, nothing decoded */
    int rc = ora_turbo_decode_batch(dim, bits, proj, seed, mode, signs, in, len, NULL, UINT64_MAX, &n, fail_index);
    if (rc != ORA_OK) return rc;
    if (n_out) *n_out = n;
    if (n == 0) return ORA_OK;
    int pbits = mode ? (int)bits - 1 : (int)bits;
    uint32_t pairs = dim / 2;
    int rcodec = in[15];
    uint32_t plen = turbo_payload_len(dim, pbits, proj, mode, rcodec);
    uint32_t angle_bytes = (pairs * (uint32_t)pbits + 7) / 8;
    const float scale = sqrtf(3.14159274101257324f / 2.0f) * 1.0f / (float)proj;
    float radii[128];
    uint16_t idx[128];
    uint64_t first_bad = UINT64_MAX;
    for (uint64_t v = 0; v < n; ++v) {
        const uint8_t* p = in + 38 + v * plen;
        if (rcodec) {
            float mn = get_f32(p + pairs), mx = get_f32(p + pairs + 4);
            float span = mx - mn;
            for (uint32_t i = 0; i < pairs; ++i) radii[i] = expf(mn + span * ((float)p[i] / 255.0f));
            p += pairs + 8;
        } else {
            for (uint32_t i = 0; i < pairs; ++i) radii[i] = get_f32(p + 4 * i);
            p += 4 * pairs;
        }
        for (uint32_t i = 0; i < pairs; ++i) idx[i] = (uint16_t)read_bits(p, (size_t)i * pbits, pbits);
        p += angle_bytes;
        for (uint32_t qi = 0; qi < nq; ++qi) {
            const float* pq = prepared + (size_t)qi * (dim + (mode ? proj : 0));
            float est = 0.0f;
            for (uint32_t i = 0; i < pairs; ++i) {
                float th = dequant_angle(idx[i], pbits);
                est += radii[i] * (pq[2 * i] * cosf(th) + pq[2 * i + 1] * sinf(th));
            }
            int bad = !isfinite(est);
            float total = est;
            if (mode) {
                float e2 = -0.0f;
                for (uint32_t j = 0; j < proj; ++j) {
                    int bit = (p[j >> 3] >> (j & 7)) & 1;
                    e2 += (bit ? 1.0f : -1.0f) * pq[dim + j];
                }
                float qj = scale * e2;
                bad |= !isfinite(qj);
                total = est + qj;
            }
            bad |= !isfinite(total);
            scores[(size_t)qi * n + v] = total;
            if (bad && v < first_bad) first_bad = v;
        }
    }
    if (first_bad != UINT64_MAX) {
        if (fail_index) *fail_index = first_bad;
        return ORA_ERR_MALFORMED;
    }
    return ORA_OK;
}

/* ======================================================================
 * 8. Exported helpers used by the tests (pins of the RNG chain).
 * ====================================================================== */
void ora_chacha_words(const uint32_t* key8, int rounds, uint64_t skip_words, uint32_t* out, uint64_t n) {
    ora_rng r;
    rng_from_key(&r, key8, rounds);
    for (uint64_t i = 0; i < skip_words; ++i) (void)rng_u32(&r);
    for (uint64_t i = 0; i < n; ++i) out[i] = rng_u32(&r);
}

void ora_seed_key(uint64_t seed, uint32_t* key8) {
    ora_rng r;
    rng_seed_from_u64(&r, seed);
    memcpy(key8, r.key, 32);
}

void ora_rng_u64(uint64_t seed, uint64_t* out, uint64_t n) {
    ora_rng r;
    rng_seed_from_u64(&r, seed);
    for (uint64_t i = 0; i < n; ++i) out[i] = rng_u64(&r);
}

void ora_normal_f64(uint64_t seed, double* out, uint64_t n) {
    ora_rng r;
    rng_seed_from_u64(&r, seed);
    for (uint64_t i = 0; i < n; ++i) out[i] = rng_normal(&r);
}

void ora_gamma_f64(uint64_t seed, double shape, double* out, uint64_t n) {
    ora_rng r;
    ora_gamma g;
    rng_seed_from_u64(&r, seed);
    gamma_init(&g, shape, 1.0);
    for (uint64_t i = 0; i < n; ++i) out[i] = rng_gamma(&r, &g);
}

/* Test hook: n draws of one of the conversions above from rand_pcg's
 * Pcg32::new(state, stream) (the generator of rand's and rand_distr's
 * value-stability tests); out[i] holds the u32 / u64 / bool as an integer, or
 * the bits of the f64.  what: 0 next_u32, 1 next_u64, 2 Standard<bool>,
 * 3 Standard<f64>, 4 Open01<f64>, 5 StandardNormal<f64>, 6 Gamma(p0, p1). */
int ora_pcg_draws(uint64_t state, uint64_t stream, int what, double p0, double p1, uint64_t* out, uint64_t n) {
    ora_rng r;
    ora_gamma g;
    rng_pcg32(&r, state, stream);
    if (what == 6) {
        if (!(p0 > 1.0) || !(p1 > 0.0)) return ORA_ERR_INVALID_ARG;   /* the large-shape branch only */
        gamma_init(&g, p0, p1);
    }
    for (uint64_t i = 0; i < n; ++i) {
        double v = 0.0;
        switch (what) {
        case 0: out[i] = rng_u32(&r); continue;
        case 1: out[i] = rng_u64(&r); continue;
        case 2: out[i] = (uint64_t)rng_bool(&r); continue;
        case 3: v = rng_f64(&r); break;
        case 4: v = rng_open01(&r); break;
        case 5: v = rng_normal(&r); break;
        case 6: v = rng_gamma(&r, &g); break;
        default: return ORA_ERR_INVALID_ARG;
        }
        memcpy(&out[i], &v, 8);
    }
    return ORA_OK;
}

void ora_zig_tables(double* x257, double* f257, double* r) {
    zig_init();
    memcpy(x257, ZX, sizeof ZX);
    memcpy(f257, ZF, sizeof ZF);
    *r = ZIG_R;
}

int ora_stored_rotation(uint32_t d, uint64_t seed, double* out_rowmajor, double* gaussian_colmajor) {
    if (gaussian_colmajor) {
        ora_rng r;
        rng_seed_from_u64(&r, seed);
        for (size_t t = 0; t < (size_t)d * d; ++t) gaussian_colmajor[t] = rng_normal(&r);
    }
    return stored_rotation((int)d, seed, out_rowmajor);
}

int ora_fib_codebook(uint32_t d, uint32_t k, uint32_t n, uint64_t seed, uint32_t training,
                     uint32_t restarts, uint32_t iterations, float* out, double* init_mse,
                     double* train_mse) {
    return fib_codebook((int)d, (int)k, (int)n, seed, (int)training, (int)restarts, (int)iterations, out,
                        init_mse, train_mse, NULL, NULL);
}

/* The codebook build with its LloydReportV1 (lloyd.rs:165-176): best
 * restart, repair count and up to `cap` event rows (7 doubles each); returns
 * the event count through *n_events. */
int ora_fib_codebook_report(uint32_t d, uint32_t k, uint32_t n, uint64_t seed, uint32_t training,
                            uint32_t restarts, uint32_t iterations, float* out, double* init_mse,
                            double* train_mse, uint32_t* best_restart, double* events, uint32_t cap,
                            uint32_t* n_events) {
    ora_events ev = {NULL, 0, 0, 0, 0};
    int rc = fib_codebook((int)d, (int)k, (int)n, seed, (int)training, (int)restarts, (int)iterations, out,
                          init_mse, train_mse, best_restart, &ev);
    *n_events = (uint32_t)ev.n;
    for (int i = 0; i < ev.n && (uint32_t)i < cap; ++i) memcpy(events + 7 * (size_t)i, ev.rows + 7 * (size_t)i, 56);
    free(ev.rows);
    return rc;
}

double ora_inv_norm_cdf(double p) { return inv_norm_cdf(p); }
double ora_beta_inv(double q, double a, double b) { return beta_inv(q, a, b); }
double ora_radius_quantile(uint32_t d, uint32_t k, uint32_t idx, uint32_t n) {
    return radius_quantile((int)d, (int)k, (int)idx, (int)n);
}
int ora_roberts_kronecker(uint32_t k, uint32_t n, double* out) { return roberts_kronecker((int)k, (int)n, out); }

/* bitpack round trip used by the literal pins (turbo bitpack.rs:21-47,
 * fib bitpack.rs:4-90, gpu-backend fallback.rs:389-397). */
void ora_pack_bits(const uint32_t* values, uint64_t n, int bits, uint8_t* out) {
    memset(out, 0, (n * (uint64_t)bits + 7) / 8);
    for (uint64_t i = 0; i < n; ++i) write_bits(out, i * (uint64_t)bits, bits, values[i]);
}
int ora_unpack_bits(const uint8_t* in, uint64_t n, int bits, uint32_t* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = read_bits(in, i * (uint64_t)bits, bits);
    return padding_zero(in, n * (uint64_t)bits, (n * (uint64_t)bits + 7) / 8) ? ORA_OK : ORA_ERR_MALFORMED;
}

void ora_track_reset(int on) { g_track = on; g_margin = INFINITY; g_tail_n = 0; memset(g_cnt, 0, sizeof g_cnt); }
void ora_track_counts(uint64_t out[7]) { memcpy(out, g_cnt, sizeof g_cnt); }
double ora_track_margin(void) { return g_margin; }
uint64_t ora_track_tail_logs(double* args, double* vals, uint64_t cap) {
    const uint64_t n = g_tail_n < ORA_TAIL_LOGS ? g_tail_n : ORA_TAIL_LOGS;
    for (uint64_t i = 0; i < n && i < cap; ++i) { args[i] = g_tail_arg[i]; vals[i] = g_tail_val[i]; }
    return g_tail_n;
}
void ora_set_codebook_perturbation(double rel) { g_perturb = rel; }

/* Host glibc logf of the n floats whose bit patterns are u0, u0 + 1, ...
 * (test hook: exhaustive comparisons against the product's restatement). */
void ora_logf_bits(uint32_t u0, uint64_t n, float* out) {
    for (uint64_t i = 0; i < n; ++i) {
        const uint32_t u = u0 + (uint32_t)i;
        float x;
        memcpy(&x, &u, 4);
        out[i] = logf(x);
    }
}
