// pkv_math.h -- bit-exact scalar math shared by the gfx950 kernels and the
// host side of libpkv_hip.so.
//
// The reference codecs take atan2f / logf / expf from the host glibc
// (Rust's f32 methods lower to libm on linux-gnu; turbo-quant/src/polar.rs:415,
// radius.rs:61,143).  To make TQB1 angle bins and BlockLogU8 bytes identical
// on the GPU, this header restates the published algorithms glibc 2.35 uses
// for those functions, operation by operation:
//   * atan2f / atanf: the fdlibm single-precision routines (Sun Microsystems
//     1993, freely redistributable), float arithmetic, no contraction;
//   * logf / expf: the table-driven double-precision evaluations of Arm's
//     optimized-routines (MIT / Apache-2.0), which glibc adopted in 2.28.
// The restatements were checked against the host libm (logf on every positive
// float, expf on every finite float with 2 disagreements at |x| > 32, atan2f on
// 3e8 random pairs); tests/test_host_side.py re-runs sampled versions of those
// checks through pkv_host_* exports.
//
// Everything here must be compiled with -ffp-contract=off.
#pragma once
#include <stdint.h>

#if defined(__HIP__) || defined(__HIPCC__)
#define PKV_HD __host__ __device__ inline __attribute__((always_inline))
#else
#define PKV_HD static inline
#endif

namespace pkv {

PKV_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
PKV_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
PKV_HD uint64_t d2u(double d) { return __builtin_bit_cast(uint64_t, d); }
PKV_HD double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }
PKV_HD float fabs_f(float x) { return u2f(f2u(x) & 0x7fffffffu); }
PKV_HD bool isfinite_f(float x) { return (f2u(x) & 0x7f800000u) != 0x7f800000u; }

// f32_rounding_stable(v, |v| 2^-50), read off v's bits, for 2^-126 <= |v| <
// 2^127: the f32 rounding boundaries inside v's binade [2^e, 2^(e+1)) are the
// values whose low 29 f64 mantissa bits are 2^28 (the one below the binade
// lies 2^(e-25) away), and |v| 2^-50 < 8 ulp64(v), so a distance of more
// than 8 ulp64 from the nearest such value leaves every value within |v|
// 2^-50 rounding like v.  False below 2^-126 (zero included): the caller then
// takes its exact path.
PKV_HD bool f32_rounding_stable_rel50(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(b), hi = static_cast<uint32_t>(b >> 32) & 0x7fffffffu;
    return hi >= 0x38100000u && (lo & 0x1fffffffu) - 0x10000000u + 8u > 16u;
}

// ---------------------------------------------------------------- atan2f
// fdlibm s_atanf.c / e_atan2f.c (single precision).
PKV_HD float fd_atanf(float x) {
    const float atanhi[4] = {4.6364760399e-01f, 7.8539812565e-01f, 9.8279368877e-01f, 1.5707962513e+00f};
    const float atanlo[4] = {5.0121582440e-09f, 3.7748947079e-08f, 3.4473217170e-08f, 7.5497894159e-08f};
    const float aT0 = 3.3333334327e-01f, aT1 = -2.0000000298e-01f, aT2 = 1.4285714924e-01f,
                aT3 = -1.1111110449e-01f, aT4 = 9.0908870101e-02f, aT5 = -7.6918758452e-02f,
                aT6 = 6.6610731184e-02f, aT7 = -5.8335702866e-02f, aT8 = 4.9768779427e-02f,
                aT9 = -3.6531571299e-02f, aT10 = 1.6285819933e-02f;
    int32_t hx = (int32_t)f2u(x);
    int32_t ix = hx & 0x7fffffff;
    int id;
    if (ix >= 0x4c000000) {
        if (ix > 0x7f800000) return x + x;
        return hx > 0 ? atanhi[3] + atanlo[3] : -atanhi[3] - atanlo[3];
    }
    if (ix < 0x3ee00000) {
        if (ix < 0x31000000) return x;
        id = -1;
    } else {
        x = fabs_f(x);
        if (ix < 0x3f980000) {
            if (ix < 0x3f300000) { id = 0; x = (2.0f * x - 1.0f) / (2.0f + x); }
            else { id = 1; x = (x - 1.0f) / (x + 1.0f); }
        } else {
            if (ix < 0x401c0000) { id = 2; x = (x - 1.5f) / (1.0f + 1.5f * x); }
            else { id = 3; x = -1.0f / x; }
        }
    }
    float z = x * x;
    float w = z * z;
    float s1 = z * (aT0 + w * (aT2 + w * (aT4 + w * (aT6 + w * (aT8 + w * aT10)))));
    float s2 = w * (aT1 + w * (aT3 + w * (aT5 + w * (aT7 + w * aT9))));
    if (id < 0) return x - x * (s1 + s2);
    float hi = id == 0 ? atanhi[0] : id == 1 ? atanhi[1] : id == 2 ? atanhi[2] : atanhi[3];
    float lo = id == 0 ? atanlo[0] : id == 1 ? atanlo[1] : id == 2 ? atanlo[2] : atanlo[3];
    z = hi - ((x * (s1 + s2) - lo) - x);
    return hx < 0 ? -z : z;
}

PKV_HD float fd_atan2f(float y, float x) {
    const float pi_o_4 = 7.8539818525e-01f, pi_o_2 = 1.5707963705e+00f, pi = 3.1415927410e+00f,
                pi_lo = -8.7422776573e-08f;
    int32_t hx = (int32_t)f2u(x), hy = (int32_t)f2u(y);
    int32_t ix = hx & 0x7fffffff, iy = hy & 0x7fffffff;
    if (ix > 0x7f800000 || iy > 0x7f800000) return x + y;
    if (hx == 0x3f800000) return fd_atanf(y);
    int m = ((hy >> 31) & 1) | ((hx >> 30) & 2);
    if (iy == 0) {
        if (m <= 1) return y;
        return m == 2 ? pi : -pi;
    }
    if (ix == 0) return hy < 0 ? -pi_o_2 : pi_o_2;
    if (ix == 0x7f800000) {
        if (iy == 0x7f800000) {
            if (m == 0) return pi_o_4;
            if (m == 1) return -pi_o_4;
            if (m == 2) return 3.0f * pi_o_4;
            return -3.0f * pi_o_4;
        }
        if (m == 0) return 0.0f;
        if (m == 1) return -0.0f;
        return m == 2 ? pi : -pi;
    }
    if (iy == 0x7f800000) return hy < 0 ? -pi_o_2 : pi_o_2;
    int32_t k = (iy - ix) >> 23;
    float z;
    if (k > 26) z = pi_o_2 + 0.5f * pi_lo;
    else if (hx < 0 && k < -26) z = 0.0f;
    else z = fd_atanf(fabs_f(y / x));
    if (m == 0) return z;
    if (m == 1) return u2f(f2u(z) ^ 0x80000000u);
    if (m == 2) return pi - (z - pi_lo);
    return (z - pi_lo) - pi;
}

// ---------------------------------------------------------------- turbo angle bin
// encode_pair (turbo-quant/src/polar.rs:413-421): index of the angle of (a, b).
PKV_HD uint32_t angle_bin_exact(float a, float b, uint32_t pbits) {
    const float PI = 3.14159265358979323846f;
    float theta = fd_atan2f(b, a);
    uint32_t levels = 1u << pbits;
    float normalized = (theta + PI) / (2.0f * PI);
    float f = __builtin_floorf(normalized * (float)levels);
    uint32_t u = (f > 0.0f) ? (uint32_t)f : 0u;   // `as u32` saturates; f <= levels here
    return u & (levels - 1u);
}

// Fast exact bin for pbits == 3 (8 octants).  The bin thresholds sit within
// ~1.2e-6 rad of the octant lines once the rounding of (theta + PI) / (2 PI)
// and the <= 2 ulp error of the libm atan2f are counted.  When (a, b) is at
// least 2^-16 (relative) away from every octant boundary line (b = 0, a = 0,
// |a| = |b|) the angle is >= 7.6e-6 rad from the lines, so the octant decides
// the bin; otherwise (about 4e-5 of random pairs) the full formula runs.
PKV_HD uint32_t octant_bin(float a, float b, bool& safe) {
    float aa = fabs_f(a), ab = fabs_f(b);
    float mx = aa > ab ? aa : ab;
    float mn = aa > ab ? ab : aa;
    float eps = mx * 1.52587890625e-05f;   // 2^-16, exact scaling
    float gap = fabs_f(aa - ab);
    safe = (mn > eps) && (gap > eps) && (mx > 1.0e-30f) && (mx < 1.0e30f);
    bool bpos = b > 0.0f, apos = a > 0.0f, bsmall = ab < aa;
    uint32_t bin;
    if (bpos) bin = apos ? (bsmall ? 4u : 5u) : (bsmall ? 7u : 6u);
    else bin = apos ? (bsmall ? 3u : 2u) : (bsmall ? 0u : 1u);
    return bin;
}

// octant_bin in integer arithmetic on the bit patterns (no compare masks):
// for finite floats, |x| orders like its bit pattern with the sign cleared,
// and a difference of two such patterns is negative exactly when the first is
// smaller.  The bin of (bpos, apos, bsmall) comes from an 8-entry table of
// 3-bit fields.  Agrees with octant_bin on every input (NaN included: both
// mark it unsafe).
PKV_HD uint32_t octant_bin_u(float a, float b, uint32_t& safe) {
    uint32_t xa, xb;
    __builtin_memcpy(&xa, &a, 4);
    __builtin_memcpy(&xb, &b, 4);
    const uint32_t ua = xa & 0x7fffffffu, ub = xb & 0x7fffffffu;
    const uint32_t bsmall = (ub - ua) >> 31;                       // |b| < |a|
    const uint32_t apos = ((0u - xa) & ~xa) >> 31;                 // a > 0
    const uint32_t bpos = ((0u - xb) & ~xb) >> 31;                 // b > 0
    const uint32_t idx = (bpos << 2) | (apos << 1) | bsmall;
    // idx: 0 -> 1, 1 -> 0, 2 -> 2, 3 -> 3, 4 -> 6, 5 -> 7, 6 -> 5, 7 -> 4
    const uint32_t lut = 1u | 0u << 3 | 2u << 6 | 3u << 9 | 6u << 12 | 7u << 15 | 5u << 18 | 4u << 21;
    const uint32_t bin = (lut >> (3u * idx)) & 7u;
    const uint32_t mx = ua > ub ? ua : ub, mn = ua > ub ? ub : ua;
    // eps = mx * 2^-16 (exact while mx > 2^-110; smaller mx is unsafe below)
    const uint32_t eps = mx - (16u << 23);
    float fa, fb;
    __builtin_memcpy(&fa, &ua, 4);
    __builtin_memcpy(&fb, &ub, 4);
    const float g = fa - fb;
    uint32_t ug;
    __builtin_memcpy(&ug, &g, 4);
    ug &= 0x7fffffffu;                                              // |aa - ab|
    const uint32_t lo = 0x0da24260u, hi = 0x7149f2cau;             // 1e-30f, 1e30f
    safe = ((eps - mn) & (eps - ug) & (lo - mx) & (mx - hi)) >> 31;
    return bin;
}

// octant_bin_u for the batched encodes: the bin from three sign bits
// (bit 2: b is not negative; bit 1: sign(a) != sign(b); bit 0: (|b| < |a|)
// == (sign(a) != sign(b)) -- the same table as octant_bin wherever a and b
// are non-zero, which every safe pair is), and the safety test as four
// unsigned compares of the same bit patterns (lane masks on the device, so a
// wave can test them all at once).  safe agrees with octant_bin_u on every
// input; the bin of an unsafe pair is not used.
// The two failing conditions come out separately (near an octant line; |a|,
// |b| outside the range the line test covers) so that a kernel can take each
// lane mask straight from its compare.
PKV_HD uint32_t octant_bin_m2(float a, float b, bool& near_line, bool& out_of_range) {
    uint32_t xa, xb;
    __builtin_memcpy(&xa, &a, 4);
    __builtin_memcpy(&xb, &b, 4);
    const uint32_t ua = xa & 0x7fffffffu, ub = xb & 0x7fffffffu;
    const uint32_t t = xa ^ xb;
    const uint32_t e = ~((ub - ua) ^ t);   // bit 31: (|b| < |a|) xnor (sign(a) xor sign(b))
    const uint32_t bin = ((~xb >> 29) & 4u) | ((t >> 30) & 2u) | (e >> 31);
    const uint32_t mx = ua > ub ? ua : ub, mn = ua > ub ? ub : ua;
    const uint32_t eps = mx - (16u << 23);   // wraps for mx < 2^-110, which fails the range test
    float fa, fb;
    __builtin_memcpy(&fa, &ua, 4);
    __builtin_memcpy(&fb, &ub, 4);
    const float g = fa - fb;
    uint32_t ug;
    __builtin_memcpy(&ug, &g, 4);
    ug &= 0x7fffffffu;
    const uint32_t m3 = mn < ug ? mn : ug;
    near_line = !(eps < m3);
    // 1e-30f < mx < 1e30f as one unsigned compare
    out_of_range = !(mx - 0x0da24261u < 0x7149f2cau - 0x0da24261u);
    return bin;
}

// octant_bin_m2 in float form, for the batched encodes' fast path (five
// instructions for the test on gfx950, |.| being a free source modifier):
// g = |a| - |b|, unsafe = !(max(|a|, |b|, 2^-31) < min(|a|, |b|, |g|) * 2^16).
// A pair it passes is one octant_bin_m2 passes, with the same bin, provided
// fl(fl(a^2) + fl(b^2)) is finite (the kernels send every pair of a vector
// whose radii do not sum to a finite value down the exact path):
//   * m3 * 2^16 is exact (no overflow: m3 <= mx < 2^64 when a^2, b^2 are
//     finite), so m3 > mx 2^-16 = eps of octant_bin_m2 (exact for mx >
//     2^-110), and m3 > 2^-47, so mx > 2^-47 > 1e-30; mx < 2^64 < 1e30;
//   * bin bit 0: the sign of g is set exactly when |a| < |b| (a difference of
//     unequal floats keeps its sign; |a| == |b| fails the test through
//     |g| = 0), so sign(g) xor sign(a) xor sign(b) is octant_bin_m2's
//     ~((ub - ua) ^ t) >> 31.
// The 2^-31 floor also keeps every passed pair's fl(a^2) + fl(b^2) >= 2^-94,
// inside sqrt_normal's domain.
PKV_HD uint32_t octant_bin_f(float a, float b, bool& unsafe) {
    const float fa = __builtin_fabsf(a), fb = __builtin_fabsf(b);
    const float g = fa - fb;
    const float mx = __builtin_fmaxf(__builtin_fmaxf(fa, fb), 0x1p-31f);
    const float m3 = __builtin_fminf(__builtin_fminf(fa, fb), __builtin_fabsf(g));
    unsafe = !(mx < m3 * 65536.0f);
    uint32_t xa, xb, xg;
    __builtin_memcpy(&xa, &a, 4);
    __builtin_memcpy(&xb, &b, 4);
    __builtin_memcpy(&xg, &g, 4);
    const uint32_t t = xa ^ xb, c = xg ^ t;
    return ((~xb >> 29) & 4u) | ((t >> 30) & 2u) | (c >> 31);
}

PKV_HD uint32_t octant_bin_m(float a, float b, bool& safe) {
    bool near_line, out_of_range;
    const uint32_t bin = octant_bin_m2(a, b, near_line, out_of_range);
    safe = !near_line && !out_of_range;
    return bin;
}

PKV_HD uint32_t angle_bin3(float a, float b) {
    bool safe;
    uint32_t bin = octant_bin(a, b, safe);
    return safe ? bin : angle_bin_exact(a, b, 3);
}

// ---------------------------------------------------------------- logf / expf
struct LogfEntry { double invc, logc; };

#define PKV_LOGF_TABLE \
    {0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2}, {0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2}, \
    {0x1.49539f0f010bp+0, -0x1.01eae7f513a67p-2}, {0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3}, \
    {0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3}, {0x1.25e227b0b8eap+0, -0x1.1aa2bc79c81p-3}, \
    {0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4}, {0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4}, \
    {0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5}, {0x1p+0, 0x0p+0}, \
    {0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5}, {0x1.ca4b31f026aap-1, 0x1.c5e53aa362eb4p-4}, \
    {0x1.b2036576afce6p-1, 0x1.526e57720db08p-3}, {0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3}, \
    {0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2}, {0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2}

// logf for x >= FLT_MIN (the only domain the radii codec uses:
// radius.rs:61 clamps to f32::MIN_POSITIVE first).  `tab` is the 16-entry
// table above (in LDS or constant memory on the device).
PKV_HD float og_logf_normal(float x, const LogfEntry* tab) {
    const double Ln2 = 0x1.62e42fefa39efp-1;
    const double A0 = -0x1.00ea348b88334p-2, A1 = 0x1.5575b0be00b6ap-2, A2 = -0x1.ffffef20a4123p-2;
    uint32_t ix = f2u(x);
    if (ix == 0x3f800000u) return 0.0f;
    if (ix >= 0x7f800000u) return x;           // +inf (NaN / negatives never reach here)
    uint32_t tmp = ix - 0x3f330000u;
    int i = (int)((tmp >> 19) & 15u);
    int k = ((int32_t)tmp) >> 23;
    uint32_t iz = ix - (tmp & (0x1ffu << 23));
    double invc = tab[i].invc, logc = tab[i].logc;
    double z = (double)u2f(iz);
    double r = z * invc - 1.0;
    double y0 = logc + (double)k * Ln2;
    double r2 = r * r;
    double y = A1 * r + A2;
    y = A0 * r2 + y;
    y = y * r2 + (y0 + r);
    return (float)y;
}

// tab[i] = bits(RN(2^(i/32))) - (i << 47); the doubles are the correctly
// rounded values of 2^(i/32) (regenerate with any multiprecision library).
#define PKV_EXP2F_TABLE \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull

// expf via the 32-entry 2^(i/32) table.
PKV_HD float og_expf(float x, const uint64_t* tab) {
    const double N = 32.0;
    const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double C0 = 0x1.c6af84b912394p-5 / N / N / N, C1 = 0x1.ebfce50fac4f3p-3 / N / N,
                 C2 = 0x1.62e42ff0c52d6p-1 / N;
    const double SHIFT = 0x1.8p+52;
    uint32_t ux = f2u(x);
    uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {            // |x| >= 88 or NaN / inf
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return u2f(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    double xd = (double)x;
    double z = InvLn2N * xd;
    double kd = z + SHIFT;
    uint64_t ki = d2u(kd);
    kd -= SHIFT;
    double r = z - kd;
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    double s = u2d(t);
    double zz = C0 * r + C1;
    double r2 = r * r;
    double y = C2 * r + 1.0;
    y = zz * r2 + y;
    y = y * s;
    return (float)y;
}

// ---------------------------------------------------------------- fp16
// IEEE binary16 round-to-nearest-even (the `half` crate's f16::from_f32).
PKV_HD uint16_t f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | (man ? (0x7e00u | (man >> 13)) : 0x7c00u));
    int e = (int)exp - 112;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        int shift = 14 - e;
        uint32_t half = 1u << (shift - 1);
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t q = m >> shift;
        if (rem > half || (rem == half && (q & 1u))) q += 1u;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((uint32_t)e << 10) | (man >> 13);
    uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u;
    return (uint16_t)(sign | q);
}

PKV_HD float f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        // subnormal: exact as m * 2^-24
        float v = (float)m * 5.9604644775390625e-08f;
        return u2f(f2u(v) | sign);
    }
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

}  // namespace pkv
