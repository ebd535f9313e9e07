// pkv_lloyd.hip -- Lloyd-Max refinement of the fib codebook on the device.
//
// Reference: FibCodebookV1::build -> refine_codebook (fib-quant/src/lloyd.rs:
// 106-182): for every restart, `iterations` rounds of assign_samples
// (nearest_index, lloyd.rs:319-337) and update_centroids (lloyd.rs:222-317,
// SplitHighestDistortion), then mse_for_codebook (lloyd.rs:339-357).  The
// host draws the training samples and the restarts' rotated starts (the
// seeded RNG chain, spherical_beta.rs / rotation.rs) and picks the best
// restart by the reference's rule; this kernel runs every restart at once,
// one workgroup each.
//
// Bit-exactness: every f64 quantity is formed in the reference's order.
// Distances sum their k squared differences in dimension order (no fused
// multiply-add: the library is built with -ffp-contract=off); per-cell sums,
// distortions and the MSE add samples in sample order.  Those ordered sums
// run one lane per (cell, dimension), each scanning every sample and adding
// 0.0 for the samples of other cells: a running sum that starts at +0.0 is
// never -0.0 under round-to-nearest, and x + 0.0 == x for every other x, so
// the extra additions change no bit.  Division and square root are the IEEE
// (correctly rounded) f64 operations.  A sample's distance to its own
// centroid in update_centroids is the distance nearest_index returned for it
// (same operands, same order), so it is kept from the assignment step.
#include <hip/hip_runtime.h>

#include "pkv_internal.h"

namespace pkv {

namespace {
constexpr uint32_t LL_THREADS = 256;
constexpr uint32_t LL_BATCH = 16;   // samples whose loads are issued before their in-order additions
constexpr size_t LL_STAGED_MAX = 112 * 1024;   // dynamic LDS for a staged training set (+ ~38 KiB static)
}

// STAGED: the training set, the distances and the assignments live in
// dynamic LDS (ns * (8k + 9) bytes); otherwise the samples are read from
// global memory and the scratch arrays are the restart's slices of bd_all /
// asg_all.  The ordered scans below read every sample once per iteration, so
// their load latency is what staging saves.
template <bool STAGED>
__global__ __launch_bounds__(LL_THREADS) void lloyd_kernel(const double* __restrict__ g_samples, uint32_t ns,
                                                           uint32_t k, uint32_t n, const double* __restrict__ starts,
                                                           uint32_t iterations, double* __restrict__ out_cb,
                                                           double* __restrict__ out_mse, double* __restrict__ init_mse,
                                                           uint32_t* __restrict__ status, double* __restrict__ bd_all,
                                                           uint8_t* __restrict__ asg_all) {
    __shared__ double cb[LLOYD_MAX_NK], sums[LLOYD_MAX_NK];
    __shared__ double dist[LLOYD_MAX_N], fard[LLOYD_MAX_N];
    __shared__ uint32_t cnt[LLOYD_MAX_N], fari[LLOYD_MAX_N];
    __shared__ uint32_t fail;
    extern __shared__ double dyn[];
    const uint32_t r = blockIdx.x, tid = threadIdx.x, nk = n * k;
    const double* samples = g_samples;
    double* bd = bd_all + static_cast<uint64_t>(r) * ns;
    uint8_t* asg = asg_all + static_cast<uint64_t>(r) * ns;
    if constexpr (STAGED) {
        double* s_l = dyn;
        for (uint32_t i = tid; i < ns * k; i += LL_THREADS) s_l[i] = g_samples[i];
        samples = s_l;
        bd = dyn + static_cast<size_t>(ns) * k;
        asg = reinterpret_cast<uint8_t*>(bd + ns);
    }
    for (uint32_t i = tid; i < nk; i += LL_THREADS) cb[i] = starts[static_cast<uint64_t>(r) * nk + i];
    if (tid == 0) fail = 0u;
    __syncthreads();

    // nearest_index for every sample: index (first strict minimum) and distance
    auto assign = [&]() {
        for (uint32_t i = tid; i < ns; i += LL_THREADS) {
            const double* s = samples + static_cast<uint64_t>(i) * k;
            uint32_t best = 0;
            double bdist = __builtin_inf();
            for (uint32_t w = 0; w < n; ++w) {
                double d = 0.0;
                for (uint32_t t = 0; t < k; ++t) {
                    const double dl = s[t] - cb[w * k + t];
                    d += dl * dl;
                }
                if (d < bdist) {
                    bdist = d;
                    best = w;
                }
            }
            asg[i] = static_cast<uint8_t>(best);
            bd[i] = bdist;
        }
        __syncthreads();
    };
    // mse_for_codebook of the current assignment, in sample order (lane 0);
    // loads go out 16 samples ahead of the additions that wait for them
    auto mse = [&]() -> double {
        double sum = 0.0;
        uint32_t i = 0;
        for (; i + LL_BATCH <= ns; i += LL_BATCH) {
            double v[LL_BATCH];
#pragma unroll
            for (uint32_t u = 0; u < LL_BATCH; ++u) v[u] = bd[i + u];
#pragma unroll
            for (uint32_t u = 0; u < LL_BATCH; ++u) sum += v[u];
        }
        for (; i < ns; ++i) sum += bd[i];
        return sum / static_cast<double>(ns);
    };

    if (r == 0) {   // the initial codebook is restart 0's start
        assign();
        if (tid == 0) *init_mse = mse();
    }
    for (uint32_t it = 0; it < iterations; ++it) {
        assign();
        // jobs [0, nk): per-(cell, dimension) sums; [nk, nk + n): per-cell
        // count, distortion and farthest sample (first strict maximum)
        for (uint32_t j = tid; j < nk + n; j += LL_THREADS) {
            if (j < nk) {
                const uint32_t w = j / k, t = j % k;
                double sum = 0.0;
                uint32_t i = 0;
                for (; i + LL_BATCH <= ns; i += LL_BATCH) {
                    double x[LL_BATCH];
                    uint32_t a[LL_BATCH];
#pragma unroll
                    for (uint32_t u = 0; u < LL_BATCH; ++u) {
                        a[u] = asg[i + u];
                        x[u] = samples[static_cast<uint64_t>(i + u) * k + t];
                    }
#pragma unroll
                    for (uint32_t u = 0; u < LL_BATCH; ++u) sum += a[u] == w ? x[u] : 0.0;
                }
                for (; i < ns; ++i) sum += asg[i] == w ? samples[static_cast<uint64_t>(i) * k + t] : 0.0;
                sums[j] = sum;
            } else {
                const uint32_t w = j - nk;
                uint32_t c = 0, fi = 0;
                double dsum = 0.0, fd = -1.0;
                auto take = [&](uint32_t i, uint32_t a, double sd) {
                    const bool mine = a == w;
                    c += mine ? 1u : 0u;
                    dsum += mine ? sd : 0.0;
                    const bool further = mine && sd > fd;
                    fd = further ? sd : fd;
                    fi = further ? i : fi;
                };
                uint32_t i = 0;
                for (; i + LL_BATCH <= ns; i += LL_BATCH) {
                    double v[LL_BATCH];
                    uint32_t a[LL_BATCH];
#pragma unroll
                    for (uint32_t u = 0; u < LL_BATCH; ++u) {
                        a[u] = asg[i + u];
                        v[u] = bd[i + u];
                    }
#pragma unroll
                    for (uint32_t u = 0; u < LL_BATCH; ++u) take(i + u, a[u], v[u]);
                }
                for (; i < ns; ++i) take(i, asg[i], bd[i]);
                cnt[w] = c;
                dist[w] = dsum;
                fard[w] = fd;
                fari[w] = fi;
            }
        }
        __syncthreads();
        for (uint32_t j = tid; j < nk; j += LL_THREADS)
            if (cnt[j / k] > 0u) cb[j] = sums[j] / static_cast<double>(cnt[j / k]);
        __syncthreads();
        if (tid == 0) {   // empty cells: split the highest-distortion donor (rare)
            for (uint32_t e = 0; e < n && !fail; ++e) {
                if (cnt[e] != 0u) continue;
                int donor = -1;   // Iterator::max_by keeps the last maximum
                for (uint32_t w = 0; w < n; ++w)
                    if (cnt[w] > 1u && (donor < 0 || !(dist[w] < dist[donor]))) donor = static_cast<int>(w);
                if (donor < 0) {
                    fail = 1u;
                    break;
                }
                const uint32_t dn = static_cast<uint32_t>(donor);
                const double* far = samples + static_cast<uint64_t>(fari[dn]) * k;
                double rn2 = 0.0;
                for (uint32_t t = 0; t < k; ++t) {
                    const double res = far[t] - cb[dn * k + t];
                    rn2 += res * res;
                }
                const double rn = __builtin_sqrt(rn2);
                if (!(rn < __builtin_inf()) || rn <= 2.220446049250313e-16) {
                    fail = 1u;
                    break;
                }
                for (uint32_t t = 0; t < k; ++t) {
                    const double dir = (far[t] - cb[dn * k + t]) / rn;
                    const double cen = cb[dn * k + t];
                    cb[dn * k + t] = cen - 1.0e-6 * dir;
                    cb[e * k + t] = cen + 1.0e-6 * dir;
                }
                cnt[dn] -= 1u;
                cnt[e] = 1u;
                dist[dn] = 0.0;
                dist[e] = 0.0;
            }
        }
        __syncthreads();
        if (fail) break;
    }
    if (!fail) assign();
    if (tid == 0) {
        out_mse[r] = fail ? __builtin_nan("") : mse();
        status[r] = fail;
    }
    for (uint32_t i = tid; i < nk; i += LL_THREADS) out_cb[static_cast<uint64_t>(r) * nk + i] = cb[i];
}

int launch_lloyd(const double* samples, uint32_t ns, uint32_t k, uint32_t n, const double* starts, uint32_t restarts,
                 uint32_t iterations, double* out_cb, double* out_mse, double* init_mse, uint32_t* status,
                 double* bd_scratch, uint8_t* asg_scratch, void* stream) {
    hipStream_t st = static_cast<hipStream_t>(stream);
    const size_t staged = static_cast<size_t>(ns) * (8u * k + 9u);
    if (staged <= LL_STAGED_MAX) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(lloyd_kernel<true>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(staged));
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(lloyd_kernel<true>, dim3(restarts), dim3(LL_THREADS), staged, st, samples, ns, k, n, starts,
                           iterations, out_cb, out_mse, init_mse, status, bd_scratch, asg_scratch);
    } else {
        hipLaunchKernelGGL(lloyd_kernel<false>, dim3(restarts), dim3(LL_THREADS), 0, st, samples, ns, k, n, starts,
                           iterations, out_cb, out_mse, init_mse, status, bd_scratch, asg_scratch);
    }
    return hipGetLastError();
}

}  // namespace pkv
