// Round metrics on the device: mean over eras of the Pearson correlation of target and
// predictions (PackBoost._era_correlation_np, booster.py:909-929). Rows are era-major, so era
// e is the row range [era_off[e], era_off[e+1]).
//
// One workgroup per era, two passes in double (means, then centred sums), each reduced in a
// fixed order (per-thread strided sums, then a fixed tree), so results are identical run to
// run. An era counts when it has >= 2 rows, both population standard deviations exceed 1e-12
// and the correlation is finite, as in the reference; the mean over counted eras is taken by
// one thread in era order (NaN when none counts).
#include "pb_internal.h"

namespace pb {
namespace {

__device__ double block_sum(double v, double* sh) {
    // fixed-order tree: lanes of a wave, then the waves in order
#pragma unroll
    for (int m = kWave / 2; m >= 1; m >>= 1) v += __shfl_down(v, m);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    __syncthreads();
    if (lane == 0) sh[wave] = v;
    __syncthreads();
    double t = 0.0;
    for (int w = 0; w < kBlock / kWave; ++w) t += sh[w];
    return t;  // every thread holds the total
}

__global__ __launch_bounds__(kBlock) void era_corr_kernel(const float* __restrict__ y,
                                                      const float* __restrict__ p,
                                                      const int32_t* __restrict__ era_off,
                                                      double* __restrict__ era_corr) {
    __shared__ double sh[kBlock / kWave];
    const int e = blockIdx.x;
    const int r0 = era_off[e], r1 = era_off[e + 1];
    const int n = r1 - r0;
    double sy = 0.0, sp = 0.0;
    for (int r = r0 + (int)threadIdx.x; r < r1; r += kBlock) {
        sy += (double)y[r];
        sp += (double)p[r];
    }
    sy = block_sum(sy, sh);
    sp = block_sum(sp, sh);
    const double my = n > 0 ? sy / n : 0.0, mp = n > 0 ? sp / n : 0.0;
    double syy = 0.0, spp = 0.0, syp = 0.0;
    for (int r = r0 + (int)threadIdx.x; r < r1; r += kBlock) {
        const double dy = (double)y[r] - my, dp = (double)p[r] - mp;
        syy += dy * dy;
        spp += dp * dp;
        syp += dy * dp;
    }
    syy = block_sum(syy, sh);
    spp = block_sum(spp, sh);
    syp = block_sum(syp, sh);
    if (threadIdx.x == 0) {
        double c = __longlong_as_double(0x7ff8000000000000ll);  // NaN: era not counted
        if (n >= 2) {
            const double sdy = sqrt(syy / n), sdp = sqrt(spp / n);
            if (sdy > 1e-12 && sdp > 1e-12) {
                const double v = (syp / n) / (sdy * sdp);
                if (isfinite(v)) c = v;
            }
        }
        era_corr[e] = c;
    }
}

__global__ void era_corr_mean_kernel(const double* __restrict__ era_corr, int32_t E,
                                     double* __restrict__ out) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    double s = 0.0;
    int k = 0;
    for (int e = 0; e < E; ++e) {
        const double c = era_corr[e];
        if (!isnan(c)) {
            s += c;
            ++k;
        }
    }
    out[0] = k > 0 ? s / k : __longlong_as_double(0x7ff8000000000000ll);
}

}  // namespace

hipError_t launch_era_corr(const float* y, const float* p, const int32_t* era_off, int32_t E,
                           double* era_corr, double* out, hipStream_t s) {
    hipLaunchKernelGGL(era_corr_kernel, dim3(E), dim3(kBlock), 0, s, y, p, era_off, era_corr);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(era_corr_mean_kernel, dim3(1), dim3(64), 0, s, era_corr, E, out);
    return hipGetLastError();
}

}  // namespace pb
