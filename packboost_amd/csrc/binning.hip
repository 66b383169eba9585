// Quantile binning on the device: the reference's quantile_bin / apply_bins (data.py:44-111).
//
//  * edges: for each column, the interior quantiles np.quantile(x, q, method="linear") of the
//    column's values, cast to float32. NumPy's arithmetic (numpy lib/_function_base_impl.py,
//    _quantile / _get_indexes / _lerp) is restated exactly, in double without contraction:
//        v = (n - 1) * q;  i = floor(v);  j = i + 1;  (both n - 1 when v >= n - 1)
//        g = v - i;  a = x(i), b = x(j) (float32, sorted ascending);  d = b - a (float32)
//        e = g >= 0.5 ? b - d * (1 - g) : a + d * g          (double), then float32
//    A column holding a NaN gets NaN edges (NumPy sorts NaN last and propagates it).
//  * bins: searchsorted(edges, x, side="left") clipped to [0, max_bins - 1], with NumPy's
//    NaN-last order (NaN > every number), written column-major for the histogram kernel,
//    optionally gathering rows through a permutation (era-major order).
#include <algorithm>

#include "pb_internal.h"

namespace pb {
namespace {

__global__ void quantile_edges_kernel(const float* __restrict__ sorted, int64_t n, int64_t ld,
                                      int32_t F, const double* __restrict__ q, int32_t nq,
                                      float* __restrict__ edges, int32_t edge_stride) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)F * nq) return;
    const int f = (int)(t / nq);
    const int k = (int)(t - (int64_t)f * nq);
    const float* col = sorted + (int64_t)f * ld;
    float out;
    if (n <= 0) {
        out = __int_as_float(0x7fc00000);
    } else if (isnan(col[n - 1])) {
        out = __int_as_float(0x7fc00000);
    } else {
        const double v = (double)(n - 1) * q[k];
        double prev = floor(v);
        double next = prev + 1.0;
        if (v >= (double)(n - 1)) {
            prev = (double)(n - 1);
            next = (double)(n - 1);
        }
        if (v < 0.0) {
            prev = 0.0;
            next = 0.0;
        }
        const double g = v - floor(v);
        const float a = col[(int64_t)prev];
        const float b = col[(int64_t)next];
        const float d = b - a;
        const double e = (g >= 0.5) ? ((double)b - (double)d * (1.0 - g))
                                    : ((double)a + (double)d * g);
        out = (float)e;
    }
    edges[(int64_t)k * edge_stride + f] = out;
}

// NumPy's float order for searchsorted: a < b, with NaN after every number
__device__ __forceinline__ bool np_less(float a, float b) {
    return a < b || (isnan(b) && !isnan(a));
}

__global__ __launch_bounds__(kBlock) void apply_bins_kernel(
    const float* __restrict__ xt, int64_t n, int64_t ld_x, const float* __restrict__ edges,
    int32_t ne, int32_t edge_stride, int32_t max_bins, const int64_t* __restrict__ perm,
    uint8_t* __restrict__ bins, int64_t ld_out, int32_t rows_per_block) {
    __shared__ float s_edges[256];
    const int f = blockIdx.y;
    for (int i = threadIdx.x; i < ne; i += kBlock) s_edges[i] = edges[(int64_t)i * edge_stride + f];
    __syncthreads();
    const float* col = xt + (int64_t)f * ld_x;
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_block;
    const int64_t r1 = min(n, r0 + rows_per_block);
    for (int64_t r = r0 + threadIdx.x; r < r1; r += kBlock) {
        const float x = col[perm ? perm[r] : r];
        int lo = 0, hi = ne;
        while (lo < hi) {
            const int mid = lo + ((hi - lo) >> 1);
            if (np_less(s_edges[mid], x))
                lo = mid + 1;
            else
                hi = mid;
        }
        bins[(int64_t)f * ld_out + r] = (uint8_t)min(lo, max_bins - 1);
    }
}

// Nibble layout for nb <= 16: every 8 rows of a uint8 column (bytes b0..b7) become one dword
// whose byte j is b_j | b_{j+4} << 4. One thread converts 16 rows (one 16-byte load, one
// 8-byte store); bins above 15 lose their high bits (callers guarantee bins < nb <= 16).
// Rows n .. ld-1 (padding) are written as bin 0: the histogram reads them unmasked.
__global__ __launch_bounds__(kBlock) void pack_bins4_kernel(const uint8_t* __restrict__ bins,
                                                         int64_t ld, int64_t n,
                                                         int64_t units_per_col, int64_t units,
                                                         uint8_t* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < units; t += stride) {
        const int64_t f = t / units_per_col;
        const int64_t u = t - f * units_per_col;
        uint4 v = *reinterpret_cast<const uint4*>(bins + f * ld + u * 16);
        const int64_t r0 = u * 16;  // first row of this unit
        if (r0 + 16 > n) {
            uint32_t wv[4] = {v.x, v.y, v.z, v.w};
    #pragma unroll
            for (int q = 0; q < 4; ++q)
    #pragma unroll
                for (int b = 0; b < 4; ++b)
                    if (r0 + 4 * q + b >= n) wv[q] &= ~(0xffu << (8 * b));
            v = make_uint4(wv[0], wv[1], wv[2], wv[3]);
        }
        uint2 o;
        o.x = (v.x & 0x0f0f0f0fu) | ((v.y & 0x0f0f0f0fu) << 4);
        o.y = (v.z & 0x0f0f0f0fu) | ((v.w & 0x0f0f0f0fu) << 4);
        *reinterpret_cast<uint2*>(out + f * (ld / 2) + u * 8) = o;
    }
}

}  // namespace

hipError_t launch_pack_bins4(const uint8_t* bins, int64_t n, int64_t ld, int32_t F, uint8_t* out,
                             hipStream_t s) {
    const int64_t per_col = ld / 16;
    const int64_t units = per_col * F;
    const int grid = (int)std::min<int64_t>((units + kBlock - 1) / kBlock, 65536);
    hipLaunchKernelGGL(pack_bins4_kernel, dim3(std::max(grid, 1)), dim3(kBlock), 0, s, bins, ld, n,
                       per_col, units, out);
    return hipGetLastError();
}

hipError_t launch_quantile_edges(const float* sorted, int64_t n, int64_t ld, int32_t F,
                                 const double* q, int32_t nq, float* edges, int32_t edge_stride,
                                 hipStream_t s) {
    const int64_t work = (int64_t)F * nq;
    const int grid = (int)((work + kBlock - 1) / kBlock);
    hipLaunchKernelGGL(quantile_edges_kernel, dim3(grid), dim3(kBlock), 0, s, sorted, n, ld, F, q,
                       nq, edges, edge_stride);
    return hipGetLastError();
}

hipError_t launch_apply_bins(const float* xt, int64_t n, int64_t ld_x, int32_t F,
                             const float* edges, int32_t ne, int32_t edge_stride, int32_t max_bins,
                             const int64_t* perm, uint8_t* bins, int64_t ld_out, hipStream_t s) {
    const int rows_per_block = 8192;
    const int64_t gx = (n + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL(apply_bins_kernel, dim3((unsigned)gx, (unsigned)F), dim3(kBlock), 0, s, xt,
                       n, ld_x, edges, ne, edge_stride, max_bins, perm, bins, ld_out,
                       rows_per_block);
    return hipGetLastError();
}

}  // namespace pb
