// Kernel 4 — batched prediction over column-major uint8 bins.
//
// Reference semantics: a row goes left iff bin <= threshold until it reaches a leaf
// (booster.py:131-169, frontier_cuda.cu:193-233). predict_pack_cuda returns
// tree_weight * sum of the pack's leaf values (frontier_cuda.cu:925-986); the CPU path of
// PackBoost.predict accumulates pred += weight * value tree by tree (booster.py:709-712).
// Malformed child indices or split features end the walk with 0 (leaf index -1), like the
// reference's guards; tree spans are clamped to the node arrays.
//
// `sequential` selects the CPU path's order: out = sum_t (weight * value_t), one float32
// rounding per product and per add, trees in order.
//
// One lane per row: a wavefront reads 64 consecutive rows of the same column while its rows
// sit in the same node, and the forest arrays are small enough to stay in L2.
#include <algorithm>

#include "pb_internal.h"

namespace pb {
namespace {

__device__ __forceinline__ float walk(const uint8_t* __restrict__ bins, int64_t ld, int64_t row,
                                      const int32_t* __restrict__ feature,
                                      const int32_t* __restrict__ threshold,
                                      const int32_t* __restrict__ left,
                                      const int32_t* __restrict__ right,
                                      const float* __restrict__ value,
                                      const uint8_t* __restrict__ is_leaf, int32_t lo, int32_t hi,
                                      int32_t F, int32_t* leaf_out) {
    int node = lo;
    const int steps = hi - lo;
    for (int it = 0; it < steps; ++it) {
        if (is_leaf[node]) {
            *leaf_out = node;
            return value[node];
        }
        const int f = feature[node];
        if (f < 0 || f >= F) break;
        const int v = bins[(int64_t)f * ld + row];
        const int nxt = (v <= threshold[node]) ? left[node] : right[node];
        if (nxt < lo || nxt >= hi) break;
        node = nxt;
    }
    *leaf_out = -1;
    return 0.0f;
}

__global__ __launch_bounds__(kBlock) void predict_pack_kernel(
    const uint8_t* __restrict__ bins, int64_t N, int64_t ld, int32_t F,
    const int32_t* __restrict__ feature, const int32_t* __restrict__ threshold,
    const int32_t* __restrict__ left_abs, const int32_t* __restrict__ right_abs,
    const float* __restrict__ value, const uint8_t* __restrict__ is_leaf,
    const int32_t* __restrict__ offsets, int32_t B, int32_t total_nodes, float tree_weight,
    int32_t sequential, float* __restrict__ out, int32_t* __restrict__ leaf) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t r = (int64_t)blockIdx.x * kBlock + threadIdx.x; r < N; r += stride) {
        float s = 0.0f;
        for (int t = 0; t < B; ++t) {
            int32_t lf;
            // a tree's span, clamped to the node arrays (offsets come from the caller)
            const int32_t lo = min(max(offsets[t], 0), total_nodes);
            const int32_t hi = min(max(offsets[t + 1], lo), total_nodes);
            const float v = walk(bins, ld, r, feature, threshold, left_abs, right_abs, value,
                                 is_leaf, lo, hi, F, &lf);
            s = sequential ? (s + tree_weight * v) : (s + v);
            if (leaf) leaf[(int64_t)t * N + r] = lf;
        }
        out[r] = sequential ? s : tree_weight * s;
    }
}

__global__ __launch_bounds__(kBlock) void predict_bins_kernel(
    const uint8_t* __restrict__ bins, int64_t N, int64_t ld, int32_t F,
    const int32_t* __restrict__ feature, const int32_t* __restrict__ threshold,
    const int32_t* __restrict__ left, const int32_t* __restrict__ right,
    const float* __restrict__ value, const uint8_t* __restrict__ is_leaf, int32_t num_nodes,
    float* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t r = (int64_t)blockIdx.x * kBlock + threadIdx.x; r < N; r += stride) {
        int32_t lf;
        out[r] = walk(bins, ld, r, feature, threshold, left, right, value, is_leaf, 0, num_nodes,
                      F, &lf);
    }
}

// Compiled forest: one 16-byte record per node {feature | threshold << 24, left, right,
// value bits}; a leaf has feature field 0xFFFFFF. A lane walks kTreeGroup trees at once, all
// one level per step, so their record and bin loads overlap; the leaf values are then added
// in tree order, one float32 rounding per product and per add (PackBoost.predict's order).
// The grid can be capped so that the rows in flight keep their bins in the caches.
constexpr uint32_t kLeafFeature = kLeafFeatureBits;

template <int kTreeGroup>
__global__ __launch_bounds__(kBlock) void forest_kernel(
    const uint8_t* __restrict__ bins, int64_t N, int64_t ld, const int4* __restrict__ rec,
    const int32_t* __restrict__ roots, int32_t T, int32_t depth, float tree_weight,
    float* __restrict__ out, int32_t* __restrict__ leaf) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t r = (int64_t)blockIdx.x * kBlock + threadIdx.x; r < N; r += stride) {
        float s = 0.0f;
        for (int t0 = 0; t0 < T; t0 += kTreeGroup) {
            int node[kTreeGroup];
#pragma unroll
            for (int j = 0; j < kTreeGroup; ++j) node[j] = roots[min(t0 + j, T - 1)];
            for (int lvl = 0; lvl < depth; ++lvl) {
#pragma unroll
                for (int j = 0; j < kTreeGroup; ++j) {
                    const int4 q = rec[node[j]];
                    const uint32_t f = (uint32_t)q.x & 0xFFFFFFu;
                    if (f != kLeafFeature) {
                        const uint32_t thr = (uint32_t)q.x >> 24;
                        const uint32_t b = bins[(int64_t)f * ld + r];
                        node[j] = (b <= thr) ? q.y : q.z;
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < kTreeGroup; ++j) {
                if (t0 + j < T) {
                    const float v = __int_as_float(rec[node[j]].w);
                    s = s + tree_weight * v;
                    if (leaf) leaf[(int64_t)(t0 + j) * N + r] = node[j];
                }
            }
        }
        out[r] = s;
    }
}

int grid_rows(int64_t N) {
    int64_t g = (N + kBlock - 1) / kBlock;
    if (g < 1) g = 1;
    if (g > 65536) g = 65536;
    return (int)g;
}

}  // namespace

hipError_t launch_predict_pack(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                               const int32_t* feature, const int32_t* threshold,
                               const int32_t* left_abs, const int32_t* right_abs,
                               const float* value, const uint8_t* is_leaf,
                               const int32_t* offsets, int32_t B, int32_t total_nodes,
                               float tree_weight, int32_t sequential, float* out, int32_t* leaf,
                               hipStream_t s) {
    hipLaunchKernelGGL(predict_pack_kernel, dim3(grid_rows(N)), dim3(kBlock), 0, s, bins, N, ld,
                       F, feature, threshold, left_abs, right_abs, value, is_leaf, offsets, B,
                       total_nodes, tree_weight, sequential, out, leaf);
    return hipGetLastError();
}

hipError_t launch_forest(const uint8_t* bins, int64_t N, int64_t ld, const int4* rec,
                         const int32_t* roots, int32_t T, int32_t depth, float tree_weight,
                         float* out, int32_t* leaf, int32_t group, int32_t max_grid,
                         hipStream_t s) {
    int grid = grid_rows(N);
    if (max_grid > 0) grid = std::min(grid, max_grid);
    switch (group) {
        case 4:
            hipLaunchKernelGGL(forest_kernel<4>, dim3(grid), dim3(kBlock), 0, s, bins, N, ld, rec,
                               roots, T, depth, tree_weight, out, leaf);
            break;
        case 16:
            hipLaunchKernelGGL(forest_kernel<16>, dim3(grid), dim3(kBlock), 0, s, bins, N, ld, rec,
                               roots, T, depth, tree_weight, out, leaf);
            break;
        case 32:
            hipLaunchKernelGGL(forest_kernel<32>, dim3(grid), dim3(kBlock), 0, s, bins, N, ld, rec,
                               roots, T, depth, tree_weight, out, leaf);
            break;
        default:
            hipLaunchKernelGGL(forest_kernel<8>, dim3(grid), dim3(kBlock), 0, s, bins, N, ld, rec,
                               roots, T, depth, tree_weight, out, leaf);
    }
    return hipGetLastError();
}

hipError_t launch_predict_bins(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                               const int32_t* feature, const int32_t* threshold,
                               const int32_t* left, const int32_t* right, const float* value,
                               const uint8_t* is_leaf, int32_t num_nodes, float* out,
                               hipStream_t s) {
    hipLaunchKernelGGL(predict_bins_kernel, dim3(grid_rows(N)), dim3(kBlock), 0, s, bins, N, ld,
                       F, feature, threshold, left, right, value, is_leaf, num_nodes, out);
    return hipGetLastError();
}

}  // namespace pb
