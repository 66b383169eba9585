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
#include <type_traits>

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

// Tiled forest walk. The compiled forest also holds every tree as a complete heap of the
// forest's depth D (a leaf above depth D becomes always-left splits down to its leftmost heap
// leaf), grouped in blocks of TB = forest_tree_block(D) trees of kForestBlockWords dwords:
// tree k of a block takes dwords k * 2^(D+1) .. (k + 1) * 2^(D+1) - 1, node i (counted from 1,
// children 2i and 2i + 1) at dword i: the records of its internal nodes (i < 2^D) and the
// values of its leaves (i >= 2^D); dword 0 holds, as a float, how many consecutive trees of the
// forest the tree stands for (a fitted pack repeats one tree B times: it is walked once and its
// value counted B times; padding trees hold 0). A record packs the bit position of its feature in its word of a row
// tile (bits 0-4), the byte offset of that word row in the tile (bits 5-23; a multiple of
// 4 * rows) and the threshold (bits 24-31). Trees past the forest's last one pad the last
// block with always-left records and zero leaf values.
// A workgroup owns a tile of R rows (32 or 64). It stages the tile's bins in LDS once, packed
// `bits` per bin (3 or 4 when every threshold of the forest is below 7 or 15: a bin above that
// is clamped, which changes no comparison; else 8) and row-interleaved: word (j, r) holds the
// features of word j of row r, so the rows of a word sit in distinct banks and any mix of
// features reads without bank conflicts. The tree blocks then pass through LDS in turn (each
// thread copies its share of the next block into registers while the current block is
// walked), and NT / R tree streams (a lane per row) walk them, G trees per lane at once: every
// load of the walk is an LDS load. Per level a lane reads the bin word of its node, compares,
// and reads the chosen child's record (five VALU instructions per node). Each stream adds
// count * float32(weight * leaf value) of its trees in double (one fma: the product is exact);
// the streams' sums are added in a fixed order and rounded once to float32.

typedef __attribute__((address_space(3))) uint32_t lds_word;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16-byte copies of tree blocks


// LDS dword at byte address `a` of the kernel's (only) LDS allocation.
__device__ __forceinline__ uint32_t lds_at(uint32_t a) { return *reinterpret_cast<const lds_word*>((size_t)a); }

// Bins of rows r0 .. r0 + R - 1 into the packed, row-interleaved tile. The rows are read four
// at a time as one dword per feature column, which the caller allows by a row stride that is
// a multiple of 4 (and 4-byte aligned columns): rows past the column's end read as 0.
template <int BITS, int NT>
__device__ __forceinline__ void stage_tile(const uint8_t* __restrict__ bins, int64_t ld, const ForestTile& ft,
                                           int64_t r0, int R, uint32_t* tile) {
    constexpr int PW = 32 / BITS;
    constexpr uint32_t kClamp = (1u << BITS) - 1u;
    const int words = ft.tile_words / R;
    for (int idx = threadIdx.x; idx < words * (R / 4); idx += NT) {
        const int j = idx / (R / 4);
        const int q = idx - j * (R / 4);
        const int64_t rr = r0 + 4 * q;
        // unconditional loads from clamped (always valid) addresses, so that all of them are
        // in flight at once; the out-of-range values are zeroed afterwards
        const bool row_ok = rr < ld;
        const int64_t rc = row_ok ? rr : 0;
        uint32_t d[PW];
#pragma unroll
        for (int k = 0; k < PW; ++k) {
            const int fc = min(j * PW + k, ft.features - 1);
            // streamed once: a non-temporal load keeps the bins from evicting the tree
            // blocks, which every tile re-reads, from L2
            d[k] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(bins + (int64_t)fc * ld + rc));
        }
#pragma unroll
        for (int k = 0; k < PW; ++k) d[k] = (row_ok && j * PW + k < ft.features) ? d[k] : 0u;
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            uint32_t w = 0u;
#pragma unroll
            for (int k = 0; k < PW; ++k) w |= min((d[k] >> (8 * m)) & 0xffu, kClamp) << (BITS * k);
            tile[j * R + 4 * q + m] = w;
        }
    }
}

// LDS holds the kernel at two workgroups per CU (NT / 128 waves per SIMD), which sets the
// register budget of a lane: all of it goes to the trees a lane walks at once.
template <int D, int R, int NT, bool LEAF, bool RUNS>
__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(NT / 128, NT / 128))) void forest_tile_kernel(
    const uint8_t* __restrict__ bins, int64_t N, int64_t ld, ForestTile ft, const u32x4* __restrict__ blocks,
    const int32_t* __restrict__ lid, const int32_t* __restrict__ tfirst, int32_t T, float tree_weight,
    float* __restrict__ out, int32_t* __restrict__ leaf) {
    extern __shared__ uint32_t lds[];
    constexpr int NL = 1 << D;
    constexpr int S = NT / R;                     // tree streams
    constexpr int TB = forest_tree_block(D);      // trees per block
    constexpr int G = TB / S >= 8 ? 8 : (TB / S >= 1 ? TB / S : 1);  // trees a lane walks at once
    static_assert(TB % (S * G) == 0 || TB < S, "a block splits evenly over streams and lanes");
    constexpr int PER = kForestBlockWords / (4 * NT);  // 16-byte copies of a block per thread
    static_assert(PER * 4 * NT == kForestBlockWords, "whole 16-byte copies per thread");
    static_assert(NT * 8 <= kForestBlockWords * 4, "the streams' sums fit the block's LDS");
    const uint32_t bits = (uint32_t)ft.bits;
    // LDS: the tile, then the current tree block (at the end, the streams' sums [S][R])
    const uint32_t lds0 = (uint32_t)(size_t)(lds_word*)lds;
    const uint32_t rec_b = lds0 + (uint32_t)ft.tile_words * 4u;
    u32x4* tblock = reinterpret_cast<u32x4*>(lds + ft.tile_words);
    double* part = reinterpret_cast<double*>(lds + ft.tile_words);
    // workgroups are dealt round-robin over the 8 XCDs: ids w and w + 8 (same XCD, dispatched
    // one after the other) take neighbouring tiles, whose bins share 128-byte lines when R = 64
    // (64 bytes per feature column), so that one XCD's L2 fetches each line once. The ids of a
    // last, partial group of 16 keep their own tile.
    const int w = blockIdx.x;
    const int tile = w < (int)(gridDim.x & ~15u) ? (w & ~15) | ((w & 7) << 1) | ((w >> 3) & 1) : w;
    const int64_t r0 = (int64_t)tile * R;

    if (ft.bits == 3)
        stage_tile<3, NT>(bins, ld, ft, r0, R, lds);
    else if (ft.bits == 4)
        stage_tile<4, NT>(bins, ld, ft, r0, R, lds);
    else
        stage_tile<8, NT>(bins, ld, ft, r0, R, lds);

    const int row = threadIdx.x & (R - 1);
    // a stream is uniform over a wavefront when R = 64
    const int stream = R == 64 ? __builtin_amdgcn_readfirstlane(threadIdx.x / R) : threadIdx.x / R;
    // the kernel declares no static LDS, so the tile starts at LDS address 0 and a row's word j
    // sits at j*R*4 | row*4 (disjoint bits): a record's masked offset ORs with rowoff
    const uint32_t rowoff = lds0 + (uint32_t)row * 4u;
    const int64_t r = r0 + row;
    double acc = 0.0;
    u32x4 pre[PER];
#pragma unroll
    for (int k = 0; k < PER; ++k) pre[k] = blocks[threadIdx.x + k * NT];
    for (int b = 0; b < ft.blocks; ++b) {
        __syncthreads();  // the tile is staged; the last block's walks are done
#pragma unroll
        for (int k = 0; k < PER; ++k) tblock[threadIdx.x + k * NT] = pre[k];
        __syncthreads();
        {
            // the next block (the last one again after the last: an unconditional load keeps
            // the copies in registers)
            const u32x4* src = blocks + (int64_t)min(b + 1, ft.blocks - 1) * (kForestBlockWords / 4) + threadIdx.x;
#pragma unroll
            for (int k = 0; k < PER; ++k) pre[k] = src[k * NT];
        }
        for (int k0 = stream; k0 < TB; k0 += S * G) {
            // per tree: i = heap index of the current node counted from 1 (children 2i and
            // 2i + 1); node i's record (internal) or leaf value (i >= 2^D) at byte base + 4i
            uint32_t i[G], q[G], base[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
                base[g] = rec_b + (uint32_t)(k0 + g * S) * (4u << (D + 1));
                i[g] = 1u;
                q[g] = D > 0 ? lds_at(base[g] + 4u) : 0u;
            }
#pragma unroll
            for (int lvl = 0; lvl < D; ++lvl) {
                // per level: the bin word of each tree's node, the comparison (right = bin >
                // threshold as a lane mask; i = i + i + right as one add with carry-in), then
                // the chosen child's record
                uint32_t w[G];
#pragma unroll
                for (int g = 0; g < G; ++g) w[g] = lds_at((q[g] & 0x00FFFFE0u) | rowoff);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const uint64_t right = __builtin_amdgcn_uicmp(__builtin_amdgcn_ubfe(w[g], q[g], bits), q[g] >> 24, 34);
                    uint64_t co;
                    asm("v_addc_co_u32_e64 %0, %1, %2, %2, %3" : "=v"(i[g]), "=s"(co) : "v"(i[g]), "s"(right));
                }
                if (lvl + 1 < D) {
#pragma unroll
                    for (int g = 0; g < G; ++g) q[g] = lds_at(base[g] + 4u * i[g]);
                }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                // dword 0: how many consecutive trees of the forest this one stands for (RUNS:
                // some tree stands for more than one; a branch on it per tree cost 7%)
                const float lv = tree_weight * __uint_as_float(lds_at(base[g] + 4u * i[g]));
                const float m = RUNS ? __uint_as_float(lds_at(base[g])) : 1.0f;
                if (RUNS)
                    acc = __builtin_fma((double)lv, (double)m, acc);
                else
                    acc += (double)lv;
                if (LEAF) {
                    const int t = b * TB + k0 + g * S;
                    if (t < T && r < N) {
                        const int t0 = tfirst[t];
                        for (int j = 0; j < (int)m; ++j)
                            leaf[(int64_t)(t0 + j) * N + r] = lid[(int64_t)(t0 + j) * NL + (int)i[g] - NL];
                    }
                }
            }
        }
    }
    __syncthreads();  // every walk of the last block is done: its LDS takes the sums
    part[stream * R + row] = acc;
    __syncthreads();
    if (threadIdx.x < R) {
        double sum = 0.0;
#pragma unroll
        for (int s = 0; s < S; ++s) sum += part[s * R + threadIdx.x];
        const int64_t rr = r0 + threadIdx.x;
        if (rr < N) out[rr] = (float)sum;
    }
}

template <int D>
hipError_t launch_tile_d(const uint8_t* bins, int64_t N, int64_t ld, const ForestTile& ft, const uint32_t* blocks,
                         const int32_t* lid, const int32_t* tfirst, int32_t T, float w, float* out, int32_t* leaf,
                         hipStream_t s) {
    const size_t lds = forest_tile_lds_bytes(ft);
    const int64_t tiles = (N + ft.rows - 1) / ft.rows;
    if (tiles > INT32_MAX || ft.tree_block != forest_tree_block(D) || (ft.rows != 32 && ft.rows != 64) ||
        (ft.threads != 256 && ft.threads != 512 && ft.threads != 1024))
        return hipErrorInvalidValue;
    auto go = [&](auto kern) -> hipError_t {
        const void* fn = reinterpret_cast<const void*>(kern);
        if (lds > 64 * 1024) {
            hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(kern, dim3((unsigned)tiles), dim3(ft.threads), lds, s, bins, N, ld, ft,
                           reinterpret_cast<const u32x4*>(blocks), lid, tfirst, T, w, out, leaf);
        return hipGetLastError();
    };
    auto pick = [&](auto runs) -> hipError_t {
        constexpr bool RU = decltype(runs)::value;
        if (ft.threads == 1024) {
            if (leaf) return ft.rows == 64 ? go(forest_tile_kernel<D, 64, 1024, true, RU>) : go(forest_tile_kernel<D, 32, 1024, true, RU>);
            return ft.rows == 64 ? go(forest_tile_kernel<D, 64, 1024, false, RU>) : go(forest_tile_kernel<D, 32, 1024, false, RU>);
        }
        if (ft.threads == 512) {
            if (leaf) return ft.rows == 64 ? go(forest_tile_kernel<D, 64, 512, true, RU>) : go(forest_tile_kernel<D, 32, 512, true, RU>);
            return ft.rows == 64 ? go(forest_tile_kernel<D, 64, 512, false, RU>) : go(forest_tile_kernel<D, 32, 512, false, RU>);
        }
        if (leaf) return ft.rows == 64 ? go(forest_tile_kernel<D, 64, 256, true, RU>) : go(forest_tile_kernel<D, 32, 256, true, RU>);
        return ft.rows == 64 ? go(forest_tile_kernel<D, 64, 256, false, RU>) : go(forest_tile_kernel<D, 32, 256, false, RU>);
    };
    return ft.runs ? pick(std::true_type{}) : pick(std::false_type{});
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

ForestTile forest_tile_shape(int32_t features, int32_t max_threshold, int32_t depth, int32_t trees) {
    ForestTile ft{};
    ft.features = std::max(1, features);
    ft.bits = max_threshold < 7 ? 3 : max_threshold < 15 ? 4 : 8;
    const int per_word = 32 / ft.bits;
    const int words = (ft.features + per_word - 1) / per_word;
    ft.tree_block = forest_tree_block(depth);
    ft.blocks = (std::max(0, trees) + ft.tree_block - 1) / ft.tree_block;
    // 64-row tiles while two workgroups still fit a CU, else 32
    ft.rows = 64;
    ft.tile_words = words * ft.rows;
    if (forest_tile_lds_bytes(ft) > kForestTileTargetLds) {
        ft.rows = 32;
        ft.tile_words = words * ft.rows;
    }
    // as many tree streams as keep every stream busy with at least one tree of a block, up to
    // 1024 threads: the walk is bound by instruction issue and LDS latency, which the waves
    // of two such workgroups per CU (eight per SIMD) hide
    ft.threads = std::min(1024, std::max(256, ft.rows * ft.tree_block));
    return ft;
}

size_t forest_tile_lds_bytes(const ForestTile& ft) { return ((size_t)ft.tile_words + kForestBlockWords) * 4; }

uint32_t forest_tile_record(const ForestTile& ft, int32_t feature, int32_t threshold) {
    const int per_word = 32 / ft.bits;
    const uint32_t j = (uint32_t)(feature / per_word);
    const uint32_t shift = (uint32_t)((feature % per_word) * ft.bits);  // < 32
    return (j * (uint32_t)ft.rows * 4u) | shift | ((uint32_t)threshold << 24);
}

hipError_t launch_forest_tile(const uint8_t* bins, int64_t N, int64_t ld, const ForestTile& ft,
                              const uint32_t* blocks, const int32_t* lid, const int32_t* tfirst, int32_t T,
                              int32_t depth, float tree_weight, float* out, int32_t* leaf, hipStream_t s) {
    if (ld % 4 != 0 || reinterpret_cast<uintptr_t>(bins) % 4 != 0 || ft.blocks < 1) return hipErrorInvalidValue;
    switch (depth) {
        case 0: return launch_tile_d<0>(bins, N, ld, ft, blocks, lid, tfirst, T, tree_weight, out, leaf, s);
        case 1: return launch_tile_d<1>(bins, N, ld, ft, blocks, lid, tfirst, T, tree_weight, out, leaf, s);
        case 2: return launch_tile_d<2>(bins, N, ld, ft, blocks, lid, tfirst, T, tree_weight, out, leaf, s);
        case 3: return launch_tile_d<3>(bins, N, ld, ft, blocks, lid, tfirst, T, tree_weight, out, leaf, s);
        case 4: return launch_tile_d<4>(bins, N, ld, ft, blocks, lid, tfirst, T, tree_weight, out, leaf, s);
        case 5: return launch_tile_d<5>(bins, N, ld, ft, blocks, lid, tfirst, T, tree_weight, out, leaf, s);
        case 6: return launch_tile_d<6>(bins, N, ld, ft, blocks, lid, tfirst, T, tree_weight, out, leaf, s);
        case 7: return launch_tile_d<7>(bins, N, ld, ft, blocks, lid, tfirst, T, tree_weight, out, leaf, s);
        case 8: return launch_tile_d<8>(bins, N, ld, ft, blocks, lid, tfirst, T, tree_weight, out, leaf, s);
        default: return hipErrorInvalidValue;
    }
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
