// Kernel 3 — row-to-node partition, plus the round's gradient and pack-aggregation passes.
//
// The reference keeps per-node, per-era row lists and splits them stably into left/right
// lists (frontier_cpu.cpp:446-497; partition_frontier_cuda, frontier_cuda.cu:719-851).
// Here every row carries two uint16 ids instead: `nid`, its slot in the active frontier of
// the current depth (PB_INACTIVE once its node stopped growing), and `tnode`, the
// TreeBuilder id of the node it sits in. Row order never changes, so the per-era order the
// reference's lists preserve is implicit, and the partition is one coalesced pass:
//   child = left_id + (bin[feature][row] > threshold)  (left iff bin <= threshold)
// All B trees of a pack share one frontier (they are identical, booster.py:503-519 +
// shard dedup at booster.py:1048-1062), so one id pair per row covers the whole pack.
#include "pb_internal.h"

namespace pb {
namespace {

constexpr int kMaxRulesLds = 2048;

// pb_round_end's inputs, for the round's last partition (partition_kernel<true>)
struct RoundEndArgs {
    const float* values;      // leaf value per TreeBuilder id
    int32_t B;                // pack size
    float lr;
    float* preds;             // [N], 16-byte aligned
    int64_t N;
    pb_round_header* header;  // written by the first workgroup (may be null)
};

// One pack step of a row's prediction: its leaf value added B times in float32, times lr, added
// to the prediction (the reference's pack aggregation, booster.py:585-597).
__device__ __forceinline__ float pack_step(float p, float v, int32_t B, float lr) {
    float s = 0.0f;
    for (int t = 0; t < B; ++t) s = s + v;
    const float tmp = lr * s;
    return p + tmp;
}

// END: the round's last depth, which also does pb_round_end's work: every row's prediction
// takes its final node's leaf value (rows whose node stopped at an earlier depth too), with
// the same float operations as round_end_kernel, so the round needs no separate pass over the
// rows' tree nodes and predictions.
template <bool END>
__global__ __launch_bounds__(kBlock) void partition_kernel(const uint8_t* __restrict__ bins,
                                                       int64_t ld, int32_t nibble,
                                                       int64_t rows_padded,
                                                       const SplitRule* __restrict__ rules,
                                                       const Frontier* st, int32_t depth,
                                                       uint16_t* __restrict__ nid,
                                                       uint16_t* __restrict__ tnode,
                                                       RoundEndArgs re) {
    __shared__ SplitRule s_rules[kMaxRulesLds];
    const int Ua = st->u_active[depth];
    if (END && re.header && blockIdx.x == 0) write_round_header(st, re.header);
    if (!END && Ua <= 0) return;
    const bool in_lds = Ua <= kMaxRulesLds;
    // 8 rows per thread (rows_padded is a multiple of 16): one 16-byte load of their node ids and
    // one of their tree nodes, then their bin gathers all in flight before any result is needed.
    // The first group's node ids and tree nodes are loaded before the rules are staged in LDS, so
    // the two loads overlap.
    const int64_t stride = (int64_t)gridDim.x * kBlock * 8;
    int64_t r = ((int64_t)blockIdx.x * kBlock + threadIdx.x) * 8;
    uint4 nn = make_uint4(0u, 0u, 0u, 0u), tt = nn;
    if (r < rows_padded) {
        nn = *reinterpret_cast<const uint4*>(nid + r);
        tt = *reinterpret_cast<const uint4*>(tnode + r);
    }
    // END: the 8 rows' predictions, read with their ids (rows at or past N are not read)
    float pr[8];
    auto load_preds = [&](int64_t r) {
        if (r + 8 <= re.N) {
            const float4 p0 = *reinterpret_cast<const float4*>(re.preds + r);
            const float4 p1 = *reinterpret_cast<const float4*>(re.preds + r + 4);
            pr[0] = p0.x; pr[1] = p0.y; pr[2] = p0.z; pr[3] = p0.w;
            pr[4] = p1.x; pr[5] = p1.y; pr[6] = p1.z; pr[7] = p1.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) pr[j] = r + j < re.N ? re.preds[r + j] : 0.0f;
        }
    };
    if (END) load_preds(r);
    if (in_lds) {
        for (int u = threadIdx.x; u < Ua; u += kBlock) s_rules[u] = rules[u];
        __syncthreads();
    }
    // the 8 rows of group r that sit in an active node move to their child (left iff bin <=
    // threshold); their new ids are stored
    auto split_rows = [&](int64_t r, uint32_t (&nw)[4], const uint32_t (&n8)[8], uint32_t (&tw)[4]) {
        SplitRule rr[8];
        uint32_t bin[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t u = n8[j];
            bin[j] = 0u;
            if (u >= (uint32_t)Ua) continue;
            rr[j] = in_lds ? s_rules[u] : rules[u];
            if (rr[j].feature < 0) continue;
            const int64_t row = r + j;
            const uint8_t* colp = bins + (int64_t)rr[j].feature * ld;
            // nibble layout: 4 bytes per 8 rows, row i of a group in byte i & 3, high nibble
            // for i >= 4
            bin[j] = nibble ? ((uint32_t)colp[(row >> 3) * 4 + (row & 3)] >> (uint32_t)((row & 4) ? 4 : 0)) & 0xfu
                            : (uint32_t)colp[row];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t u = n8[j];
            if (u >= (uint32_t)Ua) continue;
            const int q = j >> 1, sh = (j & 1) * 16;
            uint32_t nv, tv;
            if (rr[j].feature < 0) {
                nv = PB_INACTIVE;
                tv = (tw[q] >> sh) & 0xffffu;
            } else {
                const uint32_t side = bin[j] > (uint32_t)rr[j].threshold ? 1u : 0u;
                tv = (uint32_t)rr[j].left_id + side;
                nv = rr[j].next_slot[side];
            }
            nw[q] = (nw[q] & ~(0xffffu << sh)) | (nv << sh);
            tw[q] = (tw[q] & ~(0xffffu << sh)) | (tv << sh);
        }
        *reinterpret_cast<uint4*>(nid + r) = make_uint4(nw[0], nw[1], nw[2], nw[3]);
        *reinterpret_cast<uint4*>(tnode + r) = make_uint4(tw[0], tw[1], tw[2], tw[3]);
    };
    for (; r < rows_padded; r += stride) {
        if (r != ((int64_t)blockIdx.x * kBlock + threadIdx.x) * 8) {  // later groups
            nn = *reinterpret_cast<const uint4*>(nid + r);
            tt = *reinterpret_cast<const uint4*>(tnode + r);
            if (END) load_preds(r);
        }
        uint32_t nw[4] = {nn.x, nn.y, nn.z, nn.w};
        uint32_t n8[8];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            n8[q * 2] = nw[q] & 0xffffu;
            n8[q * 2 + 1] = nw[q] >> 16;
        }
        bool any = false;
#pragma unroll
        for (int j = 0; j < 8; ++j) any = any || n8[j] < (uint32_t)Ua;
        uint32_t tw[4] = {tt.x, tt.y, tt.z, tt.w};
        if (any) split_rows(r, nw, n8, tw);  // else PB_INACTIVE or stale rows only
        if (END) {
            // each row's final node: its leaf value, added as in round_end_kernel
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t tv = (tw[j >> 1] >> ((j & 1) * 16)) & 0xffffu;
                pr[j] = pack_step(pr[j], re.values[tv], re.B, re.lr);
            }
            if (r + 8 <= re.N) {
                *reinterpret_cast<float4*>(re.preds + r) = make_float4(pr[0], pr[1], pr[2], pr[3]);
                *reinterpret_cast<float4*>(re.preds + r + 4) = make_float4(pr[4], pr[5], pr[6], pr[7]);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (r + j < re.N) re.preds[r + j] = pr[j];
            }
        }
    }
}

// grad = preds - y (booster.py:2149-2151); hess == 1 is implicit (counts). Every row starts in
// the root; the pad rows [N, rows_padded) are parked with grad 0 and PB_INACTIVE. Also the sum
// of |grad| over each window of kGradWinRows consecutive rows (4 per thread, then a fixed
// reduction tree, so the sums do not depend on scheduling), which bounds the eras' fixed-point
// scales. The first thread also resets the frontier of the round. VEC: the 4 rows of a thread
// move as one 16-byte (grad, preds, y) and 8-byte (node ids, tree nodes) access (the host checks
// the alignment; rows_padded is a multiple of 16).
template <bool VEC>
__global__ __launch_bounds__(kBlock) void round_begin_kernel(const float* __restrict__ preds,
                                                         const float* __restrict__ y,
                                                         float* __restrict__ grad,
                                                         uint16_t* __restrict__ nid,
                                                         uint16_t* __restrict__ tnode, int64_t N,
                                                         int64_t rows_padded, int32_t root_active,
                                                         float* __restrict__ win_sum, Frontier* st,
                                                         int32_t* cur_ids) {
    __shared__ float s_sum[kBlock / kWave];
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        for (int d = 0; d <= PB_MAX_DEPTH; ++d) st->u_active[d] = 0;
        st->u_active[0] = root_active;
        st->tree_size = 1;
        st->reserved[kNonFinite] = 0;
        cur_ids[0] = 0;
    }
    const uint16_t n_root = root_active ? (uint16_t)0 : (uint16_t)PB_INACTIVE;
    const int64_t nwin = (rows_padded + kGradWinRows - 1) / kGradWinRows;
    for (int64_t w = blockIdx.x; w < nwin; w += gridDim.x) {
        const int64_t r0 = w * kGradWinRows + (int64_t)threadIdx.x * 4;
        float s = 0.0f;
        if (VEC) {
            if (r0 < rows_padded) {  // r0 + 3 < rows_padded too
                float4 gv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                ushort4 nv = make_ushort4(PB_INACTIVE, PB_INACTIVE, PB_INACTIVE, PB_INACTIVE);
                if (r0 + 3 < N) {
                    const float4 p = *reinterpret_cast<const float4*>(preds + r0);
                    const float4 t = *reinterpret_cast<const float4*>(y + r0);
                    gv = make_float4(p.x - t.x, p.y - t.y, p.z - t.z, p.w - t.w);
                    s = s + fabsf(gv.x);
                    s = s + fabsf(gv.y);
                    s = s + fabsf(gv.z);
                    s = s + fabsf(gv.w);
                    nv = make_ushort4(n_root, n_root, n_root, n_root);
                } else {
                    float* g4 = reinterpret_cast<float*>(&gv);
                    uint16_t* n4 = reinterpret_cast<uint16_t*>(&nv);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (r0 + j < N) {
                            g4[j] = preds[r0 + j] - y[r0 + j];
                            s = s + fabsf(g4[j]);
                            n4[j] = n_root;
                        }
                    }
                }
                *reinterpret_cast<float4*>(grad + r0) = gv;
                *reinterpret_cast<ushort4*>(nid + r0) = nv;
                *reinterpret_cast<ushort4*>(tnode + r0) = make_ushort4(0, 0, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int64_t r = r0 + j;
                if (r >= rows_padded) break;
                float g = 0.0f;
                if (r < N) {
                    g = preds[r] - y[r];
                    s = s + fabsf(g);
                }
                grad[r] = g;
                nid[r] = r < N ? n_root : (uint16_t)PB_INACTIVE;
                tnode[r] = 0;
            }
        }
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) s = s + __shfl_xor(s, m);
        __syncthreads();  // the previous window's partial sums have been read
        if ((threadIdx.x & (kWave - 1)) == 0) s_sum[threadIdx.x / kWave] = s;
        __syncthreads();
        if (threadIdx.x == 0) {
            float t = s_sum[0];
            for (int i = 1; i < kBlock / kWave; ++i) t = t + s_sum[i];
            win_sum[w] = t;
        }
    }
}

// One thread per era: the era's |grad| sum is at most the sum over the windows it overlaps;
// sh_era[e] = era_grad_scale of that bound.
// Also flags the round (Frontier::reserved[kNonFinite]) when an era's |grad| bound is not finite:
// a NaN or infinite gradient (or one whose window sum overflows float) has no fixed-point value.
__global__ __launch_bounds__(kBlock) void era_scale_kernel(const int32_t* __restrict__ era_off, int32_t E,
                                                       const float* __restrict__ win_sum,
                                                       int32_t* __restrict__ sh_era, Frontier* st) {
    const int e = blockIdx.x * kBlock + threadIdx.x;
    if (e >= E) return;
    const int64_t r0 = era_off[e], r1 = era_off[e + 1];
    double b = 0.0;
    if (r1 > r0)
        for (int64_t w = r0 / kGradWinRows; w <= (r1 - 1) / kGradWinRows; ++w) b += (double)win_sum[w];
    if (!isfinite(b)) st->reserved[kNonFinite] = 1;
    sh_era[e] = era_grad_scale(b * (1.0 + 1.0 / 1024.0));
}

// feats[j][k] = window[off + j][k] for j < D, where off is the number of feature subsets the
// previous round drew: the depths whose frontier had active nodes (booster.py:516-519). The
// caller's window holds that round's draws and the D after each possible count.
__global__ void select_subsets_kernel(const pb_round_header* prev, int32_t D, int32_t K,
                                      const int32_t* __restrict__ window, int32_t* __restrict__ feats) {
    int off = 0;
    if (prev)
        while (off < D && prev->u_active[off] > 0) ++off;
    const int64_t n = (int64_t)D * K;
    for (int64_t i = threadIdx.x; i < n; i += blockDim.x) feats[i] = window[(int64_t)off * K + i];
}

// pack_sum[r] = sum_{t<B} value[leaf(r)] in float32, tree order (booster.py:586-598, the
// B trees are identical); preds += float32(lr) * pack_sum as two rounded float32 ops
// (torch: tmp = lr * pack_sum; preds += tmp). VEC: 4 rows per thread with one 8-byte tree-node
// and one 16-byte prediction access (the host checks the alignment), the last N % 4 rows one by
// one.

template <bool VEC>
__global__ __launch_bounds__(kBlock) void round_end_kernel(const uint16_t* __restrict__ tnode,
                                                       const float* __restrict__ values,
                                                       int32_t B, float lr,
                                                       float* __restrict__ preds, int64_t N,
                                                       const Frontier* st, pb_round_header* header) {
    if (header && blockIdx.x == 0) write_round_header(st, header);  // the round's last kernel
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    const int64_t t0 = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    if (VEC) {
        const int64_t n4 = N / 4;
        for (int64_t q = t0; q < n4; q += stride) {
            const ushort4 tn = *reinterpret_cast<const ushort4*>(tnode + 4 * q);
            float4 p = *reinterpret_cast<const float4*>(preds + 4 * q);
            p.x = pack_step(p.x, values[tn.x], B, lr);
            p.y = pack_step(p.y, values[tn.y], B, lr);
            p.z = pack_step(p.z, values[tn.z], B, lr);
            p.w = pack_step(p.w, values[tn.w], B, lr);
            *reinterpret_cast<float4*>(preds + 4 * q) = p;
        }
        for (int64_t r = 4 * n4 + t0; r < N; r += stride) preds[r] = pack_step(preds[r], values[tnode[r]], B, lr);
    } else {
        for (int64_t r = t0; r < N; r += stride) preds[r] = pack_step(preds[r], values[tnode[r]], B, lr);
    }
}

bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

int grid_for(int64_t work, int per_block, int cap) {
    int64_t g = (work + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (int)g;
}

}  // namespace

hipError_t launch_partition(const uint8_t* bins, int64_t ld, int32_t nibble, int64_t rows_padded,
                            const SplitRule* rules, const Frontier* st, int32_t depth,
                            uint16_t* nid, uint16_t* tnode, hipStream_t s) {
    const int grid = grid_for(rows_padded / 8, kBlock, 8192);
    hipLaunchKernelGGL(partition_kernel<false>, dim3(grid), dim3(kBlock), 0, s, bins, ld, nibble,
                       rows_padded, rules, st, depth, nid, tnode, RoundEndArgs{});
    return hipGetLastError();
}

hipError_t launch_partition_end(const uint8_t* bins, int64_t ld, int32_t nibble, int64_t rows_padded,
                                const SplitRule* rules, const Frontier* st, int32_t depth, uint16_t* nid,
                                uint16_t* tnode, const float* values, int32_t pack_size, float lr,
                                float* preds, int64_t N, pb_round_header* header, hipStream_t s) {
    if (!aligned(preds, 16) || N > rows_padded) return hipErrorInvalidValue;
    const int grid = grid_for(rows_padded / 8, kBlock, 8192);
    hipLaunchKernelGGL(partition_kernel<true>, dim3(grid), dim3(kBlock), 0, s, bins, ld, nibble,
                       rows_padded, rules, st, depth, nid, tnode,
                       RoundEndArgs{values, pack_size, lr, preds, N, header});
    return hipGetLastError();
}

hipError_t launch_select_subsets(const pb_round_header* prev, int32_t D, int32_t K,
                                 const int32_t* window, int32_t* feats, hipStream_t s) {
    hipLaunchKernelGGL(select_subsets_kernel, dim3(1), dim3(kBlock), 0, s, prev, D, K, window, feats);
    return hipGetLastError();
}

hipError_t launch_round_begin(const float* preds, const float* y, float* grad, uint16_t* nid,
                              uint16_t* tnode, int64_t N, int64_t rows_padded, int32_t root_active,
                              const int32_t* era_off, int32_t E, float* win_sum, int32_t* sh_era,
                              Frontier* st, int32_t* cur_ids, hipStream_t s) {
    const int grid = grid_for(rows_padded, kGradWinRows, 1024);
    const bool vec = (rows_padded % 16 == 0) && aligned(preds, 16) && aligned(y, 16) && aligned(grad, 16) &&
                     aligned(nid, 8) && aligned(tnode, 8);
    if (vec)
        hipLaunchKernelGGL(round_begin_kernel<true>, dim3(grid), dim3(kBlock), 0, s, preds, y, grad, nid,
                           tnode, N, rows_padded, root_active, win_sum, st, cur_ids);
    else
        hipLaunchKernelGGL(round_begin_kernel<false>, dim3(grid), dim3(kBlock), 0, s, preds, y, grad, nid,
                           tnode, N, rows_padded, root_active, win_sum, st, cur_ids);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(era_scale_kernel, dim3((E + kBlock - 1) / kBlock), dim3(kBlock), 0, s, era_off,
                       E, win_sum, sh_era, st);
    return hipGetLastError();
}

hipError_t launch_round_end(const uint16_t* tnode, const float* values, int32_t pack_size,
                            float lr, float* preds, int64_t N, const Frontier* st, pb_round_header* header,
                            hipStream_t s) {
    if (aligned(tnode, 8) && aligned(preds, 16)) {
        const int grid = grid_for(std::max<int64_t>(1, N / 4), kBlock, 8192);
        hipLaunchKernelGGL(round_end_kernel<true>, dim3(grid), dim3(kBlock), 0, s, tnode, values, pack_size,
                           lr, preds, N, st, header);
    } else {
        const int grid = grid_for(N, kBlock, 8192);
        hipLaunchKernelGGL(round_end_kernel<false>, dim3(grid), dim3(kBlock), 0, s, tnode, values, pack_size,
                           lr, preds, N, st, header);
    }
    return hipGetLastError();
}

}  // namespace pb
