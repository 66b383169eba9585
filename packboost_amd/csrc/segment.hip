// Segment mode: from a chosen depth on, a round keeps the fit's rows sorted by (era, frontier
// slot) in buffers of the context, so that the fused scorer (seg_score_kernel) finds a node's
// rows of an era as one contiguous run of row ids (and gradients) and reads their bins from the
// caller's columns through the ids. Every round starts from the caller's era-major order
// (seg_begin). After each depth every era's rows are partitioned stably into the next depth's
// slots: for each era, the slots' left and right children that stay in the frontier, in
// next-slot order, then every row that left the frontier (rows of nodes that did not split or
// of children below 2 * min_samples_leaf, then the rows that had already left). Only the row
// ids, gradients and tree nodes move; the split rules read the caller's columns at the ids.
//
// The partition works on chunks of up to 256 rows of one (era, slot) segment, the slots
// counted 0 .. U with U standing for the era's tail of rows no longer in the frontier:
//   seg_chunks   (one workgroup)    exclusive prefix of the chunk counts per (era, slot);
//   seg_count    (one per chunk)    rows of the chunk that go left (bin <= threshold);
//   seg_scan     (one workgroup)    exclusive prefixes of the left and right counts over chunks;
//   seg_bases    (one per era)      the first destination row of each (era, slot, side);
//   seg_scatter  (one per chunk)    every row to its place (a ballot ranks it among the rows
//                                   of its side in the chunk), with its gradient, row id and
//                                   tree node (the child's id for a split node).
// At the last depth no row moves: seg_final sets the tree node of each split node's rows.
// Row counts are 32-bit: N < 2^31.
#include <algorithm>

#include "pb_internal.h"

namespace pb {
namespace {

constexpr int kSegChunk = kBlock;  // rows per chunk, one per thread

// end of segment `x` (era e, slot v <= U): the next slot's start, or the era's end for the tail
__device__ __forceinline__ int32_t seg_end(const SegState& s, const int32_t* seg, int e, int v, int U) {
    return v < U ? seg[(int64_t)e * s.segw + v + 1] : s.era_off[e + 1];
}

// the (era, slot) entry of chunk q: the last x with cp[x] <= q (cp ascending, cp[0] = 0)
__device__ __forceinline__ int chunk_entry(const int32_t* cp, int n, int q) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cp[mid] <= q) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// Exclusive prefix of one value per thread over the workgroup; *total gets the sum. Ends with
// a barrier, so the next call may reuse the scratch.
__device__ __forceinline__ int32_t wg_scan_excl(int32_t v, int32_t* total) {
    __shared__ int32_t s_w[kBlock / kWave];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    int32_t incl = v;
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
        const int32_t o = __shfl_up(incl, m);
        if (lane >= m) incl += o;
    }
    if (lane == kWave - 1) s_w[wave] = incl;
    __syncthreads();
    int32_t before = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < kBlock / kWave; ++w) {
        before += w < wave ? s_w[w] : 0;
        sum += s_w[w];
    }
    *total = sum;
    __syncthreads();
    return before + incl - v;
}

// Exclusive scan of n int32 values in place by one workgroup: vals[i] <- sum of vals[0 .. i-1],
// vals[n] <- the total. Each thread sums a contiguous strip (16-byte aligned, read four values
// at a time), the strip sums are scanned across the workgroup by wavefront shuffles, and each
// thread rewrites its strip from its offset.
__device__ void block_scan_excl(int32_t* vals, int n) {
    const int tid = threadIdx.x;
    const int per = ((n + kBlock - 1) / kBlock + 3) & ~3;
    const int i0 = min(n, tid * per), i1 = min(n, i0 + per);
    int32_t sum = 0;
    int i = i0;
#pragma unroll 4
    for (; i + 4 <= i1; i += 4) {
        const int4 v = *reinterpret_cast<const int4*>(vals + i);
        sum += v.x + v.y + v.z + v.w;
    }
    for (; i < i1; ++i) sum += vals[i];
    int32_t total;
    int32_t run = wg_scan_excl(sum, &total);
    if (tid == 0) vals[n] = total;
    i = i0;
#pragma unroll 4
    for (; i + 4 <= i1; i += 4) {
        const int4 v = *reinterpret_cast<const int4*>(vals + i);
        int4 o;
        o.x = run;
        run += v.x;
        o.y = run;
        run += v.y;
        o.z = run;
        run += v.z;
        o.w = run;
        run += v.w;
        *reinterpret_cast<int4*>(vals + i) = o;
    }
    for (; i < i1; ++i) {
        const int32_t v = vals[i];
        vals[i] = run;
        run += v;
    }
}

// Round start: the rows in the caller's (era-major) order, with their gradients and the root
// as tree node.
__global__ __launch_bounds__(kBlock) void seg_begin_kernel(const float* __restrict__ grad, int32_t* __restrict__ srow,
                                                     float* __restrict__ gs, uint16_t* __restrict__ stn, int64_t N,
                                                     const int32_t* __restrict__ era_off, int32_t E, int32_t segw,
                                                     int32_t* __restrict__ seg) {
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < N; i += stride) {
        srow[i] = (int32_t)i;
        gs[i] = grad[i];
        stn[i] = 0;
    }
    // the root: slot 0 of era e is the whole era (an inactive root has U = 0 slots, and the
    // same entry is the start of the tail)
    for (int64_t e = (int64_t)blockIdx.x * kBlock + threadIdx.x; e < E; e += stride) {
        seg[e * segw] = era_off[e];
        seg[e * segw + 1] = era_off[e + 1];
    }
}

__global__ __launch_bounds__(kBlock) void seg_chunks_kernel(SegState s, const int32_t* __restrict__ seg,
                                                      int32_t depth) {
    // the chunk counts of a contiguous strip of (era, slot) entries per thread, summed, scanned
    // across the workgroup, then written as exclusive prefixes (the counts are recomputed, not
    // stored and read back)
    const int U = s.st->u_active[depth];
    const int n = s.E * (U + 1);
    const int per = (n + kBlock - 1) / kBlock;
    const int i0 = min(n, (int)threadIdx.x * per), i1 = min(n, i0 + per);
    auto chunks = [&](int e, int v) -> int32_t {
        const int32_t len = seg_end(s, seg, e, v, U) - seg[(int64_t)e * s.segw + v];
        return (len + kSegChunk - 1) / kSegChunk;
    };
    const int e0 = i0 / (U + 1);
    const int v0 = i0 - e0 * (U + 1);
    int32_t sum = 0;
    for (int i = i0, e = e0, v = v0; i < i1; ++i) {
        sum += chunks(e, v);
        if (++v > U) {
            v = 0;
            ++e;
        }
    }
    int32_t total;
    int32_t run = wg_scan_excl(sum, &total);
    if (threadIdx.x == 0) s.cp[n] = total;
    for (int i = i0, e = e0, v = v0; i < i1; ++i) {
        const int32_t c = chunks(e, v);
        s.cp[i] = run;
        run += c;
        if (++v > U) {
            v = 0;
            ++e;
        }
    }
}

// the chunk's segment, its rows [r0, r1), and whether its slot split (then rule)
struct ChunkInfo {
    int x, e, v, U;
    int32_t r0, r1;
    bool split;
    SplitRule rule;
};

__device__ __forceinline__ bool chunk_info(const SegState& s, const int32_t* seg, int32_t depth, int q,
                                           ChunkInfo& ci) {
    ci.U = s.st->u_active[depth];
    const int n = s.E * (ci.U + 1);
    if (q >= s.cp[n]) return false;
    ci.x = chunk_entry(s.cp, n, q);
    ci.e = ci.x / (ci.U + 1);
    ci.v = ci.x - ci.e * (ci.U + 1);
    const int32_t start = seg[(int64_t)ci.e * s.segw + ci.v];
    ci.r0 = start + (q - s.cp[ci.x]) * kSegChunk;
    ci.r1 = min(ci.r0 + kSegChunk, seg_end(s, seg, ci.e, ci.v, ci.U));
    ci.split = false;
    if (ci.v < ci.U) {
        ci.rule = s.rules[ci.v];
        ci.split = ci.rule.feature >= 0;
    }
    return true;
}

// Whether sorted row r goes left under the slot's rule (the caller's column at the row's id).
__device__ __forceinline__ bool seg_goes_left(const SegState& s, const SegBuffers& src, const uint8_t* bins,
                                              const SplitRule& rule, int32_t r) {
    return (int32_t)bins[(int64_t)rule.feature * s.ld + src.row[r]] <= rule.threshold;
}

__global__ __launch_bounds__(kBlock) void seg_count_kernel(SegState s, const int32_t* __restrict__ seg,
                                                     SegBuffers src, const uint8_t* __restrict__ bins,
                                                     int32_t depth) {
    ChunkInfo ci;
    if (!chunk_info(s, seg, depth, blockIdx.x, ci)) return;
    const int32_t r = ci.r0 + (int32_t)threadIdx.x;
    const bool in = r < ci.r1;
    int left = 0;
    if (in) left = ci.split ? (seg_goes_left(s, src, bins, ci.rule, r) ? 1 : 0) : 1;
    __shared__ int s_cnt[kBlock / kWave];
    int c = __popcll(__ballot(left != 0));
    if ((threadIdx.x & (kWave - 1)) == 0) s_cnt[threadIdx.x / kWave] = c;
    __syncthreads();
    if (threadIdx.x == 0) {
        int nl = 0;
        for (int w = 0; w < kBlock / kWave; ++w) nl += s_cnt[w];
        s.cnt_l[blockIdx.x] = nl;
        s.cnt_r[blockIdx.x] = (ci.r1 - ci.r0) - nl;  // 0 unless the slot split
    }
}

__global__ __launch_bounds__(kBlock) void seg_scan_kernel(SegState s, int32_t depth) {
    const int U = s.st->u_active[depth];
    const int nq = s.cp[s.E * (U + 1)];
    block_scan_excl(s.cnt_l, nq);
    __syncthreads();
    block_scan_excl(s.cnt_r, nq);
}

// One workgroup per era: the first destination row of each (slot, side) and the next depth's
// segment starts. The children that stay in the frontier come first, in (slot, side) order (the
// order in which the decision step numbers the next slots), then the rows that leave it (a
// non-split slot's rows count as its left side), then the era's old tail.
__global__ __launch_bounds__(kBlock) void seg_bases_kernel(SegState s, const int32_t* __restrict__ seg,
                                                     int32_t* __restrict__ seg_next, int32_t depth) {
    const int e = blockIdx.x;
    const int U = s.st->u_active[depth];
    const int Un = s.st->u_active[depth + 1];
    const int64_t xb = (int64_t)e * (U + 1);
    const int n = 2 * U;  // (slot, side) items, item i = 2 slot + side
    auto tot = [&](int v, int side) -> int32_t {
        const int32_t* p = side ? s.cnt_r : s.cnt_l;
        return p[s.cp[xb + v + 1]] - p[s.cp[xb + v]];
    };
    const int32_t e0 = s.era_off[e];
    // pass 1: the children that stay in the frontier
    int32_t carry = 0, slots = 0;
    for (int i0 = 0; i0 < n; i0 += kBlock) {
        const int i = i0 + (int)threadIdx.x;
        int32_t sz = 0, keep = 0;
        int v = 0, side = 0;
        if (i < n) {
            v = i >> 1;
            side = i & 1;
            const SplitRule r = s.rules[v];
            if (r.feature >= 0 && r.next_slot[side] != PB_INACTIVE) {
                keep = 1;
                sz = tot(v, side);
            }
        }
        int32_t ts, tk;
        const int32_t off = wg_scan_excl(sz, &ts);
        const int32_t rank = wg_scan_excl(keep, &tk);
        if (keep) {
            s.base[(xb + v) * 2 + side] = e0 + carry + off;
            seg_next[(int64_t)e * s.segw + slots + rank] = e0 + carry + off;
        }
        carry += ts;
        slots += tk;
    }
    if (threadIdx.x == 0) seg_next[(int64_t)e * s.segw + Un] = e0 + carry;  // start of the tail
    // pass 2: the rows that leave the frontier
    for (int i0 = 0; i0 < n; i0 += kBlock) {
        const int i = i0 + (int)threadIdx.x;
        int32_t sz = 0, leave = 0;
        int v = 0, side = 0;
        if (i < n) {
            v = i >> 1;
            side = i & 1;
            const SplitRule r = s.rules[v];
            if (r.feature >= 0 ? r.next_slot[side] == PB_INACTIVE : side == 0) {
                leave = 1;
                sz = tot(v, side);
            }
        }
        int32_t ts;
        const int32_t off = wg_scan_excl(sz, &ts);
        if (leave) s.base[(xb + v) * 2 + side] = e0 + carry + off;
        carry += ts;
    }
    if (threadIdx.x == 0) s.base[(xb + U) * 2] = e0 + carry;  // the rows already in the tail keep their order
}

__global__ __launch_bounds__(kBlock) void seg_scatter_kernel(SegState s, const int32_t* __restrict__ seg,
                                                       SegBuffers src, SegBuffers dst,
                                                       const uint8_t* __restrict__ bins, int32_t depth) {
    ChunkInfo ci;
    if (!chunk_info(s, seg, depth, blockIdx.x, ci)) return;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int32_t r = ci.r0 + tid;
    const bool in = r < ci.r1;
    int side = 0;
    if (in && ci.split) side = seg_goes_left(s, src, bins, ci.rule, r) ? 0 : 1;
    // rank among the rows of the same side before this one in the chunk
    __shared__ int s_cnt[2][kBlock / kWave];
    const unsigned long long m1 = __ballot(in && side == 1);
    const unsigned long long m0 = __ballot(in && side == 0);
    const unsigned long long below = lane == 0 ? 0ull : (~0ull >> (kWave - lane));
    if (lane == 0) {
        s_cnt[0][wave] = __popcll(m0);
        s_cnt[1][wave] = __popcll(m1);
    }
    __syncthreads();
    if (!in) return;
    int rank = __popcll((side ? m1 : m0) & below);
    for (int w = 0; w < wave; ++w) rank += s_cnt[side][w];
    const int32_t* pre = side ? s.cnt_r : s.cnt_l;
    const int32_t d = s.base[(int64_t)ci.x * 2 + side] + (pre[blockIdx.x] - pre[s.cp[ci.x]]) + rank;
    if ((uint32_t)d >= (uint32_t)s.N) return;  // only reachable with inconsistent segments
    dst.g[d] = src.g[r];
    dst.row[d] = src.row[r];
    dst.tnode[d] = ci.split ? (uint16_t)(ci.rule.left_id + side) : src.tnode[r];
}

__global__ __launch_bounds__(kBlock) void seg_final_kernel(SegState s, const int32_t* __restrict__ seg,
                                                     SegBuffers cur, const uint8_t* __restrict__ bins,
                                                     int32_t depth) {
    ChunkInfo ci;
    if (!chunk_info(s, seg, depth, blockIdx.x, ci)) return;
    const int32_t r = ci.r0 + (int32_t)threadIdx.x;
    if (r >= ci.r1 || !ci.split) return;
    cur.tnode[r] = (uint16_t)(ci.rule.left_id + (seg_goes_left(s, cur, bins, ci.rule, r) ? 0 : 1));
}

// preds[row] += float32(lr) * (B float32 adds of the leaf value), the operations of
// round_end_kernel, through the sorted rows' ids
__global__ __launch_bounds__(kBlock) void seg_round_end_kernel(const uint16_t* __restrict__ stn,
                                                         const int32_t* __restrict__ srow,
                                                         const float* __restrict__ values, int32_t B,
                                                         float lr, float* __restrict__ preds, int64_t N,
                                                         const Frontier* st, pb_round_header* header) {
    if (header && blockIdx.x == 0) write_round_header(st, header);  // the round's last kernel
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < N; i += stride) {
        const float v = values[stn[i]];
        float sum = 0.0f;
        for (int t = 0; t < B; ++t) sum = sum + v;
        const float tmp = lr * sum;
        const int32_t r = srow[i];
        preds[r] = preds[r] + tmp;
    }
}

int grid_of_rows(int64_t n) { return (int)std::max<int64_t>(1, std::min<int64_t>((n + kBlock - 1) / kBlock, 8192)); }

}  // namespace

int64_t seg_chunk_bound(int64_t N, int32_t E, int32_t segw) {
    return (N + kSegChunk - 1) / kSegChunk + (int64_t)E * segw;
}

hipError_t launch_seg_begin(const float* grad, int32_t* srow, float* gs, uint16_t* stn, int64_t N,
                            const int32_t* era_off, int32_t E, int32_t segw, int32_t* seg, hipStream_t s) {
    hipLaunchKernelGGL(seg_begin_kernel, dim3(grid_of_rows(std::max<int64_t>(N, E))), dim3(kBlock), 0, s, grad,
                       srow, gs, stn, N, era_off, E, segw, seg);
    return hipGetLastError();
}

hipError_t launch_seg_partition(const SegState& st, const int32_t* seg, int32_t* seg_next, const SegBuffers& src,
                                const SegBuffers& dst, const uint8_t* bins, int32_t depth, bool last,
                                hipStream_t s) {
    const int64_t bound = seg_chunk_bound(st.N, st.E, st.segw);
    if (bound > INT32_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(seg_chunks_kernel, dim3(1), dim3(kBlock), 0, s, st, seg, depth);
    if (last) {
        hipLaunchKernelGGL(seg_final_kernel, dim3((unsigned)bound), dim3(kBlock), 0, s, st, seg, src, bins, depth);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(seg_count_kernel, dim3((unsigned)bound), dim3(kBlock), 0, s, st, seg, src, bins, depth);
    hipLaunchKernelGGL(seg_scan_kernel, dim3(1), dim3(kBlock), 0, s, st, depth);
    hipLaunchKernelGGL(seg_bases_kernel, dim3(st.E), dim3(kBlock), 0, s, st, seg, seg_next,
                       depth);
    hipLaunchKernelGGL(seg_scatter_kernel, dim3((unsigned)bound), dim3(kBlock), 0, s, st, seg, src, dst, bins, depth);
    return hipGetLastError();
}

hipError_t launch_seg_round_end(const uint16_t* stn, const int32_t* srow, const float* values, int32_t B,
                                float lr, float* preds, int64_t N, const Frontier* st, pb_round_header* header,
                                hipStream_t s) {
    hipLaunchKernelGGL(seg_round_end_kernel, dim3(grid_of_rows(N)), dim3(kBlock), 0, s, stn, srow, values, B, lr,
                       preds, N, st, header);
    return hipGetLastError();
}

}  // namespace pb
