// Kernel 1 — per-(era, node, feature, bin) count/grad histogram over column-major uint8 bins.
//
// Reference semantics: frontier_cpu.cpp:261-321 builds, for each sampled feature,
// count[n][e][b] (int64) and grad[n][e][b] (float32, summed in row order), then a float32
// running sum over bins gives prefix[b < nb-1] and the era total. This kernel produces the
// same prefix/total planes for all sampled features of a depth at once; the counts are
// exact and the grad prefixes are exact fixed-point sums rounded once to float32.
//
// Design (gfx950):
//  * One workgroup owns one (era, feature tile). Rows are era-major, so an era is a
//    contiguous byte range of every feature column: loads are coalesced dwords (4 rows per
//    lane, 1024 rows per workgroup pass) and no global atomics are needed.
//  * Each lane keeps the row state of its 4 rows (LDS byte offset of the row's node and the
//    packed value below) in registers and reuses it across all features of the tile.
//  * One 64-bit LDS atomic carries (fixed-point grad << 16) + 1, so the count (low 16 bits)
//    and the grad sum (high 48 bits) accumulate in a single ds_add_u64. Integer addition is
//    order-independent, so the result is deterministic run to run; grad is quantised as
//    round(g * 2^s) with max|g| * 2^s < 2^30, far finer than float32 rounding of the
//    reference's row-order sum.
//  * Joint bins (P = 2 for nb <= 16, P = 3 for nb <= 6): the P features of a group share one
//    atomic on the joint cell (b1 * nb + b2, or (b1 * nb + b2) * nb + b3). The joint index is
//    below 256, so for 4 rows it comes from 32-bit multiply-adds of the packed bin dwords.
//    The flush recovers every marginal by integer sums over the other features' bins, so the
//    histogram is exactly the one-feature-per-atomic result with 1/P of the LDS atomics.
//  * The histogram is replicated `C` times in LDS, interleaved per word, and lane l adds
//    into copy l % C: with C = 32 the 32 lanes an LDS cycle serves for 64-bit operands land in
//    distinct 8-byte slots, so same-cell rows never serialise (measured on gfx950: 16 copies
//    still conflict). The host trades C against features per workgroup under an LDS budget.
//  * Lanes whose 4 rows all lie outside the era (or in no active node) skip their atomics.
//  * blockIdx -> (era, tile) is XCD-aware: the 8 XCDs receive blocks round-robin, so all
//    feature tiles of one era run on the same XCD and share the era's row state in its L2.
#include <algorithm>

#include "pb_internal.h"

namespace pb {
namespace {

// 32-bit product that the compiler keeps as its own instruction (see the joint index).
__device__ __forceinline__ uint32_t mul_sep(uint32_t x, uint32_t y) {
    uint32_t p = x * y;
    asm volatile("" : "+v"(p));
    return p;
}

template <int FT, int P>
__global__ __launch_bounds__(kBlock) void hist_era_kernel(HistArgs a) {
    static_assert(FT % P == 0, "feature tile must hold whole groups");
    constexpr int G = FT / P;  // atomic groups (single features or feature pairs) per tile
    extern __shared__ unsigned long long lds[];
    const int Ua = a.st->u_active[a.depth];
    if (Ua <= 0) return;
    const int nb = a.nb;
    const int cells_node = (P == 3) ? nb * nb * nb : (P == 2) ? nb * nb : nb;  // joint cells/node
    const int C = 1 << a.clog2;
    const int UT = a.node_tile;                      // nodes held in LDS per work item
    const int words_group = UT * cells_node * C;     // LDS words per group
    const float gmax = __uint_as_float(a.st->gmax_bits);
    int ex = 0;
    (void)frexpf(gmax, &ex);
    // scale 2^sh with max|g| * 2^sh < 2^30; capped so that 2^sh stays a finite float
    const int sh = (gmax > 0.f) ? min(kGradScaleLog2 - ex, 127) : 0;
    const float scale = ldexpf(1.0f, sh);
    const uint32_t copy = threadIdx.x & (C - 1);
    const uint32_t bin_shift = (uint32_t)a.clog2 + 3u;  // cell -> byte offset of its C copies

    // Work items (era, feature tile), XCD-aware: item i goes to XCD i % 8, and all tiles of an
    // era share one XCD. The grid is a multiple of 8, so a workgroup's items stay on its XCD;
    // looping lets a workgroup's plane stores drain while it already builds its next item.
    const int per_era = a.ntiles * a.node_tiles;
    const int n_items = ((a.E + 7) / 8) * 8 * per_era;
    for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
        const int xcd = item & 7;
        const int i = item >> 3;
        const int era = (i / per_era) * 8 + xcd;
        const int rem_i = i - (i / per_era) * per_era;
        const int tile = rem_i / a.node_tiles;
        const int u0 = (rem_i - tile * a.node_tiles) * UT;  // first node of this item
        const int Un = min(UT, Ua - u0);                    // its nodes, UT or fewer
        const int k0 = tile * FT;
        const int nf = min(FT, a.K - k0);
        if (era >= a.E || nf <= 0 || Un <= 0) continue;  // uniform over the workgroup

        const int ng = (nf + P - 1) / P;
        const int words = ng * words_group;
        __syncthreads();  // the previous item's flush is done with the LDS
        for (int x = threadIdx.x; x < words; x += kBlock) lds[x] = 0ull;

        const int r0 = a.era_off[era];
        const int r1 = a.era_off[era + 1];
        const int a0 = r0 & ~3;

        const uint8_t* col[FT];
    #pragma unroll
        for (int kk = 0; kk < FT; ++kk) {
            const int kq = k0 + (kk < nf ? kk : nf - 1);
            col[kk] = a.bins + (int64_t)a.feats[kq] * a.ld;
        }
        __syncthreads();

        char* lds_bytes = reinterpret_cast<char*>(lds);
        const uint32_t cells_c = (uint32_t)(cells_node * C);
        // Software pipeline: the next pass's loads are in flight while this pass does its
        // atomics. Columns past the tile's last feature alias that feature (always in bounds);
        // their groups add into LDS that the flush never reads. A lane with no rows in the era
        // loads its first position (in bounds) and its rows fail the range check. Offsets are
        // 32-bit (ld * F < 2^32 is not needed: columns are addressed from their own base).
        constexpr int kStride = kBlock * 4;
        int c = a0 + (int)threadIdx.x * 4;
        uint32_t w[FT];
        uint2 nn;
        float4 gg;
        {
            const uint32_t cl = (uint32_t)(c < r1 ? c : a0);
    #pragma unroll
            for (int kk = 0; kk < FT; ++kk)
                w[kk] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(col[kk] + cl));
            nn = *reinterpret_cast<const uint2*>(a.nid + cl);
            gg = *reinterpret_cast<const float4*>(a.grad + cl);
        }
        for (; c < r1; c += kStride) {
            // Unconditional loads keep the wait counts exact (a branch around them makes the
            // compiler wait for everything): a lane's last pass re-reads offset 0 of each array,
            // one hot line, and never uses the values.
            const int cn = c + kStride;
            const uint32_t on = (uint32_t)(cn < r1 ? cn : 0);
            uint32_t wn[FT];
    #pragma unroll
            for (int kk = 0; kk < FT; ++kk)
                wn[kk] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(col[kk] + on));
            const uint2 nnn = *reinterpret_cast<const uint2*>(a.nid + on);
            const float4 ggn = *reinterpret_cast<const float4*>(a.grad + on);
            const uint32_t n4[4] = {nn.x & 0xffffu, nn.x >> 16, nn.y & 0xffffu, nn.y >> 16};
            const float g4[4] = {gg.x, gg.y, gg.z, gg.w};
            uint32_t base[4];  // byte offset of (node, cell 0, this lane's copy) in a group's block
            unsigned long long qv[4];
            uint32_t keep = 0u;  // 0xff in byte j iff row c+j is counted; other bytes read as bin 0
    #pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int r = c + j;
                const uint32_t nl = n4[j] - (uint32_t)u0;  // node within the item's tile
                const bool ok = (r >= r0) && (r < r1) && (nl < (uint32_t)Un);
                const uint32_t nj = ok ? nl : 0u;
                base[j] = (__umul24(nj, cells_c) + copy) * 8u;  // nj < 2^16, cells_c < 2^24
                const long long q = (long long)__float2int_rn(g4[j] * scale);
                qv[j] = ok ? (((unsigned long long)q << kCountBits) + 1ull) : 0ull;
                keep |= ok ? (0xffu << (8 * j)) : 0u;
            }
            if (keep != 0u) {  // lanes without a counted row skip the atomics
    #pragma unroll
                for (int gi = 0; gi < G; ++gi) {
                    const int kk = gi * P;
                    char* hk = lds_bytes + (uint32_t)(gi * words_group) * 8u;
                    uint32_t wk;
                    // The products stay apart from the adds (mul_sep): fused into v_mad_u64_u32,
                    // the 64-bit addend's unused high half may alias a register of the next
                    // pass's loads and make the atomics wait for them.
                    if (P == 3) {
                        // (b1 * nb + b2) * nb + b3 <= nb^3 - 1 <= 215 for nb <= 6: every partial
                        // result stays below 256, so no byte carries into the next row's byte
                        const uint32_t w2 = (kk + 1 < nf) ? w[kk + 1] : 0u;
                        const uint32_t w3 = (kk + 2 < nf) ? w[kk + 2] : 0u;
                        const uint32_t t = mul_sep(w[kk] & keep, (uint32_t)nb) + (w2 & keep);
                        wk = mul_sep(t, (uint32_t)nb) + (w3 & keep);
                    } else if (P == 2) {
                        // joint index per byte: b1 * nb + b2 <= 255 (no carry between bytes);
                        // a lone last feature pairs with bin 0
                        const uint32_t w2 = (kk + 1 < nf) ? w[kk + 1] : 0u;
                        wk = mul_sep(w[kk] & keep, (uint32_t)nb) + (w2 & keep);
                    } else {
                        wk = w[kk] & keep;
                    }
    #pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint32_t boff = ((wk >> (8 * j)) & 0xffu) << bin_shift;
                        atomicAdd(reinterpret_cast<unsigned long long*>(hk + base[j] + boff), qv[j]);
                    }
                }
            }
    #pragma unroll
            for (int kk = 0; kk < FT; ++kk) w[kk] = wn[kk];
            nn = nnn;
            gg = ggn;
        }
        __syncthreads();

        // Flush. (1) Fold the C copies of every cell into copy 0 (all threads).
        const int cells_total = ng * UT * cells_node;
        if (C > 1) {
            for (int x = threadIdx.x; x < cells_total; x += kBlock) {
                unsigned long long* cp = lds + (int64_t)x * C;
                unsigned long long tot = 0ull;
                for (int cc = 0; cc < C; ++cc) tot += cp[cc];
                cp[0] = tot;
            }
            __syncthreads();
        }
        // (2) Output element (node u, feature kk, bin bb) of the prefix planes, with bb the fastest
        // index: a node's [nf][nb] output run is contiguous, so consecutive threads store
        // consecutive addresses. Each element is the exact integer prefix (count | fixed-point
        // grad) over the feature's bins 0..bb, converted once: the count exactly, the grad as the
        // float32 rounding of the exact sum.
        const double inv_scale = ldexp(1.0, -sh);
        if (P == 1) {
            // single features own their cells: prefix them in place, one thread per (node, feature)
            for (int p = threadIdx.x; p < nf * Un; p += kBlock) {
                const int u = p / nf;
                const int kk = p - u * nf;
                unsigned long long* hc = lds + ((int64_t)kk * words_group + (int64_t)u * cells_node * C);
                unsigned long long run = 0ull;
                for (int bb = 0; bb < nb; ++bb) {
                    run += hc[bb * C];
                    hc[bb * C] = run;
                }
            }
            __syncthreads();
        }
        const int run_len = nf * nb;
        const int items = Un * run_len;
        // marginal of element (u, kk, bb) alone (P == 1: the prefix, already in place)
        auto marginal = [&](int it, bool prefix) -> unsigned long long {
            const int u = it / run_len;
            const int rem = it - u * run_len;
            const int kk = rem / nb;
            const int bb = rem - kk * nb;
            const int gi = kk / P;
            const int side = kk - gi * P;  // which feature of the group (b1, b2, b3)
            const unsigned long long* hc =
                lds + ((int64_t)gi * words_group + (int64_t)u * cells_node * C);
            const int b_lo = prefix ? 0 : bb;
            unsigned long long tot = 0ull;
            if (P == 3) {
                const int nb2 = nb * nb;
                const int stride = side == 0 ? nb2 : (side == 1 ? nb : 1);
                const int s1 = side == 0 ? nb : nb2;   // stride of the first other feature
                const int s2 = side == 2 ? nb : 1;     // stride of the second other feature
                for (int b = b_lo; b <= bb; ++b)
                    for (int o1 = 0; o1 < nb; ++o1)
                        for (int o2 = 0; o2 < nb; ++o2) tot += hc[(b * stride + o1 * s1 + o2 * s2) * C];
            } else if (P == 2) {
                for (int b = b_lo; b <= bb; ++b)
                    for (int o = 0; o < nb; ++o)
                        tot += hc[(side == 0 ? (b * nb + o) : (o * nb + b)) * C];
            } else {
                tot = hc[bb * C];
            }
            return tot;
        };
        auto emit = [&](int it, unsigned long long tot) {
            const int u = it / run_len;
            const int rem = it - u * run_len;
            const uint32_t cnt = (uint32_t)(tot & ((1ull << kCountBits) - 1ull));
            const long long Q = ((long long)(tot - cnt)) >> kCountBits;
            const int64_t o = ((int64_t)era * a.U + u0 + u) * a.K * nb + (int64_t)k0 * nb + rem;
            a.out_cnt[o] = (int32_t)cnt;
            a.out_g[o] = (float)((double)Q * inv_scale);
        };
        constexpr int kMaxItems = 16;  // marginals a thread holds in registers
        if (P == 1) {
            for (int it = threadIdx.x; it < items; it += kBlock) emit(it, marginal(it, false));
        } else if (items <= kMaxItems * kBlock) {
            // marginals into registers, then compact them over the (no longer needed) joint cells
            // and prefix from there: nb reads per element instead of (bb + 1) * nb
            unsigned long long m[kMaxItems];
    #pragma unroll
            for (int i = 0; i < kMaxItems; ++i) {
                const int it = (int)threadIdx.x + i * kBlock;
                m[i] = (it < items) ? marginal(it, false) : 0ull;
            }
            __syncthreads();
    #pragma unroll
            for (int i = 0; i < kMaxItems; ++i) {
                const int it = (int)threadIdx.x + i * kBlock;
                if (it < items) lds[it] = m[i];
            }
            __syncthreads();
            for (int it = threadIdx.x; it < items; it += kBlock) {
                const int bb = (it % run_len) % nb;
                unsigned long long tot = 0ull;
                for (int b = it - bb; b <= it; ++b) tot += lds[b];
                emit(it, tot);
            }
        } else {
            for (int it = threadIdx.x; it < items; it += kBlock) emit(it, marginal(it, true));
        }
    }  // work items
}

template <int FT, int P>
hipError_t launch_ft(const HistArgs& a, int grid, size_t lds_bytes, hipStream_t s) {
    const void* fn = reinterpret_cast<const void*>(&hist_era_kernel<FT, P>);
    if (lds_bytes > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds_bytes);
        if (e != hipSuccess) return e;
    }
    // as many workgroups as are resident at once (times a.rounds), a multiple of 8
    if (a.resident_cus > 0) {
        int per_cu = 0;
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kBlock, lds_bytes);
        if (e != hipSuccess) return e;
        const int64_t want = (int64_t)std::max(1, per_cu) * a.resident_cus * std::max(1, a.rounds);
        grid = (int)std::max<int64_t>(8, std::min<int64_t>(grid, want) / 8 * 8);
    }
    hipLaunchKernelGGL((hist_era_kernel<FT, P>), dim3(grid), dim3(kBlock), lds_bytes, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_hist(const HistArgs& a, int pairs, int grid, size_t lds_bytes, hipStream_t s) {
    if (pairs == 3) {
        switch (a.ftile) {
            case 3: return launch_ft<3, 3>(a, grid, lds_bytes, s);
            case 6: return launch_ft<6, 3>(a, grid, lds_bytes, s);
            case 12: return launch_ft<12, 3>(a, grid, lds_bytes, s);
            default: return hipErrorInvalidValue;
        }
    }
    if (pairs == 2) {
        switch (a.ftile) {
            case 2: return launch_ft<2, 2>(a, grid, lds_bytes, s);
            case 4: return launch_ft<4, 2>(a, grid, lds_bytes, s);
            case 8: return launch_ft<8, 2>(a, grid, lds_bytes, s);
            case 16: return launch_ft<16, 2>(a, grid, lds_bytes, s);
            case 32: return launch_ft<32, 2>(a, grid, lds_bytes, s);
            default: return hipErrorInvalidValue;
        }
    }
    switch (a.ftile) {
        case 1: return launch_ft<1, 1>(a, grid, lds_bytes, s);
        case 2: return launch_ft<2, 1>(a, grid, lds_bytes, s);
        case 4: return launch_ft<4, 1>(a, grid, lds_bytes, s);
        case 8: return launch_ft<8, 1>(a, grid, lds_bytes, s);
        case 16: return launch_ft<16, 1>(a, grid, lds_bytes, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace pb
