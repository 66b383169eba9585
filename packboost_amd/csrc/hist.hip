// Kernel 1 — per-(era, node, feature, bin) count/grad histogram over column-major uint8 bins.
//
// Reference semantics: frontier_cpu.cpp:261-321 builds, for each sampled feature,
// count[n][e][b] (int64) and grad[n][e][b] (float32, summed in row order), then a float32
// running sum over bins gives prefix[b < nb-1] and the era total. This kernel produces the
// same prefix/total planes for all sampled features of a depth at once.
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
//  * Joint bins (P = 2, for nb <= 16): the two features of a pair share one atomic on the
//    joint cell (b1 * nb + b2). b1 * nb + b2 <= 255, so the joint index of 4 rows comes
//    from a single 32-bit multiply-add of the two packed bin dwords. The flush recovers both
//    marginals by integer sums over the other feature's bins, so the histogram is exactly
//    the one-feature-per-atomic result with half the LDS atomics.
//  * The histogram is replicated `C` times in LDS, interleaved per word, and lane l adds
//    into copy l % C: with C = 32 the 32 lanes an LDS cycle serves for 64-bit operands land in
//    distinct 8-byte slots, so same-cell rows never serialise (measured on gfx950: 16 copies
//    still conflict). The host trades C against features per workgroup under an LDS budget.
//  * Lanes whose 4 rows all lie outside the era (or in no active node) skip their atomics.
//  * blockIdx -> (era, tile) is XCD-aware: the 8 XCDs receive blocks round-robin, so all
//    feature tiles of one era run on the same XCD and share the era's row state in its L2.
#include "pb_internal.h"

namespace pb {
namespace {

template <int FT, int P>
__global__ __launch_bounds__(kBlock) void hist_era_kernel(HistArgs a) {
    static_assert(FT % P == 0, "feature tile must hold whole groups");
    constexpr int G = FT / P;  // atomic groups (single features or feature pairs) per tile
    extern __shared__ unsigned long long lds[];
    const int b = blockIdx.x;
    const int xcd = b & 7;
    const int i = b >> 3;
    const int era = (i / a.ntiles) * 8 + xcd;
    const int tile = i - (i / a.ntiles) * a.ntiles;
    if (era >= a.E) return;
    const int Ua = a.st->u_active[a.depth];
    if (Ua <= 0) return;
    const int k0 = tile * FT;
    const int nf = min(FT, a.K - k0);
    if (nf <= 0) return;

    const int nb = a.nb;
    const int cells_node = (P == 2) ? nb * nb : nb;  // joint cells per node
    const int C = 1 << a.clog2;
    const int words_group = a.U * cells_node * C;    // LDS words per group
    const int ng = (nf + P - 1) / P;
    const int words = ng * words_group;
    for (int x = threadIdx.x; x < words; x += kBlock) lds[x] = 0ull;

    const float gmax = __uint_as_float(a.st->gmax_bits);
    int ex = 0;
    (void)frexpf(gmax, &ex);
    // scale 2^sh with max|g| * 2^sh < 2^30; capped so that 2^sh stays a finite float
    const int sh = (gmax > 0.f) ? min(kGradScaleLog2 - ex, 127) : 0;
    const float scale = ldexpf(1.0f, sh);

    const int r0 = a.era_off[era];
    const int r1 = a.era_off[era + 1];
    const int a0 = r0 & ~3;
    const uint32_t copy = threadIdx.x & (C - 1);
    const uint32_t bin_shift = (uint32_t)a.clog2 + 3u;  // cell -> byte offset of its C copies

    const uint8_t* col[FT];
#pragma unroll
    for (int kk = 0; kk < FT; ++kk) {
        const int kq = k0 + (kk < nf ? kk : nf - 1);
        col[kk] = a.bins + (int64_t)a.feats[kq] * a.ld;
    }
    __syncthreads();

    char* lds_bytes = reinterpret_cast<char*>(lds);
    for (int c = a0 + (int)threadIdx.x * 4; c < r1; c += kBlock * 4) {
        uint32_t w[FT];
#pragma unroll
        for (int kk = 0; kk < FT; ++kk) {
            if (kk < nf) w[kk] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(col[kk] + c));
        }
        const uint2 nn = *reinterpret_cast<const uint2*>(a.nid + c);
        const float4 gg = *reinterpret_cast<const float4*>(a.grad + c);
        const uint32_t n4[4] = {nn.x & 0xffffu, nn.x >> 16, nn.y & 0xffffu, nn.y >> 16};
        const float g4[4] = {gg.x, gg.y, gg.z, gg.w};
        uint32_t base[4];  // byte offset of (node, cell 0, this lane's copy) in a group's block
        unsigned long long qv[4];
        uint32_t keep = 0u;  // 0xff in byte j iff row c+j is counted; other bytes read as bin 0
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int r = c + j;
            const bool ok = (r >= r0) && (r < r1) && (n4[j] < (uint32_t)Ua);
            base[j] = (ok ? (n4[j] * (uint32_t)(cells_node * C) + copy) : copy) * 8u;
            const long long q = (long long)__float2int_rn(g4[j] * scale);
            qv[j] = ok ? (((unsigned long long)q << kCountBits) + 1ull) : 0ull;
            keep |= ok ? (0xffu << (8 * j)) : 0u;
        }
        if (keep == 0u) continue;  // no counted row in this lane
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            const int kk = gi * P;
            if (kk < nf) {
                char* hk = lds_bytes + (uint32_t)(gi * words_group) * 8u;
                uint32_t wk;
                if (P == 2) {
                    // joint index per byte: b1 * nb + b2 <= 255 (no carry between bytes);
                    // a lone last feature pairs with bin 0
                    const uint32_t w2 = (kk + 1 < nf) ? w[kk + 1] : 0u;
                    wk = (w[kk] & keep) * (uint32_t)nb + (w2 & keep);
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
    }
    __syncthreads();

    // Flush. (1) Fold the C copies of every cell into copy 0 (all threads).
    const int cells_total = ng * a.U * cells_node;
    if (C > 1) {
        for (int x = threadIdx.x; x < cells_total; x += kBlock) {
            unsigned long long* cp = lds + (int64_t)x * C;
            unsigned long long tot = 0ull;
            for (int cc = 0; cc < C; ++cc) tot += cp[cc];
            cp[0] = tot;
        }
        __syncthreads();
    }
    // (2) One thread per (node, feature): marginal per bin (joint cells summed over the pair's
    // other feature), decoded count / fixed-point grad, float32 running sums (prefix, total).
    const double inv_scale = ldexp(1.0, -sh);
    const int pairs = nf * Ua;
    for (int p = threadIdx.x; p < pairs; p += kBlock) {
        const int u = p / nf;
        const int kk = p - u * nf;
        const int gi = kk / P;
        const int side = kk - gi * P;  // 0: first feature of the pair (b1), 1: second (b2)
        const unsigned long long* hc =
            lds + ((int64_t)gi * words_group + (int64_t)u * cells_node * C);
        const int64_t ob = (((int64_t)era * a.U + u) * a.K + (k0 + kk)) * nb;
        int32_t rc = 0;
        float rg = 0.0f;
        for (int bb = 0; bb < nb; ++bb) {
            unsigned long long tot = 0ull;
            if (P == 2) {
                for (int o = 0; o < nb; ++o) {
                    const int cell = side == 0 ? (bb * nb + o) : (o * nb + bb);
                    tot += hc[cell * C];
                }
            } else {
                tot = hc[bb * C];
            }
            const uint32_t cnt = (uint32_t)(tot & ((1ull << kCountBits) - 1ull));
            const long long Q = ((long long)(tot - cnt)) >> kCountBits;
            const float gb = (float)((double)Q * inv_scale);
            rc += (int32_t)cnt;
            rg = rg + gb;
            a.out_cnt[ob + bb] = rc;
            a.out_g[ob + bb] = rg;
        }
    }
}

template <int FT, int P>
hipError_t launch_ft(const HistArgs& a, int grid, size_t lds_bytes, hipStream_t s) {
    if (lds_bytes > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&hist_era_kernel<FT, P>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds_bytes);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((hist_era_kernel<FT, P>), dim3(grid), dim3(kBlock), lds_bytes, s, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_hist(const HistArgs& a, int pairs, int grid, size_t lds_bytes, hipStream_t s) {
    if (pairs == 2) {
        switch (a.ftile) {
            case 2: return launch_ft<2, 2>(a, grid, lds_bytes, s);
            case 4: return launch_ft<4, 2>(a, grid, lds_bytes, s);
            case 8: return launch_ft<8, 2>(a, grid, lds_bytes, s);
            case 16: return launch_ft<16, 2>(a, grid, lds_bytes, s);
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
