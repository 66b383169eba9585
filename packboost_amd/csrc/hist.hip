// Kernel 1 — per-(era, node, feature, bin) count/grad histogram over column-major uint8 bins.
//
// Reference semantics: frontier_cpu.cpp:261-321 builds, for each sampled feature,
// count[n][e][b] (int64) and grad[n][e][b] (float32, summed in row order), then a float32
// running sum over bins gives prefix[b < nb-1] and the era total. This kernel produces the
// same prefixes for all sampled features of a depth at once, plus one era total per node
// (the compact planes of pb_internal.h); the counts are exact and the grad prefixes are exact
// fixed-point sums rounded once to float32, so the total is the same for every feature.
//
// Design (gfx950):
//  * One workgroup owns one (era, feature tile). Rows are era-major, so an era is a
//    contiguous byte range of every feature column: loads are coalesced dwords (4 rows per
//    lane in uint8 columns, 8 in nibble columns) and no global atomics are needed.
//  * Each lane forms the row state of its rows (LDS byte offset of the row's node and the
//    packed value below) once per pass and reuses it across all features of the tile.
//  * One 64-bit LDS atomic carries (fixed-point grad << 16) + 1, so the count (low 16 bits)
//    and the grad sum (high 48 bits) accumulate in a single ds_add_u64. Integer addition is
//    order-independent, so the result is deterministic run to run; grad is quantised as
//    round(g * 2^s), with s set per round and era so that the era's sum of |q| stays below
//    2^45 (era_grad_scale), far finer than float32 rounding of the reference's row-order sum.
//    (A per-round 8-byte addend array instead of the 4-byte gradient measured slower: the
//    row-side loads are re-read by every feature tile.)
//  * Joint bins (P = 2 for nb <= 16, P = 3 for nb <= 6): the P features of a group share one
//    atomic on the joint cell (b1 * nb + b2, or (b1 * nb + b2) * nb + b3). The joint index is
//    below 256, so for 4 rows it comes from byte-wise multiply-adds of the packed bin dwords.
//    The flush recovers every marginal by integer sums over the other features' bins, so the
//    histogram is exactly the one-feature-per-atomic result with 1/P of the LDS atomics.
//  * The histogram is replicated `C` times in LDS, interleaved per word, and lane l adds into
//    copy l % C. gfx950 serves a wave's 64-bit LDS atomics in 32-lane halves; lanes of a half
//    that share a copy collide when their cells alias one bank (measured: about 6.5 cycles per
//    conflict-free wave-level ds_add_u64, 10.6 at C = 8 over 25 joint cells, 6.7 at C >= 16).
//    Copies cost LDS (occupancy) and a fold per era, and with eras of a few thousand rows the
//    kernel waits on memory more than on the LDS, so the host keeps the LDS per workgroup
//    small and takes the copies that fit.
//  * Nibble layout (NIB, nb <= 16): every 4 bytes of a column hold 8 rows, byte j = row j in
//    the low nibble and row j + 4 in the high one, so one dword load brings 8 rows and
//    (w & 0x0f0f0f0f), ((w >> 4) & 0x0f0f0f0f) are the byte-per-row dwords of rows 0-3 and
//    4-7: the bin bytes read per depth halve and the per-quad code is the uint8 one.
//  * Lanes whose 4 rows all lie outside the era (or in no active node) skip their atomics.
//  * blockIdx -> (era, tile) is XCD-aware: the 8 XCDs receive blocks round-robin, so all
//    feature tiles of one era run on the same XCD and share the era's row state in its L2.
#include <algorithm>
#include <type_traits>

#include "pb_internal.h"

namespace pb {
namespace {

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// floor(n / d) for n, d < 2^16 as one multiply-high by m = ceil(2^32 / d): with e = m - 2^32 / d
// in [0, 1), n * m / 2^32 = n / d + n * e / 2^32 and n * e / 2^32 < 1 / d, so the floor is exact.
// d == 1 (m would be 2^32) returns n.
struct DivU16 {
    uint32_t m;
    bool one;
    __device__ explicit DivU16(int d)
        : m((uint32_t)(0xFFFFFFFFull / (unsigned long long)d + 1ull)), one(d == 1) {}
    __device__ uint32_t div(uint32_t n) const { return one ? n : __umulhi(n, m); }
};

// Byte-wise x * m + y for four bytes at once, when every byte's result stays below 256: in
// each 16-bit half (hi * 256 + lo) * m + (yh * 256 + yl) = (hi * m + yh) * 256 + (lo * m + yl)
// with no carry out of the low byte, so one full-rate packed 16-bit multiply-add
// (v_pk_mad_u16) replaces a quarter-rate 32-bit multiply.
__device__ __forceinline__ uint32_t mad_bytes(uint32_t x, uint32_t m, uint32_t y) {
    const u16x2 a = __builtin_bit_cast(u16x2, x);
    const u16x2 b = __builtin_bit_cast(u16x2, y);
    const u16x2 mm = {(unsigned short)m, (unsigned short)m};
    return __builtin_bit_cast(uint32_t, (u16x2)(a * mm + b));
}

// Waves per SIMD: six (at most 80 VGPRs) for more loads in flight per CU (measured 6% faster
// over the depths of a 2.4M-row, 5-bin round than the unconstrained 4-wave build); five for the
// 16-feature pair tile (measured); four for the 16-feature single-feature tile, which spills at
// 80 VGPRs and fits 92 without spills (its 128-bin depth measured 7% faster that way), and for
// the 32-feature pair tile (chosen only when the feature tile is forced), which spills at 96.
template <int FT, int P>
constexpr int hist_waves_per_eu() {
    return (P == 2 && FT >= 32) ? 4 : (P == 2 && FT >= 16) ? 5 : (P == 1 && FT >= 16) ? 4 : 6;
}

template <int FT, int P, bool NIB, int BS>
__global__ __launch_bounds__(BS) __attribute__((amdgpu_waves_per_eu(hist_waves_per_eu<FT, P>())))
void hist_era_kernel(HistArgs a, const int4* __restrict__ seg_info, const int32_t* __restrict__ feats) {
    // seg_info / feats are separate restrict arguments (the same pointers as in `a`): nothing the
    // kernel writes can alias them, so their workgroup-uniform loads go through the scalar cache
    static_assert(FT % P == 0, "feature tile must hold whole groups");
    constexpr int RL = NIB ? 8 : 4;  // rows per lane per pass (rows per bin dword)
    constexpr int G = FT / P;  // atomic groups (single features or feature pairs) per tile
    extern __shared__ unsigned long long lds[];
    const int Ua = a.st->u_active[a.depth];
    if (Ua <= 0) return;
    const int nb = a.nb;
    const int cells_node = (P == 3) ? nb * nb * nb : (P == 2) ? nb * nb : nb;  // joint cells/node
    const int C = 1 << a.clog2;
    const int UT = a.node_tile;                      // nodes held in LDS per work item
    const int words_group = hist_group_words(UT * cells_node * C, P, nb, C, G);  // LDS words per group
    const uint32_t copy = threadIdx.x & (C - 1);
    const uint32_t bin_shift = (uint32_t)a.clog2 + 3u;  // cell -> byte offset of its C copies

    // Work items (segment, feature tile), XCD-aware: item i goes to XCD i % 8, and all tiles of
    // a segment share one XCD. A segment is an era, or part of one above the host's segment
    // size. The grid is a multiple of 8, so a workgroup's items stay on its XCD; looping lets a
    // workgroup's plane stores drain while it already builds its next item.
    const int per_era = a.ntiles * a.node_tiles;
    const int n_items = ((a.S + 7) / 8) * 8 * per_era;
    for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
        const int xcd = item & 7;
        const int i = item >> 3;
        const int seg = (i / per_era) * 8 + xcd;
        const int rem_i = i - (i / per_era) * per_era;
        const int tile = rem_i / a.node_tiles;
        const int u0 = (rem_i - tile * a.node_tiles) * UT;  // first node of this item
        const int Un = min(UT, Ua - u0);                    // its nodes, UT or fewer
        const int k0 = tile * FT;
        const int nf = min(FT, a.K - k0);
        if (seg >= a.S || nf <= 0 || Un <= 0) continue;  // uniform over the workgroup
        const int4 si = seg_info[seg];  // one load: rows, era and slot of the segment
        const int era = si.z;
        const int slot = si.w;  // >= 0: add into the era's sums
        const int sh = a.sh_era[era];  // rows add round(grad * 2^sh)
        const float scale = ldexpf(1.0f, sh);

        const int ng = (nf + P - 1) / P;
        const int words = ng * words_group;
        __syncthreads();  // the previous item's flush is done with the LDS
        for (int x = threadIdx.x; x < words; x += BS) lds[x] = 0ull;

        const int r0 = si.x;
        const int r1 = si.y;
        const int a0 = r0 & ~(RL - 1);

        const uint8_t* col[FT];
    #pragma unroll
        for (int kk = 0; kk < FT; ++kk) {
            const int kq = k0 + (kk < nf ? kk : nf - 1);
            col[kk] = a.bins + (int64_t)feats[kq] * a.ld;
        }
        __syncthreads();

        char* lds_bytes = reinterpret_cast<char*>(lds);
        const uint32_t cells_c8 = (uint32_t)(cells_node * C) * 8u;  // bytes per node
        const uint32_t copy8 = copy * 8u;
        // Software pipeline: the next pass's loads are in flight while this pass does its
        // atomics. Columns past the tile's last feature alias that feature (always in bounds);
        // their groups add into LDS that the flush never reads. A lane with no rows in the era
        // loads its first position (in bounds) and its rows fail the range check. Offsets are
        // 32-bit (ld * F < 2^32 is not needed: columns are addressed from their own base).
        constexpr int kStride = BS * RL;
        constexpr uint32_t kByteShift = NIB ? 1u : 0u;  // row -> byte offset of its bin dword
        int c = a0 + (int)threadIdx.x * RL;
        uint32_t w[FT];
        uint4 nn;   // node ids of the lane's rows (.x, .y used when RL == 4)
        float4 gg[RL / 4];
        {
            const uint32_t cl = (uint32_t)(c < r1 ? c : a0);
    #pragma unroll
            for (int kk = 0; kk < FT; ++kk)
                w[kk] = __builtin_nontemporal_load(
                    reinterpret_cast<const uint32_t*>(col[kk] + (cl >> kByteShift)));
            if (NIB) {
                nn = *reinterpret_cast<const uint4*>(a.nid + cl);
            } else {
                const uint2 n2 = *reinterpret_cast<const uint2*>(a.nid + cl);
                nn = make_uint4(n2.x, n2.y, 0u, 0u);
            }
    #pragma unroll
            for (int h = 0; h < RL / 4; ++h) gg[h] = *reinterpret_cast<const float4*>(a.grad + cl + 4 * h);
        }
        // One pass over a lane's RL rows from row cc: bins wv, node ids nv and grads gv.
        const uint32_t seg_len = (uint32_t)(r1 - r0);
        auto pass = [&](const uint32_t (&wv)[FT], const uint4& nv, const float4 (&gv)[RL / 4], int cc) {
    #pragma unroll
            for (int h = 0; h < RL / 4; ++h) {  // quads of rows cc + 4h .. cc + 4h + 3
                const uint32_t nq0 = h ? nv.z : nv.x;
                const uint32_t nq1 = h ? nv.w : nv.y;
                const uint32_t n4[4] = {nq0 & 0xffffu, nq0 >> 16, nq1 & 0xffffu, nq1 >> 16};
                const float g4[4] = {gv[h].x, gv[h].y, gv[h].z, gv[h].w};
                const uint32_t rq = (uint32_t)(cc + 4 * h - r0);  // first row of the quad, from r0
                uint32_t base[4];  // byte offset of (node, cell 0, this lane's copy) in a group's block
                unsigned long long qv[4];
                uint32_t keep = 0u;  // uint8 bins: 0xff in byte j iff row cc+4h+j is counted
    #pragma unroll
                for (int j = 0; j < 4; ++j) {
                    // row cc+4h+j is counted: in the segment and in one of the item's nodes (each
                    // test one unsigned compare; the flag stays a lane mask, no branch per row)
                    const uint32_t nj = n4[j] - (uint32_t)u0;  // node within the tile
                    const bool ok = (nj < (uint32_t)Un) & (rq + (uint32_t)j < seg_len);
                    base[j] = __umul24(ok ? nj : 0u, cells_c8) + copy8;  // nj < 2^16, cells_c8 < 2^24
                    // (q << 16) + 1 with q = round(g * 2^sh) (grad_addend), computed for every row
                    // and masked to 0 if not counted
                    qv[j] = grad_addend(g4[j], scale) & (0ull - (unsigned long long)ok);
                    if (!NIB) keep |= ok ? (0xffu << (8 * j)) : 0u;
                }
                // some row of the quad is counted (a counted row's addend has its low bit set)
                const bool any = ((uint32_t)(qv[0] | qv[1] | qv[2] | qv[3]) & 1u) != 0u;
                // this quad's byte-per-row bin dwords. uint8 columns: bytes of uncounted rows are
                // masked to bin 0 (the caller's padding rows may hold anything). Nibble columns:
                // every row holds a valid bin (rows past N are zero, pb_pack_bins4), and uncounted
                // rows add zero, so no mask is needed.
                const uint32_t kmask = NIB ? 0xffffffffu : keep;
                auto wq = [&](int kk) -> uint32_t {
                    return NIB ? ((wv[kk] >> (4 * h)) & 0x0f0f0f0fu) : (wv[kk] & kmask);
                };
                if (any) {  // lanes without a counted row skip the atomics
    #pragma unroll
                    for (int gi = 0; gi < G; ++gi) {
                        const int kk = gi * P;
                        char* hk = lds_bytes + (uint32_t)(gi * words_group) * 8u;
                        // Joint index per byte, below 256 so no byte carries into the next row's:
                        // (b1 * nb + b2) * nb + b3 <= nb^3 - 1 <= 215 for nb <= 6, b1 * nb + b2 <=
                        // 255 for nb <= 16. A group's partners past the tile's last feature read
                        // that feature's column (valid bins); the flush sums the partners out of
                        // the marginals of the real features.
                        uint32_t wk;
                        if (P == 3)
                            wk = mad_bytes(mad_bytes(wq(kk), (uint32_t)nb, wq(kk + 1)), (uint32_t)nb, wq(kk + 2));
                        else if (P == 2)
                            wk = mad_bytes(wq(kk), (uint32_t)nb, wq(kk + 1));
                        else
                            wk = wq(kk);
    #pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const uint32_t boff = ((wk >> (8 * j)) & 0xffu) << bin_shift;
                            atomicAdd(reinterpret_cast<unsigned long long*>(hk + base[j] + boff), qv[j]);
                        }
                    }
                }
            }  // quads
        };
        // The pass's loads for row cn. Unconditional loads keep the wait counts exact (a branch
        // around them makes the compiler wait for everything): a lane past the segment re-reads
        // offset 0 of each array, one hot line, and never uses the values.
        auto load = [&](uint32_t (&wv)[FT], uint4& nv, float4 (&gv)[RL / 4], int cn) {
            const uint32_t on = (uint32_t)(cn < r1 ? cn : 0);
    #pragma unroll
            for (int kk = 0; kk < FT; ++kk)
                wv[kk] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(col[kk] + (on >> kByteShift)));
            if (NIB) {
                nv = *reinterpret_cast<const uint4*>(a.nid + on);
            } else {
                const uint2 n2 = *reinterpret_cast<const uint2*>(a.nid + on);
                nv = make_uint4(n2.x, n2.y, 0u, 0u);
            }
    #pragma unroll
            for (int h = 0; h < RL / 4; ++h) gv[h] = *reinterpret_cast<const float4*>(a.grad + on + 4 * h);
        };
        // Software pipeline, unrolled by two so the two register sets alternate without copies:
        // the next pass's loads are in flight while this pass does its atomics.
        uint32_t w2[FT];
        uint4 nn2;
        float4 gg2[RL / 4];
        for (; c < r1; c += 2 * kStride) {
            load(w2, nn2, gg2, c + kStride);
            pass(w, nn, gg, c);
            if (c + kStride >= r1) break;
            load(w, nn, gg, c + 2 * kStride);
            pass(w2, nn2, gg2, c + kStride);
        }
        __syncthreads();

        // Flush. (1) Fold the C copies of every cell into copy 0. A cell's copies are C adjacent
        // words, so each wave reads 64 consecutive words (64 / C whole cells, no bank conflicts;
        // a thread walking one cell's copies would make all lanes hit one bank), sums every C
        // lanes with DPP row shifts (an inclusive scan inside each 16-lane row, then a row
        // broadcast for C = 32; lanes shifted in from outside a row read 0), so lane C-1 of every
        // C-lane group holds its cell's total, and writes it back to copy 0.
        const int cells_total = ng * UT * cells_node;
        if (C > 1) {
            const int total_words = cells_total * C;
            const int lane = (int)(threadIdx.x & (kWave - 1));
            // four 64-word windows per wave at a time, their reads issued together (each window
            // is written only inside itself, so the reads of the next windows cannot see a write)
            constexpr int kFoldBatch = 4;
            for (int wb0 = (int)(threadIdx.x / kWave) * kWave; wb0 < total_words; wb0 += kFoldBatch * BS) {
                unsigned long long vb[kFoldBatch];
    #pragma unroll
                for (int k = 0; k < kFoldBatch; ++k) {
                    const int wi = wb0 + k * BS + lane;
                    vb[k] = lds[min(wi, total_words - 1)];
                }
    #pragma unroll
                for (int k = 0; k < kFoldBatch; ++k) {
                    const int wi = wb0 + k * BS + lane;
                    unsigned long long v = wi < total_words ? vb[k] : 0ull;
                    v += dpp_u64<0x111>(v);                 // row_shr:1
                    if (C > 2) v += dpp_u64<0x112>(v);      // row_shr:2
                    if (C > 4) v += dpp_u64<0x114>(v);      // row_shr:4
                    if (C > 8) v += dpp_u64<0x118>(v);      // row_shr:8
                    if (C > 16) v += dpp_u64<0x142>(v);     // row_bcast:15 (row r's lane 15 -> row r+1)
                    if ((lane & (C - 1)) == C - 1 && wi < total_words) lds[wi - (C - 1)] = v;
                }
            }
            __syncthreads();
        }
        // (2) Output element (node u, feature kk, bin bb) of the prefix planes, with bb the fastest
        // index: a node's [nf][nb] output run is contiguous, so consecutive threads store
        // consecutive addresses. Each element is the exact integer prefix (count | fixed-point
        // grad) over the feature's bins 0..bb, converted once: the count exactly, the grad as the
        // float32 rounding of the exact sum.
        // A word's grad field w = Q * 2^kCountBits (count bits cleared) as a float: Q * 2^-sh
        // rounded once. |Q| < 2^45, so high half * 2^32 + low half is exact in double (the fma
        // has nothing to round) and the scaling by a power of two is exact: no 64-bit shift.
        const int grad_exp = -kCountBits - sh;
        auto grad_f32 = [&](unsigned long long word) -> float {
            const uint32_t lo = (uint32_t)word & ~((1u << kCountBits) - 1u);
            return (float)ldexp(fma((double)(int32_t)(uint32_t)(word >> 32), 0x1p32, (double)lo), grad_exp);
        };
        // Element it = (u * nf + kk) * nb + bb. Its digits come from two exact multiply-high
        // divisions by the uniform nb and nf (a runtime integer division is a long VALU sequence
        // and the flush decodes every element).
        struct Digits {
            int u, kk, bb;
        };
        const DivU16 div_nb(nb), div_nf(nf);
        auto split = [&](int it) -> Digits {
            const uint32_t q = div_nb.div((uint32_t)it);
            const uint32_t u = div_nf.div(q);
            return Digits{(int)u, (int)(q - u * (uint32_t)nf), (int)((uint32_t)it - q * (uint32_t)nb)};
        };
        if (P == 1 && slot < 0) {
            // single features own their cells: prefix each (node, feature) row of nb cells in
            // place (the count and the fixed-point grad share one integer word, so one integer
            // scan does both)
            if (nb >= 32) {
                // many bins: one wavefront per row, 64 cells per step (a DPP scan inside each
                // 16-lane row, then the row totals broadcast across), the running total carried
                // from step to step; a thread walking a row alone would chain nb dependent LDS
                // round trips
                const int lane = (int)(threadIdx.x & (kWave - 1));
                for (int p = (int)(threadIdx.x / kWave); p < nf * Un; p += BS / kWave) {
                    const int u = (int)div_nf.div((uint32_t)p);
                    const int kk = p - u * nf;
                    unsigned long long* hc = lds + ((int64_t)kk * words_group + (int64_t)u * cells_node * C);
                    // the row's 64-cell steps (NS of them, nb <= 64 * NS) read together; each step
                    // writes only its own cells
                    auto scan_row = [&](auto nsteps) {
                        constexpr int NS = decltype(nsteps)::value;
                        unsigned long long seg[NS];
    #pragma unroll
                        for (int q = 0; q < NS; ++q) seg[q] = hc[min(q * kWave + lane, nb - 1) * C];
                        unsigned long long carry = 0ull;
    #pragma unroll
                        for (int q = 0; q < NS; ++q) {
                            const int b = q * kWave + lane;
                            unsigned long long v = b < nb ? seg[q] : 0ull;
                            v += dpp_u64<0x111>(v);        // row_shr:1
                            v += dpp_u64<0x112>(v);        // row_shr:2
                            v += dpp_u64<0x114>(v);        // row_shr:4
                            v += dpp_u64<0x118>(v);        // row_shr:8: inclusive scan per 16-lane row
                            v += dpp_u64<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
                            v += dpp_u64<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
                            v += carry;
                            if (b < nb) hc[b * C] = v;
                            carry = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), kWave - 1) << 32) |
                                    (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, kWave - 1);
                        }
                    };
                    if (nb <= kWave)
                        scan_row(std::integral_constant<int, 1>{});
                    else if (nb <= 2 * kWave)
                        scan_row(std::integral_constant<int, 2>{});
                    else
                        scan_row(std::integral_constant<int, 4>{});
                }
            } else {
                // few bins: one thread per (node, feature) row
                for (int p = threadIdx.x; p < nf * Un; p += BS) {
                    const int u = (int)div_nf.div((uint32_t)p);
                    const int kk = p - u * nf;
                    unsigned long long* hc = lds + ((int64_t)kk * words_group + (int64_t)u * cells_node * C);
                    unsigned long long run = 0ull;
                    for (int bb = 0; bb < nb; ++bb) {
                        run += hc[bb * C];
                        hc[bb * C] = run;
                    }
                }
            }
            __syncthreads();
        }
        const int items = Un * nf * nb;
        // The thread's element indices below depend only on the thread and nb, so the compiler
        // would hoist their digit divisions out of the item loop and hold them in registers across
        // the row passes; an opaque copy of the thread index keeps them here.
        int tx = (int)threadIdx.x;
        __asm__ volatile("" : "+v"(tx));
        // Sums over one partner's nb bins are read as one batch of W loads (clamped to the last
        // bin, the extra values dropped), so their LDS round trips overlap: the LDS is busy with
        // the other workgroups' atomics, and a dependent read per cell made the flush a chain of
        // nb^(P-1) round trips.
        auto rsum = [&](const unsigned long long* base, int step, auto width) -> unsigned long long {
            constexpr int W = decltype(width)::value;
            unsigned long long v[W];
    #pragma unroll
            for (int o = 0; o < W; ++o) v[o] = base[min(o, nb - 1) * step];
            unsigned long long r = 0ull;
    #pragma unroll
            for (int o = 0; o < W; ++o) r += (o < nb) ? v[o] : 0ull;
            return r;
        };
        // marginal of element (u, kk, bb) alone, or (prefix) its bins 0..bb; P == 1: the prefix,
        // already in place
        auto marginal = [&](const Digits& d, bool prefix) -> unsigned long long {
            const int gi = d.kk / P;
            const int side = d.kk - gi * P;  // which feature of the group (b1, b2, b3)
            const unsigned long long* hc =
                lds + ((int64_t)gi * words_group + (int64_t)d.u * cells_node * C);
            const int bb = d.bb;
            const int b_lo = prefix ? 0 : bb;
            unsigned long long tot = 0ull;
            if (P == 3) {
                const int nb2 = nb * nb;
                const int stride = side == 0 ? nb2 : (side == 1 ? nb : 1);
                const int s1 = side == 0 ? nb : nb2;   // stride of the first other feature
                const int s2 = side == 2 ? nb : 1;     // stride of the second other feature
                for (int b = b_lo; b <= bb; ++b) {
                    if (nb == 5) {
                        // the 25 partner cells of the bin in two batches (15 and 10 reads)
                        // instead of five dependent ones
                        auto batch = [&](auto lo, auto hi) {
                            constexpr int L = decltype(lo)::value, H = decltype(hi)::value;
                            unsigned long long v[(H - L) * 5];
#pragma unroll
                            for (int o1 = L; o1 < H; ++o1)
#pragma unroll
                                for (int o2 = 0; o2 < 5; ++o2)
                                    v[(o1 - L) * 5 + o2] = hc[(b * stride + o1 * s1 + o2 * s2) * C];
#pragma unroll
                            for (int o = 0; o < (H - L) * 5; ++o) tot += v[o];
                        };
                        batch(std::integral_constant<int, 0>{}, std::integral_constant<int, 3>{});
                        batch(std::integral_constant<int, 3>{}, std::integral_constant<int, 5>{});
                        continue;
                    }
                    for (int o1 = 0; o1 < nb; ++o1) {
                        const unsigned long long* base = hc + (b * stride + o1 * s1) * C;
                        tot += (nb <= 4) ? rsum(base, s2 * C, std::integral_constant<int, 4>{})
                                         : rsum(base, s2 * C, std::integral_constant<int, 6>{});
                    }
                }
            } else if (P == 2) {
                const int step = (side == 0 ? 1 : nb) * C;  // the partner's bins
                for (int b = b_lo; b <= bb; ++b) {
                    const unsigned long long* base = hc + (side == 0 ? b * nb : b) * C;
                    tot += (nb <= 4)   ? rsum(base, step, std::integral_constant<int, 4>{})
                           : (nb == 5) ? rsum(base, step, std::integral_constant<int, 5>{})
                           : (nb <= 8) ? rsum(base, step, std::integral_constant<int, 8>{})
                                       : rsum(base, step, std::integral_constant<int, 16>{});
                }
            } else {
                tot = hc[bb * C];
            }
            return tot;
        };
        // compact planes: prefixes t < nb-1 per (node, feature); the era total (bin nb-1) once
        // per node, from the depth's first feature
        const int pt = nb - 1;
        if (slot >= 0) {
            // part of a split era: add this segment's per-bin cells, exact integers, into the
            // era's sums (integer adds: the order of the segments does not matter)
            const int64_t srow0 = ((int64_t)slot * a.acc_U + u0) * a.acc_K + k0;
            for (int it = tx; it < items; it += BS) {
                const Digits d = split(it);
                const unsigned long long m = marginal(d, false);
                const uint32_t cnt = (uint32_t)(m & ((1ull << kCountBits) - 1ull));
                if (cnt == 0u) continue;
                const long long Q = ((long long)(m - cnt)) >> kCountBits;
                const int64_t o = (srow0 + (int64_t)d.u * a.acc_K + d.kk) * nb + d.bb;
                atomicAdd(a.acc_cnt + o, cnt);
                atomicAdd(a.acc_g + o, (unsigned long long)Q);
            }
            continue;
        }
        const int64_t row0 = ((int64_t)era * a.U + u0) * a.K + k0;  // (node u0, feature k0)
        auto emit = [&](const Digits& d, unsigned long long tot) {
            const uint32_t cnt = (uint32_t)(tot & ((1ull << kCountBits) - 1ull));
            const float gs = grad_f32(tot);
            if (d.bb < pt) {
                const int64_t o = (row0 + (int64_t)d.u * a.K + d.kk) * pt + d.bb;
                if (a.out_cnt32)
                    a.out_cnt32[o] = cnt;
                else
                    a.out_cnt[o] = (uint16_t)cnt;
                a.out_g[o] = gs;
            } else if (k0 + d.kk == 0) {
                const int64_t o = (int64_t)era * a.U + u0 + d.u;
                a.out_tot_cnt[o] = (int32_t)cnt;
                a.out_tot_g[o] = gs;
            }
        };
        // 5 bins (config of the 2.4M x 2376 panel): a (node, feature)'s 4 prefixes go out as one
        // 8-byte count store and one 16-byte grad store (the run of 4 is aligned: its element
        // index is a multiple of 4), instead of 8 scalar stores
        const bool vec5 = nb == 5 && !a.out_cnt32 && !(reinterpret_cast<uintptr_t>(a.out_cnt) & 7) &&
                          !(reinterpret_cast<uintptr_t>(a.out_g) & 15);
        auto emit5 = [&](int u, int kk, const unsigned long long (&m)[5]) {
            unsigned long long run = 0ull;
            ushort4 cv;
            float4 gv;
            uint16_t* cp = reinterpret_cast<uint16_t*>(&cv);
            float* gp = reinterpret_cast<float*>(&gv);
    #pragma unroll
            for (int bb = 0; bb < 4; ++bb) {
                run += m[bb];
                const uint32_t cnt = (uint32_t)(run & ((1ull << kCountBits) - 1ull));
                cp[bb] = (uint16_t)cnt;
                gp[bb] = grad_f32(run);
            }
            const int64_t o = (row0 + (int64_t)u * a.K + kk) * 4;
            *reinterpret_cast<ushort4*>(a.out_cnt + o) = cv;
            *reinterpret_cast<float4*>(a.out_g + o) = gv;
            if (k0 + kk == 0) emit(Digits{u, kk, 4}, run + m[4]);
        };
        constexpr int kMaxItems = 8;  // marginals a thread holds in registers
        if (P == 2 && NIB && vec5) {
            // 5 bins, nibble columns: one thread per (node, pair), pairs fastest. It reads the
            // pair's 25 joint cells once, sums the rows of the 5 x 5 block (cell b1 * 5 + b2) into
            // the first feature's marginals and its columns into the second's, and emits both.
            // Consecutive lanes take one node's pairs, so a wavefront's plane stores cover a few
            // whole runs of consecutive features instead of one 8- or 16-byte piece per node;
            // the padded group stride (hist_group_words) keeps their cell reads on distinct LDS
            // banks. A thread per (node, feature) read every cell twice. (The uint8
            // instantiations keep that form: this one spills there at their register budget.)
            // (Tiles of one or two pairs keep nodes fastest: their few groups gain little, and
            // that order keeps the one-pair instantiation within its registers.)
            const DivU16 div_ng(ng), div_un(Un);
            for (int t = tx; t < Un * ng; t += BS) {
                int u, g;
                if (G >= 4) {
                    u = (int)div_ng.div((uint32_t)t);
                    g = t - u * ng;
                } else {
                    g = (int)div_un.div((uint32_t)t);
                    u = t - g * Un;
                }
                const unsigned long long* hc =
                    lds + ((int64_t)g * words_group + (int64_t)u * cells_node * C);
                unsigned long long m0[5], m1[5];
                // the block's rows b1 = 0-2 (15 cells), then 3-4 (10), each as one batch of
                // reads, within the register budget of every pair instantiation
                {
                    unsigned long long v[15];
    #pragma unroll
                    for (int j = 0; j < 15; ++j) v[j] = hc[j * C];
    #pragma unroll
                    for (int b = 0; b < 5; ++b) m1[b] = v[b] + v[5 + b] + v[10 + b];
    #pragma unroll
                    for (int r = 0; r < 3; ++r)
                        m0[r] = v[r * 5] + v[r * 5 + 1] + v[r * 5 + 2] + v[r * 5 + 3] + v[r * 5 + 4];
                }
                {
                    unsigned long long v[10];
    #pragma unroll
                    for (int j = 0; j < 10; ++j) v[j] = hc[(15 + j) * C];
    #pragma unroll
                    for (int b = 0; b < 5; ++b) m1[b] += v[b] + v[5 + b];
    #pragma unroll
                    for (int r = 0; r < 2; ++r)
                        m0[3 + r] = v[r * 5] + v[r * 5 + 1] + v[r * 5 + 2] + v[r * 5 + 3] + v[r * 5 + 4];
                }
                emit5(u, 2 * g, m0);
                if (2 * g + 1 < nf) emit5(u, 2 * g + 1, m1);  // the partner past the tile's end: none
            }
        } else if (P == 2 && nb <= 8) {
            // One thread per (node, feature) of a pair: it reads the pair's nb x nb joint cells
            // once, sums its feature's marginals (side 0 over rows of the cell block, side 1 over
            // columns), and emits the running sums. Every cell is read twice (once per side)
            // instead of once per marginal element and again for its prefix.
            const int ng2 = ng * 2;
            const DivU16 div_ng2(ng2);
            for (int t = tx; t < Un * ng2; t += BS) {
                const int u = (int)div_ng2.div((uint32_t)t);
                const int kk = t - u * ng2;  // feature of the tile: group kk / 2, side kk % 2
                if (kk >= nf) continue;       // the partner past the tile's last feature
                const int side = kk & 1;
                const unsigned long long* hc =
                    lds + ((int64_t)(kk >> 1) * words_group + (int64_t)u * cells_node * C);
                const int s_out = (side ? 1 : nb) * C;  // from one marginal bin to the next
                const int s_in = (side ? nb : 1) * C;   // over the partner's bins
                if (vec5) {  // all 25 cells read as one batch
                    unsigned long long m[5];
    #pragma unroll
                    for (int bb = 0; bb < 5; ++bb)
                        m[bb] = rsum(hc + bb * s_out, s_in, std::integral_constant<int, 5>{});
                    emit5(u, kk, m);
                    continue;
                }
                unsigned long long run = 0ull;
                for (int bb = 0; bb < nb; ++bb) {
                    const unsigned long long* base = hc + bb * s_out;
                    run += (nb <= 4)   ? rsum(base, s_in, std::integral_constant<int, 4>{})
                           : (nb == 5) ? rsum(base, s_in, std::integral_constant<int, 5>{})
                                       : rsum(base, s_in, std::integral_constant<int, 8>{});
                    emit(Digits{u, kk, bb}, run);
                }
            }
        } else if (P == 1) {
            // kEmitBatch elements per thread at a time: their LDS reads first, then the stores
            constexpr int kEmitBatch = 4;
            for (int it0 = tx; it0 < items; it0 += kEmitBatch * BS) {
                Digits dd[kEmitBatch];
                unsigned long long v[kEmitBatch];
    #pragma unroll
                for (int q = 0; q < kEmitBatch; ++q) {
                    dd[q] = split(min(it0 + q * BS, items - 1));
                    v[q] = marginal(dd[q], false);
                }
    #pragma unroll
                for (int q = 0; q < kEmitBatch; ++q)
                    if (it0 + q * BS < items) emit(dd[q], v[q]);
            }
        } else if (P == 3 && NIB && vec5) {
            // 5 bins, nibble columns, in two steps. (1) One thread per (node, group, plane b1 of
            // the first feature), planes fastest, then nodes (a half-wave's plane and node
            // offsets, 25 b1 + 125 u words, then fall on distinct LDS bank pairs at 2, 4 and 8
            // nodes, where nodes fastest put two lanes on one bank pair). It reads the plane's
            // 25 cells (b2 * 5 + b3) once, in two batches, and forms the first feature's marginal
            // at b1 (all 25), the second feature's partial marginals over this plane (rows, by
            // b2) and the third's (columns, by b3). It writes those 11 sums over the plane's first words: no other thread reads
            // the plane. (2) One thread per (node, feature) adds its 5 marginals from the 5
            // planes' sums and emits them. Each cell is read once, where a thread per marginal
            // element read it three times.
            const int ng5 = ng * 5;
            const DivU16 div_un(Un);
            for (int t = tx; t < Un * ng5; t += BS) {
                const int q = t / 5;  // (node, group)
                const int b1 = t - q * 5;
                const int g = (int)div_un.div((uint32_t)q);
                const int u = q - g * Un;
                unsigned long long* pl =
                    lds + ((int64_t)g * words_group + (int64_t)u * cells_node * C + (int64_t)b1 * 25 * C);
                unsigned long long s2[5], s3[5];
                {
                    unsigned long long v[15];
    #pragma unroll
                    for (int j = 0; j < 15; ++j) v[j] = pl[j * C];
    #pragma unroll
                    for (int b = 0; b < 5; ++b) s3[b] = v[b] + v[5 + b] + v[10 + b];
    #pragma unroll
                    for (int q = 0; q < 3; ++q) s2[q] = v[q * 5] + v[q * 5 + 1] + v[q * 5 + 2] + v[q * 5 + 3] + v[q * 5 + 4];
                }
                {
                    unsigned long long v[10];
    #pragma unroll
                    for (int j = 0; j < 10; ++j) v[j] = pl[(15 + j) * C];
    #pragma unroll
                    for (int b = 0; b < 5; ++b) s3[b] += v[b] + v[5 + b];
    #pragma unroll
                    for (int q = 0; q < 2; ++q)
                        s2[3 + q] = v[q * 5] + v[q * 5 + 1] + v[q * 5 + 2] + v[q * 5 + 3] + v[q * 5 + 4];
                }
                pl[0] = s2[0] + s2[1] + s2[2] + s2[3] + s2[4];
    #pragma unroll
                for (int b = 0; b < 5; ++b) {
                    pl[1 + b] = s2[b];
                    pl[6 + b] = s3[b];
                }
            }
            __syncthreads();
            for (int t = tx; t < Un * nf; t += BS) {
                const int u = (int)div_nf.div((uint32_t)t);
                const int kk = t - u * nf;
                const int g = kk / 3;
                const int side = kk - g * 3;
                const unsigned long long* pl0 =
                    lds + ((int64_t)g * words_group + (int64_t)u * cells_node * C);
                unsigned long long m[5];
                if (side == 0) {  // plane bb's total
    #pragma unroll
                    for (int bb = 0; bb < 5; ++bb) m[bb] = pl0[bb * 25 * C];
                } else {  // bin bb's partial sums of the 5 planes
                    const int off = side == 1 ? 1 : 6;
                    unsigned long long v[25];
    #pragma unroll
                    for (int p = 0; p < 5; ++p)
    #pragma unroll
                        for (int bb = 0; bb < 5; ++bb) v[p * 5 + bb] = pl0[p * 25 * C + off + bb];
    #pragma unroll
                    for (int bb = 0; bb < 5; ++bb) m[bb] = v[bb] + v[5 + bb] + v[10 + bb] + v[15 + bb] + v[20 + bb];
                }
                emit5(u, kk, m);
            }
        } else if (items <= kMaxItems * BS) {
            // marginals into registers, then compact them over the (no longer needed) joint cells
            // and prefix from there: nb reads per element instead of (bb + 1) * nb
            unsigned long long m[kMaxItems];
    #pragma unroll
            for (int i = 0; i < kMaxItems; ++i) {
                const int it = tx + i * BS;
                m[i] = (it < items) ? marginal(split(it), false) : 0ull;
            }
            __syncthreads();
    #pragma unroll
            for (int i = 0; i < kMaxItems; ++i) {
                const int it = tx + i * BS;
                if (it < items) lds[it] = m[i];
            }
            __syncthreads();
            // prefix over bins 0..bb of the compacted marginals, its loads as one batch
            auto prefix = [&](int it, int bb, auto width) -> unsigned long long {
                constexpr int W = decltype(width)::value;
                unsigned long long v[W];
    #pragma unroll
                for (int o = 0; o < W; ++o) v[o] = lds[it - bb + min(o, bb)];
                unsigned long long r = 0ull;
    #pragma unroll
                for (int o = 0; o < W; ++o) r += (o <= bb) ? v[o] : 0ull;
                return r;
            };
            if (vec5) {
                // one thread per (node, feature): its 5 compacted marginals, then emit5
                for (int t = tx; t < Un * nf; t += BS) {
                    const int u = (int)div_nf.div((uint32_t)t);
                    unsigned long long m[5];
    #pragma unroll
                    for (int bb = 0; bb < 5; ++bb) m[bb] = lds[t * 5 + bb];
                    emit5(u, t - u * nf, m);
                }
            } else
            for (int it = tx; it < items; it += BS) {
                const Digits d = split(it);
                const unsigned long long tot =
                    (nb <= 4)   ? prefix(it, d.bb, std::integral_constant<int, 4>{})
                    : (nb == 5) ? prefix(it, d.bb, std::integral_constant<int, 5>{})
                    : (nb <= 8) ? prefix(it, d.bb, std::integral_constant<int, 8>{})
                                : prefix(it, d.bb, std::integral_constant<int, 16>{});
                emit(d, tot);
            }
        } else {
            for (int it = tx; it < items; it += BS) {
                const Digits d = split(it);
                emit(d, marginal(d, true));
            }
        }
    }  // work items
}

template <int FT, int P, bool NIB, int BS>
hipError_t launch_bs(const HistArgs& a, int grid, size_t lds_bytes, hipStream_t s) {
    const void* fn = reinterpret_cast<const void*>(&hist_era_kernel<FT, P, NIB, BS>);
    if (lds_bytes > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)lds_bytes);
        if (e != hipSuccess) return e;
    }
    // as many workgroups as are resident at once (times a.rounds), a multiple of 8
    if (a.resident_cus > 0) {
        int per_cu = 0;
        hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, BS, lds_bytes);
        if (e != hipSuccess) return e;
        const int64_t want = (int64_t)std::max(1, per_cu) * a.resident_cus * std::max(1, a.rounds);
        grid = (int)std::max<int64_t>(8, std::min<int64_t>(grid, want) / 8 * 8);
    }
    hipLaunchKernelGGL((hist_era_kernel<FT, P, NIB, BS>), dim3(grid), dim3(BS), lds_bytes, s, a, a.seg_info,
                       a.feats);
    return hipGetLastError();
}

// Workgroup size: 2 waves when the histogram is small (more resident workgroups per CU, each
// streaming its era in more passes; measured 6% faster over the depths of a 5-bin round),
// 4 waves when the LDS per workgroup caps residency anyway.
template <int FT, int P, bool NIB>
hipError_t launch_ft(const HistArgs& a, int grid, size_t lds_bytes, hipStream_t s) {
    if (a.block == 128) return launch_bs<FT, P, NIB, 128>(a, grid, lds_bytes, s);
    if (a.block == 256) return launch_bs<FT, P, NIB, 256>(a, grid, lds_bytes, s);
    return hipErrorInvalidValue;
}

template <bool NIB>
hipError_t launch_layout(const HistArgs& a, int pairs, int grid, size_t lds_bytes, hipStream_t s) {
    if (pairs == 3) {
        switch (a.ftile) {
            case 3: return launch_ft<3, 3, NIB>(a, grid, lds_bytes, s);
            case 6: return launch_ft<6, 3, NIB>(a, grid, lds_bytes, s);
            case 12: return launch_ft<12, 3, NIB>(a, grid, lds_bytes, s);
            default: return hipErrorInvalidValue;
        }
    }
    if (pairs == 2) {
        switch (a.ftile) {
            case 2: return launch_ft<2, 2, NIB>(a, grid, lds_bytes, s);
            case 4: return launch_ft<4, 2, NIB>(a, grid, lds_bytes, s);
            case 8: return launch_ft<8, 2, NIB>(a, grid, lds_bytes, s);
            case 16: return launch_ft<16, 2, NIB>(a, grid, lds_bytes, s);
            case 32: return launch_ft<32, 2, NIB>(a, grid, lds_bytes, s);
            default: return hipErrorInvalidValue;
        }
    }
    switch (a.ftile) {
        case 1: return launch_ft<1, 1, NIB>(a, grid, lds_bytes, s);
        case 2: return launch_ft<2, 1, NIB>(a, grid, lds_bytes, s);
        case 4: return launch_ft<4, 1, NIB>(a, grid, lds_bytes, s);
        case 8: return launch_ft<8, 1, NIB>(a, grid, lds_bytes, s);
        case 16: return launch_ft<16, 1, NIB>(a, grid, lds_bytes, s);
        default: return hipErrorInvalidValue;
    }
}

// One thread per (split era, node, feature): prefix over the bins of the exact sums, the same
// conversion as the histogram flush (count exact, grad rounded once to float32), then the
// sums are cleared for the next depth.
__global__ __launch_bounds__(kBlock) void finalize_kernel(FinalizeArgs f) {
    const int Ua = f.st->u_active[f.depth];
    const int64_t n = (int64_t)f.n_acc * Ua * f.K;
    const int pt = f.nb - 1;
    const int64_t stride = (int64_t)gridDim.x * kBlock;
    for (int64_t t = (int64_t)blockIdx.x * kBlock + threadIdx.x; t < n; t += stride) {
        const int64_t sk = t / f.K;
        const int k = (int)(t - sk * f.K);
        const int slot = (int)(sk / Ua);
        const int u = (int)(sk - (int64_t)slot * Ua);
        const int era = f.acc_era[slot];
        const double inv_scale = ldexp(1.0, -f.sh_era[era]);
        uint32_t* ac = f.acc_cnt + (((int64_t)slot * f.acc_U + u) * f.acc_K + k) * f.nb;
        unsigned long long* ag = f.acc_g + (((int64_t)slot * f.acc_U + u) * f.acc_K + k) * f.nb;
        const int64_t o = (((int64_t)era * f.U + u) * f.K + k) * pt;
        uint32_t c = 0u;
        long long q = 0;
        for (int b = 0; b < f.nb; ++b) {
            c += ac[b];
            q += (long long)ag[b];
            ac[b] = 0u;
            ag[b] = 0ull;
            const float gs = (float)((double)q * inv_scale);  // exact in double: |q| < 2^45
            if (b < pt) {
                if (f.out_cnt32)
                    f.out_cnt32[o + b] = c;
                else
                    f.out_cnt[o + b] = (uint16_t)c;
                f.out_g[o + b] = gs;
            } else if (k == 0) {
                f.out_tot_cnt[(int64_t)era * f.U + u] = (int32_t)c;
                f.out_tot_g[(int64_t)era * f.U + u] = gs;
            }
        }
    }
}

}  // namespace

hipError_t launch_finalize(const FinalizeArgs& f, hipStream_t s) {
    const int64_t n = (int64_t)f.n_acc * f.U * f.K;
    const int grid = (int)std::max<int64_t>(1, std::min<int64_t>((n + kBlock - 1) / kBlock, 4096));
    hipLaunchKernelGGL(finalize_kernel, dim3(grid), dim3(kBlock), 0, s, f);
    return hipGetLastError();
}

hipError_t launch_hist(const HistArgs& a, int pairs, int grid, size_t lds_bytes, hipStream_t s) {
    if (a.nibble) {
        if (a.nb > 16) return hipErrorInvalidValue;
        return launch_layout<true>(a, pairs, grid, lds_bytes, s);
    }
    return launch_layout<false>(a, pairs, grid, lds_bytes, s);
}

}  // namespace pb
