// Internal declarations shared by the HIP kernels and the C-ABI host layer.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/packboost_hip.h"

namespace pb {

constexpr int kWave = 64;          // CDNA wavefront width
constexpr int kBlock = 256;        // threads per workgroup for the row kernels
constexpr int kCountBits = 16;     // low bits of a histogram word hold the row count
constexpr int kMaxEraRowsDirect = (1 << kCountBits) - 1;
constexpr uint32_t kLeafFeatureBits = 0xFFFFFFu;  // compiled-forest leaf marker
constexpr int kGradWinRows = kBlock * 4;  // rows per window of the round's |grad| sums

// Frontier state of the round in flight; lives in device memory and is only written
// by kernels, so a whole round is enqueued without host round trips.
struct Frontier {
    int32_t u_active[PB_MAX_DEPTH + 1];  // active nodes per depth
    int32_t tree_size;                   // next TreeBuilder id
    int32_t reserved[7];                 // [kNonFinite]: the round's gradients were not all finite
};
constexpr int kNonFinite = 0;

// The round's header (pb_round_header) from the frontier state, written by the first
// workgroup's threads of a kernel that runs after the round's last decision step.
__device__ __forceinline__ void write_round_header(const Frontier* st, pb_round_header* h) {
    const int i = (int)threadIdx.x;
    if (i <= PB_MAX_DEPTH) h->u_active[i] = st->u_active[i];
    if (i == 0) h->tree_size = st->tree_size;
    if (i < 6) h->reserved[i] = i == 0 ? st->reserved[kNonFinite] : 0;
}

// Fixed-point gradient scale of one era: rows add q = round(g * 2^sh) into the 48-bit grad field
// of a histogram word. round_begin sums |g| over windows of kGradWinRows consecutive rows, and
// era_scale_kernel bounds the era's sum of |g| by the sum of the windows that overlap it
// (times 1 + 2^-10 for the float rounding of those sums), so
//   sum over the era of |q| <= 2^sh * bound + rows / 2 < 2^45
// with sh = 44 - ceil(log2(bound)): every cell, prefix, era total and split-era sum fits the
// field with room to spare, and each row carries about 44 - log2(bound / |g|) bits, far finer
// than the float32 rounding of the reference's row-order sums unless an era holds rows whose
// |g| differ by many orders of magnitude. Capped so that 2^sh is a finite float.
__device__ __forceinline__ int era_grad_scale(double bound) {
    if (!(bound > 0.0)) return 0;
    int ex = 0;
    (void)frexp(bound, &ex);  // bound < 2^ex
    return min(44 - ex, 126);
}

// v moved across lanes by the DPP control CTRL (both 32-bit halves); lanes with no source in
// range, and the rows outside ROW_MASK, read 0 (bound_ctrl, old value 0).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long v) {
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, ROW_MASK, 0xf, true);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, ROW_MASK, 0xf, true);
    return ((unsigned long long)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Inclusive scan of v over the 64 lanes of a wavefront: a scan inside each 16-lane row by DPP
// row shifts, then the row totals broadcast across rows (no LDS round trip).
__device__ __forceinline__ unsigned long long wave_scan_incl_u64(unsigned long long v) {
    v += dpp_u64<0x111>(v);       // row_shr:1
    v += dpp_u64<0x112>(v);       // row_shr:2
    v += dpp_u64<0x114>(v);       // row_shr:4
    v += dpp_u64<0x118>(v);       // row_shr:8
    v += dpp_u64<0x142, 0xa>(v);  // row_bcast:15 into rows 1 and 3
    v += dpp_u64<0x143, 0xc>(v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// One row's 64-bit histogram addend (q << 16) + 1 with q = round(g * scale) (|q| < 2^45): the
// count 1 in the low 16 bits, the fixed-point grad above it. g * scale is exact in float (scale
// is a power of two); adding 1.5 * 2^52 to it in double rounds it to an integer with ties to
// even (as rintf does) and leaves that integer in the low mantissa bits, so the double's bit
// pattern minus that of 1.5 * 2^52 (low word 0) is q in two's complement for |q| < 2^51. Six
// instructions where float floor/split conversions took nine; double adds issue at the full
// rate on gfx950.
__device__ __forceinline__ unsigned long long grad_addend(float g, float scale) {
    const double y = (double)(g * scale) + 6755399441055744.0;
    const unsigned long long b = (unsigned long long)__double_as_longlong(y);
    const uint32_t lo = (uint32_t)b;                       // q's low word
    const uint32_t hi = (uint32_t)(b >> 32) - 0x43380000u;  // q's high word
    const uint32_t ahi = __builtin_amdgcn_alignbit(hi, lo, 32 - kCountBits);  // (q << 16) >> 32
    return ((unsigned long long)ahi << 32) | ((lo << kCountBits) | 1u);
}

// LDS words per feature group of hist_era_kernel: `cells` words (a group's joint cells over the
// item's nodes, times the copies), padded for 5-bin pairs with one copy in tiles of 4 or more
// groups. Their flush gives the lanes of a wavefront the groups of one node, then the next
// node's (so that each node's plane stores are contiguous); a group stride that is an odd
// multiple of 32 / groups words (groups rounded up to a power of two) puts the 32 lanes of a
// half-wave, whose node offsets 25 u differ modulo 32 / groups, on distinct pairs of LDS banks.
__host__ __device__ inline int hist_group_words(int cells, int P, int nb, int C, int groups) {
    if (!(P == 2 && nb == 5 && C == 1 && groups >= 4)) return cells;
    int g2 = 1;
    while (g2 < groups) g2 *= 2;
    const int q = 32 / (g2 < 32 ? g2 : 32);
    int s = (cells + q - 1) / q * q;
    if (((s / q) & 1) == 0) s += q;
    return s;
}

// IEEE 1/n for an integer-valued float n in [1, 2^20]: the hardware reciprocal (within one ulp)
// and one Newton step with fused multiply-adds give the correctly rounded value, checked bit for
// bit against the IEEE division for every n in that range on gfx950. The scorers' unit-weight
// Welford factor w / wsum = 1 / n takes it in place of a table lookup that put an LDS round trip
// on the era chain.
__device__ __forceinline__ float exact_recip(float n) {
    const float r = __builtin_amdgcn_rcpf(n);
    const float e = __builtin_fmaf(-n, r, 1.0f);
    return __builtin_fmaf(e, r, r);
}

// Per active node of the current depth, read by the partition kernel.
struct SplitRule {
    int32_t feature;    // -1: node did not split
    int32_t threshold;
    int32_t left_id;    // TreeBuilder id of the left child (right = left + 1)
    uint16_t next_slot[2];  // slot in the next frontier (PB_INACTIVE if not active)
};

struct NodeTotal {
    int32_t count;
    float grad;
};

struct HistArgs {
    int32_t resident_cus;  // > 0: loop work items over a resident grid on this many CUs
    int32_t rounds;        // resident grids' worth of workgroups (1 = one per slot)
    const uint8_t* bins;
    int64_t ld;            // byte stride between columns of `bins`
    int32_t nibble;        // 1: two rows per byte (nb <= 16), 0: one uint8 per row
    int32_t block;         // threads per workgroup: 128 or 256
    const float* grad;
    const uint16_t* nid;
    const int32_t* feats;
    int32_t K;
    int32_t ntiles;
    int32_t ftile;
    int32_t U;      // node stride of the output planes (max nodes)
    int32_t node_tile;   // nodes per work item (LDS tile), node_tiles * node_tile >= U
    int32_t node_tiles;
    int32_t nb;
    int32_t clog2;  // log2 of LDS histogram copies
    const Frontier* st;
    int32_t depth;
    uint16_t* out_cnt;     // compact planes (plane_cells / plane_tot_off), 16-bit counts
    uint32_t* out_cnt32;   // the same with 32-bit counts (an era above 65535 rows), or null
    int32_t* out_tot_cnt;
    float* out_g;
    float* out_tot_g;
    // Work segments: seg_info[s] = (first row, end row, era, slot), at most 65535 rows. An era
    // of several segments (slot >= 0) is summed exactly over its segments in acc_cnt / acc_g
    // ([slot][U][K][nb], raw per-bin counts and fixed-point grads) and turned into planes by
    // finalize_kernel; other eras (slot -1) write their planes directly.
    const int4* seg_info;
    int32_t S;
    uint32_t* acc_cnt;
    unsigned long long* acc_g;
    int32_t acc_U, acc_K;  // node and feature strides of acc_cnt / acc_g (their allocation)
    const int32_t* sh_era;  // [E] fixed-point gradient scale exponent of each era
};

// Planes of the eras split into several segments (see HistArgs): prefix over bins of the
// exact sums, then the same rounding and layout as the histogram kernel's own flush.
struct FinalizeArgs {
    uint32_t* acc_cnt;
    unsigned long long* acc_g;
    const int32_t* acc_era;  // [n_acc] era of each slot
    int32_t n_acc;
    int32_t U, K, nb;        // plane strides and the depth's feature count
    int32_t acc_U, acc_K;    // node and feature strides of acc_cnt / acc_g
    const int32_t* sh_era;   // [E] fixed-point gradient scale exponent of each era
    const Frontier* st;
    int32_t depth;
    uint16_t* out_cnt;
    uint32_t* out_cnt32;
    int32_t* out_tot_cnt;
    float* out_g;
    float* out_tot_g;
};
hipError_t launch_finalize(const FinalizeArgs& f, hipStream_t s);

// Histogram planes (compact form). For T = nb - 1 thresholds of U node slots and K features:
//   count buffer: uint16 [E][U][K][T] prefix counts (rows with bin <= t; an era holds at most
//                 65535 rows), then int32 [E][U] era totals at element plane_tot_off;
//   grad buffer:  float  [E][U][K][T] prefix grads, then float [E][U] era totals at the same
//                 element offset.
// The totals are the same for every feature (exact fixed-point sums), so they are stored once.
__host__ __device__ inline int64_t plane_cells(int64_t E, int64_t U, int64_t K, int64_t nb) {
    return E * U * K * (nb - 1);
}
__host__ __device__ inline int64_t plane_tot_off(int64_t E, int64_t U, int64_t K, int64_t nb) {
    return (plane_cells(E, U, K, nb) + 63) / 64 * 64;  // 4-byte elements into either buffer
}
__host__ __device__ inline int64_t plane_elems(int64_t E, int64_t U, int64_t K, int64_t nb) {
    return plane_tot_off(E, U, K, nb) + E * U;
}

constexpr int kScoreChunkEras = 24;  // eras whose plane cells a scorer chunk stages at once

// Every candidate of one depth, [U][K][T] in the reference's visiting order (subset feature,
// then threshold index), for the decision step's sequential pick: score (-inf for a candidate
// the reference skips), left count, left grad; band is that step's scratch ([U][K * T] indices).
struct SeqCands {
    float* score;
    int32_t* lt;
    float* lg;
    int32_t* band;
};

struct ScoreArgs {
    const uint16_t* cnt;     // prefix counts [E][U][K][nb-1]
    const uint32_t* cnt32;   // the same as 32-bit counts (eras above 65535 rows), or null
    const int32_t* tot_cnt;  // [E][U]
    const float* g;          // prefix grads [E][U][K][nb-1]
    const float* tot_g;      // [E][U]
    int32_t E;
    int32_t U;
    int32_t K;
    int32_t nb;
    int32_t T;             // thresholds per feature
    const int32_t* feats;
    const int32_t* thr_tab;  // [K][T] or null for the full sweep 0..nb-2
    float lambda_l2;
    float lambda_dro;
    float dir_w;
    float era_alpha;
    int32_t msl;
    const Frontier* st;
    int32_t depth;
    pb_candidate* cand_w;    // [U][W] wavefront winners, W = ntiles * wpt
    pb_candidate* cand_all;  // optional [U][K][T]
    NodeTotal* ntot;         // [U]
    int32_t fts;             // features per workgroup
    int32_t ntiles;          // feature tiles per node
    int32_t ec;              // eras staged in LDS per chunk
    int32_t wpt;             // wavefront winners per tile (ceil(fts * T / 64))
    int32_t rt;              // size of the 1/n table (equal era weights)
    int32_t staged;          // T >= 64: 1 = LDS-staged two-phase kernel, 0 = wide kernel
    int32_t pc_classic;      // T <= 63 with unit era weights (PB_SCORE_PC): 0 = des_score_pcu_kernel
                             // for one pair per producer thread, else des_score_pc_kernel;
                             // 1 = des_score_pc_kernel always; 2 = des_score_pcu_kernel always
    SeqCands seq;            // every candidate, for the sequential pick
    int32_t skip_last;       // 1: nb = the reference's num_bins + 1, the last bin its skipped
                             // rows (pb_split_params.skip_last_bin); des_score_kernel only
};

// Launch shape of the scorer for K features and T thresholds (shared by the context's
// buffer sizing and the launch).
struct ScoreShape {
    int32_t fts, ntiles, ec, wpt, rt;
    size_t lds_bytes;
};
ScoreShape score_shape(int32_t K, int32_t T, int32_t E, int32_t nodes, int32_t target_wgs);
ScoreShape score_shape_classic(int32_t K, int32_t T, int32_t E);

// Launchers (defined in the .hip files; all return hipError_t of the launch).
hipError_t launch_hist(const HistArgs& a, int pairs, int grid, size_t lds_bytes, hipStream_t s);
hipError_t launch_score(const ScoreArgs& a, int grid, size_t lds_bytes, hipStream_t s);
hipError_t launch_kcuts(const uint16_t* cnt, const uint32_t* cnt32, const int32_t* tot_cnt, int32_t E,
                        int32_t U, int32_t K, int32_t nb, int32_t skip, int32_t k, int32_t mass,
                        const Frontier* st, int32_t depth, int32_t* thr_tab, hipStream_t s);
// The candidates of the depth the decision step picks from: the scorer's wavefront winners
// (cand_w [U][W]) and every candidate in visiting order (seq, K features x T thresholds of the
// ids feats / thresholds thr_tab, or 0..T-1 when thr_tab is null).
struct DecideCands {
    const pb_candidate* cand_w;
    int32_t W;
    SeqCands seq;
    int32_t K, T;
    const int32_t* feats;
    const int32_t* thr_tab;
};
hipError_t launch_decide(const DecideCands& dc, int32_t max_nodes, const NodeTotal* ntot,
                         Frontier* st, int32_t depth, int32_t msl, double lambda_l2,
                         const int32_t* cur_ids, int32_t* next_ids, SplitRule* rules,
                         pb_decision* dec, float* values, pb_candidate* node_best,
                         hipStream_t s);
// Segment mode (segment.hip, score.hip). Rows are kept sorted by (era, frontier slot): in era
// e, slot u's rows are [seg[e * segw + u], seg[e * segw + u + 1]) of the sorted buffers, and
// [seg[e * segw + U], era end) holds the rows no longer in the frontier (U = active slots).
// One workgroup per (slot, tile of FT features) walks the eras in order, builds each era's
// histogram of its node's rows in LDS (bins read from the caller's columns through the sorted
// row ids) and runs the DES recurrence on it: the candidates and wavefront winners are those of
// the plane scorers, bit for bit, without the planes.
struct SegScoreArgs {
    const uint8_t* bins;   // the caller's bins, uint8 [F][ld]
    const int32_t* row;    // the sorted rows' ids
    int64_t ld;
    const float* g;        // sorted gradients [N]
    const int32_t* seg;    // [E][segw] segment starts of the current depth
    int32_t segw;
    const int32_t* sh_era;  // per-era fixed-point scale exponent
    const int32_t* feats;
    int32_t K;
    int32_t E, nb, T;       // T = nb - 1 thresholds (full sweep)
    float lambda_l2, lambda_dro, dir_w, era_alpha;
    int32_t msl;
    const Frontier* st;
    int32_t depth;
    pb_candidate* cand_w;  // [U][ntiles * wpt]
    int32_t ntiles, wpt, fts;
    SeqCands seq;
    NodeTotal* ntot;
    int32_t rt;            // size of the 1/n table (equal era weights)
    int32_t mu;            // node slots per tile in the grid (the launch's max_nodes)
    int32_t tile_major;    // 1: XCD-aware tile-major block order (nodes fastest), 0: node-major
};
constexpr int kSegMaxFt = 4;  // 8 measured slower: 123 VGPRs hold it to 4 waves per SIMD (FT 4: 6)
// The sorted rows of segment mode: per row its gradient, original row id and tree node id.
struct SegBuffers {
    float* g;
    int32_t* row;
    uint16_t* tnode;
};
// The partition's shape and workspace (segment.hip).
struct SegState {
    int64_t N, ld;
    int32_t E, segw;
    const int32_t* era_off;
    const Frontier* st;
    const SplitRule* rules;
    int32_t* cp;     // [E * segw + 1] chunk prefix per (era, slot)
    int32_t* cnt_l;  // [seg_chunk_bound + 1] left rows per chunk, then their prefix
    int32_t* cnt_r;
    int32_t* base;   // [E * segw][2] first destination row of each (era, slot, side)
};
int64_t seg_chunk_bound(int64_t N, int32_t E, int32_t segw);
hipError_t launch_seg_begin(const float* grad, int32_t* srow, float* gs, uint16_t* stn, int64_t N,
                            const int32_t* era_off, int32_t E, int32_t segw, int32_t* seg, hipStream_t s);
// Partition of depth `depth` from src (segments seg) into dst (segments seg_next); at the last
// depth (`last`) only the tree nodes of src change. The split rules read bins [F][ld] at the
// rows' ids.
hipError_t launch_seg_partition(const SegState& st, const int32_t* seg, int32_t* seg_next, const SegBuffers& src,
                                const SegBuffers& dst, const uint8_t* bins, int32_t depth, bool last,
                                hipStream_t s);
hipError_t launch_seg_round_end(const uint16_t* stn, const int32_t* srow, const float* values, int32_t B,
                                float lr, float* preds, int64_t N, const Frontier* st, pb_round_header* header,
                                hipStream_t s);
// Features per workgroup for `nodes` active slots and K features: enough workgroups to fill
// the device (about 1024), at most kSegMaxFt.
int32_t seg_score_fts(int32_t nodes, int32_t K);
size_t seg_score_lds_bytes(int32_t fts, int32_t rt);
hipError_t launch_seg_score(const SegScoreArgs& a, int32_t max_nodes, hipStream_t s);

// One winner per node of candidate records [M][n] in visiting order, by the reference's
// sequential scan (band: int32 [M][n] scratch).
hipError_t launch_pick_sequential(const pb_candidate* cand, int32_t M, int64_t n, int32_t* band,
                                  pb_candidate* out, hipStream_t s);
hipError_t launch_select_subsets(const pb_round_header* prev, int32_t D, int32_t K,
                                 const int32_t* window, int32_t* feats, hipStream_t s);
hipError_t launch_partition(const uint8_t* bins, int64_t ld, int32_t nibble, int64_t rows_padded,
                            const SplitRule* rules, const Frontier* st, int32_t depth,
                            uint16_t* nid, uint16_t* tnode, hipStream_t s);
// The round's last partition together with launch_round_end's work (preds 16-byte aligned,
// N <= rows_padded; hipErrorInvalidValue otherwise, and nothing is launched).
hipError_t launch_partition_end(const uint8_t* bins, int64_t ld, int32_t nibble, int64_t rows_padded,
                                const SplitRule* rules, const Frontier* st, int32_t depth, uint16_t* nid,
                                uint16_t* tnode, const float* values, int32_t pack_size, float lr,
                                float* preds, int64_t N, pb_round_header* header, hipStream_t s);
// Also writes win_sum [ceil(rows_padded / kGradWinRows)] (sum of |grad| per window) and
// sh_era [E] (era_grad_scale of each era, eras at era_off [E+1]).
hipError_t launch_round_begin(const float* preds, const float* y, float* grad, uint16_t* nid,
                              uint16_t* tnode, int64_t N, int64_t rows_padded, int32_t root_active,
                              const int32_t* era_off, int32_t E, float* win_sum, int32_t* sh_era,
                              Frontier* st, int32_t* cur_ids, hipStream_t s);
hipError_t launch_round_end(const uint16_t* tnode, const float* values, int32_t pack_size,
                            float lr, float* preds, int64_t N, const Frontier* st, pb_round_header* header,
                            hipStream_t s);
hipError_t launch_pack_bins4(const uint8_t* bins, int64_t n, int64_t ld, int32_t F, uint8_t* out,
                             hipStream_t s);
// Row-list kernels (rowlist.hip). Workspace: rowlist_work_elems(segments) int32, whose first
// four entries are status flags (segment, row id, feature, capacity) left set after the call.
int64_t rowlist_work_elems(int64_t segments);
// pb_rowlist_partition_noalloc: the same stages with the workspace in a fixed device array of
// kNoAllocScratchInts int32 per device (no allocation); status [4] is the caller's.
constexpr int64_t kNoAllocScratchInts = int64_t(1) << 22;  // 16 MiB
constexpr int kNoAllocMaxDevices = 64;
int64_t rowlist_noalloc_max_segments();
hipError_t noalloc_scratch(int32_t** out);
hipError_t launch_rowlist_partition_noalloc(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                                            const int32_t* rows, int64_t R, const int32_t* nrs,
                                            const int32_t* nes, int32_t S, int32_t E,
                                            const int32_t* feat, const int32_t* thr, int32_t* left_out,
                                            int32_t* right_out, int64_t cap, int32_t* left_splits,
                                            int32_t* right_splits, int32_t* status, hipStream_t s);
hipError_t launch_rowlist_partition(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                                    const int32_t* rows, int64_t R, const int32_t* nrs,
                                    const int32_t* nes, int32_t S, int32_t E, const int32_t* feat,
                                    const int32_t* thr, int32_t* left_out, int32_t* right_out,
                                    int64_t cap, int32_t* left_splits, int32_t* right_splits,
                                    int32_t* work, hipStream_t s);
hipError_t launch_rowlist_gather(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                                 const int32_t* feats, int32_t K, const float* values,
                                 const int32_t* rows, int64_t R, const int32_t* nrs,
                                 const int32_t* nes, int32_t m0, int32_t m1, int32_t E,
                                 uint8_t* out_bins, int64_t out_ld, float* out_values,
                                 uint16_t* out_slot, int32_t* era_off, int32_t* work, hipStream_t s);
hipError_t launch_best_thresholds(const pb_candidate* cand, int32_t M, int32_t K, int32_t T,
                                  float* score, int32_t* thr, float* left_grad, float* left_hess,
                                  int64_t* left_count, hipStream_t s);
hipError_t launch_quantile_edges(const float* sorted, int64_t n, int64_t ld, int32_t F,
                                 const double* q, int32_t nq, float* edges, int32_t edge_stride,
                                 hipStream_t s);
hipError_t launch_apply_bins(const float* xt, int64_t n, int64_t ld_x, int32_t F,
                             const float* edges, int32_t ne, int32_t edge_stride, int32_t max_bins,
                             const int64_t* perm, uint8_t* bins, int64_t ld_out, hipStream_t s);
hipError_t launch_era_corr(const float* y, const float* p, const int32_t* era_off, int32_t E,
                           double* era_corr, double* out, hipStream_t s);
hipError_t launch_forest(const uint8_t* bins, int64_t N, int64_t ld, const int4* rec,
                         const int32_t* roots, int32_t T, int32_t depth, float tree_weight,
                         float* out, int32_t* leaf, int32_t group, int32_t max_grid,
                         hipStream_t s);
// Tiled walk of a compiled forest stored as complete heaps (predict.hip): forests of depth
// <= kForestTileMaxDepth whose row tile and tree block fit kForestTileMaxLds bytes of LDS.
constexpr int kForestTileMaxDepth = 8;
constexpr size_t kForestTileMaxLds = 144 * 1024;
constexpr size_t kForestTileTargetLds = 80 * 1024;  // two workgroups per CU
constexpr int kForestBlockWords = 4096;             // dwords of one tree block (16 KB)
// Trees per block at depth D: each tree takes 2^(D+1) dwords (its complete heap, slot 0 unused).
constexpr int forest_tree_block(int D) { return kForestBlockWords >> (D + 1); }
struct ForestTile {
    int32_t features;    // feature columns in the tile (the forest's largest feature + 1)
    int32_t bits;        // bits per bin in the tile (3, 4 or 8)
    int32_t rows;        // rows per tile (32 or 64)
    int32_t tile_words;  // dwords of the packed tile
    int32_t tree_block;  // trees per block (forest_tree_block of the depth)
    int32_t blocks;      // tree blocks (the last one padded with trees that add 0)
    int32_t threads;     // threads per workgroup (256, 512 or 1024)
    int32_t runs;        // 1: some heap tree stands for a run of identical trees (dword 0 counts)
};
ForestTile forest_tile_shape(int32_t features, int32_t max_threshold, int32_t depth, int32_t trees);
size_t forest_tile_lds_bytes(const ForestTile& ft);
uint32_t forest_tile_record(const ForestTile& ft, int32_t feature, int32_t threshold);
hipError_t launch_forest_tile(const uint8_t* bins, int64_t N, int64_t ld, const ForestTile& ft,
                              const uint32_t* blocks, const int32_t* lid, const int32_t* tfirst, int32_t T,
                              int32_t depth, float tree_weight, float* out, int32_t* leaf, hipStream_t s);
hipError_t launch_predict_pack(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                               const int32_t* feature, const int32_t* threshold,
                               const int32_t* left_abs, const int32_t* right_abs,
                               const float* value, const uint8_t* is_leaf,
                               const int32_t* offsets, int32_t B, int32_t total_nodes,
                               float tree_weight, int32_t sequential, float* out, int32_t* leaf,
                               hipStream_t s);
hipError_t launch_predict_bins(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                               const int32_t* feature, const int32_t* threshold,
                               const int32_t* left, const int32_t* right, const float* value,
                               const uint8_t* is_leaf, int32_t num_nodes, float* out,
                               hipStream_t s);

}  // namespace pb
