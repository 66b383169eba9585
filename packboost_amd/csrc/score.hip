// Kernel 2 — DES split scoring with wavefront-shuffle argmax, plus the per-depth decision
// step (node argmax over wavefront winners, child ids, leaf values, next frontier).
//
// Reference semantics (frontier_cpu.cpp:342-444): for every (node, threshold) and each era
// with rows, in era order:
//     L = prefix count, R = total - L, GL = prefix grad, GR = total grad - GL
//     left_total += L; left_grad += GL
//     w = (L > 0 && R > 0) ? era_weight : 0;  skip if w <= 0
//     gain = 0.5f * (GL*GL/(L+lambda) + GR*GR/(R+lambda)) - 0.5f*(G*G)/(count+lambda)
//     weighted Welford update of (mean, M2, wsum); optional direction agreement
// then score = mean - lambda_dro * sqrt(max(0, M2 / max(wsum, 1e-12))) (+ dir term) and
// the candidate is rejected unless both sides hold >= min_samples_leaf rows.
// Every float operation below is issued in that order with no contraction (the library
// is compiled with -ffp-contract=off), so given identical histogram planes the scores are
// bit-identical to the reference's.
//
// One lane owns one (node, feature, threshold) candidate and walks the eras; the lanes of a
// wavefront all belong to one node (the candidate space of a node is padded to 64), so
// a 6-step xor-shuffle argmax yields the wavefront's winner under a strict order (higher
// score; on an exactly equal score the larger left count, then larger feature id, then larger
// threshold). Every candidate is also kept in visiting order, and the decision step replays
// the reference's sequential pick with its 1e-12 tie window (frontier_cpu.cpp:415-426) over the
// candidates near the top score (sequential_pick).
#include <algorithm>

#include <type_traits>
#include <utility>

#include "pb_internal.h"

namespace pb {
namespace {

struct Cand {
    float score;
    int lt;
    float lg;
    int f;
    int thr;
    int valid;
};

// a beats b: valid first, then higher score, then (exact score tie) larger left count, larger
// feature id, larger threshold. Written without early returns: with early returns the gfx950
// backend of this toolchain emitted a winner update that kept the old feature/threshold on
// the tie path (the IR was right, the machine code was not), so both the comparison and the
// update below are plain boolean algebra and per-field selects.
__device__ __forceinline__ bool better(const Cand& a, const Cand& b) {
    const bool a_ok = a.valid != 0;
    const bool b_ok = b.valid != 0;
    const bool s_gt = a.score > b.score;
    const bool s_eq = a.score == b.score;
    const bool tie_win = (a.lt > b.lt) | ((a.lt == b.lt) & ((a.f > b.f) | ((a.f == b.f) & (a.thr > b.thr))));
    return a_ok & ((!b_ok) | s_gt | (s_eq & tie_win));
}

__device__ __forceinline__ void take_if(bool take, const Cand& c, Cand& best) {
    best.score = take ? c.score : best.score;
    best.lt = take ? c.lt : best.lt;
    best.lg = take ? c.lg : best.lg;
    best.f = take ? c.f : best.f;
    best.thr = take ? c.thr : best.thr;
    best.valid = take ? c.valid : best.valid;
}

__device__ __forceinline__ Cand shfl_xor_cand(const Cand& c, int m) {
    Cand o;
    o.score = __shfl_xor(c.score, m);
    o.lt = __shfl_xor(c.lt, m);
    o.lg = __shfl_xor(c.lg, m);
    o.f = __shfl_xor(c.f, m);
    o.thr = __shfl_xor(c.thr, m);
    o.valid = __shfl_xor(c.valid, m);
    return o;
}

__device__ __forceinline__ void store_cand(pb_candidate* dst, const Cand& c) {
    dst->score = c.score;
    dst->left_total = c.lt;
    dst->left_grad = c.lg;
    dst->feature = c.f;
    dst->threshold = c.thr;
    dst->valid = c.valid;
    dst->reserved[0] = 0;
    dst->reserved[1] = 0;
}

__device__ __forceinline__ Cand load_cand(const pb_candidate* src) {
    Cand c;
    c.score = src->score;
    c.lt = src->left_total;
    c.lg = src->left_grad;
    c.f = src->feature;
    c.thr = src->threshold;
    c.valid = src->valid;
    return c;
}

// Width of the first tie band of the sequential pick (64 x 1e-12, widened past the float
// rounding of |s - best| <= 1e-12f).
constexpr double kTieBand0 = 64.0e-12 * (1.0 + 1.0e-6);

// After the wavefront argmax (`win`, held by every lane): how many of the wavefront's valid
// candidates (own score `mine`, -inf if invalid) score below its winner but within kTieBand0
// of it. Stored with the winner, it tells the decision step whether the node's tie band holds
// any score other than the top one: when every candidate within kTieBand0 of the top score M
// scores exactly M, the sequential scan takes only score-M candidates after the first one, by
// the order (left count, feature, threshold), and that is the strict argmax.
__device__ __forceinline__ int wave_band_count(const Cand& win, float mine) {
    const bool near = win.valid && mine < win.score && (double)mine >= (double)win.score - kTieBand0;
    return __popcll(__ballot(near));
}

__device__ __forceinline__ void store_winner(pb_candidate* dst, const Cand& c, int band) {
    store_cand(dst, c);
    dst->reserved[0] = band;
}

// Every candidate of the depth in the reference's visiting order (per node: subset feature k,
// then threshold index t), for the sequential pick of the decision step: its score (-inf when
// the reference would skip it: below min_samples_leaf, no rows, or NaN), left count and left
// grad.
__device__ __forceinline__ void store_seq(const ScoreArgs& a, int64_t i, const Cand& c) {
    a.seq.score[i] = c.valid ? c.score : -INFINITY;
    a.seq.lt[i] = c.lt;
    a.seq.lg[i] = c.lg;
}

// Scorer. One workgroup owns one (node, tile of `fts` features) = fts * T candidates and walks
// the eras in chunks of `ec`, software-pipelined:
//   every thread holds kPairs (candidate, era) pairs of the NEXT chunk in registers (the four
//   plane values each needs), so the chunk's global loads are in flight while
//   phase A (all threads) turns the current pairs into gain / weight / direction in LDS and
//   phase B (one thread per candidate) runs the weighted Welford recurrence in era order over
//   the previous chunk. LDS is double-buffered, so one barrier per chunk orders the stages.
// With equal era weights (era_alpha == 0) the Welford factor w / wsum is 1 / n for the n-th
// valid era, read from a table of IEEE divisions 1.0f / n (bit-identical to the division).
constexpr int kPairs = 4;

struct PairIn {
    int ctot, L;
    float Gt, GL;
};

// C32: the planes carry 32-bit counts (an era above 65535 rows). SKIP: the planes hold one bin
// more than the reference's num_bins, the rows whose bin is >= num_bins (ScoreArgs.skip_last):
// an era's totals for a feature are then its prefix through bin num_bins - 1 (the last plane
// cell) while the era weight and the node's row and gradient totals stay those of all rows
// (frontier_cpu.cpp:174-206, 278-281, 296-314).
template <bool C32, bool SKIP>
__global__ __launch_bounds__(kBlock) void des_score_kernel(ScoreArgs a) {
    extern __shared__ unsigned char smem[];
    const int tid = threadIdx.x;
    const int u = blockIdx.x / a.ntiles;
    const int tile = blockIdx.x - u * a.ntiles;
    const int Ua = a.st->u_active[a.depth];
    if (u >= Ua) return;
    const int k0 = tile * a.fts;
    const int nf = min(a.fts, a.K - k0);
    if (nf <= 0) return;
    const int T = a.T;
    const int nb = a.nb;
    const int ncand = nf * T;
    const int cstride = a.fts * T;  // LDS row stride (max candidates of a tile)
    const int EC = a.ec;
    const int RT = a.rt;
    const int buf_words = EC * cstride;

    float* recip = reinterpret_cast<float*>(smem);
    float* base_f = recip + RT;
    // buffer b: sG, sGL, sL, sWD (each EC x cstride), then sCt, sGt (each EC)
    const int buf_stride = 4 * buf_words + 2 * EC;

    const float lam = a.lambda_l2;
    const float alpha = a.era_alpha;
    const bool use_dir = a.dir_w != 0.0f;
    const bool unit_w = !(alpha > 0.0f);
    const int pt = nb - 1;  // prefix cells per (node, feature) in the compact planes
    const int64_t ustride = (int64_t)a.K * pt;
    const int64_t estride = (int64_t)a.U * ustride;
    const int64_t node_off = (int64_t)u * ustride;
    const int nchunks = (a.E + EC - 1) / EC;

    PairIn pin[kPairs];
    int cful[SKIP ? kPairs : 1];    // SKIP: the era's rows (all bins) and their gradient sum
    float gful[SKIP ? kPairs : 1];
    auto prefetch = [&](int chunk) {
        const int e0 = chunk * EC;
        const int ne = min(EC, a.E - e0);
#pragma unroll
        for (int i = 0; i < kPairs; ++i) {
            const int pidx = tid + i * kBlock;
            pin[i].ctot = 0;
            pin[i].L = 0;
            pin[i].Gt = 0.0f;
            pin[i].GL = 0.0f;
            if (SKIP) {
                cful[SKIP ? i : 0] = 0;
                gful[SKIP ? i : 0] = 0.0f;
            }
            if (pidx < ne * ncand) {
                const int el = pidx / ncand;
                const int c = pidx - el * ncand;
                const int kk = c / T;
                const int t = c - kk * T;
                const int k = k0 + kk;
                const int thr = a.thr_tab ? a.thr_tab[k * T + t] : t;
                const int64_t off = (int64_t)(e0 + el) * estride + node_off + (int64_t)k * pt;
                const int64_t to = (int64_t)(e0 + el) * a.U + u;
                if (SKIP) {
                    pin[i].ctot = C32 ? (int)a.cnt32[off + pt - 1] : (int)a.cnt[off + pt - 1];
                    pin[i].Gt = a.g[off + pt - 1];
                    cful[SKIP ? i : 0] = a.tot_cnt[to];
                    gful[SKIP ? i : 0] = a.tot_g[to];
                } else {
                    pin[i].ctot = a.tot_cnt[to];
                    pin[i].Gt = a.tot_g[to];
                }
                pin[i].L = C32 ? (int)a.cnt32[off + thr] : (int)a.cnt[off + thr];
                pin[i].GL = a.g[off + thr];
            }
        }
    };

    const bool owner = tid < ncand;
    float wsum = 0.0f, mean = 0.0f, M2 = 0.0f, agn = 0.0f, agd = 0.0f, lg = 0.0f, tg = 0.0f;
    int lt = 0, tc = 0;

    prefetch(0);
    for (int ch = 0; ch < nchunks; ++ch) {
        const int e0 = ch * EC;
        const int ne = min(EC, a.E - e0);
        float* sG = base_f + (ch & 1) * buf_stride;
        float* sGL = sG + buf_words;
        int32_t* sL = reinterpret_cast<int32_t*>(sGL + buf_words);
        float* sWD = reinterpret_cast<float*>(sL + buf_words);
        int32_t* sCt = reinterpret_cast<int32_t*>(sWD + buf_words);
        float* sGt = reinterpret_cast<float*>(sCt + EC);
        // phase A on the prefetched pairs of this chunk
#pragma unroll
        for (int i = 0; i < kPairs; ++i) {
            const int pidx = tid + i * kBlock;
            if (pidx < ne * ncand) {
                const int el = pidx / ncand;
                const int c = pidx - el * ncand;
                const int ctot = pin[i].ctot;
                float gain = 0.0f, wd = 0.0f, GL = 0.0f;
                int L = -1;  // -1: the node has no rows in this era (skipped entirely)
                if (ctot != 0) {
                    const float Gt = pin[i].Gt;
                    L = pin[i].L;
                    GL = pin[i].GL;
                    const int R = ctot - L;
                    const float GR = Gt - GL;
                    const float wera = (alpha > 0.0f) ? ((float)(SKIP ? cful[SKIP ? i : 0] : ctot) + alpha) : 1.0f;
                    const float w = (L > 0 && R > 0) ? wera : 0.0f;
                    if (w > 0.0f) {
                        const float dL = (float)L + lam;
                        const float dR = (float)R + lam;
                        const float pden = (float)ctot + lam;
                        const float parent = (pden > 0.0f) ? (0.5f * (Gt * Gt)) / pden : 0.0f;
                        gain = 0.5f * ((GL * GL) / dL + (GR * GR) / dR) - parent;
                        bool pos = true;
                        if (use_dir) {
                            const float lv = -GL / dL;
                            const float rv = -GR / dR;
                            pos = lv > rv;
                        }
                        wd = pos ? w : -w;
                    }
                }
                sG[el * cstride + c] = gain;
                sGL[el * cstride + c] = GL;
                sL[el * cstride + c] = L;
                sWD[el * cstride + c] = wd;
                if (c == 0) {  // the node's totals over all of the era's rows
                    sCt[el] = SKIP ? cful[SKIP ? i : 0] : ctot;
                    sGt[el] = SKIP ? gful[SKIP ? i : 0] : pin[i].Gt;
                }
            }
        }
        if (ch + 1 < nchunks) prefetch(ch + 1);  // loads in flight across phase B
        __syncthreads();
        if (owner) {
            // eras in batches of kRecBatch: the batch's records first (their LDS reads in flight
            // together), then the weight-sum chain with its table lookups, then the era-ordered
            // sums and the mean/M2 chain; every float operation and its order per candidate are
            // those of the one-era-at-a-time recurrence
            constexpr int kRecBatch = 4;
            for (int b0 = 0; b0 < ne; b0 += kRecBatch) {
                int Lb[kRecBatch], ctb[kRecBatch];
                float GLb[kRecBatch], wdb[kRecBatch], gb[kRecBatch], gtb[kRecBatch];
#pragma unroll
                for (int j = 0; j < kRecBatch; ++j) {
                    const int el = min(b0 + j, ne - 1);  // past the chunk: read but not used
                    Lb[j] = sL[el * cstride + tid];
                    GLb[j] = sGL[el * cstride + tid];
                    wdb[j] = sWD[el * cstride + tid];
                    gb[j] = sG[el * cstride + tid];
                    ctb[j] = sCt[el];
                    gtb[j] = sGt[el];
                }
                float facb[kRecBatch], wb[kRecBatch];
#pragma unroll
                for (int j = 0; j < kRecBatch; ++j) {
                    const float w = (b0 + j < ne) ? fabsf(wdb[j]) : 0.0f;
                    const bool act = w > 0.0f;  // implies has; wsum + w > 0 then holds
                    const float wn = wsum + w;
                    const int wi = (int)wn;
                    facb[j] = (unit_w && wi < RT) ? (act ? exact_recip(wn) : 0.0f) : w / (act ? wn : 1.0f);
                    wsum = wn;  // + (+0) when inactive
                    wb[j] = w;
                }
#pragma unroll
                for (int j = 0; j < kRecBatch; ++j) {
                    if (b0 + j >= ne) break;  // uniform
                    const int L = Lb[j];
                    const bool has = L >= 0;
                    lt += has ? L : 0;
                    lg = has ? lg + GLb[j] : lg;
                    tc += ctb[j];
                    tg = (ctb[j] != 0) ? tg + gtb[j] : tg;
                    const float w = wb[j];
                    const float gain = gb[j];
                    // an inactive era (w = +0, gain = +0, factor 0) adds +-0 to every sum, which
                    // keeps its bits (no sum is ever -0): the reference's `continue`
                    const float delta = gain - mean;
                    const float mean_n = mean + facb[j] * delta;
                    M2 = M2 + (w * delta) * (gain - mean_n);
                    mean = mean_n;
                    if (use_dir) {
                        agn = agn + w * ((wdb[j] > 0.0f) ? 1.0f : -1.0f);
                        agd = agd + w;
                    }
                }
            }
        }
    }

    Cand c;
    c.lt = lt;
    c.lg = lg;
    c.valid = 0;
    c.score = 0.0f;
    c.f = -1;
    c.thr = -1;
    if (owner) {
        const int kk = tid / T;
        const int t = tid - kk * T;
        const int k = k0 + kk;
        c.f = a.feats[k];
        c.thr = a.thr_tab ? a.thr_tab[k * T + t] : t;
        const int rt = tc - lt;
        const float ws = (wsum < 1e-12f) ? 1e-12f : wsum;
        const float var = M2 / ws;
        const float sd = sqrtf((0.0f < var) ? var : 0.0f);
        float score = mean - a.lambda_dro * sd;
        if (use_dir && agd > 0.0f) score = score + a.dir_w * (agn / agd);
        c.score = score;
        // a node without rows never splits (the reference skips it, frontier_cpu.cpp:191-193)
        c.valid = (tc > 0 && lt >= a.msl && rt >= a.msl && !isnan(score)) ? 1 : 0;
        if (a.cand_all) store_cand(a.cand_all + ((int64_t)u * a.K + k) * T + t, c);
        store_seq(a, ((int64_t)u * a.K + k) * T + t, c);
        if (tile == 0 && tid == 0) {
            a.ntot[u].count = tc;
            a.ntot[u].grad = tg;
        }
    }
    const int wave = tid / kWave;
    if (wave < a.wpt) {
        const float mine = c.valid ? c.score : -INFINITY;
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) {
            const Cand o = shfl_xor_cand(c, m);
            take_if(better(o, c), o, c);
        }
        const int band = wave_band_count(c, mine);
        if ((tid & (kWave - 1)) == 0) {
            const int W = a.ntiles * a.wpt;
            store_winner(a.cand_w + (int64_t)u * W + tile * a.wpt + wave, c, band);
        }
    }
}

// Wide scorer for T >= 64 thresholds per feature (the default for that case). One workgroup
// owns one (node, feature); thread t owns threshold t and walks the eras itself: the era's
// record (gain, weight, direction) and the Welford step are computed by the same thread, in
// the same float operations and order as des_score_kernel's two phases. The plane values of
// kWidePf eras are loaded per batch into registers, two batches in flight (one being
// consumed while the next one loads), so a workgroup waits on memory once per kWidePf eras
// and needs no LDS staging or barriers (LDS holds only the 1/n table).
constexpr int kWidePf = 8;

// one batch of kWidePf eras: this thread's plane values, and the (era, node) totals with
// lane j of every wavefront holding era e0 + j (read back with readlane, so the totals of
// two batches stay in two vector registers instead of 2 * kWidePf scalar ones)
struct EraBatch {
    int L[kWidePf];
    float GL[kWidePf];
    int ct;
    float Gt;
    float parent;  // lane j: 0.5 * Gt^2 / (ct + lambda) of era e0 + j, 0 without rows
};

template <bool C32>
__global__ __launch_bounds__(kBlock) void des_score_wide_kernel(ScoreArgs a) {
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int u = blockIdx.x / a.ntiles;
    const int k = blockIdx.x - u * a.ntiles;  // one feature per workgroup
    const int Ua = a.st->u_active[a.depth];
    if (u >= Ua) return;
    const int T = a.T;
    const int RT = a.rt;

    const bool owner = tid < T;
    const int t = owner ? tid : T - 1;  // idle lanes mirror the last threshold (never owners)
    const int thr = a.thr_tab ? a.thr_tab[k * T + t] : t;
    const float lam = a.lambda_l2;
    const float alpha = a.era_alpha;
    const bool use_dir = a.dir_w != 0.0f;
    const bool unit_w = !(alpha > 0.0f);
    const int pt = a.nb - 1;
    const int64_t estride = (int64_t)a.U * a.K * pt;
    const int64_t cell0 = ((int64_t)u * a.K + k) * pt + thr;
    const int E = a.E;

    auto load = [&](int e0, EraBatch& b) {
        b.ct = 0;
        b.Gt = 0.0f;
        if (lane < kWidePf && e0 + lane < E) {
            const int64_t to = (int64_t)(e0 + lane) * a.U + u;
            b.ct = a.tot_cnt[to];
            b.Gt = a.tot_g[to];
        }
        b.parent = 0.0f;
#pragma unroll
        for (int j = 0; j < kWidePf; ++j) {
            b.L[j] = 0;
            b.GL[j] = 0.0f;
            if (e0 + j < E) {
                const int64_t off = (int64_t)(e0 + j) * estride + cell0;
                b.L[j] = C32 ? (int)a.cnt32[off] : (int)a.cnt[off];
                b.GL[j] = a.g[off];
            }
        }
    };

    // the parent term of era e0 + lane, once per era (lanes 0 .. kWidePf - 1), after the
    // batch's totals have arrived
    auto parents = [&](EraBatch& b) {
        const float pden = (float)b.ct + lam;
        b.parent = (b.ct != 0 && pden > 0.0f) ? (0.5f * (b.Gt * b.Gt)) / pden : 0.0f;
    };

    float wsum = 0.0f, mean = 0.0f, M2 = 0.0f, agn = 0.0f, agd = 0.0f, lg = 0.0f, tg = 0.0f;
    int lt = 0, tc = 0;
    auto step = [&](const EraBatch& b, int j) {
        const int ctot = __builtin_amdgcn_readlane(b.ct, j);
        if (ctot == 0) return;  // the node has no rows in this era (or past E): skipped
        const float Gt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b.Gt), j));
        const int L = b.L[j];
        const float GL = b.GL[j];
        const int R = ctot - L;
        const float GR = Gt - GL;
        const float wera = (alpha > 0.0f) ? ((float)ctot + alpha) : 1.0f;
        const float w = (L > 0 && R > 0) ? wera : 0.0f;
        float gain = 0.0f;
        bool pos = true;
        if (w > 0.0f) {
            const float dL = (float)L + lam;
            const float dR = (float)R + lam;
            const float parent = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(b.parent), j));
            gain = 0.5f * ((GL * GL) / dL + (GR * GR) / dR) - parent;
            if (use_dir) {
                const float lv = -GL / dL;
                const float rv = -GR / dR;
                pos = lv > rv;
            }
        }
        lt += L;
        lg = lg + GL;
        tc += ctot;
        tg = tg + Gt;
        const bool act = w > 0.0f;
        const float wn = wsum + w;
        const int wi = (int)wn;
        const float fac = (unit_w && wi < RT) ? (act ? exact_recip(wn) : 0.0f) : w / (act ? wn : 1.0f);
        // an inactive era (w = +0, gain = +0, factor 0) adds +-0 to every sum, which keeps its
        // bits (no sum is ever -0): the reference's `continue`, with no selects
        wsum = wn;
        const float delta = gain - mean;
        const float mean_n = mean + fac * delta;
        M2 = M2 + (w * delta) * (gain - mean_n);
        mean = mean_n;
        if (use_dir) {
            agn = agn + w * (pos ? 1.0f : -1.0f);
            agd = agd + w;
        }
    };

    EraBatch ba, bb;
    load(0, ba);
    for (int e0 = 0; e0 < E; e0 += 2 * kWidePf) {
        load(e0 + kWidePf, bb);
        parents(ba);
#pragma unroll
        for (int j = 0; j < kWidePf; ++j) step(ba, j);
        load(e0 + 2 * kWidePf, ba);
        parents(bb);
#pragma unroll
        for (int j = 0; j < kWidePf; ++j) step(bb, j);
    }

    Cand c;
    c.lt = lt;
    c.lg = lg;
    c.valid = 0;
    c.score = 0.0f;
    c.f = -1;
    c.thr = -1;
    if (owner) {
        c.f = a.feats[k];
        c.thr = thr;
        const int rt = tc - lt;
        const float ws = (wsum < 1e-12f) ? 1e-12f : wsum;
        const float var = M2 / ws;
        const float sd = sqrtf((0.0f < var) ? var : 0.0f);
        float score = mean - a.lambda_dro * sd;
        if (use_dir && agd > 0.0f) score = score + a.dir_w * (agn / agd);
        c.score = score;
        c.valid = (tc > 0 && lt >= a.msl && rt >= a.msl && !isnan(score)) ? 1 : 0;
        if (a.cand_all) store_cand(a.cand_all + ((int64_t)u * a.K + k) * T + t, c);
        store_seq(a, ((int64_t)u * a.K + k) * T + t, c);
        if (k == 0 && tid == 0) {
            a.ntot[u].count = tc;
            a.ntot[u].grad = tg;
        }
    }
    const int wave = tid / kWave;
    if (wave < a.wpt) {
        const float mine = c.valid ? c.score : -INFINITY;
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) {
            const Cand o = shfl_xor_cand(c, m);
            take_if(better(o, c), o, c);
        }
        const int band = wave_band_count(c, mine);
        if ((tid & (kWave - 1)) == 0) {
            const int W = a.ntiles * a.wpt;
            store_winner(a.cand_w + (int64_t)u * W + k * a.wpt + wave, c, band);
        }
    }
}

// Producer/consumer scorer for T <= 63 thresholds per feature. A workgroup owns up to 63
// candidates (63 / T features of one node):
//   wave 0 (consumer): one lane per candidate runs the Welford recurrence over the eras;
//   waves 1-3 (producers): compute each (candidate, era) record — gain, left grad, left
//   count, signed weight — for the NEXT chunk of eras into a double-buffered LDS ring,
//   with the chunk after that already in flight in registers.
// One barrier per chunk hands a buffer from the producers to the consumer, so the
// consumer's sequential chain (the part that cannot be parallelised without changing the
// reference's float order) runs at full wavefront width while its inputs are made alongside.
constexpr int kPcEras = kScoreChunkEras;  // eras per chunk
constexpr int kPcProducers = kBlock - kWave;
constexpr int kPcThreadsPerEra = kPcProducers / kPcEras;              // 8
constexpr int kPcPairs = (kWave + kPcThreadsPerEra - 1) / kPcThreadsPerEra;  // 8 pairs per thread

template <bool C32>
// three workgroups fit a CU's LDS: the register budget is held to the same occupancy
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(3))) void des_score_pc_kernel(ScoreArgs a) {
    extern __shared__ unsigned char smem[];
    const int tid = threadIdx.x;
    const int u = blockIdx.x / a.ntiles;
    const int tile = blockIdx.x - u * a.ntiles;
    const int Ua = a.st->u_active[a.depth];
    if (u >= Ua) return;
    const int k0 = tile * a.fts;
    const int nf = min(a.fts, a.K - k0);
    if (nf <= 0) return;
    const int T = a.T;
    const int nb = a.nb;
    const int ncand = nf * T;  // <= 63; lane 63 carries the node totals
    const int RT = a.rt;

    float* recip = reinterpret_cast<float*>(smem);
    float4* ring = reinterpret_cast<float4*>(recip + ((RT + 3) & ~3));  // [2][kPcEras][64]

    for (int i = tid; i < RT; i += kBlock) recip[i] = (i == 0) ? 0.0f : 1.0f / (float)i;

    const float lam = a.lambda_l2;
    const float alpha = a.era_alpha;
    const bool use_dir = a.dir_w != 0.0f;
    const bool unit_w = !(alpha > 0.0f);
    const int pt = nb - 1;  // prefix cells per (node, feature) in the compact planes
    const int64_t ustride = (int64_t)a.K * pt;
    const int64_t estride = (int64_t)a.U * ustride;
    const int64_t node_off = (int64_t)u * ustride;
    const int nchunks = (a.E + kPcEras - 1) / kPcEras;
    const bool consumer = tid < kWave;
    const int ptid = tid - kWave;

    // Producer slot i of this thread always maps to the same (era-in-chunk, candidate): the 8
    // producer threads of era el = ptid / 8 take candidates ptid % 8 + 8 i, so every pair of a
    // thread belongs to one era, whose totals are loaded and whose parent term is divided once
    // per thread. The plane offsets are precomputed once, so a chunk costs only loads and the
    // gain math. Only the first `np` slots can hold a record (workgroup-uniform): fewer
    // candidates per workgroup mean fewer pairs per producer lane.
    static_assert(kPcEras * kPcThreadsPerEra == kPcProducers, "one era per 8 producer threads");
    const int np = (ncand + kPcThreadsPerEra - 1) / kPcThreadsPerEra;
    const int my_el = ptid / kPcThreadsPerEra;  // the era (in chunk) of all of this thread's pairs
    int slot_el[kPcPairs], slot_c[kPcPairs];
    // plane element of the slot's (era in chunk, candidate) relative to the chunk's first era,
    // threshold included (the host checks that it fits 31 bits)
    int32_t slot_off[kPcPairs];
#pragma unroll
    for (int i = 0; i < kPcPairs; ++i) {
        const int c = ptid % kPcThreadsPerEra + kPcThreadsPerEra * i;
        const int cc = min(c, ncand - 1);
        const int kk = cc / T;
        const int t = cc - kk * T;
        const int k = k0 + kk;
        slot_el[i] = (ptid >= 0 && c < ncand) ? my_el : kPcEras;  // kPcEras: unused
        slot_c[i] = c;
        const int thr = a.thr_tab ? a.thr_tab[k * T + t] : t;
        slot_off[i] = (int32_t)((int64_t)my_el * estride + node_off + (int64_t)k * pt + thr);
    }

    // inputs of the next two chunks, in two register sets (chunk c in set c % 2, the set index
    // always a compile-time constant): this thread's era totals, and per pair the prefix count
    // and grad. Loading two chunks ahead covers the plane loads' latency when three workgroups
    // per CU stream a deep frontier's planes.
    // Loads without a branch (an element outside the chunk, the last era or this thread's
    // candidates reads the chunk's first one, always in bounds, and bit 0 of pok[S] says the
    // era is real, and with it the thread's pairs), so the compiler's wait counts stay exact and
    // the next chunk's loads stay in flight while this one is made.
    int pct[2] = {0, 0};
    float pGt[2] = {0.0f, 0.0f};
    uint32_t pok[2] = {0u, 0u};
    int pL[2][kPcPairs];
    float pGL[2][kPcPairs];
    auto prefetch = [&](int chunk, auto set) {
        constexpr int S = decltype(set)::value;
        const bool live = chunk < nchunks;
        const int e0 = live ? chunk * kPcEras : 0;
        const int ne = min(kPcEras, a.E - e0);
        const int64_t eoff = (int64_t)e0 * estride;
        const bool era_ok = live && slot_el[0] < ne;  // slot 0 is valid whenever any slot is
        const int64_t to = (int64_t)(e0 + (era_ok ? my_el : 0)) * a.U + u;  // era total
        pct[S] = a.tot_cnt[to];
        pGt[S] = a.tot_g[to];
        uint32_t ok = era_ok ? 1u : 0u;
#pragma unroll
        for (int i = 0; i < kPcPairs; ++i) {
            if (i >= np) break;
            const bool pair_ok = live && slot_el[i] < ne;
            const int64_t off = eoff + (pair_ok ? slot_off[i] : 0);
            pL[S][i] = C32 ? (int)a.cnt32[off] : (int)a.cnt[off];
            pGL[S][i] = a.g[off];
        }
        pok[S] = ok;
    };
    // Branch-free per pair (the same float operations as the reference, evaluated for every
    // pair and selected), so the divide sequences of all pairs interleave. The parent term
    // depends on the era only and is computed once per thread, with the same operations.
    auto produce = [&](int chunk, auto set) {
        constexpr int S = decltype(set)::value;
        float4* buf = ring + (chunk & 1) * kPcEras * kWave;
        const uint32_t ok = pok[S];
        const int ctot = (ok & 1u) ? pct[S] : 0;
        const bool has = ctot != 0;
        const float Gt = (ok & 1u) ? pGt[S] : 0.0f;
        const float wera = (alpha > 0.0f) ? ((float)ctot + alpha) : 1.0f;
        const float pden = (float)ctot + lam;
        const float pq = (0.5f * (Gt * Gt)) / pden;
        const float parent = (pden > 0.0f) ? pq : 0.0f;
#pragma unroll
        for (int i = 0; i < kPcPairs; ++i) {
            if (i >= np) break;
            // a pair's values are real whenever its era is (ok bit 0; a thread's pairs share one
            // era), and every output below is masked by `has` (false unless the era is real), so
            // the values of a pair outside the chunk reach no output and are not masked here
            const int Lc = pL[S][i];
            const float GLc = pGL[S][i];
            const int R = ctot - Lc;
            const float GR = Gt - GLc;
            const bool act = has && Lc > 0 && R > 0;
            const float w = act ? wera : 0.0f;  // wera >= 1 for an era with rows
            const float dL = (float)Lc + lam;
            const float dR = (float)R + lam;
            const float gfull = 0.5f * ((GLc * GLc) / dL + (GR * GR) / dR) - parent;
            bool pos = true;
            if (use_dir) {
                const float lv = -GLc / dL;
                const float rv = -GR / dR;
                pos = lv > rv;
            }
            const float gain = act ? gfull : 0.0f;
            const float wd = pos ? w : -w;  // +-0 when inactive: the consumer reads |wd| first
            // An era without rows of the node contributes L = 0, GL = +0 and weight 0, which
            // leaves every consumer sum bit-unchanged: the reference skips such eras
            // (frontier_cpu.cpp:367-369), and x + (+0) == x for every x the sums can hold
            // (they start at +0 and never become -0).
            const int L = has ? Lc : 0;
            const float GL = has ? GLc : 0.0f;
            const int el = slot_el[i];
            const int c = slot_c[i];
            // eras past the end of the last chunk get neutral records (no rows, zero
            // weight: their era total is masked to zero), so the consumer reads whole
            // batches unconditionally
            if (el < kPcEras) {
                buf[el * kWave + c] = make_float4(gain, GL, __int_as_float(L), wd);
                if (c == 0) {
                    // lane 63 pseudo-candidate: its left count / left grad sums become the
                    // node's row count and float32 era-order grad total
                    buf[el * kWave + (kWave - 1)] =
                        make_float4(0.0f, has ? Gt : 0.0f, __int_as_float(ctot), 0.0f);
                }
            }
        }
    };

    float wsum = 0.0f, mean = 0.0f, M2 = 0.0f, agn = 0.0f, agd = 0.0f, lg = 0.0f;
    int lt = 0;
    int nact = 0;  // active eras so far (unit weights: wsum == nact exactly)
    int tc = 0;
    float tg = 0.0f;
    const bool owner = tid < ncand;
    // Consumer: eras in batches of 8 — all record reads first, then the weight-sum chain with
    // its (independent) factor lookups, then the mean/M2 chain. With unit era weights (TABLE)
    // the factor w / wsum is 1/n, read from the table of IEEE 1/n (bit-identical), and
    // w * delta == delta; otherwise it is the IEEE division. The lookups are issued off the
    // mean/M2 chain (computing 1/n with exact_recip instead measured slower here: more VALU on
    // the consumer wave). Inactive eras get factor 0 and weight 0, which keep mean/M2 exactly.
    // TABLE and DIR are compile-time, so the loop has no branches.
    const bool table = unit_w && a.E < RT;
    auto consume = [&](int chunk, auto table_flag, auto dir_flag) {
        constexpr bool TABLE = decltype(table_flag)::value;
        constexpr bool DIR = decltype(dir_flag)::value;
        const float4* buf = ring + (chunk & 1) * kPcEras * kWave;
        static_assert(kPcEras % 8 == 0, "batches of 8 eras must tile a chunk");
        // All kPcEras rows of a chunk hold records (eras past the last one are neutral: no rows,
        // zero weight, which leave every sum bit-unchanged), so the batches are unrolled and
        // batch bi + 1's records are read while batch bi runs its chains.
        constexpr int kBatches = kPcEras / 8;
        float4 rec[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) rec[j] = buf[j * kWave + tid];
#pragma unroll
        for (int bi = 0; bi < kBatches; ++bi) {
            float4 nxt[8];
            if (bi + 1 < kBatches) {
#pragma unroll
                for (int j = 0; j < 8; ++j) nxt[j] = buf[((bi + 1) * 8 + j) * kWave + tid];
            }
            float fac[8], wv[8];
            bool actv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float w = fabsf(rec[j].w);
                const bool act = w > 0.0f;  // implies a row-bearing era; wsum + w > 0 then holds
                if (TABLE) {
                    nact += act ? 1 : 0;
                    fac[j] = recip[act ? nact : 0];
                } else {
                    const float wn = wsum + w;
                    fac[j] = w / (act ? wn : 1.0f);
                    wsum = wn;  // + (+0) when inactive
                }
                wv[j] = w;
                actv[j] = act;
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                lt += __float_as_int(rec[j].z);
                lg = lg + rec[j].y;
                const float gain = rec[j].x;
                const bool act = actv[j];
                // An inactive era has factor 0 and weight 0 (gain +0): mean + 0 * delta and
                // M2 + (+-0) leave both sums bit-unchanged (neither is ever -0: they start at +0
                // and an IEEE sum is -0 only when both terms are), the reference's `continue`,
                // with no select on the mean's chain.
                const float delta = gain - mean;
                const float mean_n = mean + fac[j] * delta;
                const float wdelta = TABLE ? (act ? delta : 0.0f) : wv[j] * delta;
                M2 = M2 + wdelta * (gain - mean_n);
                mean = mean_n;
                if (DIR) {
                    const float w = wv[j];
                    agn = agn + w * ((rec[j].w > 0.0f) ? 1.0f : -1.0f);  // + (+-0) when inactive
                    agd = agd + w;
                }
            }
            if (bi + 1 < kBatches) {
#pragma unroll
                for (int j = 0; j < 8; ++j) rec[j] = nxt[j];
            }
        }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    if (!consumer) {
        prefetch(0, S0{});
        prefetch(1, S1{});
        produce(0, S0{});
        prefetch(2, S0{});
    }
    __syncthreads();
    // Chunk ch: the consumer runs it while the producers make chunk ch + 1 (register set
    // (ch + 1) % 2) and then load chunk ch + 3 into the set they just used. The two roles run
    // separate loops (whole wavefronts, so each role's registers are its own) that pass the same
    // number of barriers: one per chunk. The role is read from the first lane, so the branch is
    // a scalar one: a wavefront runs only its own loop and its own barriers.
    if (__builtin_amdgcn_readfirstlane(consumer ? 1 : 0) != 0) {
        for (int ch = 0; ch < nchunks; ++ch) {
            if (owner || tid == kWave - 1) {
                if (table) {
                    if (use_dir)
                        consume(ch, std::true_type{}, std::true_type{});
                    else
                        consume(ch, std::true_type{}, std::false_type{});
                } else {
                    if (use_dir)
                        consume(ch, std::false_type{}, std::true_type{});
                    else
                        consume(ch, std::false_type{}, std::false_type{});
                }
            }
            __syncthreads();
        }
    } else {
        for (int ch = 0; ch < nchunks; ch += 2) {
            if (ch + 1 < nchunks) {
                produce(ch + 1, S1{});
                prefetch(ch + 3, S1{});
            }
            __syncthreads();
            if (ch + 1 < nchunks) {
                if (ch + 2 < nchunks) {
                    produce(ch + 2, S0{});
                    prefetch(ch + 4, S0{});
                }
                __syncthreads();
            }
        }
    }
    if (consumer) {
        if (table) wsum = (float)nact;  // exact: a sum of ones below 2^24
        tc = __shfl(lt, kWave - 1);
        tg = __shfl(lg, kWave - 1);
    }

    if (consumer) {
        Cand c;
        c.lt = lt;
        c.lg = lg;
        c.valid = 0;
        c.score = 0.0f;
        c.f = -1;
        c.thr = -1;
        if (owner) {
            const int kk = tid / T;
            const int t = tid - kk * T;
            const int k = k0 + kk;
            c.f = a.feats[k];
            c.thr = a.thr_tab ? a.thr_tab[k * T + t] : t;
            const int rt = tc - lt;
            const float ws = (wsum < 1e-12f) ? 1e-12f : wsum;
            const float var = M2 / ws;
            const float sd = sqrtf((0.0f < var) ? var : 0.0f);
            float score = mean - a.lambda_dro * sd;
            if (use_dir && agd > 0.0f) score = score + a.dir_w * (agn / agd);
            c.score = score;
            // a node without rows never splits (the reference skips it, frontier_cpu.cpp:191-193)
            c.valid = (tc > 0 && lt >= a.msl && rt >= a.msl && !isnan(score)) ? 1 : 0;
            if (a.cand_all) store_cand(a.cand_all + ((int64_t)u * a.K + k) * T + t, c);
        store_seq(a, ((int64_t)u * a.K + k) * T + t, c);
            if (tile == 0 && tid == 0) {
                a.ntot[u].count = tc;
                a.ntot[u].grad = tg;
            }
        }
        const float mine = c.valid ? c.score : -INFINITY;
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) {
            const Cand o = shfl_xor_cand(c, m);
            take_if(better(o, c), o, c);
        }
        const int band = wave_band_count(c, mine);
        if (tid == 0) store_winner(a.cand_w + (int64_t)u * a.ntiles + tile, c, band);
    }
}

// f(std::integral_constant<int, 0>{}), ..., f(std::integral_constant<int, N - 1>{}), in order
template <typename F, int... J>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, J...>) {
    (f(std::integral_constant<int, J>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}

// Producer/consumer scorer for unit era weights (era_alpha <= 0) without the direction term,
// T <= 63: the layout and the producers' gain math of des_score_pc_kernel, with the work that
// does not depend on the era chain taken off the consumer wave. With unit weights the Welford
// factor w / wsum is 1 / n, n the candidate's count of valid eras so far: the producers count
// them (per chunk, one bit per (candidate, era) in an LDS mask, then a popcount below the
// era's bit plus the count of the earlier chunks) and read the IEEE 1/n (the table of
// des_score_pc_kernel) into the record, 0 for an era that is not valid; the left counts (an
// integer sum, order-free) are added up in LDS by the producers. A record is (gain, left
// grad, factor, weight 1 or 0), and per era the consumer runs
//     lg = lg + GL;  delta = gain - mean;  mean' = mean + f * delta;
//     M2 = M2 + (w * delta) * (gain - mean');  mean = mean'
// which is the reference's recurrence (frontier_cpu.cpp:376-393) bit for bit: for a valid era
// f = 1/n and w * delta == delta; an invalid era has f = +0 and w = +0 (and gain = +0), so
// mean + (+-0) == mean and M2 + (+-0) == M2 exactly (mean is never -0: it starts at +0 and an
// IEEE sum is -0 only when both terms are), which is the reference's `continue`. Eight VALU
// operations per era and no LDS lookup on the chain, where des_score_pc_kernel takes about
// fifteen. The producers run two chunks ahead of the consumer (a chunk's masks are complete
// one barrier after its gains), still one barrier per chunk.
// NP: the most (candidate, era) pairs a producer thread holds (ceil(candidates / 8)); PF: the
// chunks whose plane values are in flight in the producers' registers. A workgroup with few
// candidates (a shallow depth: one feature of four thresholds) has the registers for a deep
// prefetch, and needs it: each chunk's loads then carry little work to hide their latency.
template <bool C32, int NP, int PF>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(3))) void des_score_pcu_kernel(ScoreArgs a) {
    extern __shared__ unsigned char smem[];
    const int tid = threadIdx.x;
    const int u = blockIdx.x / a.ntiles;
    const int tile = blockIdx.x - u * a.ntiles;
    const int Ua = a.st->u_active[a.depth];
    if (u >= Ua) return;
    const int k0 = tile * a.fts;
    const int nf = min(a.fts, a.K - k0);
    if (nf <= 0) return;
    const int T = a.T;
    const int nb = a.nb;
    const int ncand = nf * T;  // <= 63; lane 63 carries the node totals
    const int RT = a.rt;

    float* recip = reinterpret_cast<float*>(smem);
    float4* ring = reinterpret_cast<float4*>(recip + ((RT + 3) & ~3));  // [2][kPcEras][64]
    uint32_t* vmask = reinterpret_cast<uint32_t*>(ring + 2 * kPcEras * kWave);  // [3][64]
    int32_t* vbase = reinterpret_cast<int32_t*>(vmask + 3 * kWave);            // [2][64]
    int32_t* ltsum = vbase + 2 * kWave;                                         // [64]
    static_assert(kPcEras == 3 * 8, "one byte of a 32-bit mask per producer wave");

    for (int i = tid; i < RT; i += kBlock) recip[i] = (i == 0) ? 0.0f : 1.0f / (float)i;
    for (int i = tid; i < 3 * kWave; i += kBlock) vbase[i] = 0;  // counts, left sums

    const float lam = a.lambda_l2;
    const int pt = nb - 1;
    const int64_t ustride = (int64_t)a.K * pt;
    const int64_t estride = (int64_t)a.U * ustride;
    const int64_t node_off = (int64_t)u * ustride;
    const int nchunks = (a.E + kPcEras - 1) / kPcEras;
    const bool consumer = tid < kWave;
    const int ptid = tid - kWave;

    // the producer slots of des_score_pc_kernel: thread -> one era of each chunk; slot i holds
    // candidate c0 + 8 i, and bit i of slot_ok says it is a candidate of this workgroup
    const int np = min(NP, (ncand + kPcThreadsPerEra - 1) / kPcThreadsPerEra);
    const int my_el = ptid / kPcThreadsPerEra;
    const uint32_t below = (1u << (consumer ? 0 : my_el)) - 1u;  // mask bits of earlier eras
    const int c0 = ptid % kPcThreadsPerEra;
    uint32_t slot_ok = 0u;
    int32_t slot_off[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int c = c0 + kPcThreadsPerEra * i;
        const int cc = min(c, ncand - 1);
        const int kk = cc / T;
        const int t = cc - kk * T;
        const int k = k0 + kk;
        slot_ok |= (ptid >= 0 && c < ncand) ? (1u << i) : 0u;
        const int thr = a.thr_tab ? a.thr_tab[k * T + t] : t;
        slot_off[i] = (int32_t)((int64_t)my_el * estride + node_off + (int64_t)k * pt + thr);
    }

    // Register set S: the era total and per pair the prefix count and grad of one chunk, read
    // without a branch (a chunk past the end, an era past the last one or a slot without a
    // candidate reads the chunk's first elements, always in bounds) so that the compiler's
    // wait counts stay exact and the loads of later chunks stay in flight; bit 0 of pok[S]
    // says the era is real, and with it the pairs of the thread's candidate slots.
    int pct[PF];
    float pGt[PF];
    uint32_t pok[PF];
    int pL[PF][NP];
    float pGL[PF][NP];
    auto prefetch = [&](int chunk, auto set) {
        constexpr int S = decltype(set)::value;
        const bool live = chunk < nchunks;
        const int e0 = live ? chunk * kPcEras : 0;
        const int ne = min(kPcEras, a.E - e0);
        const bool era_ok = live && (slot_ok & 1u) && my_el < ne;
        const int64_t eoff = (int64_t)e0 * estride;
        const uint16_t* cb = a.cnt + eoff;
        const uint32_t* cb32 = a.cnt32 + eoff;
        const float* gb = a.g + eoff;
        const int64_t to = (int64_t)(e0 + (era_ok ? my_el : 0)) * a.U + u;
        pct[S] = a.tot_cnt[to];
        pGt[S] = a.tot_g[to];
        uint32_t ok = era_ok ? 1u : 0u;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            const bool pair_ok = era_ok && ((slot_ok >> i) & 1u);
            const uint32_t o = pair_ok ? (uint32_t)slot_off[i] : 0u;
            pL[S][i] = C32 ? (int)cb32[o] : (int)cb[o];
            pGL[S][i] = gb[o];
        }
        pok[S] = ok;
    };
    // Two producer phases per chunk, one interval apart. Phase 1 (chunk c): gains (the
    // reference's float operations, branch-free) and left grads kept in registers, and the
    // validity of every (candidate, era) pair as a mask: a producer wave holds 8 eras of the
    // chunk (lane = 8 * era + c0), so a ballot over its lanes gathers, per candidate, the byte
    // of its 8 eras, which the wave's era-0 lanes store as byte (wave - 1) of the candidate's
    // 24-bit mask in buffer c % 3 (no atomics; every byte of the mask is rewritten each time).
    // Left counts and the node's rows are summed in registers, into LDS once at the end.
    // Phase 2 (chunk c, the next interval, when its mask is complete): each valid era's 1/n,
    // the whole record into ring buffer c % 2, and the count base of chunk c + 1.
    float hg[NP], hgl[NP];
    int lt_reg[NP];
#pragma unroll
    for (int i = 0; i < NP; ++i) lt_reg[i] = 0;
    int ct_reg = 0;
    uint32_t hv = 0u;  // bit i: slot i's era is valid
    float hgt = 0.0f;  // the era's grad total (the lane-63 record)
    const int wbyte = (tid / kWave) - 1;  // producer wave 1-3: byte 0-2 of a mask
    const int lane = tid & (kWave - 1);
    auto produce1 = [&](int chunk, auto set) {
        constexpr int S = decltype(set)::value;
        const uint32_t ok = pok[S];
        const int ctot = (ok & 1u) ? pct[S] : 0;
        const bool has = ctot != 0;
        ct_reg += (c0 == 0 && (slot_ok & 1u)) ? ctot : 0;  // the node's rows, once per era
        const float Gt = (ok & 1u) ? pGt[S] : 0.0f;
        const float pden = (float)ctot + lam;
        const float pq = (0.5f * (Gt * Gt)) / pden;
        const float parent = (pden > 0.0f) ? pq : 0.0f;
        uint8_t* mskb = reinterpret_cast<uint8_t*>(vmask + (chunk % 3) * kWave);
        hv = 0u;
        hgt = has ? Gt : 0.0f;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            if (i >= np) break;
            // as in des_score_pc_kernel: every output is masked by `has` (or by the slot's
            // validity), so a pair outside the chunk needs no mask of its own
            const int Lc = pL[S][i];
            const float GLc = pGL[S][i];
            const int R = ctot - Lc;
            const float GR = Gt - GLc;
            const bool act = has && Lc > 0 && R > 0;
            const float dL = (float)Lc + lam;
            const float dR = (float)R + lam;
            const float gfull = 0.5f * ((GLc * GLc) / dL + (GR * GR) / dR) - parent;
            const int c = c0 + kPcThreadsPerEra * i;
            const bool valid = (slot_ok >> i) & 1u;
            hg[i] = act ? gfull : 0.0f;
            hgl[i] = has ? GLc : 0.0f;
            hv |= act ? (1u << i) : 0u;
            lt_reg[i] += (valid && has) ? Lc : 0;
            // bits c0 + 8 k of the ballot: era 8 (wave - 1) + k of candidate c
            const unsigned long long bal = __ballot(valid && act);
            const unsigned long long x = (bal >> c0) & 0x0101010101010101ull;
            if (lane < kPcThreadsPerEra && valid)
                mskb[c * 4 + wbyte] = (uint8_t)((x * 0x0102040810204080ull) >> 56);
        }
    };
    auto produce2 = [&](int chunk) {
        float4* buf = ring + (chunk & 1) * kPcEras * kWave;
        const uint32_t* msk = vmask + (chunk % 3) * kWave;
        const int32_t* base = vbase + (chunk & 1) * kWave;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            if (i >= np) break;
            const int c = c0 + kPcThreadsPerEra * i;
            if ((slot_ok >> i) & 1u) {
                const uint32_t m = msk[c] & 0x00FFFFFFu;  // bytes 0-2: the three producer waves
                const int b = base[c];
                const int n = b + __popc(m & below) + 1;
                const bool v = (hv >> i) & 1u;
                buf[my_el * kWave + c] = make_float4(hg[i], hgl[i], v ? recip[n] : 0.0f, v ? 1.0f : 0.0f);
                // lane 63 pseudo-candidate: its left grad sum becomes the node's float32
                // era-order grad total
                if (c == 0) buf[my_el * kWave + (kWave - 1)] = make_float4(0.0f, hgt, 0.0f, 0.0f);
                if (my_el == 0) vbase[((chunk + 1) & 1) * kWave + c] = b + __popc(m);
            }
        }
    };

    float mean = 0.0f, M2 = 0.0f, lg = 0.0f;
    const bool owner = tid < ncand;
    // one chunk's eras in batches of 8 (records of the next batch read while this one runs)
    auto consume = [&](int chunk) {
        const float4* buf = ring + (chunk & 1) * kPcEras * kWave;
        static_assert(kPcEras % 8 == 0, "batches of 8 eras must tile a chunk");
        constexpr int kBatches = kPcEras / 8;
        float4 rec[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) rec[j] = buf[j * kWave + tid];
#pragma unroll
        for (int bi = 0; bi < kBatches; ++bi) {
            float4 nxt[8];
            if (bi + 1 < kBatches) {
#pragma unroll
                for (int j = 0; j < 8; ++j) nxt[j] = buf[((bi + 1) * 8 + j) * kWave + tid];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                lg = lg + rec[j].y;
                const float gain = rec[j].x;
                const float delta = gain - mean;
                const float mean_n = mean + rec[j].z * delta;
                M2 = M2 + (rec[j].w * delta) * (gain - mean_n);
                mean = mean_n;
            }
            if (bi + 1 < kBatches) {
#pragma unroll
                for (int j = 0; j < 8; ++j) rec[j] = nxt[j];
            }
        }
    };
    // One barrier per chunk: in the interval of chunk ch the consumer runs ch while the
    // producers finish ch + 1 (phase 2), start ch + 2 (phase 1, its plane values from register
    // set (ch + 2) % PF) and load ch + 2 + PF into that set. Before it: the first PF chunks'
    // loads, chunk 0's two phases and chunk 1's phase 1 (three barriers both roles pass). The
    // producers' loop runs a whole multiple of PF intervals with no branch in it (chunks past
    // the last one load in-bounds elements marked invalid, so their phases add nothing), which
    // keeps the compiler's load wait counts exact: each chunk waits for its own loads only.
    const int nint = (nchunks + PF - 1) / PF * PF;
    if (!consumer) {
        static_for<PF>([&](auto j) { prefetch(decltype(j)::value, j); });
        __syncthreads();  // the LDS arrays are initialised
        produce1(0, std::integral_constant<int, 0>{});
        prefetch(PF, std::integral_constant<int, 0>{});
        __syncthreads();  // chunk 0's masks are complete
        produce2(0);
        produce1(1, std::integral_constant<int, 1 % PF>{});
        prefetch(PF + 1, std::integral_constant<int, 1 % PF>{});
    } else {
        __syncthreads();
        __syncthreads();
    }
    __syncthreads();
    if (__builtin_amdgcn_readfirstlane(consumer ? 1 : 0) != 0) {
        // every lane of the consumer wave runs the chain (lanes past the candidates read
        // records that were never written and store nothing)
        for (int ch = 0; ch < nint; ++ch) {
            if (ch < nchunks) consume(ch);
            __syncthreads();
        }
    } else {
        for (int ch = 0; ch < nint; ch += PF) {
            static_for<PF>([&](auto j) {  // interval ch + J; set (J + 2) % PF == (ch + J + 2) % PF
                constexpr int J = decltype(j)::value;
                produce2(ch + J + 1);
                produce1(ch + J + 2, std::integral_constant<int, (J + 2) % PF>{});
                prefetch(ch + J + 2 + PF, std::integral_constant<int, (J + 2) % PF>{});
                __syncthreads();
            });
        }
        // left counts of every candidate and the node's rows, exact integer sums
#pragma unroll
        for (int i = 0; i < NP; ++i)
            if (i < np && ((slot_ok >> i) & 1u)) atomicAdd(ltsum + c0 + kPcThreadsPerEra * i, lt_reg[i]);
        if (c0 == 0) atomicAdd(ltsum + (kWave - 1), ct_reg);
    }
    __syncthreads();

    if (consumer) {
        const int lt = ltsum[tid];
        const int tc = ltsum[kWave - 1];
        const float tg = __shfl(lg, kWave - 1);
        const float wsum = (float)vbase[(nchunks & 1) * kWave + (owner ? tid : 0)];  // valid eras
        Cand c;
        c.lt = lt;
        c.lg = lg;
        c.valid = 0;
        c.score = 0.0f;
        c.f = -1;
        c.thr = -1;
        if (owner) {
            const int kk = tid / T;
            const int t = tid - kk * T;
            const int k = k0 + kk;
            c.f = a.feats[k];
            c.thr = a.thr_tab ? a.thr_tab[k * T + t] : t;
            const int rt = tc - lt;
            const float ws = (wsum < 1e-12f) ? 1e-12f : wsum;
            const float var = M2 / ws;
            const float sd = sqrtf((0.0f < var) ? var : 0.0f);
            const float score = mean - a.lambda_dro * sd;
            c.score = score;
            c.valid = (tc > 0 && lt >= a.msl && rt >= a.msl && !isnan(score)) ? 1 : 0;
            if (a.cand_all) store_cand(a.cand_all + ((int64_t)u * a.K + k) * T + t, c);
            store_seq(a, ((int64_t)u * a.K + k) * T + t, c);
            if (tile == 0 && tid == 0) {
                a.ntot[u].count = tc;
                a.ntot[u].grad = tg;
            }
        }
        const float mine = c.valid ? c.score : -INFINITY;
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) {
            const Cand o = shfl_xor_cand(c, m);
            take_if(better(o, c), o, c);
        }
        const int band = wave_band_count(c, mine);
        if (tid == 0) store_winner(a.cand_w + (int64_t)u * a.ntiles + tile, c, band);
    }
}

// K-cut threshold table (frontier_cpu.cpp:35-109, 322-335): per sampled feature, the
// candidate thresholds are either evenly spaced or placed on the CDF of the feature's bin
// counts summed over every active node and era. One lane per feature; k <= nb-1 <= 254.
__device__ void even_cuts(int nb, int k, int32_t* out) {
    const int max_thr = max(1, nb - 1);
    const int kk = max(1, min(k, max_thr));
    int n = 0;
    if (kk == 1) {
        out[n++] = 0;
    } else {
        const double step = (double)(max_thr - 1) / (double)(kk - 1);
        for (int i = 0; i < kk; ++i) {
            const double v = round((double)i * step);  // std::round: half away from zero
            int idx = (int)llround(v);
            idx = max(0, min(idx, max_thr - 1));
            out[n++] = idx;
        }
    }
    // already ascending; drop duplicates and pad with the last value (frontier_cpu.cpp:51-55)
    int m = 0;
    for (int i = 0; i < n; ++i)
        if (m == 0 || out[m - 1] != out[i]) out[m++] = out[i];
    while (m < kk) { out[m] = out[m - 1]; ++m; }
}

// K-cut thresholds per feature (frontier_cpu.cpp:36-101, 322-330): even cuts, or mass cuts
// from the feature's count distribution over the depth's nodes and eras. One workgroup per
// feature (kKcutsBlock threads):
//   (1) cdf[b] = sum over (era, node) of the plane's prefix count of bin b (the planes hold
//       running sums over the bins, so these are the cumulative counts; bin nb-1's is the era
//       total). Thread t sums bin t % nb over every (1024 / nb)-th (era, node) pair in a
//       register, then adds it into the LDS cdf once.
//   (2) thread i < kk takes the lower bound of target i over cdf;
//   (3) thread 0 de-duplicates and tops up with even cuts (at most 2 x 254 values).
// skip: the planes hold nb + 1 bins, the last one the rows the reference leaves out of the
// histogram (frontier_cpu.cpp:278-281); the mass then counts bins < nb only, the last of them
// from the final plane cell instead of the (all-bins) era total.
constexpr int kKcutsBlock = 1024;

__global__ __launch_bounds__(kKcutsBlock) void kcuts_kernel(const uint16_t* cnt, const uint32_t* cnt32,
                                                           const int32_t* tot_cnt, int32_t E, int32_t U,
                                                           int32_t K, int32_t nb, int32_t skip, int32_t k,
                                                           int32_t mass, const Frontier* st, int32_t depth,
                                                           int32_t* thr_tab) {
    const int kf = blockIdx.x;
    if (kf >= K) return;
    const int tid = threadIdx.x;
    const int max_thr = max(1, nb - 1);
    const int kk = max(1, min(k, max_thr));
    int32_t* out = thr_tab + (int64_t)kf * kk;
    __shared__ unsigned long long cdf[256];
    __shared__ int32_t buf[512];
    __shared__ int32_t ev[256];
    if (!mass) {
        if (tid == 0) {
            even_cuts(nb, k, buf);
            for (int i = 0; i < kk; ++i) out[i] = buf[i];
        }
        return;
    }
    for (int b = tid; b < 256; b += kKcutsBlock) cdf[b] = 0ull;
    __syncthreads();
    const int Ua = st->u_active[depth];
    const int pt = nb - 1 + (skip ? 1 : 0);  // plane cells per (era, node, feature)
    const int G = kKcutsBlock / nb;          // pairs summed side by side per bin (nb <= 255)
    if (tid < G * nb) {
        const int b = tid % nb;
        const int g = tid / nb;
        unsigned long long acc = 0ull;
        const int P = E * Ua;
        // four pairs per step, their loads issued together
        for (int p0 = g; p0 < P; p0 += 4 * G) {
            unsigned long long v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int pi = p0 + q * G;
                v[q] = 0ull;
                if (pi < P) {
                    const int e = pi / Ua;
                    const int u = pi - e * Ua;
                    const int64_t base = (((int64_t)e * U + u) * K + kf) * pt;
                    if (b < nb - 1)
                        v[q] = cnt32 ? cnt32[base + b] : cnt[base + b];
                    else
                        v[q] = skip ? (cnt32 ? cnt32[base + nb - 1] : cnt[base + nb - 1])
                                    : (unsigned long long)tot_cnt[(int64_t)e * U + u];
                }
            }
            acc += (v[0] + v[1]) + (v[2] + v[3]);
        }
        atomicAdd(&cdf[b], acc);
    }
    __syncthreads();
    const long long total = (long long)cdf[nb - 1];
    if (total <= 0) {  // uniform: every thread reads the same cdf
        if (tid == 0) {
            even_cuts(nb, k, buf);
            for (int i = 0; i < kk; ++i) out[i] = buf[i];
        }
        return;
    }
    const double upper = (double)total * (1.0 - 1e-12);
    for (int i = tid; i < kk; i += kKcutsBlock) {
        const double alpha = (kk == 1) ? 0.0 : (double)i / (double)(kk - 1);
        const double target = upper * alpha;
        int idx = nb - 1;  // lower_bound over cdf; end() -> last index
        for (int b = 0; b < nb; ++b)
            if (!((double)(long long)cdf[b] < target)) { idx = b; break; }
        buf[i] = max(0, min(idx - 1, max_thr - 1));
    }
    __syncthreads();
    if (tid != 0) return;
    // buf[0..kk) ascends with the targets (the reference sorts it, which keeps it); unique, then
    // top up with the even cuts: the sorted, de-duplicated union (frontier_cpu.cpp:86-101),
    // formed by one merge of the two ascending lists
    int m = 0;
    for (int i = 0; i < kk; ++i)
        if (m == 0 || buf[m - 1] != buf[i]) buf[m++] = buf[i];
    if (m < kk) {
        even_cuts(nb, kk, ev);
        int32_t* mg = buf + 256;  // the merge's output, after buf's m values
        int ia = 0, ib = 0, n = 0;
        while (ia < m || ib < kk) {
            const bool take_a = ib >= kk || (ia < m && buf[ia] <= ev[ib]);
            const int v = take_a ? buf[ia++] : ev[ib++];
            if (n == 0 || mg[n - 1] != v) mg[n++] = v;
        }
        for (int i = 0; i < n; ++i) buf[i] = mg[i];
        m = n;
    }
    for (int i = 0; i < kk; ++i) {
        const int v = (i < m) ? buf[i] : buf[m - 1];
        out[i] = max(0, min(v, max_thr - 1));
    }
}

// Block-wide exclusive scan of one int per thread (256 threads); returns the total.
__device__ int block_exclusive_scan(int v, int* out_excl, int* s_wave) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    int incl = v;
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
        const int o = __shfl_up(incl, m);
        if (lane >= m) incl += o;
    }
    if (lane == kWave - 1) s_wave[wave] = incl;
    __syncthreads();
    int before = 0, total = 0;
    for (int w = 0; w < kBlock / kWave; ++w) {
        before += (w < wave) ? s_wave[w] : 0;
        total += s_wave[w];
    }
    __syncthreads();
    *out_excl = before + incl - v;
    return total;
}

// Decision step (booster.py:527-563 on the unique frontier), one workgroup:
//  1. one wavefront per node reduces the node's W wavefront winners (same order as the
//     scorer: valid, score, left count, feature, threshold);
//  2. per node, in parallel: split or leaf, child counts, float32 child / leaf values computed
//     in double like the reference's Python (-G / (H + lambda));
//  3. exclusive scans over the frontier order give the children's TreeBuilder ids
//     (tree_size + 2 * splits before) and their slots in the next frontier (children with
//     >= 2 * min_samples_leaf rows, left before right).
// The reference scans a node's candidates in order (subset feature, then threshold) and
// replaces its best when a candidate scores higher, or scores within 1e-12 (a float difference)
// and has more left rows, then a larger feature id, then a larger threshold
// (frontier_cpu.cpp:415-426). That relation is not transitive, so the scan order matters when
// scores lie within 1e-12 of each other. One wavefront replays it exactly from `best`, the
// node's candidate of the highest score M under the strict order of `better`:
//  * the first candidate i* of score M is always taken (every earlier score is below M), so
//    the scan's result is the scan from i* with best = c(i*);
//  * each later replacement lowers the best score by at most 1e-12, so a scan whose band
//    [M - w, M] holds fewer than w / 1e-12 candidates never takes one outside the band.
// The band doubles from w = 64e-12 until that holds, its indices are compacted in order into
// `band`, and lane 0 scans them. Scores above about 1e-5 in magnitude have float spacing beyond
// 1e-12, so there the band holds only exact ties and the pick is the strict order's.
__device__ void sequential_pick(const DecideCands& dc, int u, Cand& best) {
    const int lane = (int)(threadIdx.x & (kWave - 1));
    if (!best.valid) return;  // wave-uniform
    const int64_t n = (int64_t)dc.K * dc.T;
    const float* sc = dc.seq.score + (int64_t)u * n;
    const double M = (double)best.score;
    // the band's width w = 2^k * 1e-12 (widened as kTieBand0): the first k from 6 whose band
    // holds fewer than 2^k candidates (or 2^k > n); eight widths counted per pass over the scores
    double w = 0.0;
    for (int k0 = 6;; k0 += 8) {
        int c[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) c[q] = 0;
        for (int64_t i = lane; i < n; i += kWave) {
            const double d = M - (double)sc[i];
#pragma unroll
            for (int q = 0; q < 8; ++q) c[q] += (d <= ldexp(kTieBand0, k0 + q - 6)) ? 1 : 0;
        }
        int k_hit = -1;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            int64_t cq = c[q];
#pragma unroll
            for (int m = 1; m < kWave; m <<= 1) cq += __shfl_xor(cq, m);
            const int k = k0 + q;
            if (k_hit < 0 && (cq < (int64_t(1) << k) || (int64_t(1) << k) > n)) k_hit = k;
        }
        if (k_hit >= 0) {  // uniform
            w = ldexp(kTieBand0, k_hit - 6);
            break;
        }
    }
    int32_t* band = dc.seq.band + (int64_t)u * n;
    int64_t pos = 0;
    for (int64_t b0 = 0; b0 < n; b0 += kWave) {
        const int64_t i = b0 + lane;
        const bool in = i < n && M - (double)sc[i] <= w;
        const unsigned long long m = __ballot(in);
        if (in) band[pos + __popcll(m & ((1ull << lane) - 1ull))] = (int32_t)i;
        pos += __popcll(m);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    // The scan over the band in visiting order, 64 candidates per window: every lane loads
    // one candidate and tests it against the best so far. A window where no lane would replace
    // it is passed over; otherwise the scan runs through the window from the first lane that
    // would, on values read from the lanes' registers (uniform across the wavefront), so a band
    // where nearly every candidate replaces the last one costs register steps, not a chain of
    // dependent loads.
    float c_s = 0.0f, c_lg = 0.0f;
    int c_lt = 0, c_f = -1, c_thr = -1;
    float b_s = best.score, b_lg = best.lg;
    int b_lt = best.lt, b_f = best.f, b_thr = best.thr;
    bool started = false;
    for (int64_t j0 = 0; j0 < pos; j0 += kWave) {  // wave-uniform
        const int64_t j = j0 + lane;
        bool take = false;
        if (j < pos) {
            const int32_t i = band[j];
            const int kk = i / dc.T;
            const int t = i - kk * dc.T;
            c_s = sc[i];
            c_lt = dc.seq.lt[(int64_t)u * n + i];
            c_lg = dc.seq.lg[(int64_t)u * n + i];
            c_f = dc.feats[kk];
            c_thr = dc.thr_tab ? dc.thr_tab[kk * dc.T + t] : t;
            const bool first = !started && ((double)c_s == M);
            const bool s_gt = c_s > b_s;
            const bool near = fabsf(c_s - b_s) <= 1e-12f;
            const bool tie_win = (c_lt > b_lt) | ((c_lt == b_lt) & ((c_f > b_f) | ((c_f == b_f) & (c_thr > b_thr))));
            take = first | (started & (s_gt | (near & tie_win)));
        }
        const unsigned long long m = __ballot(take);
        if (m == 0ull) continue;
        const int l0 = __ffsll((long long)m) - 1;
        const int l1 = (int)min<int64_t>((int64_t)kWave, pos - j0);
        for (int l = l0; l < l1; ++l) {  // uniform: the same steps on every lane
            const float sv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c_s), l));
            const int lt = __builtin_amdgcn_readlane(c_lt, l);
            const int f = __builtin_amdgcn_readlane(c_f, l);
            const int thr = __builtin_amdgcn_readlane(c_thr, l);
            const bool first = !started && ((double)sv == M);
            const bool s_gt = sv > b_s;
            const bool near = fabsf(sv - b_s) <= 1e-12f;
            const bool tie_win = (lt > b_lt) | ((lt == b_lt) & ((f > b_f) | ((f == b_f) & (thr > b_thr))));
            if (first | (started & (s_gt | (near & tie_win)))) {
                b_s = sv;
                b_lt = lt;
                b_lg = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c_lg), l));
                b_f = f;
                b_thr = thr;
                started = true;
            }
        }
    }
    best.score = b_s;
    best.lt = b_lt;
    best.lg = b_lg;
    best.f = b_f;
    best.thr = b_thr;
    best.valid = 1;
}

// Candidates of the node scoring below its best score M but within kTieBand0 of it, as far
// as the wavefront winners show them: a winner in [M - kTieBand0, M) is one, and a winner
// scoring M brings its wavefront's count of such candidates (a candidate in that band belongs
// to a wavefront whose winner scores between it and M, so none is missed). Zero means the
// strict argmax is the sequential pick. Summed by the calling threads over winners w0,
// w0 + step, ...
__device__ __forceinline__ int band_bound_part(const DecideCands& dc, int u, int W, int w0, int step,
                                               const Cand& best) {
    int n = 0;
    if (!best.valid) return 0;
    for (int w = w0; w < W; w += step) {
        const pb_candidate* r = dc.cand_w + (int64_t)u * W + w;
        if (r->valid && (double)r->score >= (double)best.score - kTieBand0)
            n += (r->score < best.score ? 1 : 0) + r->reserved[0];
    }
    return n;
}

// Phase 1 of the decision step when the candidate set is wide (many wavefront winners per node,
// e.g. 254 thresholds x 500 features): one workgroup per node slot reduces that node's W winners
// under the strict order of `better` (so the winner is the same whatever the reduction order),
// then its first wavefront replays the reference's sequential pick.
__global__ __launch_bounds__(kBlock) void node_best_kernel(DecideCands dc, const Frontier* st,
                                                        int32_t depth, pb_candidate* node_best) {
    __shared__ Cand s_best[kBlock / kWave];
    const int u = blockIdx.x;
    if (u >= st->u_active[depth]) return;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int W = dc.W;
    Cand best;
    best.valid = 0; best.score = 0.0f; best.lt = 0; best.lg = 0.0f; best.f = -1; best.thr = -1;
    for (int w = threadIdx.x; w < W; w += kBlock) {
        const Cand c = load_cand(dc.cand_w + (int64_t)u * W + w);
        take_if(better(c, best), c, best);
    }
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
        const Cand o = shfl_xor_cand(best, m);
        take_if(better(o, best), o, best);
    }
    __shared__ int s_band[kBlock / kWave];
    if (lane == 0) s_best[wave] = best;
    __syncthreads();
    best = s_best[0];
    for (int i = 1; i < kBlock / kWave; ++i) take_if(better(s_best[i], best), s_best[i], best);
    int band = band_bound_part(dc, u, W, threadIdx.x, kBlock, best);
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) band += __shfl_xor(band, m);
    if (lane == 0) s_band[wave] = band;
    __syncthreads();
    if (wave == 0) {
        int nb = 0;
        for (int i = 0; i < kBlock / kWave; ++i) nb += s_band[i];
        if (nb > 0) sequential_pick(dc, u, best);
        if (lane == 0) store_cand(node_best + u, best);
    }
}

// W == 0: node_best already holds each node's winner (node_best_kernel ran first).
__global__ __launch_bounds__(kBlock) void decide_kernel(DecideCands dc, int32_t W,
                                                    const NodeTotal* ntot, Frontier* st,
                                                    int32_t depth, int32_t msl, double lambda_l2,
                                                    const int32_t* cur_ids, int32_t* next_ids,
                                                    SplitRule* rules, pb_decision* dec,
                                                    float* values, pb_candidate* node_best) {
    __shared__ int s_wave[kBlock / kWave];
    __shared__ int s_carry[2];
    const int Ua = st->u_active[depth];
    const int tree_size0 = st->tree_size;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    pb_decision* dd = dec + ((1 << depth) - 1);

    for (int u = wave; W > 0 && u < Ua; u += kBlock / kWave) {
        Cand best;
        best.valid = 0; best.score = 0.0f; best.lt = 0; best.lg = 0.0f; best.f = -1; best.thr = -1;
        for (int w = lane; w < W; w += kWave) {
            const Cand c = load_cand(dc.cand_w + (int64_t)u * W + w);
            take_if(better(c, best), c, best);
        }
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) {
            const Cand o = shfl_xor_cand(best, m);
            take_if(better(o, best), o, best);
        }
        int band = band_bound_part(dc, u, W, lane, kWave, best);
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) band += __shfl_xor(band, m);
        if (band > 0) sequential_pick(dc, u, best);
        if (lane == 0) store_cand(node_best + u, best);
    }
    if (threadIdx.x == 0) {
        s_carry[0] = 0;
        s_carry[1] = 0;
    }
    __syncthreads();

    for (int base = 0; base < Ua; base += kBlock) {
        const int u = base + threadIdx.x;
        const bool in = u < Ua;
        Cand best;
        best.valid = 0; best.lt = 0; best.lg = 0.0f; best.f = -1; best.thr = -1; best.score = 0.0f;
        NodeTotal nt;
        nt.count = 0;
        nt.grad = 0.0f;
        if (in) {
            best = load_cand(node_best + u);
            nt = ntot[u];
        }
        const int split = (in && best.valid) ? 1 : 0;
        const int lc = split ? best.lt : 0;
        const int rc = split ? nt.count - lc : 0;
        const int la = (split && lc >= 2 * msl) ? 1 : 0;
        const int ra = (split && rc >= 2 * msl) ? 1 : 0;
        int split_before, act_before;
        const int split_total = block_exclusive_scan(split, &split_before, s_wave);
        const int act_total = block_exclusive_scan(la + ra, &act_before, s_wave);
        split_before += s_carry[0];
        act_before += s_carry[1];
        if (in) {
            SplitRule r;
            pb_decision d;
            d.node_id = cur_ids[u];
            d.node_grad = nt.grad;
            d.node_count = nt.count;
            d.reserved = 0;
            if (split) {
                const int left_id = tree_size0 + 2 * split_before;
                r.feature = best.f;
                r.threshold = best.thr;
                r.left_id = left_id;
                r.next_slot[0] = la ? (uint16_t)act_before : (uint16_t)PB_INACTIVE;
                r.next_slot[1] = ra ? (uint16_t)(act_before + la) : (uint16_t)PB_INACTIVE;
                if (la) next_ids[act_before] = left_id;
                if (ra) next_ids[act_before + la] = left_id + 1;
                d.split = 1;
                d.feature = best.f;
                d.threshold = best.thr;
                d.score = best.score;
                d.left_grad = best.lg;
                d.left_hess = (float)lc;
                d.right_grad = nt.grad - best.lg;
                d.right_hess = (float)nt.count - d.left_hess;
                d.left_count = lc;
                d.right_count = rc;
                d.left_id = left_id;
                d.right_id = left_id + 1;
                values[left_id] = (float)(-(double)d.left_grad / ((double)d.left_hess + lambda_l2));
                values[left_id + 1] =
                    (float)(-(double)d.right_grad / ((double)d.right_hess + lambda_l2));
            } else {
                r.feature = -1;
                r.threshold = -1;
                r.left_id = -1;
                r.next_slot[0] = r.next_slot[1] = (uint16_t)PB_INACTIVE;
                d.split = 0;
                d.feature = -1;
                d.threshold = 0;
                d.score = 0.0f;
                d.left_grad = d.left_hess = d.right_grad = d.right_hess = 0.0f;
                d.left_count = d.right_count = 0;
                d.left_id = d.right_id = -1;
                values[d.node_id] = (nt.count == 0)
                    ? 0.0f
                    : (float)(-(double)nt.grad / ((double)(float)nt.count + lambda_l2));
            }
            rules[u] = r;
            dd[u] = d;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            s_carry[0] += split_total;
            s_carry[1] += act_total;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        st->tree_size = tree_size0 + 2 * s_carry[0];
        if (depth + 1 <= PB_MAX_DEPTH) st->u_active[depth + 1] = s_carry[1];
    }
}

// The sequential pick of sequential_pick for plain candidate records (pb_candidate [M][n] in
// visiting order: the cand_all output of the scorer): one wavefront per node finds the highest
// score M among the candidates the reference can take (valid, not NaN, above -inf), then
// replays the reference's scan (frontier_cpu.cpp:415-426) over the band of candidates near M,
// compacted in order into `band` ([M][n] scratch). A node without such a candidate gets
// valid = 0, feature = threshold = -1.
__global__ __launch_bounds__(kBlock) void pick_sequential_kernel(const pb_candidate* __restrict__ cand, int32_t M,
                                                                 int64_t n, int32_t* __restrict__ band_all,
                                                                 pb_candidate* __restrict__ out) {
    const int lane = (int)(threadIdx.x & (kWave - 1));
    const int u = (int)blockIdx.x * (kBlock / kWave) + (int)(threadIdx.x / kWave);
    if (u >= M) return;  // wave-uniform
    const pb_candidate* c = cand + (int64_t)u * n;
    float top = -INFINITY;
    for (int64_t i = lane; i < n; i += kWave) {
        const float sv = c[i].score;
        top = (c[i].valid != 0 && sv > top) ? sv : top;  // NaN never compares above
    }
#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) top = fmaxf(top, __shfl_xor(top, m));
    Cand cur;
    cur.score = -INFINITY;
    cur.lt = -1;
    cur.lg = 0.0f;
    cur.f = -1;
    cur.thr = -1;
    cur.valid = 0;
    if (top > -INFINITY) {  // wave-uniform
        const double Mx = (double)top;
        double w = 0.0;
        for (int k = 6;; ++k) {
            w = ldexp(kTieBand0, k - 6);
            int64_t cnt = 0;
            for (int64_t i = lane; i < n; i += kWave) cnt += (c[i].valid != 0 && (double)c[i].score >= Mx - w) ? 1 : 0;
#pragma unroll
            for (int m = 1; m < kWave; m <<= 1) cnt += __shfl_xor(cnt, m);
            if (cnt < (int64_t(1) << k) || (int64_t(1) << k) > n) break;
        }
        int32_t* band = band_all + (int64_t)u * n;
        int64_t pos = 0;
        for (int64_t b0 = 0; b0 < n; b0 += kWave) {
            const int64_t i = b0 + lane;
            const bool in = i < n && c[i].valid != 0 && (double)c[i].score >= Mx - w;
            const unsigned long long msk = __ballot(in);
            if (in) band[pos + __popcll(msk & ((1ull << lane) - 1ull))] = (int32_t)i;
            pos += __popcll(msk);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0) {
            bool started = false;
            for (int64_t j = 0; j < pos; ++j) {
                const Cand cj = load_cand(c + band[j]);
                const bool first = !started && ((double)cj.score == Mx);
                const bool s_gt = cj.score > cur.score;
                const bool near = fabsf(cj.score - cur.score) <= 1e-12f;
                const bool tie_win = (cj.lt > cur.lt) | ((cj.lt == cur.lt) & ((cj.f > cur.f) | ((cj.f == cur.f) & (cj.thr > cur.thr))));
                const bool take = first | (started & (s_gt | (near & tie_win)));
                take_if(take, cj, cur);
                started = started | first;
            }
        }
    }
    if (lane == 0) store_cand(out + u, cur);
}


// Segment-mode scorer (SegScoreArgs). Workgroup (slot u, feature tile): thread i owns the
// candidates c = i + 256 j (feature c / T of the tile, threshold c % T). Per era with rows of
// the node: (1) every thread adds its rows' addends (grad_addend, the era's scale) into the
// tile's LDS histogram [FT][256]; (2) wave w scans the bins of features w, w + 4, ... exactly
// (64-bit integer prefixes), writes each prefix count and its grad rounded once to float (the
// values the plane path writes) and clears the histogram; (3) every thread runs the wide
// scorer's era step on its candidates. Two barriers per era: the next era's histogram is built
// while no thread still reads the prefixes of this one only after the barrier that ends (1).
// DIR: the direction term is on (dir_w != 0); UNIT: equal era weights (era_alpha <= 0).
// Occupancy targets: 4 features fit 64 VGPRs (8 waves per SIMD) without the direction term and
// 77 with it (6 waves); narrower tiles keep the compiler's own allocation (4 = no constraint).
template <int FT, bool DIR>
constexpr int seg_waves_per_eu() { return FT == 4 ? (DIR ? 6 : 8) : 4; }

template <int FT, bool DIR, bool UNIT>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(seg_waves_per_eu<FT, DIR>()))) void seg_score_kernel(SegScoreArgs a) {
    constexpr int kCpt = (FT * 254 + kBlock - 1) / kBlock;  // candidates per thread (T <= 254)
    extern __shared__ unsigned char smem[];
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    // blockIdx -> (node, feature tile). tile_major (many nodes): XCD-aware, the 8 XCDs take
    // blocks round-robin and XCD x walks tiles x, x + 8, ... with the node fastest. The
    // workgroups resident on one XCD at a time are then mostly all the nodes of one tile: they
    // gather the same columns' lines era by era (a deep node holds one row in tens of a line's),
    // so the XCD's L2 serves each line to every node instead of each node fetching it.
    // Otherwise node-major: a node's tiles are consecutive blocks.
    int u, tile;
    if (a.tile_major) {
        const int i = (int)(blockIdx.x >> 3);
        const int jt = i / a.mu;
        u = i - jt * a.mu;
        tile = (int)(blockIdx.x & 7) + 8 * jt;
    } else {
        u = (int)blockIdx.x / a.ntiles;
        tile = (int)blockIdx.x - u * a.ntiles;
    }
    const int Ua = a.st->u_active[a.depth];
    if (u >= Ua || tile >= a.ntiles) return;
    const int k0 = tile * FT;
    const int nf = min(FT, a.K - k0);
    if (nf <= 0) return;
    const int nb = a.nb;
    const int T = a.T;
    const int ncand = nf * T;
    const int RT = a.rt;
    unsigned long long* hist = reinterpret_cast<unsigned long long*>(smem);  // [FT][256]
    int32_t* pc = reinterpret_cast<int32_t*>(hist + FT * 256);                 // [FT][256]
    float* pg = reinterpret_cast<float*>(pc + FT * 256);                       // [FT][256]
    float* eg = pg + FT * 256;                                                 // [2]: Gt, parent
    float* recip = eg + 4;                                                     // [RT]
    for (int i = tid; i < FT * 256; i += kBlock) hist[i] = 0ull;
    for (int i = tid; i < RT; i += kBlock) recip[i] = (i == 0) ? 0.0f : 1.0f / (float)i;

    const uint8_t* col[FT];
#pragma unroll
    for (int f = 0; f < FT; ++f) col[f] = a.bins + (int64_t)a.feats[k0 + min(f, nf - 1)] * a.ld;

    const float lam = a.lambda_l2;
    const float alpha = a.era_alpha;
    float wsum[kCpt], mean[kCpt], M2[kCpt], agn[kCpt], agd[kCpt], lg[kCpt];
    int lt[kCpt];
#pragma unroll
    for (int j = 0; j < kCpt; ++j) {
        wsum[j] = mean[j] = M2[j] = agn[j] = agd[j] = lg[j] = 0.0f;
        lt[j] = 0;
    }
    int tc = 0;
    float tg = 0.0f;
    int coff[kCpt];  // LDS index f * 256 + t of each candidate (0 past the last: never stored)
#pragma unroll
    for (int j = 0; j < kCpt; ++j) {
        const int c = tid + j * kBlock;
        const int f = c / T;
        coff[j] = c < ncand ? f * 256 + (c - f * T) : 0;
    }
    __syncthreads();

    for (int e = 0; e < a.E; ++e) {
        const int s0 = a.seg[(int64_t)e * a.segw + u];
        const int s1 = a.seg[(int64_t)e * a.segw + u + 1];
        const int ctot = s1 - s0;
        if (ctot <= 0) continue;  // workgroup-uniform: the node has no rows in this era
        const int sh = a.sh_era[e];
        const float scale = ldexpf(1.0f, sh);
        const double inv_scale = ldexp(1.0, -sh);
        // (1) histogram of the node's rows of this era
        if (ctot <= kBlock) {  // one row per thread (waves past the rows skip it)
            const int r = s0 + tid;
            if (r < s1) {
                const float gv = a.g[r];
                const int rb = a.row[r];
                uint32_t bv[FT];
#pragma unroll
                for (int f = 0; f < FT; ++f) bv[f] = col[f][rb];
                const unsigned long long add = grad_addend(gv, scale);
#pragma unroll
                for (int f = 0; f < FT; ++f)
                    if (f < nf) atomicAdd(hist + f * 256 + bv[f], add);
            }
        } else {
            // four rows per thread per step, all loads issued before the atomics
            for (int r0 = s0 + tid; r0 < s1; r0 += 4 * kBlock) {
                float gv[4];
                uint32_t bv[4][FT];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int r = min(r0 + q * kBlock, s1 - 1);
                    gv[q] = a.g[r];
                    const int rb = a.row[r];
#pragma unroll
                    for (int f = 0; f < FT; ++f) bv[q][f] = col[f][rb];
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (r0 + q * kBlock >= s1) break;
                    const unsigned long long add = grad_addend(gv[q], scale);
#pragma unroll
                    for (int f = 0; f < FT; ++f)
                        if (f < nf) atomicAdd(hist + f * 256 + bv[q][f], add);
                }
            }
        }
        __syncthreads();
        // (2) exact prefixes, one wave per feature; the era total from the tile's first feature
        for (int f = wave; f < nf; f += kBlock / kWave) {
            unsigned long long v[4];
            unsigned long long run = 0ull;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                unsigned long long* cell = hist + f * 256 + 4 * lane + j;
                run += *cell;
                v[j] = run;
                *cell = 0ull;
            }
            const unsigned long long excl = wave_scan_incl_u64(run) - run;  // lanes before this one
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int b = 4 * lane + j;
                const unsigned long long tot = excl + v[j];
                const uint32_t cnt = (uint32_t)(tot & ((1ull << kCountBits) - 1ull));
                const long long Q = ((long long)(tot - cnt)) >> kCountBits;
                const float gs = (float)((double)Q * inv_scale);
                if (b < T) {
                    pc[f * 256 + b] = (int32_t)cnt;
                    pg[f * 256 + b] = gs;
                } else if (b == nb - 1 && f == 0) {
                    const float pden = (float)ctot + lam;
                    eg[0] = gs;
                    eg[1] = (pden > 0.0f) ? (0.5f * (gs * gs)) / pden : 0.0f;
                }
            }
        }
        __syncthreads();
        // (3) the era step of every candidate (the wide scorer's operations)
        const float Gt = eg[0];
        const float parent = eg[1];
        tc += ctot;
        tg = tg + Gt;
        const float wera = UNIT ? 1.0f : (float)ctot + alpha;
        // branch-free: every candidate evaluates the era record and selects (the same float
        // operations as the wide scorer where it is taken)
#pragma unroll
        for (int j = 0; j < kCpt; ++j) {
            const int L = pc[coff[j]];
            const float GL = pg[coff[j]];
            const int R = ctot - L;
            const float GR = Gt - GL;
            const bool act = L > 0 && R > 0;
            const float w = act ? wera : 0.0f;
            const float dL = (float)L + lam;
            const float dR = (float)R + lam;
            const float gfull = 0.5f * ((GL * GL) / dL + (GR * GR) / dR) - parent;
            const float gain = act ? gfull : 0.0f;
            lt[j] += L;
            lg[j] = lg[j] + GL;
            const float wn = wsum[j] + w;
            float fac;
            if (UNIT) {
                const int wi = (int)wn;
                fac = wi < RT ? recip[act ? wi : 0] : w / (act ? wn : 1.0f);
            } else {
                fac = w / (act ? wn : 1.0f);
            }
            // an inactive era has w = +0, gain = +0 and factor 0, so every sum below takes a +-0
            // term and keeps its bits (none is ever -0: each starts at +0, and an IEEE sum is -0
            // only when both terms are): the reference's `continue`, with no selects
            wsum[j] = wn;
            const float delta = gain - mean[j];
            const float mean_n = mean[j] + fac * delta;
            M2[j] = M2[j] + (w * delta) * (gain - mean_n);
            mean[j] = mean_n;
            if (DIR) {
                const float lv = -GL / dL;
                const float rv = -GR / dR;
                const bool pos = lv > rv;
                agn[j] = agn[j] + w * (pos ? 1.0f : -1.0f);
                agd[j] = agd[j] + w;
            }
        }
    }

    // scores, the visiting-order records, and one winner per wavefront
    Cand best;
    best.score = 0.0f;
    best.lt = 0;
    best.lg = 0.0f;
    best.f = -1;
    best.thr = -1;
    best.valid = 0;
    float mine[kCpt];
#pragma unroll
    for (int j = 0; j < kCpt; ++j) {
        const int c = tid + j * kBlock;
        mine[j] = -INFINITY;
        if (c >= ncand) continue;
        const int f = c / T;
        const int t = c - f * T;
        Cand cc;
        cc.lt = lt[j];
        cc.lg = lg[j];
        cc.f = a.feats[k0 + f];
        cc.thr = t;
        const int rt = tc - lt[j];
        const float ws = (wsum[j] < 1e-12f) ? 1e-12f : wsum[j];
        const float var = M2[j] / ws;
        const float sd = sqrtf((0.0f < var) ? var : 0.0f);
        float score = mean[j] - a.lambda_dro * sd;
        if (DIR && agd[j] > 0.0f) score = score + a.dir_w * (agn[j] / agd[j]);
        cc.score = score;
        cc.valid = (tc > 0 && lt[j] >= a.msl && rt >= a.msl && !isnan(score)) ? 1 : 0;
        const int64_t i = ((int64_t)u * a.K + k0 + f) * T + t;
        a.seq.score[i] = cc.valid ? cc.score : -INFINITY;
        a.seq.lt[i] = cc.lt;
        a.seq.lg[i] = cc.lg;
        mine[j] = cc.valid ? cc.score : -INFINITY;
        take_if(better(cc, best), cc, best);
    }
    if (tile == 0 && tid == 0) {
        a.ntot[u].count = tc;
        a.ntot[u].grad = tg;
    }
    if (wave < a.wpt) {
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) {
            const Cand o = shfl_xor_cand(best, m);
            take_if(better(o, best), o, best);
        }
        // this wave's candidates below its winner but within kTieBand0 of it
        int band = 0;
#pragma unroll
        for (int j = 0; j < kCpt; ++j)
            band += (best.valid && mine[j] < best.score && (double)mine[j] >= (double)best.score - kTieBand0) ? 1 : 0;
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) band += __shfl_xor(band, m);
        if (lane == 0) store_winner(a.cand_w + (int64_t)u * (a.ntiles * a.wpt) + tile * a.wpt + wave, best, band);
    }
}

}  // namespace

ScoreShape score_shape(int32_t K, int32_t T, int32_t E, int32_t nodes, int32_t target_wgs) {
    ScoreShape sh;
    sh.rt = std::max(2, std::min<int32_t>(E + 1, 4096));
    if (T < kWave) {
        // producer/consumer kernel: a 64-lane consumer wavefront per workgroup, up to 63
        // candidate lanes + one lane for the node totals. A workgroup walks all eras in
        // order (the era recurrence is sequential), so its duration barely depends on how
        // many candidates it carries: spread the candidates over about `target_wgs`
        // workgroups (three fit in a CU's LDS) rather than packing 63 per workgroup.
        const int64_t want = std::max<int64_t>(1, target_wgs);
        const int64_t per = ((int64_t)K * std::max(1, nodes) + want - 1) / want;  // features / WG
        sh.fts = (int)std::max<int64_t>(1, std::min<int64_t>({(int64_t)K, (kWave - 1) / T, per}));
        sh.ntiles = (K + sh.fts - 1) / sh.fts;
        sh.wpt = 1;
        sh.ec = kPcEras;
        // table, record ring, then (unit-weight kernel) the valid-era masks, counts and left sums
        sh.lds_bytes = (size_t)((sh.rt + 3) & ~3) * 4 + 2 * (size_t)kPcEras * kWave * 16 + 6 * kWave * 4;
        return sh;
    }
    // many thresholds per feature (nb > 65): one feature per workgroup, all threads alternate
    // between the two phases
    sh.fts = 1;
    const int ncand = T;
    sh.ntiles = K;
    sh.wpt = (ncand + kWave - 1) / kWave;
    sh.ec = std::max(1, (kPairs * kBlock) / ncand);
    sh.lds_bytes = (size_t)sh.rt * 4 + 2 * ((size_t)sh.ec * ncand * 16 + (size_t)sh.ec * 8);
    return sh;
}

// Launch shape of des_score_kernel for any T: one feature per workgroup, its T candidates on
// the first T threads, eras staged in chunks of `ec` (about kPairs (candidate, era) pairs per
// thread).
ScoreShape score_shape_classic(int32_t K, int32_t T, int32_t E) {
    ScoreShape sh;
    sh.rt = std::max(2, std::min<int32_t>(E + 1, 4096));
    sh.fts = 1;
    sh.ntiles = K;
    sh.wpt = (T + kWave - 1) / kWave;
    sh.ec = std::max(1, (kPairs * kBlock) / std::max(1, T));
    sh.lds_bytes = (size_t)sh.rt * 4 + 2 * ((size_t)sh.ec * T * 16 + (size_t)sh.ec * 8);
    return sh;
}

// Launches kernel `fn` with `lds_bytes` of dynamic LDS (raising the limit past 64 KiB first).
template <typename K>
hipError_t launch_lds(K fn, int grid, int block, size_t lds_bytes, hipStream_t s, const ScoreArgs& a) {
    if (lds_bytes > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fn, dim3(grid), dim3(block), lds_bytes, s, a);
    return hipGetLastError();
}

template <bool C32>
hipError_t launch_score_c(const ScoreArgs& a, int grid, size_t lds_bytes, hipStream_t s) {
    // rows past the reference's bins (score_shape_classic's launch shape)
    if (a.skip_last) return launch_lds(des_score_kernel<C32, true>, grid, kBlock, lds_bytes, s, a);
    if (a.T >= kWave) {
        if (a.staged) return launch_lds(des_score_kernel<C32, false>, grid, kBlock, lds_bytes, s, a);
        // the wide scorer computes 1/n (exact_recip) instead of a table; one thread per
        // threshold, whole wavefronts up to T (T <= 254)
        return launch_lds(des_score_wide_kernel<C32>, grid, (a.T + kWave - 1) / kWave * kWave, 0, s, a);
    }
    // unit era weights, no direction term, the 1/n table covering every era: the
    // producer/consumer kernel with the factors made by the producers, its prefetch depth by
    // the pairs per producer thread (ceil(candidates per workgroup / 8))
    // Measured at the 2.4M x 2376 x 5-bin panel: with one pair per producer thread (4
    // candidates per workgroup, depths 0-2) it takes 21-23 us per depth against 29-31; from
    // two pairs on its producers' extra work outweighs the shorter chain (depth 3: 38.6
    // against 36.8 us, depth 5: 79 against 54). PB_SCORE_PC: 0 that rule, 1 never, 2 always.
    const bool unit = !(a.era_alpha > 0.0f) && a.dir_w == 0.0f && a.E < a.rt && a.pc_classic != 1;
    const int np = (a.fts * a.T + kPcThreadsPerEra - 1) / kPcThreadsPerEra;
    if (!unit || (np > 1 && a.pc_classic != 2))
        return launch_lds(des_score_pc_kernel<C32>, grid, kBlock, lds_bytes, s, a);
    if (np <= 1) return launch_lds(des_score_pcu_kernel<C32, 1, 6>, grid, kBlock, lds_bytes, s, a);
    if (np <= 2) return launch_lds(des_score_pcu_kernel<C32, 2, 4>, grid, kBlock, lds_bytes, s, a);
    if (np <= 4) return launch_lds(des_score_pcu_kernel<C32, 4, 3>, grid, kBlock, lds_bytes, s, a);
    return launch_lds(des_score_pcu_kernel<C32, 8, 2>, grid, kBlock, lds_bytes, s, a);
}

hipError_t launch_score(const ScoreArgs& a, int grid, size_t lds_bytes, hipStream_t s) {
    return a.cnt32 ? launch_score_c<true>(a, grid, lds_bytes, s) : launch_score_c<false>(a, grid, lds_bytes, s);
}

hipError_t launch_kcuts(const uint16_t* cnt, const uint32_t* cnt32, const int32_t* tot_cnt, int32_t E,
                        int32_t U, int32_t K, int32_t nb, int32_t skip, int32_t k, int32_t mass,
                        const Frontier* st, int32_t depth, int32_t* thr_tab, hipStream_t s) {
    if (K <= 0) return hipSuccess;
    hipLaunchKernelGGL(kcuts_kernel, dim3(K), dim3(kKcutsBlock), 0, s, cnt, cnt32, tot_cnt, E, U, K,
                       nb, skip, k, mass, st, depth, thr_tab);
    return hipGetLastError();
}

hipError_t launch_decide(const DecideCands& dc, int32_t max_nodes, const NodeTotal* ntot,
                         Frontier* st, int32_t depth, int32_t msl, double lambda_l2,
                         const int32_t* cur_ids, int32_t* next_ids, SplitRule* rules,
                         pb_decision* dec, float* values, pb_candidate* node_best,
                         hipStream_t s) {
    // the per-node reductions in parallel, one workgroup per node slot, for wide candidate sets
    // (one workgroup walking max_nodes x W winners took ~0.1 ms per depth at 128 x 2000) and
    // whenever there are more nodes than the decision workgroup has wavefronts (each wavefront
    // would reduce its nodes one after another: 32 nodes x 24 winners took 17 us in one
    // workgroup, against about 6 us for both launches)
    int32_t w_decide = dc.W;
    if ((int64_t)max_nodes * dc.W >= (int64_t)32 * 1024 || max_nodes > kBlock / kWave) {
        hipLaunchKernelGGL(node_best_kernel, dim3(max_nodes), dim3(kBlock), 0, s, dc, st, depth,
                           node_best);
        w_decide = 0;
    }
    hipLaunchKernelGGL(decide_kernel, dim3(1), dim3(kBlock), 0, s, dc, w_decide, ntot, st, depth,
                       msl, lambda_l2, cur_ids, next_ids, rules, dec, values, node_best);
    return hipGetLastError();
}

hipError_t launch_pick_sequential(const pb_candidate* cand, int32_t M, int64_t n, int32_t* band,
                                  pb_candidate* out, hipStream_t s) {
    if (M <= 0) return hipSuccess;
    const int per_block = kBlock / kWave;
    hipLaunchKernelGGL(pick_sequential_kernel, dim3((M + per_block - 1) / per_block), dim3(kBlock), 0, s, cand, M,
                       n, band, out);
    return hipGetLastError();
}

int32_t seg_score_fts(int32_t nodes, int32_t K) {
    int32_t ft = kSegMaxFt;
    while (ft > 1 && (int64_t)nodes * ((K + ft - 1) / ft) < 1024) ft /= 2;
    return ft;
}

size_t seg_score_lds_bytes(int32_t fts, int32_t rt) {
    return (size_t)fts * 256 * (8 + 4 + 4) + 4 * 4 + (size_t)rt * 4;
}

hipError_t launch_seg_score(const SegScoreArgs& args, int32_t max_nodes, hipStream_t s) {
    SegScoreArgs a = args;
    a.mu = max_nodes;
    // tile_major: every XCD gets ceil(ntiles / 8) tiles x max_nodes blocks (past the last tile
    // they exit)
    const int64_t grid = a.tile_major ? 8 * (int64_t)((a.ntiles + 7) / 8) * max_nodes
                                      : (int64_t)max_nodes * a.ntiles;
    if (grid <= 0) return hipSuccess;
    if (grid > INT32_MAX || a.T > 254 || a.T != a.nb - 1) return hipErrorInvalidValue;
    const size_t lds = seg_score_lds_bytes(a.fts, a.rt);
    auto go = [&](auto kern) -> hipError_t {
        const void* fn = reinterpret_cast<const void*>(kern);
        if (lds > 64 * 1024) {
            hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return e;
        }
        hipLaunchKernelGGL(kern, dim3((unsigned)grid), dim3(kBlock), lds, s, a);
        return hipGetLastError();
    };
    const bool dir = a.dir_w != 0.0f;
    const bool unit = !(a.era_alpha > 0.0f);
    auto pick = [&](auto ft) -> hipError_t {
        constexpr int FT = decltype(ft)::value;
        if (dir) return unit ? go(seg_score_kernel<FT, true, true>) : go(seg_score_kernel<FT, true, false>);
        return unit ? go(seg_score_kernel<FT, false, true>) : go(seg_score_kernel<FT, false, false>);
    };
    switch (a.fts) {
        case 1: return pick(std::integral_constant<int, 1>{});
        case 2: return pick(std::integral_constant<int, 2>{});
        case 4: return pick(std::integral_constant<int, 4>{});
        default: return hipErrorInvalidValue;
    }
}

}  // namespace pb
