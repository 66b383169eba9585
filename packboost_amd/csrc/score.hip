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
// a 6-step xor-shuffle argmax yields the wavefront's winner. Ties on the exact score are
// broken like the reference: larger left count, then larger feature id, then larger
// threshold (frontier_cpu.cpp:415-426).
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

__global__ __launch_bounds__(kBlock) void des_score_kernel(ScoreArgs a) {
    const int KT = a.K * a.T;
    const int KTpad = (KT + kWave - 1) & ~(kWave - 1);
    const int64_t gid = (int64_t)blockIdx.x * kBlock + threadIdx.x;
    const int u = (int)(gid / KTpad);
    const int j = (int)(gid - (int64_t)u * KTpad);
    const int Ua = a.st->u_active[a.depth];
    if (u >= Ua) return;  // uniform per wavefront: KTpad is a multiple of 64

    const bool lane_ok = j < KT;
    const int k = lane_ok ? j / a.T : 0;
    const int t = lane_ok ? j - k * a.T : 0;
    const int thr = a.thr_tab ? a.thr_tab[k * a.T + t] : t;
    const int nb = a.nb;
    const int64_t estride = (int64_t)a.U * a.K * nb;
    const int32_t* pc = a.cnt + ((int64_t)u * a.K + k) * nb;
    const float* pg = a.g + ((int64_t)u * a.K + k) * nb;
    const float lam = a.lambda_l2;
    const float alpha = a.era_alpha;
    const bool use_dir = a.dir_w != 0.0f;

    float wsum = 0.0f, mean = 0.0f, M2 = 0.0f, agn = 0.0f, agd = 0.0f;
    float lg = 0.0f, tg = 0.0f;
    int lt = 0, tc = 0;
    for (int e = 0; e < a.E; ++e, pc += estride, pg += estride) {
        const int ctot = pc[nb - 1];
        if (ctot == 0) continue;
        const float Gt = pg[nb - 1];
        const int L = pc[thr];
        const float GL = pg[thr];
        const int R = ctot - L;
        const float GR = Gt - GL;
        lt += L;
        lg = lg + GL;
        tc += ctot;
        tg = tg + Gt;
        const float wera = (alpha > 0.0f) ? ((float)ctot + alpha) : 1.0f;
        const float w = (L > 0 && R > 0) ? wera : 0.0f;
        if (w <= 0.0f) continue;
        const float dL = (float)L + lam;
        const float dR = (float)R + lam;
        const float pden = (float)ctot + lam;
        const float parent = (pden > 0.0f) ? (0.5f * (Gt * Gt)) / pden : 0.0f;
        const float gain = 0.5f * ((GL * GL) / dL + (GR * GR) / dR) - parent;
        const float delta = gain - mean;
        const float wn = wsum + w;
        if (wn > 0.0f) {
            const float fac = w / wn;
            mean = mean + fac * delta;
            M2 = M2 + (w * delta) * (gain - mean);
            wsum = wn;
        }
        if (use_dir) {
            const float lv = -GL / dL;
            const float rv = -GR / dR;
            const float dir = (lv > rv) ? 1.0f : -1.0f;
            agn = agn + w * dir;
            agd = agd + w;
        }
    }

    Cand c;
    c.lt = lt;
    c.lg = lg;
    c.f = lane_ok ? a.feats[k] : -1;
    c.thr = thr;
    const int rt = tc - lt;
    const float ws = (wsum < 1e-12f) ? 1e-12f : wsum;
    const float var = M2 / ws;
    const float sd = sqrtf((0.0f < var) ? var : 0.0f);
    float score = mean - a.lambda_dro * sd;
    if (use_dir && agd > 0.0f) score = score + a.dir_w * (agn / agd);
    c.score = score;
    // a node without rows never splits (the reference skips it, frontier_cpu.cpp:191-193)
    c.valid = (lane_ok && tc > 0 && lt >= a.msl && rt >= a.msl && !isnan(score)) ? 1 : 0;

    if (a.cand_all && lane_ok) store_cand(a.cand_all + ((int64_t)u * a.K + k) * a.T + t, c);
    if (j == 0) {
        a.ntot[u].count = tc;
        a.ntot[u].grad = tg;
    }

#pragma unroll
    for (int m = 1; m < kWave; m <<= 1) {
        const Cand o = shfl_xor_cand(c, m);
        take_if(better(o, c), o, c);
    }
    if ((j & (kWave - 1)) == 0) {
        const int W = KTpad / kWave;
        store_cand(a.cand_w + (int64_t)u * W + (j / kWave), c);
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

__global__ void kcuts_kernel(const int32_t* cnt, int32_t E, int32_t U, int32_t K, int32_t nb,
                             int32_t k, int32_t mass, const Frontier* st, int32_t depth,
                             int32_t* thr_tab) {
    const int kf = blockIdx.x * blockDim.x + threadIdx.x;
    if (kf >= K) return;
    const int max_thr = max(1, nb - 1);
    const int kk = max(1, min(k, max_thr));
    int32_t* out = thr_tab + (int64_t)kf * kk;
    int32_t buf[512];
    if (!mass) {
        even_cuts(nb, k, buf);
        for (int i = 0; i < kk; ++i) out[i] = buf[i];
        return;
    }
    const int Ua = st->u_active[depth];
    // cdf[b] = sum over nodes, eras of count of bin b (planes hold running sums over bins)
    long long cdf[256];
    for (int b = 0; b < nb; ++b) cdf[b] = 0;
    for (int e = 0; e < E; ++e)
        for (int u = 0; u < Ua; ++u) {
            const int32_t* p = cnt + (((int64_t)e * U + u) * K + kf) * nb;
            for (int b = 0; b < nb; ++b) cdf[b] += p[b];
        }
    const long long total = cdf[nb - 1];
    if (total <= 0) {
        even_cuts(nb, k, buf);
        for (int i = 0; i < kk; ++i) out[i] = buf[i];
        return;
    }
    const double upper = (double)total * (1.0 - 1e-12);
    int n = 0;
    for (int i = 0; i < kk; ++i) {
        const double alpha = (kk == 1) ? 0.0 : (double)i / (double)(kk - 1);
        const double target = upper * alpha;
        int idx = nb - 1;  // lower_bound over cdf; end() -> last index
        for (int b = 0; b < nb; ++b)
            if (!((double)cdf[b] < target)) { idx = b; break; }
        buf[n++] = max(0, min(idx - 1, max_thr - 1));
    }
    // sort (insertion; kk <= 254) + unique
    for (int i = 1; i < n; ++i) {
        const int v = buf[i];
        int q = i - 1;
        while (q >= 0 && buf[q] > v) { buf[q + 1] = buf[q]; --q; }
        buf[q + 1] = v;
    }
    int m = 0;
    for (int i = 0; i < n; ++i)
        if (m == 0 || buf[m - 1] != buf[i]) buf[m++] = buf[i];
    // top up with even cuts, re-sorting and de-duplicating (frontier_cpu.cpp:93-101)
    int32_t ev[256];
    if (m < kk) {
        even_cuts(nb, kk, ev);
        for (int i = 0; i < kk; ++i) buf[m + i] = ev[i];
        n = m + kk;
        for (int i = 1; i < n; ++i) {
            const int v = buf[i];
            int q = i - 1;
            while (q >= 0 && buf[q] > v) { buf[q + 1] = buf[q]; --q; }
            buf[q + 1] = v;
        }
        m = 0;
        for (int i = 0; i < n; ++i)
            if (m == 0 || buf[m - 1] != buf[i]) buf[m++] = buf[i];
    }
    for (int i = 0; i < kk; ++i) {
        const int v = (i < m) ? buf[i] : buf[m - 1];
        out[i] = max(0, min(v, max_thr - 1));
    }
}

// Decision step: one workgroup. Applies booster.py:527-563 to the unique frontier.
__global__ __launch_bounds__(kBlock) void decide_kernel(const pb_candidate* cand_w, int32_t W,
                                                    const NodeTotal* ntot, Frontier* st,
                                                    int32_t depth, int32_t msl, double lambda_l2,
                                                    const int32_t* cur_ids, int32_t* next_ids,
                                                    SplitRule* rules, pb_decision* dec,
                                                    float* values) {
    const int Ua = st->u_active[depth];
    pb_decision* dd = dec + ((1 << depth) - 1);
    const int tree_size0 = st->tree_size;
    // Sequential scan in frontier order for child ids and next-frontier slots; the number
    // of active nodes is small (<= 2^(D-1)) and this keeps the order trivially exact.
    if (threadIdx.x == 0) {
        int next_id = tree_size0;
        int slot = 0;
        for (int u = 0; u < Ua; ++u) {
            Cand best;
            best.valid = 0;
            best.score = 0.f; best.lt = 0; best.lg = 0.f; best.f = -1; best.thr = -1;
            for (int w = 0; w < W; ++w) {
                const Cand c = load_cand(cand_w + (int64_t)u * W + w);
                take_if(better(c, best), c, best);
            }
            const NodeTotal nt = ntot[u];
            SplitRule r;
            pb_decision d;
            d.node_id = cur_ids[u];
            d.node_grad = nt.grad;
            d.node_count = nt.count;
            d.reserved = 0;
            if (best.valid) {
                const int lc = best.lt;
                const int rc = nt.count - lc;
                r.feature = best.f;
                r.threshold = best.thr;
                r.left_id = next_id;
                r.next_slot[0] = (lc >= 2 * msl) ? (uint16_t)(slot++) : (uint16_t)PB_INACTIVE;
                if (r.next_slot[0] != PB_INACTIVE) next_ids[r.next_slot[0]] = next_id;
                r.next_slot[1] = (rc >= 2 * msl) ? (uint16_t)(slot++) : (uint16_t)PB_INACTIVE;
                if (r.next_slot[1] != PB_INACTIVE) next_ids[r.next_slot[1]] = next_id + 1;
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
                d.left_id = next_id;
                d.right_id = next_id + 1;
                values[next_id] = (float)(-(double)d.left_grad / ((double)d.left_hess + lambda_l2));
                values[next_id + 1] =
                    (float)(-(double)d.right_grad / ((double)d.right_hess + lambda_l2));
                next_id += 2;
            } else {
                r.feature = -1;
                r.threshold = -1;
                r.left_id = -1;
                r.next_slot[0] = r.next_slot[1] = (uint16_t)PB_INACTIVE;
                d.split = 0;
                d.feature = -1;
                d.threshold = 0;
                d.score = 0.f;
                d.left_grad = d.left_hess = d.right_grad = d.right_hess = 0.f;
                d.left_count = d.right_count = 0;
                d.left_id = d.right_id = -1;
                values[d.node_id] =
                    (float)(-(double)nt.grad / ((double)(float)nt.count + lambda_l2));
            }
            rules[u] = r;
            dd[u] = d;
        }
        st->tree_size = next_id;
        if (depth + 1 <= PB_MAX_DEPTH) st->u_active[depth + 1] = slot;
    }
}

}  // namespace

hipError_t launch_score(const ScoreArgs& a, int grid, hipStream_t s) {
    hipLaunchKernelGGL(des_score_kernel, dim3(grid), dim3(kBlock), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_kcuts(const int32_t* cnt, int32_t E, int32_t U, int32_t K, int32_t nb,
                        int32_t k, int32_t mass, const Frontier* st, int32_t depth,
                        int32_t* thr_tab, hipStream_t s) {
    const int threads = 64;
    const int grid = (K + threads - 1) / threads;
    hipLaunchKernelGGL(kcuts_kernel, dim3(grid), dim3(threads), 0, s, cnt, E, U, K, nb, k, mass,
                       st, depth, thr_tab);
    return hipGetLastError();
}

hipError_t launch_decide(const pb_candidate* cand_w, int32_t W, const NodeTotal* ntot,
                         Frontier* st, int32_t depth, int32_t msl, double lambda_l2,
                         const int32_t* cur_ids, int32_t* next_ids, SplitRule* rules,
                         pb_decision* dec, float* values, hipStream_t s) {
    hipLaunchKernelGGL(decide_kernel, dim3(1), dim3(kBlock), 0, s, cand_w, W, ntot, st, depth,
                       msl, lambda_l2, cur_ids, next_ids, rules, dec, values);
    return hipGetLastError();
}

}  // namespace pb
