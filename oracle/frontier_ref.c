/*
 * ORACLE — test infrastructure only. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker / CPU baseline; the
 * product (packboost_amd) never calls it.
 *
 * A from-scratch C/OpenMP restatement of the reference CPU split finder
 * find_best_splits_batched_cpu (packboost/backends/cpu/frontier_cpu.cpp:111-515), keeping
 * its loop structure (serial over sampled features, OpenMP over nodes, row-major bins
 * gathered row by row) and its float32 operation order, so that it is both the parity
 * oracle and a fair stand-in for the reference's CPU time. Build without -march=native or
 * -ffast-math: plain SSE2 float arithmetic, no FMA contraction, like the reference's build.
 *
 * Function map (reference lines):
 *   ctx build         frontier_cpu.cpp:142-209  (era counts, row-order grad totals, weights)
 *   histogram         frontier_cpu.cpp:261-289  (count int64 / grad float32, row order)
 *   scan              frontier_cpu.cpp:291-321  (running sums over bins, parent gain)
 *   K-cuts            frontier_cpu.cpp:35-109, 322-335
 *   score + argmax    frontier_cpu.cpp:342-444  (weighted Welford DES, tie-break)
 *   partition         frontier_cpu.cpp:446-497  (stable per era, bin <= thr -> left)
 *   decision fields   frontier_cpu.cpp:475-494
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* Planted mistakes for the tests that show the oracle's checks have teeth
 * (tests/test_oracle_closed_form.py builds one copy per value; 0 = the restatement):
 *   1 parent gain dropped          2 era weight ignores era_alpha
 *   3 M2 update uses the old mean  4 direction sign flipped
 *   5 threshold index off by one */
#ifndef ORACLE_MUTANT
#define ORACLE_MUTANT 0
#endif

#define OR_OK 0
#define OR_ERR_INVALID (-1)
#define OR_ERR_RANGE (-2)
#define OR_ERR_NOMEM (-3)

static double now_ms(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

static int cmp_i32(const void* a, const void* b) {
    int32_t x = *(const int32_t*)a, y = *(const int32_t*)b;
    return (x > y) - (x < y);
}

/* sort ascending + unique in place; returns the new length */
static int sort_unique(int32_t* v, int n) {
    if (n <= 1) return n;
    qsort(v, (size_t)n, sizeof(int32_t), cmp_i32);
    int m = 1;
    for (int i = 1; i < n; ++i)
        if (v[i] != v[m - 1]) v[m++] = v[i];
    return m;
}

/* evenly spaced cut indices (frontier_cpu.cpp:35-57); writes kk values, returns kk */
int oracle_even_cuts(int max_bins, int k, int32_t* out) {
    const int max_thr = max_bins - 1 > 1 ? max_bins - 1 : 1;
    int kk = k < max_thr ? k : max_thr;
    if (kk < 1) kk = 1;
    int n = 0;
    if (kk == 1) {
        out[0] = 0;
        return 1;
    }
    const double step = (double)(max_thr - 1) / (double)(kk - 1);
    for (int i = 0; i < kk; ++i) {
        const double val = round((double)i * step);
        int32_t idx = (int32_t)llround(val);
        if (idx > max_thr - 1) idx = max_thr - 1;
        if (idx < 0) idx = 0;
        out[n++] = idx;
    }
    n = sort_unique(out, n);
    while (n < kk) {
        out[n] = out[n - 1];
        ++n;
    }
    return kk;
}

/* CDF-placed cut indices over per-bin counts (frontier_cpu.cpp:59-109) */
int oracle_mass_cuts(const int64_t* counts, int max_bins, int k, int32_t* out) {
    const int max_thr = max_bins - 1 > 1 ? max_bins - 1 : 1;
    int kk = k < max_thr ? k : max_thr;
    if (kk < 1) kk = 1;
    int64_t total = 0;
    for (int b = 0; b < max_bins; ++b) total += counts[b];
    if (total <= 0) return oracle_even_cuts(max_bins, kk, out);
    int64_t* cdf = (int64_t*)malloc(sizeof(int64_t) * (size_t)max_bins);
    int32_t* buf = (int32_t*)malloc(sizeof(int32_t) * (size_t)(4 * kk + 8));
    int64_t acc = 0;
    for (int b = 0; b < max_bins; ++b) {
        acc += counts[b];
        cdf[b] = acc;
    }
    const double upper = (double)total * (1.0 - 1e-12);
    int n = 0;
    for (int i = 0; i < kk; ++i) {
        const double alpha = (kk == 1) ? 0.0 : (double)i / (double)(kk - 1);
        const double target = upper * alpha;
        int64_t idx = max_bins - 1;
        for (int b = 0; b < max_bins; ++b)
            if (!((double)cdf[b] < target)) {
                idx = b;
                break;
            }
        int64_t t = idx - 1;
        if (t > max_thr - 1) t = max_thr - 1;
        if (t < 0) t = 0;
        buf[n++] = (int32_t)t;
    }
    n = sort_unique(buf, n);
    while (n < kk) {
        int32_t ev[512];
        int ne = oracle_even_cuts(max_bins, kk, ev);
        for (int i = 0; i < ne; ++i) buf[n + i] = ev[i];
        n = sort_unique(buf, n + ne);
        if (n >= kk) break;
    }
    if (n > kk) n = kk;
    for (int i = 0; i < n; ++i) {
        int32_t v = buf[i];
        if (v > max_thr - 1) v = max_thr - 1;
        if (v < 0) v = 0;
        out[i] = v;
    }
    free(cdf);
    free(buf);
    return n;
}

typedef struct {
    int64_t lo, hi;      /* range of this node in rows[] */
    int64_t count;
    float grad;          /* float32 sum of era totals in era order */
    int valid;           /* has at least one row */
} node_ctx;

/* Score every threshold of one (node, feature) and update the node's running best,
 * visiting thresholds in list order (frontier_cpu.cpp:353-433). The per-era inputs are the
 * node's prefix/total planes for this feature: pc/pg [E][nb] with index nb-1 = total. The
 * era weights count all of the node's rows in the era (NodeContext::era_weights,
 * frontier_cpu.cpp:196-204): es [E+1], the node's era splits, or NULL when the feature's
 * totals hold every row (no bin >= nb). */
static void score_feature(const int64_t* pc, const float* pg, const int64_t* es, int E, int nb,
                          const int32_t* thr_list,
                          int n_thr, int32_t feature, int64_t node_count, float lambda_l2,
                          float lambda_dro, float dir_w, float era_alpha, int msl, float* best_score,
                          int32_t* best_feat, int32_t* best_thr, int64_t* best_left, float* best_lg,
                          float* cand_score, int64_t* cand_lt, float* cand_lg, uint8_t* cand_valid) {
    const int use_dir = (dir_w != 0.0f);
    for (int ti = 0; ti < n_thr; ++ti) {
        const int32_t thr = thr_list[ti];
        float wsum = 0.0f, mean = 0.0f, M2 = 0.0f, agr_num = 0.0f, agr_den = 0.0f, left_grad_sum = 0.0f;
        int64_t left_total = 0;
        for (int e = 0; e < E; ++e) {
            const int64_t total_e = pc[(int64_t)e * nb + nb - 1];
            if (total_e == 0) continue;
#if ORACLE_MUTANT == 5
            const int32_t thr_m = (thr + 1 < nb - 1) ? thr + 1 : thr;
#else
            const int32_t thr_m = thr;
#endif
            const int64_t left_e = pc[(int64_t)e * nb + thr_m];
            const int64_t right_e = total_e - left_e;
            const float left_grad_e = pg[(int64_t)e * nb + thr_m];
            const float total_grad_e = pg[(int64_t)e * nb + nb - 1];
            const float right_grad_e = total_grad_e - left_grad_e;
#if ORACLE_MUTANT == 2
            const float era_w = 1.0f;
#else
            const int64_t rows_e = es ? es[e + 1] - es[e] : total_e;
            const float era_w = (era_alpha > 0.0f) ? ((float)rows_e + era_alpha) : 1.0f;
#endif
            const float weight = (left_e > 0 && right_e > 0) ? era_w : 0.0f;
            left_total += left_e;
            left_grad_sum += left_grad_e;
            if (weight <= 0.0f) continue;
            const float denom_L = (float)left_e + lambda_l2;
            const float denom_R = (float)right_e + lambda_l2;
            const float parent_denom = (float)total_e + lambda_l2;
#if ORACLE_MUTANT == 1
            const float parent_gain = 0.0f * parent_denom;
#else
            const float parent_gain =
                (parent_denom > 0.0f) ? 0.5f * (total_grad_e * total_grad_e) / parent_denom : 0.0f;
#endif
            const float gain_e = 0.5f * ((left_grad_e * left_grad_e) / denom_L +
                                         (right_grad_e * right_grad_e) / denom_R) - parent_gain;
            const float delta = gain_e - mean;
            const float wsum_new = wsum + weight;
            if (wsum_new > 0.0f) {
                const float factor = weight / wsum_new;
#if ORACLE_MUTANT == 3
                const float mean_old = mean;
                mean += factor * delta;
                M2 += weight * delta * (gain_e - mean_old);
#else
                mean += factor * delta;
                M2 += weight * delta * (gain_e - mean);
#endif
                wsum = wsum_new;
            }
            if (use_dir) {
                const float left_val = -left_grad_e / denom_L;
                const float right_val = -right_grad_e / denom_R;
#if ORACLE_MUTANT == 4
                const float direction = (left_val > right_val) ? -1.0f : 1.0f;
#else
                const float direction = (left_val > right_val) ? 1.0f : -1.0f;
#endif
                agr_num += weight * direction;
                agr_den += weight;
            }
        }
        const int64_t right_total = node_count - left_total;
        const int ok = !(left_total < msl || right_total < msl);
        const float ws = (wsum < 1e-12f) ? 1e-12f : wsum;
        const float var = M2 / ws;
        const float std_dev = sqrtf((0.0f < var) ? var : 0.0f);
        float score = mean - lambda_dro * std_dev;
        if (use_dir && agr_den > 0.0f) score += dir_w * (agr_num / agr_den);
        if (cand_score) {
            cand_score[ti] = score;
            cand_lt[ti] = left_total;
            cand_lg[ti] = left_grad_sum;
            cand_valid[ti] = (uint8_t)ok;
        }
        if (!ok) continue;
        int better = score > *best_score;
        if (!better && fabsf(score - *best_score) <= 1e-12f) {
            if (left_total > *best_left) {
                better = 1;
            } else if (left_total == *best_left) {
                if (feature > *best_feat)
                    better = 1;
                else if (feature == *best_feat && thr > *best_thr)
                    better = 1;
            }
        }
        if (better) {
            *best_score = score;
            *best_feat = feature;
            *best_thr = thr;
            *best_left = left_total;
            *best_lg = left_grad_sum;
        }
    }
}

/*
 * Split finder over a batch of nodes (the unique shards of one depth).
 *  bins      uint8 [n_rows][n_feat] row-major
 *  rows      int64 row ids, node-major then era-major; era_splits int64 [n_nodes][n_eras+1]
 *            absolute offsets into rows (era e of node m = rows[es[m][e] .. es[m][e+1]))
 *  feats     int32 [n_sub] sampled feature ids, visited in order
 * Outputs (per node): feature (-1 = no split), threshold, score, left/right grad/hess/count;
 *  go_left  uint8 [len(rows)] partition flag per entry of rows (stable order is implied);
 *  optional planes [n_eras][n_nodes][n_sub][max_bins] (prefix count/grad, total at nb-1);
 *  optional per-candidate arrays [n_nodes][n_sub][T] (T thresholds per feature).
 *  timings[4] = hist, scan, score, partition milliseconds.
 */
int oracle_split_batch(const uint8_t* bins, int64_t n_rows, int64_t n_feat, const float* grad,
                       int32_t n_nodes, int32_t n_eras, const int64_t* rows, const int64_t* era_splits,
                       const int32_t* feats, int32_t n_sub, int32_t max_bins, int32_t k_cuts,
                       int32_t cut_mass, float lambda_l2, float lambda_dro, float dir_w,
                       float era_alpha, int32_t msl, int32_t* out_feat, int32_t* out_thr,
                       float* out_score, float* out_lgrad, float* out_lhess, float* out_rgrad,
                       float* out_rhess, int64_t* out_lcnt, int64_t* out_rcnt, uint8_t* go_left,
                       int32_t* plane_cnt, float* plane_g, float* cand_score, int64_t* cand_lt,
                       float* cand_lg, uint8_t* cand_valid, double* timings) {
    if (!bins || !grad || !rows || !era_splits || !feats || n_nodes < 0 || n_eras < 1 || max_bins < 1)
        return OR_ERR_INVALID;
    const int nb = max_bins;
    const int thresholds_full = nb - 1 > 1 ? nb - 1 : 1;
    const int E = n_eras;
    double t_hist = 0, t_scan = 0, t_score = 0, t_part = 0;

    node_ctx* ctx = (node_ctx*)calloc((size_t)(n_nodes > 0 ? n_nodes : 1), sizeof(node_ctx));
    if (!ctx) return OR_ERR_NOMEM;
    for (int m = 0; m < n_nodes; ++m) {
        const int64_t* es = era_splits + (int64_t)m * (E + 1);
        ctx[m].lo = es[0];
        ctx[m].hi = es[E];
        float total_grad = 0.0f;
        int64_t count = 0;
        for (int e = 0; e < E; ++e) {
            float era_grad = 0.0f;
            for (int64_t i = es[e]; i < es[e + 1]; ++i) {
                const int64_t r = rows[i];
                if (r < 0 || r >= n_rows) {
                    free(ctx);
                    return OR_ERR_RANGE;
                }
                era_grad += grad[r];
            }
            count += es[e + 1] - es[e];
            total_grad += era_grad;
        }
        ctx[m].count = count;
        ctx[m].grad = total_grad;
        ctx[m].valid = count > 0;
        out_feat[m] = -1;
        out_thr[m] = -1;
    }
    for (int k = 0; k < n_sub; ++k)
        if (feats[k] < 0 || feats[k] >= n_feat) {
            free(ctx);
            return OR_ERR_RANGE;
        }

    const size_t cells = (size_t)n_nodes * E * nb;
    int64_t* counts = (int64_t*)malloc(sizeof(int64_t) * (cells ? cells : 1));
    float* grads = (float*)malloc(sizeof(float) * (cells ? cells : 1));
    int64_t* pcnt = (int64_t*)malloc(sizeof(int64_t) * (cells ? cells : 1));
    float* pgrd = (float*)malloc(sizeof(float) * (cells ? cells : 1));
    float* best_score = (float*)malloc(sizeof(float) * (n_nodes ? n_nodes : 1));
    int32_t* best_feat = (int32_t*)malloc(sizeof(int32_t) * (n_nodes ? n_nodes : 1));
    int32_t* best_thr = (int32_t*)malloc(sizeof(int32_t) * (n_nodes ? n_nodes : 1));
    int64_t* best_left = (int64_t*)malloc(sizeof(int64_t) * (n_nodes ? n_nodes : 1));
    float* best_lg = (float*)malloc(sizeof(float) * (n_nodes ? n_nodes : 1));
    int64_t* mass = (int64_t*)malloc(sizeof(int64_t) * (size_t)nb);
    int32_t* thr_list = (int32_t*)malloc(sizeof(int32_t) * (size_t)(thresholds_full + 8));
    if (!counts || !grads || !pcnt || !pgrd || !best_score || !best_feat || !best_thr || !best_left ||
        !best_lg || !mass || !thr_list) {
        free(counts); free(grads); free(pcnt); free(pgrd); free(best_score); free(best_feat);
        free(best_thr); free(best_left); free(best_lg); free(mass); free(thr_list); free(ctx);
        return OR_ERR_NOMEM;
    }
    for (int m = 0; m < n_nodes; ++m) {
        best_score[m] = -INFINITY;
        best_feat[m] = -1;
        best_thr[m] = -1;
        best_left[m] = -1;
        best_lg[m] = 0.0f;
    }
    const int use_k = (k_cuts > 0) && (k_cuts < thresholds_full);
    const int T = use_k ? k_cuts : thresholds_full;

    for (int fi = 0; fi < n_sub; ++fi) {
        const int32_t f = feats[fi];
        memset(counts, 0, sizeof(int64_t) * cells);
        memset(grads, 0, sizeof(float) * cells);
        double t0 = now_ms();
#pragma omp parallel for schedule(static)
        for (int m = 0; m < n_nodes; ++m) {
            const int64_t* es = era_splits + (int64_t)m * (E + 1);
            for (int e = 0; e < E; ++e) {
                const size_t base = ((size_t)m * E + e) * nb;
                for (int64_t i = es[e]; i < es[e + 1]; ++i) {
                    const int64_t r = rows[i];
                    const int b = bins[r * n_feat + f];
                    if (b >= nb) continue;
                    counts[base + b] += 1;
                    grads[base + b] += grad[r];
                }
            }
        }
        double t1 = now_ms();
        t_hist += t1 - t0;
        for (int b = 0; b < nb; ++b) mass[b] = 0;
        for (int m = 0; m < n_nodes; ++m)
            for (int e = 0; e < E; ++e) {
                const size_t base = ((size_t)m * E + e) * nb;
                int64_t rc = 0;
                float rg = 0.0f;
                for (int b = 0; b < nb; ++b) {
                    rc += counts[base + b];
                    rg += grads[base + b];
                    mass[b] += counts[base + b];
                    pcnt[base + b] = rc;  /* b < nb-1: prefix; b = nb-1: total */
                    pgrd[base + b] = rg;
                }
                if (plane_cnt) {
                    const size_t ob = (((size_t)e * n_nodes + m) * n_sub + fi) * nb;
                    for (int b = 0; b < nb; ++b) {
                        plane_cnt[ob + b] = (int32_t)pcnt[base + b];
                        plane_g[ob + b] = pgrd[base + b];
                    }
                }
            }
        int n_thr;
        if (use_k) {
            n_thr = cut_mass ? oracle_mass_cuts(mass, nb, k_cuts, thr_list)
                             : oracle_even_cuts(nb, k_cuts, thr_list);
        } else {
            n_thr = thresholds_full;
            for (int t = 0; t < n_thr; ++t) thr_list[t] = t;
        }
        double t2 = now_ms();
        t_scan += t2 - t1;
#pragma omp parallel for schedule(static)
        for (int m = 0; m < n_nodes; ++m) {
            if (!ctx[m].valid) continue;
            const size_t base = (size_t)m * E * nb;
            const size_t co = ((size_t)m * n_sub + fi) * T;
            score_feature(pcnt + base, pgrd + base, era_splits + (int64_t)m * (E + 1), E, nb,
                          thr_list, n_thr, f, ctx[m].count,
                          lambda_l2, lambda_dro, dir_w, era_alpha, msl, &best_score[m], &best_feat[m],
                          &best_thr[m], &best_left[m], &best_lg[m], cand_score ? cand_score + co : NULL,
                          cand_lt ? cand_lt + co : NULL, cand_lg ? cand_lg + co : NULL,
                          cand_valid ? cand_valid + co : NULL);
        }
        t_score += now_ms() - t2;
    }

    double t3 = now_ms();
    for (int m = 0; m < n_nodes; ++m) {
        const int ok = ctx[m].valid && best_feat[m] >= 0 && best_thr[m] >= 0;
        for (int64_t i = ctx[m].lo; i < ctx[m].hi; ++i)
            go_left[i] = ok ? (uint8_t)(bins[rows[i] * n_feat + best_feat[m]] <= best_thr[m]) : 0;
        if (!ok) {
            out_feat[m] = -1;
            out_thr[m] = -1;
            out_score[m] = 0.0f;
            out_lgrad[m] = out_lhess[m] = out_rgrad[m] = out_rhess[m] = 0.0f;
            out_lcnt[m] = out_rcnt[m] = 0;
            continue;
        }
        out_feat[m] = best_feat[m];
        out_thr[m] = best_thr[m];
        out_score[m] = best_score[m];
        out_lgrad[m] = best_lg[m];
        out_lhess[m] = (float)best_left[m];
        out_rgrad[m] = ctx[m].grad - best_lg[m];
        out_rhess[m] = (float)ctx[m].count - out_lhess[m];
        out_lcnt[m] = best_left[m];
        out_rcnt[m] = ctx[m].count - best_left[m];
    }
    t_part = now_ms() - t3;
    if (timings) {
        timings[0] = t_hist;
        timings[1] = t_scan;
        timings[2] = t_score;
        timings[3] = t_part;
    }
    free(counts); free(grads); free(pcnt); free(pgrd); free(best_score); free(best_feat);
    free(best_thr); free(best_left); free(best_lg); free(mass); free(thr_list); free(ctx);
    return OR_OK;
}

/*
 * Scorer alone on given prefix planes [n_eras][n_nodes][n_sub][nb] (the layout the GPU
 * histogram kernel writes): per-candidate score / left total / left grad / validity
 * [n_nodes][n_sub][T], thresholds 0..nb-2 (or thr_tab [n_sub][T] when given), and the per-node
 * winner with the reference's sequential tie-break. Node counts come from the planes' totals.
 */
int oracle_score_planes(const int32_t* plane_cnt, const float* plane_g, int32_t n_eras,
                        int32_t n_nodes, int32_t n_sub, int32_t nb, const int32_t* feats,
                        const int32_t* thr_tab, int32_t T, float lambda_l2, float lambda_dro,
                        float dir_w, float era_alpha, int32_t msl, float* cand_score,
                        int64_t* cand_lt, float* cand_lg, uint8_t* cand_valid, int32_t* out_feat,
                        int32_t* out_thr, float* out_score, int64_t* out_lcnt, float* out_lgrad) {
    const int E = n_eras;
    int64_t* pc = (int64_t*)malloc(sizeof(int64_t) * (size_t)E * nb);
    float* pg = (float*)malloc(sizeof(float) * (size_t)E * nb);
    int32_t* thr_list = (int32_t*)malloc(sizeof(int32_t) * (size_t)(T > 0 ? T : 1));
    if (!pc || !pg || !thr_list) {
        free(pc); free(pg); free(thr_list);
        return OR_ERR_NOMEM;
    }
    for (int m = 0; m < n_nodes; ++m) {
        float bs = -INFINITY, blg = 0.0f;
        int32_t bf = -1, bt = -1;
        int64_t bl = -1;
        for (int fi = 0; fi < n_sub; ++fi) {
            int64_t count = 0;
            for (int e = 0; e < E; ++e) {
                const size_t ib = (((size_t)e * n_nodes + m) * n_sub + fi) * nb;
                for (int b = 0; b < nb; ++b) {
                    pc[(size_t)e * nb + b] = plane_cnt[ib + b];
                    pg[(size_t)e * nb + b] = plane_g[ib + b];
                }
                count += plane_cnt[ib + nb - 1];
            }
            for (int t = 0; t < T; ++t) thr_list[t] = thr_tab ? thr_tab[fi * T + t] : t;
            const size_t co = ((size_t)m * n_sub + fi) * T;
            if (count == 0) {
                for (int t = 0; t < T; ++t) {
                    cand_score[co + t] = 0.0f;
                    cand_lt[co + t] = 0;
                    cand_lg[co + t] = 0.0f;
                    cand_valid[co + t] = 0;
                }
                continue;
            }
            score_feature(pc, pg, NULL, E, nb, thr_list, T, feats[fi], count, lambda_l2, lambda_dro, dir_w,
                          era_alpha, msl, &bs, &bf, &bt, &bl, &blg, cand_score + co, cand_lt + co,
                          cand_lg + co, cand_valid + co);
        }
        out_feat[m] = bf;
        out_thr[m] = bt;
        out_score[m] = bs;
        out_lcnt[m] = bl;
        out_lgrad[m] = blg;
    }
    free(pc); free(pg); free(thr_list);
    return OR_OK;
}

int oracle_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
