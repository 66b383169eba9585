/*
 * packboost_hip.h — C ABI of libpackboost_hip.so, the MI355X (gfx950) backend for
 * PackBoost's pack-parallel, layer-wise tree growth and pack prediction.
 *
 * Conventions
 *   - Every entry point returns an int status: PB_OK (0) or a negative PB_ERR_* code.
 *     pb_last_error() returns a thread-local message for the last failure on the
 *     calling thread. HIP failures are reported as "HIP error: ..." so a caller that
 *     pattern-matches the reference's "CUDA error" fallback can match either spelling.
 *   - All pointers named *_dev are device pointers allocated by the caller; the
 *     library never frees caller memory. Persistent scratch belongs to pb_ctx.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream). Work is
 *     enqueued asynchronously; no entry point synchronises the device unless stated.
 *   - Row-indexed device arrays (grad, node ids, ...) must hold `rows_padded`
 *     (= N rounded up to a multiple of 16) elements from a 16-byte aligned base; the pad
 *     rows must carry node id PB_INACTIVE and grad 0. Bins are column-major uint8 [F][ld] with
 *     ld % 16 == 0, ld >= N, 16-byte aligned base, and rows sorted era-major so
 *     era e occupies rows [era_off[e], era_off[e+1]).
 *
 * The reference binds its native path through pybind11 (packboost/backends/bindings.cpp:11-24)
 * and the Python shim packboost/backends/__init__.py:9-163. Each entry point below names
 * the reference interface it replaces.
 */
#ifndef PACKBOOST_HIP_H
#define PACKBOOST_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PB_OK 0
#define PB_ERR_INVALID (-1)     /* bad argument / shape / id (reference: std::invalid_argument) */
#define PB_ERR_RANGE (-2)       /* index out of range (reference: std::out_of_range) */
#define PB_ERR_HIP (-3)         /* HIP runtime failure (reference: "CUDA error: ...") */
#define PB_ERR_UNSUPPORTED (-4) /* configuration this build does not handle */
#define PB_ERR_NOMEM (-5)

#define PB_INACTIVE 0xFFFFu     /* node id of a row that is in no active frontier node */
#define PB_MAX_DEPTH 16

typedef struct pb_ctx pb_ctx;

/* Shape of one fit. Replaces the implicit shapes the reference reads from its tensors
 * (frontier_cpu.cpp:131-140, frontier_cuda.cu:576-632). */
typedef struct {
    int64_t num_rows;      /* N */
    int64_t ld;            /* byte stride between feature columns of bins (>= N, %16 == 0) */
    int32_t num_features;  /* F */
    int32_t num_eras;      /* E (>= 1) */
    int32_t max_bins;      /* nb, 2..255 */
    int32_t max_depth;     /* D, 1..PB_MAX_DEPTH */
    int32_t max_feats;     /* largest feature subset per depth, K */
    int32_t min_samples_leaf;
} pb_dims;

/* Split-scoring hyper-parameters; the reference passes them one by one
 * (frontier_cpu.cpp:116-123) as C++ float after pybind's double->float cast, while
 * leaf values use the Python double (booster.py:545-546). They are carried here as
 * double; the scorer rounds each to float exactly as that cast does.
 * cut_selection: 0 = "even", 1 = "mass".
 * skip_last_bin: 1 when the histogram planes were built with one bin more than the
 * reference's num_bins (the context's max_bins = num_bins + 1), that last bin holding the rows
 * whose bin is >= num_bins. The reference leaves such rows out of a feature's histogram
 * (frontier_cpu.cpp:278-281, frontier_cuda.cu:451) while they still count in the node's row
 * total and go right in the partition (:464-470). pb_des_score then sweeps thresholds
 * 0..num_bins-2 only, takes each era's totals for a feature over its bins < num_bins, and the
 * era weights and the node's row count over all rows. 0: every row's bin is < max_bins. */
typedef struct {
    double lambda_l2;
    double lambda_dro;
    double direction_weight;
    double era_alpha;
    int32_t min_samples_leaf;
    int32_t k_cuts;
    int32_t cut_selection;
    int32_t skip_last_bin;
} pb_split_params;

/* One entry per active frontier node and depth: the reference's SplitDecision
 * (booster.py:205-217) without row lists, plus the node's tree ids. */
typedef struct {
    int32_t node_id;      /* TreeBuilder id of the node */
    int32_t split;        /* 1: split, 0: became a leaf (no valid candidate) */
    int32_t feature;
    int32_t threshold;
    float score;
    float left_grad;
    float left_hess;
    float right_grad;
    float right_hess;
    int32_t left_count;
    int32_t right_count;
    int32_t left_id;      /* TreeBuilder ids of the children (split only) */
    int32_t right_id;
    float node_grad;      /* sum of grad over the node's rows (float32) */
    int32_t node_count;   /* rows in the node */
    int32_t reserved;
} pb_decision;

/* Candidate record (one per wavefront winner, or per lane when dumped for tests). In a
 * wavefront winner, reserved[0] counts that wavefront's valid candidates scoring below the
 * winner but within 64e-12 of it (the decision step replays the reference's sequential scan
 * only when such candidates exist near the node's top score); elsewhere it is 0. */
typedef struct {
    float score;
    int32_t left_total;
    float left_grad;
    int32_t feature;
    int32_t threshold;
    int32_t valid;
    int32_t reserved[2];
} pb_candidate;

/* ---- library ---------------------------------------------------------------------- */
const char* pb_last_error(void);
int32_t pb_version(void);
/* Reference: _cuda_available (bindings.cpp:15-22 / backends/__init__.py:95-113). 1 if a gfx950 device is usable. */
int32_t pb_device_available(void);

/* ---- context ---------------------------------------------------------------------- */
/* Allocates the persistent scratch for one fit (frontier state, decision tables,
 * candidate buffers). era_off_host: int32 [E+1], era_off[0] = 0, era_off[E] = N.
 * Replaces the per-call context build of frontier_cpu.cpp:142-209. */
int pb_ctx_create(const pb_dims* dims, const int32_t* era_off_host, pb_ctx** out);
int pb_ctx_destroy(pb_ctx* ctx);
/* 4-byte elements each of the two histogram buffers (counts, grads) pb_hist_build fills for
 * a depth with up to `max_nodes` active nodes and K = max_feats: round_up(C, 64) + E * max_nodes
 * with C = E * max_nodes * K * (nb - 1) (layout at pb_hist_build). */
int64_t pb_hist_plane_elems(const pb_ctx* ctx, int32_t max_nodes);
/* Largest active-node count the frontier can reach at `depth`. */
int32_t pb_max_nodes(const pb_ctx* ctx, int32_t depth);
/* Device pointer of the era offsets (int32 [E+1]) the context holds. */
const int32_t* pb_era_offsets_dev(const pb_ctx* ctx);

/* ---- round driver ------------------------------------------------------------------ */
/* grad = preds - y (booster.py:2149-2151, squared loss; hess == 1, booster.py:2153-2154);
 * resets the per-round frontier: every row in root node 0 (active iff N >= 2*msl,
 * booster.py:794-796), tree size 1. Also records the bounds of the histogram's fixed-point
 * gradient scale (max |grad| and the largest |grad| sum over 1024 consecutive rows). */
int pb_round_begin(pb_ctx* ctx, const float* preds_dev, const float* y_dev, float* grad_dev,
                   uint16_t* nid_dev, uint16_t* tnode_dev, void* stream);

/* Kernel 1 — histogram build. Replaces the per-feature histogram + scan of
 * find_best_splits_batched_cpu (frontier_cpu.cpp:261-321) and the histogram part of
 * cuda_find_best_splits_kernel (frontier_cuda.cu:441-498). For every active node u,
 * era e, sampled feature k and threshold t < nb-1 it writes the prefix over bins 0..t, and
 * per (e, u) the era total (the reference's running sum at bin nb-1, the same for every
 * feature because the sums are exact). With T = nb - 1, C = E * max_nodes * K * T and
 * O = round_up(C, 64):
 *   hist_cnt_dev  as uint16 [E][max_nodes][K][T]: rows with bin <= t (as uint32 when an era
 *                 holds more than 65535 rows); as int32, elements O .. O + E*max_nodes: era
 *                 totals [E][max_nodes]
 *   hist_grad_dev float32 [E][max_nodes][K][T]: prefix grad sums; elements O ..: era totals.
 * feats_dev: int32 [K] feature ids; `depth` selects the frontier's active-node count.
 * grad_dev must hold the gradients the last pb_round_begin on this context wrote: their
 * per-era |grad| sums set the exact fixed-point scale of each era's sums.
 * Eras of any size: an era above 16384 rows is built in parts whose exact sums are added up
 * before the planes are written, so the planes do not depend on the split. */
int pb_hist_build(pb_ctx* ctx, const uint8_t* bins_dev, const float* grad_dev,
                  const uint16_t* nid_dev, const int32_t* feats_dev, int32_t K, int32_t depth,
                  int32_t max_nodes, int32_t* hist_cnt_dev, float* hist_grad_dev, void* stream);

/* Kernel 2 — DES split scoring + argmax. Replaces the scoring/tie-break loop of
 * frontier_cpu.cpp:342-444 (and frontier_cuda.cu:500-571 + booster.py:1451-1467).
 * Reads the planes written by pb_hist_build, scores every (node, feature, threshold)
 * by era-weighted Welford mean - lambda_dro * std (+ direction term), and keeps the
 * best candidate per node. cand_all_dev (optional, may be NULL) receives one record
 * per (node, feature, threshold) lane: [max_nodes][K][T]. */
int pb_des_score(pb_ctx* ctx, const int32_t* hist_cnt_dev, const float* hist_grad_dev,
                 const int32_t* feats_dev, int32_t K, int32_t depth, int32_t max_nodes,
                 const pb_split_params* params, pb_candidate* cand_all_dev, void* stream);

/* Segment mode (no counterpart in the reference's data structures; its semantics are
 * pb_grow_round's): from depth from_depth on, pb_grow_round keeps the round's row ids and
 * gradients sorted by (era, frontier slot) in buffers of the context and scores each depth with
 * one fused kernel per (node, feature tile) that streams the node's rows era by era (reading
 * their bins from bins_dev through the ids), builds each era's histogram in LDS and runs the DES
 * recurrence on it (frontier_cpu.cpp:261-444): those depths' histogram planes are never
 * written, and the candidates, decisions and predictions are bit-identical to the plane path's.
 * The shallower depths use the plane path while the context tracks the row order; between
 * depths the rows are partitioned stably into the next frontier's slots. For many bins and
 * nodes, where the planes dominate (255 bins, 128 nodes, 200 eras).
 * from_depth < 0 picks the first depth whose planes would pass 1 GiB. The context then holds
 * 2 x 10 bytes per row more. Requires eras of at most 65535 rows; pb_grow_round then scores
 * every threshold (k_cuts 0), maintains preds_dev through the rows' ids and leaves nid_dev /
 * tnode_dev unspecified. enable 0 returns to the plane path. */
int pb_set_segment_mode(pb_ctx* ctx, int32_t enable, int32_t from_depth);

/* Applies the per-node winners of the last pb_des_score: picks each node's split with the
 * reference's sequential scan (features in subset order, thresholds ascending; a candidate wins
 * with a higher score, or within 1e-12 of the best with more left rows, then a larger feature
 * id, then a larger threshold: frontier_cpu.cpp:415-426), with the feature ids that call was
 * given (pb_des_score copies them into the context on its stream, so feats_dev may be freed or
 * rewritten once pb_des_score has returned), builds the decisions of this
 * depth (booster.py:527-563: split -> children ids (len, len+1), child values
 * -G/(H+lambda); no split -> leaf value -G/(H+lambda)), assigns the next frontier
 * (children with >= 2*msl rows, booster.py:516, 794-796) and writes the depth's
 * decisions to decisions_dev + (2^depth - 1) (pb_decision [2^D - 1] per round).
 * values_dev: float32 [2^(D+1)] leaf value per TreeBuilder node id. max_nodes: the node bound
 * passed to pb_des_score (at least pb_max_nodes(ctx, depth)). */
int pb_decide(pb_ctx* ctx, int32_t depth, int32_t max_nodes, const pb_split_params* params,
              pb_decision* decisions_dev, float* values_dev, void* stream);

/* Kernel 3 — partition. Replaces the stable per-era left/right row split of
 * frontier_cpu.cpp:446-497 and partition_frontier_cuda (frontier_cuda.cu:719-851):
 * every row of a split node moves to child 2j+(bin > thr) (TreeBuilder ids) and to its
 * slot in the next frontier (PB_INACTIVE if the child is below capacity); rows of a
 * node that did not split leave the frontier. */
int pb_partition(pb_ctx* ctx, const uint8_t* bins_dev, int32_t depth, uint16_t* nid_dev,
                 uint16_t* tnode_dev, void* stream);

/* Pack aggregation (booster.py:581-599): pack_sum[r] = sum over the pack's `pack_size`
 * identical trees of float32(value[leaf(r)]) in tree order; preds += float32(lr) * pack_sum. */
int pb_round_end(pb_ctx* ctx, const uint16_t* tnode_dev, const float* values_dev,
                 int32_t pack_size, float learning_rate, float* preds_dev, void* stream);

/* Per-round summary written on the device at the end of pb_grow_round, so one small copy
 * gives the host everything it needs to rebuild the round's trees. */
typedef struct {
    int32_t u_active[PB_MAX_DEPTH + 1];  /* active unique nodes per depth */
    int32_t tree_size;                   /* nodes in each tree of the round */
    int32_t reserved[6];                 /* [0]: 1 when the round's gradients (preds - y) were
                                          * not all finite; its histograms have no meaning then
                                          * (the fixed-point sums hold no NaN or infinity) and the
                                          * caller should stop. [1..5]: 0 */
} pb_round_header;  /* 96 bytes */

/* Device buffers of one fit, bound once for pb_grow_round. All row arrays hold rows_padded
 * entries; hist planes hold pb_hist_plane_elems(ctx, pb_max_nodes(ctx, D-1)) entries. */
typedef struct {
    const uint8_t* bins_dev;     /* [F][ld] column-major */
    const uint8_t* bins4_dev;    /* NULL, or the same bins in the nibble layout of
                                  * pb_pack_bins4 ([F][ld / 2], max_bins <= 16): the
                                  * histogram and partition read it instead of bins_dev */
    const float* y_dev;
    float* preds_dev;
    float* grad_dev;
    uint16_t* nid_dev;
    uint16_t* tnode_dev;
    int32_t* hist_cnt_dev;
    float* hist_grad_dev;
    float* values_dev;           /* [2^(D+1)] */
    int32_t pack_size;
    float learning_rate;
    pb_split_params params;
} pb_fit_buffers;

/* One whole boosting round (booster.py:494-599) as a single asynchronous enqueue:
 * pb_round_begin, then for every depth pb_hist_build -> pb_des_score -> pb_decide ->
 * pb_partition, then pb_round_end (the last depth's partition and the round end run as one
 * launch when preds, nid and tnode are 16-byte aligned; the results are the same). feats_dev:
 * int32 [D][K] feature subsets (the host draws them, booster.py:519, 787-792); decisions_dev:
 * pb_decision [2^D - 1]; header_dev: the round's pb_round_header. Depths whose frontier is
 * empty run no work. */
int pb_grow_round(pb_ctx* ctx, const pb_fit_buffers* buffers, const int32_t* feats_dev, int32_t K,
                  pb_decision* decisions_dev, pb_round_header* header_dev, void* stream);

/* Feature subsets of the next round without waiting for this one. The reference draws one
 * subset per depth while the frontier has active nodes (booster.py:516-519, 787-792), so the
 * next round's D subsets are the D draws that follow the previous round's own draws, whose
 * count the host learns only from that round's header. Given window_dev = int32 [2D][K]: the
 * previous round's D draws followed by D more, this writes feats_dev[j] = window_dev[off + j]
 * (j < D) with off = the number of depths of prev_header_dev with active nodes (0 when it is
 * NULL). Enqueued between two pb_grow_round calls, it lets the host run a round ahead without
 * redoing a round that stopped early. */
int pb_select_subsets(const pb_round_header* prev_header_dev, const int32_t* window_dev, int32_t D,
                      int32_t K, int32_t* feats_dev, void* stream);

/* GPU time of the phases of pb_grow_round, from HIP events recorded on the launch stream
 * around each depth's hist / score / decide / partition launches (the device-side analogue of
 * the per-depth hist_ms / scan_ms / score_ms / partition_ms instrumentation,
 * booster.py:220-270). enable: 0 off, 1 every phase, 2 the histogram launches only (two
 * events per depth instead of five: each recorded event is a queue barrier). pb_profile_read
 * waits for the recorded rounds, fills ms[phase * PB_MAX_DEPTH + depth] (phase 0 hist,
 * 1 score, 2 decide, 3 partition) and the matching launch counts, and clears them. */
int pb_profile_enable(pb_ctx* ctx, int32_t enable);
int pb_profile_read(pb_ctx* ctx, double* ms, int64_t* launches);

/* Teacher-forces the frontier of `depth`: `num_active` active slots whose TreeBuilder ids are
 * node_ids_host (NULL: 0..num_active-1) and a tree size of `tree_size`. Lets a caller run one
 * depth on its own row -> slot assignment (nid); the reference takes that assignment as the
 * per-node era row lists of find_best_splits_batched_cpu (frontier_cpu.cpp:111-124). */
int pb_frontier_set(pb_ctx* ctx, int32_t depth, int32_t num_active, const int32_t* node_ids_host,
                    int32_t tree_size, void* stream);

/* Copies the frontier's per-depth active-node counts (int32 [PB_MAX_DEPTH+1]) and the
 * tree size to host memory; synchronises `stream`. */
int pb_frontier_counts(pb_ctx* ctx, int32_t* u_active_host, int32_t* tree_size_host, void* stream);

/* ---- quantile binning ---------------------------------------------------------------- */
/* Interior quantile edges of quantile_bin (data.py:44-56): for every column f of
 * sorted_dev (float32 [F][ld], each column's n values ascending, NaN last) and level q[k]
 * (double [num_q], the reference's linspace(0, 1, max_bins + 1)[1:-1]), edges[k][f] =
 * float32 of NumPy's method="linear" quantile, its arithmetic restated exactly; a column with
 * a NaN gets NaN edges. edges_dev: float32, row k at edges_dev + k * edge_stride. */
int pb_quantile_edges(const float* sorted_dev, int64_t n, int64_t ld, int32_t F,
                      const double* q_dev, int32_t num_q, float* edges_dev, int32_t edge_stride,
                      void* stream);

/* Layout of the bins_dev that pb_hist_build and pb_partition read: 0 = uint8 [F][ld] (the
 * default), 1 = the nibble layout of pb_pack_bins4 ([F][ld / 2], max_bins <= 16). The
 * reference's per-depth kernels take int8 feature-major bins only (frontier_cuda.cu:576-716,
 * 719-851); pb_grow_round picks its layout from pb_fit_buffers instead. */
int pb_set_bin_layout(pb_ctx* ctx, int32_t layout);

/* Nibble layout of the frontier kernels' feature-major bins (the reference builds
 * bins.t().contiguous() as int8 [F][N], booster.py:419-426): out_dev[f][ld / 2] receives, for
 * every 8 rows, one 4-byte word whose byte j holds row j in its low and row j + 4 in its high
 * nibble; rows n .. ld-1 are written as 0. For max_bins <= 16 (bins must be < 16);
 * pb_fit_buffers.bins4_dev takes the result and halves the bin bytes the histogram reads.
 * ld % 16 == 0, 0 <= n <= ld; bins_dev 16-byte aligned, out_dev 8-byte aligned. */
int pb_pack_bins4(const uint8_t* bins_dev, int64_t n, int64_t ld, int32_t F, uint8_t* out_dev,
                  void* stream);

/* apply_bins (data.py:93-111): bins[f][r] = min(searchsorted(edges[:, f], x, side="left"),
 * max_bins - 1) with NumPy's NaN-last order, x = xt[f][perm ? perm[r] : r] (xt: float32
 * [F][ld_x] column-major values; perm: optional int64 [n] row gather, e.g. the era-major
 * order). bins_dev: uint8 [F][ld_out], the histogram kernel's layout. */
int pb_apply_bins(const float* xt_dev, int64_t n, int64_t ld_x, int32_t F, const float* edges_dev,
                  int32_t num_edges, int32_t edge_stride, int32_t max_bins, const int64_t* perm_dev,
                  uint8_t* bins_dev, int64_t ld_out, void* stream);

/* ---- round metrics ------------------------------------------------------------------ */
/* Mean over eras of the Pearson correlation of y and preds (PackBoost._era_correlation_np,
 * booster.py:909-929, the train/eval corr of booster.py:474-491, 604-655), in double with a
 * fixed reduction order. Rows are era-major: era e is [era_off[e], era_off[e+1]) (device
 * int32 [E+1]). An era counts with >= 2 rows, both standard deviations > 1e-12 and a finite
 * correlation. era_corr_dev: double [E] per-era correlations (NaN where not counted);
 * out_dev: double [1], the mean (NaN if no era counts). */
int pb_era_corr(const float* y_dev, const float* preds_dev, const int32_t* era_off_dev,
                int32_t num_eras, double* era_corr_dev, double* out_dev, void* stream);

/* ---- prediction --------------------------------------------------------------------- */
/* Kernel 4 — batched pack prediction. Replaces predict_pack_cuda (frontier_cuda.cu:925-1068):
 * out[r] = tree_weight * sum_t value(leaf_t(r)) over the B trees of one packed forest
 * (the SoA layout of booster.py:730-783: feature, threshold, left_abs, right_abs int32,
 * value float32, is_leaf uint8, offsets int32 [B+1]). Traversal: left iff bin <= threshold.
 * bins_dev: column-major uint8 [F][ld], N rows. out_dev is overwritten (not accumulated).
 * leaf_dev (optional, may be NULL): int32 [B][N] absolute leaf index per tree and row. */
int pb_predict_pack(const uint8_t* bins_dev, int64_t N, int64_t ld, int32_t F,
                    const int32_t* feature_dev, const int32_t* threshold_dev,
                    const int32_t* left_abs_dev, const int32_t* right_abs_dev,
                    const float* value_dev, const uint8_t* is_leaf_dev,
                    const int32_t* offsets_dev, int32_t B, int32_t total_nodes,
                    float tree_weight, float* out_dev, int32_t* leaf_dev, void* stream);

/* Whole forest in PackBoost.predict's CPU order (booster.py:709-712): out[r] = sum over the
 * T trees in order of float32(tree_weight * value(leaf_t(r))), one float32 rounding per
 * product and per add. Same SoA layout as pb_predict_pack with offsets int32 [T+1]. */
int pb_predict_forest(const uint8_t* bins_dev, int64_t N, int64_t ld, int32_t F,
                      const int32_t* feature_dev, const int32_t* threshold_dev,
                      const int32_t* left_abs_dev, const int32_t* right_abs_dev,
                      const float* value_dev, const uint8_t* is_leaf_dev,
                      const int32_t* offsets_dev, int32_t T, int32_t total_nodes,
                      float tree_weight, float* out_dev, void* stream);

/* Compiled forest for repeated prediction (the reference re-packs per call,
 * booster.py:730-783 + predict_pack_cuda, frontier_cuda.cu:925-1068). pb_forest_create reads
 * the packed SoA forest (same arrays and layout as pb_predict_forest, offsets int32 [T+1],
 * device pointers), checks every tree (children inside the tree, no node reached twice,
 * 0 <= feature < 2^24 - 1, 0 <= threshold <= 255) and stores one 16-byte record per node
 * in device memory the handle owns, plus, for forests up to depth 8 whose row tile fits the
 * LDS, every tree as a complete heap for the tiled walk; runs of consecutive identical trees
 * (a fitted pack's B copies) are stored there once with their length.
 * pb_forest_predict: out[r] = sum over trees of float32(tree_weight * leaf value)
 * (booster.py:709-712). The tiled walk (used when the row stride and bins are 4-byte
 * aligned) adds the products in double, a run's length times its product in one exact fma,
 * and rounds once, so it agrees with pb_predict_forest's tree-order float32 sum within that
 * sum's roundings; otherwise one lane per row walks the trees in order with pb_predict_forest's
 * float32 adds, bit for bit. leaf_dev (optional): int32 [T][N] absolute leaf index per tree
 * (every tree of a run). PB_ERR_RANGE if a split feature is >= F. */
typedef struct pb_forest pb_forest;
int pb_forest_create(const int32_t* feature_dev, const int32_t* threshold_dev,
                     const int32_t* left_abs_dev, const int32_t* right_abs_dev,
                     const float* value_dev, const uint8_t* is_leaf_dev,
                     const int32_t* offsets_dev, int32_t T, int32_t total_nodes, pb_forest** out);
int pb_forest_predict(const pb_forest* forest, const uint8_t* bins_dev, int64_t N, int64_t ld,
                      int32_t F, float tree_weight, float* out_dev, int32_t* leaf_dev,
                      void* stream);
int pb_forest_destroy(pb_forest* forest);

/* Single tree. Replaces predict_bins_cuda (frontier_cuda.cu:193-233, 853-920):
 * out[r] = value(leaf(r)) with child indices relative to the tree. */
int pb_predict_bins(const uint8_t* bins_dev, int64_t N, int64_t ld, int32_t F,
                    const int32_t* feature_dev, const int32_t* threshold_dev,
                    const int32_t* left_dev, const int32_t* right_dev,
                    const float* value_dev, const uint8_t* is_leaf_dev, int32_t num_nodes,
                    float* out_dev, void* stream);

/* ---- row lists ---------------------------------------------------------------------- */
/* The reference's CUDA backend takes the rows of each frontier node as per-era lists:
 * rows_index int32 [R] with node_row_splits int32 [S+1] and node_era_splits int32 [S][E+1];
 * segment (s, e) is rows_index[node_row_splits[s] + node_era_splits[s][e] ..
 * node_row_splits[s] + node_era_splits[s][e+1]) (frontier_cuda.cu:576-598, 719-726). Bins are
 * feature-major uint8 [F][ld] with N rows (the reference's int8 [F][N], booster.py:419-426).
 *
 * These entry points are fully asynchronous and check every index on the device: after the
 * stream has run them, work_dev[0..3] are nonzero if a segment lay outside [0, R), a row id
 * outside [0, N), a feature outside [0, F), or an output would pass its capacity (nothing is
 * read or written out of range; results are then unspecified). work_dev: int32
 * [pb_rowlist_work_elems(nodes, E)], the nodes of the call. */
int64_t pb_rowlist_work_elems(int32_t num_nodes, int32_t num_eras);

/* partition_frontier_cuda (frontier_cuda.cu:719-851; the CPU path's stable per-era split,
 * frontier_cpu.cpp:446-497): every segment (s, e) splits stably into its rows with
 * bin[feat[s]][row] <= thr[s] (left) and the rest (right), in list order. left_index and
 * right_index receive the node-major, era-minor concatenation (capacity entries each; R
 * suffices for disjoint segments); left_splits / right_splits int32 [S][E+1] are absolute
 * offsets into them (entry [S-1][E] = the total). */
int pb_rowlist_partition(const uint8_t* bins_dev, int64_t N, int64_t ld, int32_t F,
                         const int32_t* rows_dev, int64_t R, const int32_t* node_row_splits_dev,
                         const int32_t* node_era_splits_dev, int32_t S, int32_t E,
                         const int32_t* feat_dev, const int32_t* thr_dev, int32_t* left_index_dev,
                         int32_t* right_index_dev, int64_t capacity, int32_t* left_splits_dev,
                         int32_t* right_splits_dev, int32_t* work_dev, void* stream);

/* No counterpart in the reference: pb_rowlist_partition for callers that cannot allocate
 * device memory (HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same inputs, outputs and results; the workspace is a fixed device array the library holds per
 * device (16 MiB, kept until the process ends) instead of work_dev, and the four status words
 * come back in status_dev (int32 [4], written by the call's own kernels). No allocation, no
 * hipMemset. At most pb_rowlist_noalloc_max_segments() (node, era) segments, S * E, per call:
 * larger calls return PB_ERR_UNSUPPORTED before any device work. Calls that overlap on one
 * device share that array and race: serialise them (one stream, or events). */
int64_t pb_rowlist_noalloc_max_segments(void);
int pb_rowlist_partition_noalloc(const uint8_t* bins_dev, int64_t N, int64_t ld, int32_t F,
                                 const int32_t* rows_dev, int64_t R, const int32_t* node_row_splits_dev,
                                 const int32_t* node_era_splits_dev, int32_t S, int32_t E,
                                 const int32_t* feat_dev, const int32_t* thr_dev,
                                 int32_t* left_index_dev, int32_t* right_index_dev, int64_t capacity,
                                 int32_t* left_splits_dev, int32_t* right_splits_dev,
                                 int32_t* status_dev, void* stream);

/* The row-gathering half of find_best_splits_batched_cuda (frontier_cuda.cu:576-716, which
 * reads bins[f][rows_index[i]] and grad[i] per list position): the listed rows of nodes
 * [node_begin, node_end) in era-major order (era, then node, then list order), the layout
 * pb_hist_build reads. Position d receives out_bins[k][d] = bins[feats[k]][row] (k < K),
 * out_values[d] = values[i] (values: float32 [R] per list position, e.g. grad) and
 * out_slot[d] = node - node_begin; era_off_dev int32 [E+1] receives the era boundaries
 * (era_off[E] = the rows gathered, at most out_ld). Positions past era_off[E] are not
 * written. Up to 65534 nodes per call. */
int pb_rowlist_gather(const uint8_t* bins_dev, int64_t N, int64_t ld, int32_t F,
                      const int32_t* feats_dev, int32_t K, const float* values_dev,
                      const int32_t* rows_dev, int64_t R, const int32_t* node_row_splits_dev,
                      const int32_t* node_era_splits_dev, int32_t node_begin, int32_t node_end,
                      int32_t E, uint8_t* out_bins_dev, int64_t out_ld, float* out_values_dev,
                      uint16_t* out_slot_dev, int32_t* era_off_dev, int32_t* work_dev, void* stream);

/* The per-(node, feature) pick of find_best_splits_batched_cuda (frontier_cuda.cu:537-560)
 * over candidate records cand_dev [M][K][T] (pb_des_score's cand_all_dev, thresholds in
 * order): the best valid score wins; within 1e-12 of it the larger left count, then the
 * larger threshold. No valid candidate, or a non-finite best, gives score -inf (or the best),
 * threshold -1 and zero sums. Outputs [M][K]: left_hess = left count (squared loss). */
int pb_best_thresholds(const pb_candidate* cand_dev, int32_t M, int32_t K, int32_t T,
                       float* scores_dev, int32_t* thresholds_dev, float* left_grad_dev,
                       float* left_hess_dev, int64_t* left_count_dev, void* stream);

/* The per-node pick of find_best_splits_batched_cpu (frontier_cpu.cpp:415-426, the scan that
 * feeds its decisions at 446-499) over candidate records cand_dev [M][K][T] in its visiting
 * order (subset feature, then threshold: pb_des_score's cand_all_dev): features and thresholds
 * are scanned in order and a candidate replaces the best when it scores higher, or scores
 * within 1e-12 (a float32 difference) and has more left rows, then a larger feature id, then a
 * larger threshold; candidates with valid == 0 or a NaN score are skipped. out_dev [M]: the
 * winner (valid = 0, feature = threshold = -1 when the node has none). band_dev: int32
 * [M][K * T] scratch. */
int pb_pick_sequential(const pb_candidate* cand_dev, int32_t M, int32_t K, int32_t T, int32_t* band_dev,
                       pb_candidate* out_dev, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* PACKBOOST_HIP_H */
