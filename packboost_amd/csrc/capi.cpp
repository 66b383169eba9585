// C-ABI host layer of libpackboost_hip.so: argument validation (mirroring the reference's
// std::invalid_argument / std::out_of_range checks, frontier_cpu.cpp:125-135,176-178,263-265),
// launch-shape selection for the kernels, the per-fit context, and error reporting.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <utility>
#include <cstdio>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "pb_internal.h"

struct pb_ctx {
    pb_dims d;
    int64_t rows_padded;
    int32_t max_era_rows;
    int32_t umax;   // largest active-node count of any depth
    int32_t wmax;   // wavefront winners per node for K features x all thresholds
    int32_t device;
    int32_t* era_off_dev;
    pb::Frontier* st;
    pb::SplitRule* rules;
    pb::NodeTotal* ntot;
    pb_candidate* cand_w;
    pb_candidate* node_best;
    int32_t* ids[2];
    int32_t* thr_tab;
    // histogram work segments (eras above seg_rows rows split into parts; see HistArgs)
    int32_t S;
    int32_t* seg_info_dev;  // [S][4] per work segment: first row, end row, era, slot of a
                            // split era (-1: the era is one segment)
    float* win_sum;         // |grad| sum per window of pb::kGradWinRows rows (round_begin)
    int32_t* sh_era;        // [E] fixed-point gradient scale exponent of each era
    int32_t n_acc;          // eras split into several segments
    int32_t* acc_era_dev;   // [n_acc]
    uint32_t* acc_cnt;      // [n_acc][umax][max_feats][nb]
    unsigned long long* acc_g;
    bool cnt32;             // planes carry 32-bit counts (an era above 65535 rows)
    int32_t last_w;
    pb::SeqCands seq;              // every candidate of a depth [umax][max_feats][tmax]
    int32_t last_K, last_T;        // shape, feature ids and threshold table of the last
    const int32_t* last_feats;     // pb_des_score, read by pb_decide
    int32_t* feats_keep;           // [max_feats] the per-phase pb_des_score's copy of its ids
    const int32_t* last_thr_tab;
    int64_t lds_budget;
    int32_t force_copies;
    int32_t force_ftile;
    int32_t force_pairs;
    int32_t hist_block;  // 0: by LDS size, else 128 or 256 threads
    int32_t score_wgs;  // workgroups the producer/consumer scorer aims for
    int32_t score_staged;  // T >= 64 thresholds: LDS-staged scorer instead of the wide one
    int32_t score_pc_classic;  // unit era weights, T <= 63: the scorer whose consumer forms 1/n
    int32_t num_cus;        // compute units of the device
    int32_t hist_resident;  // histogram: loop work items over a resident grid
    int32_t hist_rounds;
    // phase timing of pb_grow_round (pb_profile_enable): per depth, 5 events bracket the
    // hist / score / decide / partition launches on the caller's stream
    // segment mode (pb_set_segment_mode): rows sorted by (era, slot) in two buffer sets
    bool seg_mode;
    int32_t seg_from;           // first depth scored by the fused kernel
    int32_t seg_ft;             // cap on the fused kernel's features per workgroup (0: rule)
    int32_t seg_major_nodes;    // frontier bound from which the fused kernel runs tile-major
    int32_t seg_cur;            // buffer set holding the current depth's rows
    pb::SegBuffers sb[2];
    int32_t* seg[2];            // [E][segw] segment starts of the rows in sb[i]
    pb::SegState ss;            // partition shape and workspace
    int32_t profile;  // 0 off, 1 every phase, 2 the histogram only
    int32_t bin_layout;  // bins_dev of pb_hist_build / pb_partition: 0 uint8, 1 nibble
    std::vector<hipEvent_t> ev_free;
    std::vector<std::pair<int32_t, std::array<hipEvent_t, 5>>> ev_pending;
};

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* where) {
    g_err = std::string("HIP error: ") + hipGetErrorString(e) + " (" + where + ")";
    return PB_ERR_HIP;
}

#define PB_HIP(call, where)                          \
    do {                                             \
        hipError_t e_ = (call);                      \
        if (e_ != hipSuccess) return hip_fail(e_, where); \
    } while (0)

int64_t env_int(const char* name, int64_t dflt) {
    const char* v = std::getenv(name);
    if (!v || !*v) return dflt;
    return std::strtoll(v, nullptr, 10);
}

int32_t max_nodes_at(const pb_ctx* c, int32_t depth) {
    int64_t cap = int64_t(1) << std::min(depth, 30);
    if (c->d.min_samples_leaf > 0) {
        const int64_t by_rows = c->d.num_rows / (2 * (int64_t)c->d.min_samples_leaf);
        cap = std::min(cap, std::max<int64_t>(1, by_rows));
    }
    cap = std::min<int64_t>(cap, 65534);
    return (int32_t)cap;
}

int32_t thresholds_per_feature(const pb_ctx* c, const pb_split_params* p) {
    const int full = std::max(1, c->d.max_bins - 1 - (p->skip_last_bin ? 1 : 0));
    if (p->k_cuts > 0 && p->k_cuts < full) return std::max(1, std::min(p->k_cuts, full));
    return full;
}

template <typename T>
int dev_alloc(T** p, size_t n, const char* what) {
    *p = nullptr;
    if (n == 0) n = 1;
    hipError_t e = hipMalloc(reinterpret_cast<void**>(p), n * sizeof(T));
    if (e != hipSuccess) return hip_fail(e, what);
    return PB_OK;
}

void free_ctx(pb_ctx* c) {
    if (!c) return;
    (void)hipFree(c->era_off_dev);
    (void)hipFree(c->win_sum);
    (void)hipFree(c->sh_era);
    (void)hipFree(c->st);
    (void)hipFree(c->rules);
    (void)hipFree(c->ntot);
    (void)hipFree(c->cand_w);
    (void)hipFree(c->seq.score);
    (void)hipFree(c->seq.lt);
    (void)hipFree(c->seq.lg);
    (void)hipFree(c->seq.band);
    (void)hipFree(c->node_best);
    (void)hipFree(c->ids[0]);
    (void)hipFree(c->ids[1]);
    (void)hipFree(c->thr_tab);
    (void)hipFree(c->feats_keep);
    for (int i = 0; i < 2; ++i) {
        (void)hipFree(c->sb[i].g);
        (void)hipFree(c->sb[i].row);
        (void)hipFree(c->sb[i].tnode);
        (void)hipFree(c->seg[i]);
    }
    (void)hipFree(c->ss.cp);
    (void)hipFree(c->ss.cnt_l);
    (void)hipFree(c->ss.cnt_r);
    (void)hipFree(c->ss.base);
    (void)hipFree(c->seg_info_dev);
    (void)hipFree(c->acc_era_dev);
    (void)hipFree(c->acc_cnt);
    (void)hipFree(c->acc_g);
    for (auto& p : c->ev_pending)
        for (hipEvent_t e : p.second)
            if (e) c->ev_free.push_back(e);
    for (hipEvent_t e : c->ev_free) (void)hipEventDestroy(e);
    delete c;
}

}  // namespace

extern "C" {

const char* pb_last_error(void) { return g_err.c_str(); }

int32_t pb_version(void) { return 100; }  // 0.1.0

int32_t pb_device_available(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) return 0;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
    return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int pb_ctx_create(const pb_dims* dims, const int32_t* era_off_host, pb_ctx** out) {
    if (!dims || !era_off_host || !out) return fail(PB_ERR_INVALID, "pb_ctx_create: null argument");
    *out = nullptr;
    const pb_dims& d = *dims;
    if (d.num_rows < 1) return fail(PB_ERR_INVALID, "num_rows must be >= 1");
    if (d.num_rows > (int64_t(1) << 30)) return fail(PB_ERR_UNSUPPORTED, "num_rows above 2^30");
    if (d.ld < d.num_rows || d.ld % 16 != 0)
        return fail(PB_ERR_INVALID, "ld must be >= num_rows and a multiple of 16");
    if (d.num_features < 1) return fail(PB_ERR_INVALID, "num_features must be >= 1");
    if (d.num_eras < 1) return fail(PB_ERR_INVALID, "num_eras must be >= 1");
    if (d.max_bins < 2 || d.max_bins > 255) return fail(PB_ERR_INVALID, "max_bins must be in [2, 255]");
    if (d.max_depth < 1 || d.max_depth > 15) return fail(PB_ERR_UNSUPPORTED, "max_depth must be in [1, 15]");
    if (d.max_feats < 1 || d.max_feats > d.num_features)
        return fail(PB_ERR_INVALID, "max_feats must be in [1, num_features]");
    if (d.min_samples_leaf < 0) return fail(PB_ERR_INVALID, "min_samples_leaf must be >= 0");
    if (era_off_host[0] != 0 || era_off_host[d.num_eras] != d.num_rows)
        return fail(PB_ERR_INVALID, "era offsets must start at 0 and end at num_rows");
    int32_t max_era = 0;
    for (int e = 0; e < d.num_eras; ++e) {
        const int32_t len = era_off_host[e + 1] - era_off_host[e];
        if (len < 0) return fail(PB_ERR_INVALID, "era offsets must be non-decreasing");
        max_era = std::max(max_era, len);
    }

    pb_ctx* c = new pb_ctx();
    c->d = d;
    c->rows_padded = (d.num_rows + 15) / 16 * 16;
    c->max_era_rows = max_era;
    (void)hipGetDevice(&c->device);
    c->umax = 1;
    for (int dd = 0; dd < d.max_depth; ++dd) c->umax = std::max(c->umax, max_nodes_at(c, dd));
    const int tmax = std::max(1, d.max_bins - 1);
    c->score_wgs = (int32_t)env_int("PB_SCORE_WGS", 768);
    c->score_staged = env_int("PB_SCORE_STAGED", 0) != 0 ? 1 : 0;
    c->score_pc_classic = (int32_t)std::min<int64_t>(2, std::max<int64_t>(0, env_int("PB_SCORE_PC", 0)));
    c->hist_resident = (int32_t)env_int("PB_HIST_RESIDENT", 0);
    c->hist_rounds = (int32_t)env_int("PB_HIST_ROUNDS", 1);
    c->num_cus = 0;
    if (hipDeviceGetAttribute(&c->num_cus, hipDeviceAttributeMultiprocessorCount, c->device) !=
        hipSuccess)
        c->num_cus = 0;
    c->wmax = 1;
    for (int t = 1; t <= tmax; ++t)
        for (int dd = 0; dd < d.max_depth; ++dd) {
            const pb::ScoreShape sh = pb::score_shape(d.max_feats, t, d.num_eras, max_nodes_at(c, dd),
                                                        c->score_wgs);
            c->wmax = std::max(c->wmax, sh.ntiles * sh.wpt);
        }
    for (int32_t ft = 1; ft <= pb::kSegMaxFt; ft *= 2) {  // the segment-mode scorer's winners, any tile width
        const int32_t nt = (d.max_feats + ft - 1) / ft;
        c->wmax = std::max(c->wmax, nt * std::min(4, (ft * std::max(1, d.max_bins - 1) + pb::kWave - 1) / pb::kWave));
    }
    c->lds_budget = env_int("PB_HIST_LDS_BUDGET", 0);  // 0: by frontier width
    c->hist_block = (int32_t)env_int("PB_HIST_BLOCK", 0);
    c->force_pairs = (int32_t)env_int("PB_HIST_PAIRS", 0);
    c->bin_layout = 0;
    c->force_copies = (int32_t)env_int("PB_HIST_COPIES", 0);
    c->force_ftile = (int32_t)env_int("PB_HIST_FTILE", 0);

    // work segments: an era above seg_rows rows is split into equal parts of at most seg_rows
    // (<= 65535, the LDS count field) whose exact sums are added up per era
    const int64_t seg_rows = std::min<int64_t>(65535, std::max<int64_t>(256, env_int("PB_HIST_SEG_ROWS", 16384)));
    std::vector<int32_t> seg_info, acc_era;
    for (int e = 0; e < d.num_eras; ++e) {
        const int64_t len = era_off_host[e + 1] - era_off_host[e];
        const int64_t parts = len > seg_rows ? (len + seg_rows - 1) / seg_rows : 1;
        const int32_t slot = parts > 1 ? (int32_t)acc_era.size() : -1;
        if (parts > 1) acc_era.push_back(e);
        for (int64_t j = 0; j < parts; ++j) {
            seg_info.push_back((int32_t)(era_off_host[e] + len * j / parts));
            seg_info.push_back((int32_t)(era_off_host[e] + len * (j + 1) / parts));
            seg_info.push_back(e);
            seg_info.push_back(slot);
        }
    }
    c->S = (int32_t)(seg_info.size() / 4);
    c->n_acc = (int32_t)acc_era.size();
    c->cnt32 = max_era > pb::kMaxEraRowsDirect;
    const size_t acc_cells = (size_t)c->n_acc * c->umax * d.max_feats * d.max_bins;

    int rc = PB_OK;
    if ((rc = dev_alloc(&c->seg_info_dev, std::max<size_t>(4, seg_info.size()), "alloc segments")) ||
        (rc = dev_alloc(&c->acc_era_dev, std::max<size_t>(1, acc_era.size()), "alloc segment slots")) ||
        (rc = dev_alloc(&c->acc_cnt, std::max<size_t>(1, acc_cells), "alloc segment sums")) ||
        (rc = dev_alloc(&c->acc_g, std::max<size_t>(1, acc_cells), "alloc segment sums"))) {
        free_ctx(c);
        return rc;
    }
    {
        hipError_t e1 = hipSuccess;
        if (!seg_info.empty())
            e1 = hipMemcpy(c->seg_info_dev, seg_info.data(), sizeof(int32_t) * seg_info.size(),
                           hipMemcpyHostToDevice);
        if (e1 == hipSuccess && !acc_era.empty())
            e1 = hipMemcpy(c->acc_era_dev, acc_era.data(), sizeof(int32_t) * acc_era.size(),
                           hipMemcpyHostToDevice);
        if (e1 == hipSuccess && acc_cells > 0) e1 = hipMemset(c->acc_cnt, 0, sizeof(uint32_t) * acc_cells);
        if (e1 == hipSuccess && acc_cells > 0)
            e1 = hipMemset(c->acc_g, 0, sizeof(unsigned long long) * acc_cells);
        if (e1 != hipSuccess) {
            free_ctx(c);
            return hip_fail(e1, "copy segments");
        }
    }
    if ((rc = dev_alloc(&c->era_off_dev, d.num_eras + 1, "alloc era offsets")) ||
        (rc = dev_alloc(&c->win_sum, (c->rows_padded + pb::kGradWinRows - 1) / pb::kGradWinRows,
                        "alloc gradient windows")) ||
        (rc = dev_alloc(&c->sh_era, d.num_eras, "alloc era scales")) ||
        (rc = dev_alloc(&c->st, 1, "alloc frontier")) ||
        (rc = dev_alloc(&c->rules, c->umax, "alloc split rules")) ||
        (rc = dev_alloc(&c->ntot, c->umax, "alloc node totals")) ||
        (rc = dev_alloc(&c->cand_w, (size_t)c->umax * c->wmax, "alloc candidates")) ||
        (rc = dev_alloc(&c->seq.score, (size_t)c->umax * d.max_feats * tmax, "alloc candidates")) ||
        (rc = dev_alloc(&c->seq.lt, (size_t)c->umax * d.max_feats * tmax, "alloc candidates")) ||
        (rc = dev_alloc(&c->seq.lg, (size_t)c->umax * d.max_feats * tmax, "alloc candidates")) ||
        (rc = dev_alloc(&c->seq.band, (size_t)c->umax * d.max_feats * tmax, "alloc candidates")) ||
        (rc = dev_alloc(&c->node_best, c->umax, "alloc node winners")) ||
        (rc = dev_alloc(&c->ids[0], std::max(c->umax, 2) * 2, "alloc frontier ids")) ||
        (rc = dev_alloc(&c->ids[1], std::max(c->umax, 2) * 2, "alloc frontier ids")) ||
        (rc = dev_alloc(&c->thr_tab, (size_t)d.max_feats * tmax, "alloc threshold table")) ||
        (rc = dev_alloc(&c->feats_keep, (size_t)d.max_feats, "alloc feature ids"))) {
        free_ctx(c);
        return rc;
    }
    hipError_t e = hipMemcpy(c->era_off_dev, era_off_host, sizeof(int32_t) * (d.num_eras + 1),
                             hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        free_ctx(c);
        return hip_fail(e, "copy era offsets");
    }
    e = hipMemset(c->sh_era, 0, sizeof(int32_t) * d.num_eras);
    if (e == hipSuccess) e = hipMemset(c->st, 0, sizeof(pb::Frontier));
    if (e != hipSuccess) {
        free_ctx(c);
        return hip_fail(e, "clear frontier");
    }
    *out = c;
    return PB_OK;
}

int pb_ctx_destroy(pb_ctx* ctx) {
    free_ctx(ctx);
    return PB_OK;
}

int64_t pb_hist_plane_elems(const pb_ctx* c, int32_t max_nodes) {
    if (!c) return -1;
    return pb::plane_elems(c->d.num_eras, max_nodes, c->d.max_feats, c->d.max_bins);
}

int32_t pb_max_nodes(const pb_ctx* c, int32_t depth) {
    if (!c || depth < 0) return -1;
    return max_nodes_at(c, depth);
}

const int32_t* pb_era_offsets_dev(const pb_ctx* c) { return c ? c->era_off_dev : nullptr; }

int pb_round_begin(pb_ctx* c, const float* preds, const float* y, float* grad, uint16_t* nid,
                   uint16_t* tnode, void* stream) {
    if (!c || !preds || !y || !grad || !nid || !tnode)
        return fail(PB_ERR_INVALID, "pb_round_begin: null argument");
    const int64_t N = c->d.num_rows;
    const int32_t root_active = (N >= 2 * (int64_t)c->d.min_samples_leaf) ? 1 : 0;
    PB_HIP(pb::launch_round_begin(preds, y, grad, nid, tnode, N, c->rows_padded, root_active,
                                  c->era_off_dev, c->d.num_eras, c->win_sum, c->sh_era, c->st,
                                  c->ids[0], (hipStream_t)stream),
           "round_begin launch");
    return PB_OK;
}

namespace {

// pb_hist_build over either bin layout: uint8 columns of stride ld (nibble 0) or the
// two-rows-per-byte columns of stride ld / 2 that pb_pack_bins4 writes (nibble 1).
int hist_build(pb_ctx* c, const uint8_t* bins, int64_t ld_bytes, int32_t nibble, const float* grad,
               const uint16_t* nid, const int32_t* feats, int32_t K, int32_t depth,
               int32_t max_nodes, int32_t* hist_cnt, float* hist_grad, void* stream) {
    if (!c || !bins || !grad || !nid || !feats || !hist_cnt || !hist_grad)
        return fail(PB_ERR_INVALID, "pb_hist_build: null argument");
    if (K < 1 || K > c->d.max_feats) return fail(PB_ERR_INVALID, "pb_hist_build: K out of range");
    if (depth < 0 || depth >= c->d.max_depth) return fail(PB_ERR_RANGE, "pb_hist_build: depth out of range");
    if (max_nodes < max_nodes_at(c, depth))
        return fail(PB_ERR_INVALID, "pb_hist_build: max_nodes below the frontier bound of this depth");
    if ((reinterpret_cast<uintptr_t>(bins) & 15) || (reinterpret_cast<uintptr_t>(grad) & 15) ||
        (reinterpret_cast<uintptr_t>(nid) & (nibble ? 15 : 7)))
        return fail(PB_ERR_INVALID,
                    "pb_hist_build: bins/grad must be 16-byte and nid 8-byte (nibble bins: 16-byte) aligned");

    const int nb = c->d.max_bins;
    // Launch shape, from sweeps on MI355X at the 2.4M x 2376 x 5-bin panel: feature pairs (or
    // triples) share one atomic on joint bins when nb * nb <= 256; the LDS per workgroup stays
    // within a small budget (occupancy beats copies), the largest feature tile that fits comes
    // first, then as many histogram copies as fit in half of that.
    int P = (nb <= 16 && K >= 2) ? 2 : 1;
    // feature triples while their joint histogram stays small (at most 512 cells per copy:
    // depths 0-2 at 5 bins), where a third fewer atomics beat the larger flush; at 5-6 bins up
    // to 1000 cells (8 nodes at 5 bins) with 12-feature tiles in a 40 KB budget (config 3's
    // depth 3: 121 against 135 us for 16-feature pair tiles; 16 nodes measured slower)
    const int64_t tri_cells = (int64_t)max_nodes * nb * nb * nb;
    if (nb <= 6 && K >= 3 && (tri_cells <= 512 || (nb >= 5 && tri_cells <= 1000))) P = 3;
    if (c->force_pairs == 1 || (c->force_pairs == 2 && nb <= 16) ||
        (c->force_pairs == 3 && nb <= 6 && K >= 3))
        P = c->force_pairs;
    const int64_t cells_node = (P == 3 ? nb * nb * nb : P == 2 ? nb * nb : nb);
    // budget: 20 KB for narrow frontiers (2-wave workgroups), 26 KB from 16 nodes on, where
    // 16-feature pair tiles and 4-wave workgroups measured faster (config 3 depths 4-5)
    int64_t budget = c->lds_budget > 0 ? c->lds_budget : (max_nodes >= 16 ? 26 * 1024 : 20000);
    if (c->lds_budget <= 0 && P == 3 && tri_cells > 512) budget = 40000;
    int64_t cap = std::max<int64_t>(budget, 4 * 1024);
    // node tiles when one feature's node x bin histogram does not fit: single features, up
    // to 32 KiB of LDS, as many nodes per tile as fit (swept at 1M rows x 500 features x 255
    // bins, depths 4-7: 32 KiB beat 12-24 KiB (more tiles re-read the rows) and 48-160 KiB
    // (fewer resident workgroups), also where two features per item would fit in 64 KiB)
    int node_tile = max_nodes;
    if ((int64_t)max_nodes * cells_node * 8 > cap) {
        P = 1;
        cap = c->lds_budget > 0 ? std::min<int64_t>(std::max<int64_t>(c->lds_budget, (int64_t)nb * 8),
                                                   160 * 1024)
                                : std::max<int64_t>(cap, 32 * 1024);
        node_tile = (int)std::max<int64_t>(1, std::min<int64_t>(max_nodes, cap / ((int64_t)nb * 8)));
    }
    const int node_tiles = (max_nodes + node_tile - 1) / node_tile;
    const int64_t cells_group =
        (int64_t)node_tile * (P == 3 ? nb * nb * nb : P == 2 ? nb * nb : nb);
    const int64_t groups_k = (K + P - 1) / P;
    // FT <= 16 (more registers cost occupancy); triples: FT <= 12
    const int max_groups = (P == 3) ? 4 : (P == 2) ? 8 : 16;
    int64_t groups = max_groups;
    if (c->force_ftile > 0) groups = std::max<int64_t>(1, std::min(c->force_ftile, P == 2 ? 32 : 16) / P);
    while (groups > 1 && groups * cells_group * 8 > cap) groups /= 2;
    int64_t need = 1;
    while (need < groups_k) need *= 2;  // no more groups than the features present need
    groups = std::min<int64_t>(groups, need);
    int clog2 = 0;
    if (c->force_copies > 0) {
        while ((1 << (clog2 + 1)) <= c->force_copies && clog2 < 5) ++clog2;
    } else {
        while (clog2 < 5 && groups * cells_group * (int64_t(2) << clog2) * 8 <= cap / 2) ++clog2;
    }
    const int64_t per_group = cells_group * (int64_t(1) << clog2) * 8;
    while (groups > 1 && groups * per_group > 160 * 1024) groups /= 2;  // forced copies
    const int ftile = (int)groups * P;
    const size_t lds_bytes =
        (size_t)groups * 8 *
        (size_t)pb::hist_group_words((int)(per_group / 8), P, nb, 1 << clog2, (int)groups);
    if (lds_bytes > 160 * 1024)
        return fail(PB_ERR_UNSUPPORTED,
                    "pb_hist_build: one feature's node x bin histogram exceeds the 160 KiB LDS");

    pb::HistArgs a{};
    a.resident_cus = c->hist_resident ? c->num_cus : 0;
    a.rounds = c->hist_rounds;
    a.bins = bins;
    a.ld = ld_bytes;
    a.nibble = nibble;
    // 4-wave workgroups: an era takes fewer passes, and each workgroup's fixed costs (segment
    // set-up, flush) are shared by twice the rows (measured faster at every depth of a 2.4M-row,
    // 5-bin round than 2-wave workgroups)
    a.block = (c->hist_block == 128 || c->hist_block == 256) ? c->hist_block : 256;
    a.grad = grad;
    a.nid = nid;
    a.feats = feats;
    a.K = K;
    a.ntiles = (K + ftile - 1) / ftile;
    a.ftile = ftile;
    a.U = max_nodes;
    a.node_tile = node_tile;
    a.node_tiles = node_tiles;
    a.nb = nb;
    a.clog2 = clog2;
    a.st = c->st;
    a.depth = depth;
    {
        const int64_t to = pb::plane_tot_off(c->d.num_eras, max_nodes, K, c->d.max_bins);
        a.out_cnt = reinterpret_cast<uint16_t*>(hist_cnt);
        a.out_cnt32 = c->cnt32 ? reinterpret_cast<uint32_t*>(hist_cnt) : nullptr;
        a.out_tot_cnt = hist_cnt + to;
        a.out_g = hist_grad;
        a.out_tot_g = hist_grad + to;
    }
    a.seg_info = reinterpret_cast<const int4*>(c->seg_info_dev);
    a.S = c->S;
    a.acc_cnt = c->acc_cnt;
    a.acc_g = c->acc_g;
    a.acc_U = c->umax;  // active nodes < umax whatever max_nodes the caller passes
    a.acc_K = c->d.max_feats;
    a.sh_era = c->sh_era;
    const int eras8 = (a.S + 7) / 8 * 8;  // segments, a multiple of the 8 XCDs
    const int64_t grid = (int64_t)eras8 * a.ntiles * node_tiles;
    if (grid > INT32_MAX) return fail(PB_ERR_UNSUPPORTED, "pb_hist_build: grid too large");
    PB_HIP(pb::launch_hist(a, P, (int)grid, lds_bytes, (hipStream_t)stream), "hist launch");
    if (c->n_acc > 0) {
        pb::FinalizeArgs f;
        f.acc_cnt = c->acc_cnt;
        f.acc_g = c->acc_g;
        f.acc_era = c->acc_era_dev;
        f.n_acc = c->n_acc;
        f.U = max_nodes;
        f.K = K;
        f.nb = nb;
        f.acc_U = a.acc_U;
        f.acc_K = a.acc_K;
        f.sh_era = c->sh_era;
        f.st = c->st;
        f.depth = depth;
        f.out_cnt = a.out_cnt;
        f.out_cnt32 = a.out_cnt32;
        f.out_tot_cnt = a.out_tot_cnt;
        f.out_g = a.out_g;
        f.out_tot_g = a.out_tot_g;
        PB_HIP(pb::launch_finalize(f, (hipStream_t)stream), "finalize launch");
    }
    return PB_OK;
}

int partition(pb_ctx* c, const uint8_t* bins, int64_t ld_bytes, int32_t nibble, int32_t depth,
              uint16_t* nid, uint16_t* tnode, void* stream) {
    if (!c || !bins || !nid || !tnode) return fail(PB_ERR_INVALID, "pb_partition: null argument");
    if (depth < 0 || depth >= c->d.max_depth) return fail(PB_ERR_RANGE, "pb_partition: depth out of range");
    if ((reinterpret_cast<uintptr_t>(nid) & 15) || (reinterpret_cast<uintptr_t>(tnode) & 15))
        return fail(PB_ERR_INVALID, "pb_partition: nid/tnode must be 16-byte aligned");
    PB_HIP(pb::launch_partition(bins, ld_bytes, nibble, c->rows_padded, c->rules, c->st, depth, nid,
                                tnode, (hipStream_t)stream),
           "partition launch");
    return PB_OK;
}

}  // namespace

int pb_hist_build(pb_ctx* c, const uint8_t* bins, const float* grad, const uint16_t* nid,
                  const int32_t* feats, int32_t K, int32_t depth, int32_t max_nodes,
                  int32_t* hist_cnt, float* hist_grad, void* stream) {
    if (!c) return fail(PB_ERR_INVALID, "pb_hist_build: null argument");
    const int32_t nib = c->bin_layout;
    return hist_build(c, bins, nib ? c->d.ld / 2 : c->d.ld, nib, grad, nid, feats, K, depth,
                      max_nodes, hist_cnt, hist_grad, stream);
}

int pb_set_bin_layout(pb_ctx* c, int32_t layout) {
    if (!c) return fail(PB_ERR_INVALID, "pb_set_bin_layout: null context");
    if (layout != 0 && layout != 1) return fail(PB_ERR_INVALID, "pb_set_bin_layout: layout must be 0 or 1");
    if (layout == 1 && c->d.max_bins > 16)
        return fail(PB_ERR_INVALID, "pb_set_bin_layout: the nibble layout needs max_bins <= 16");
    c->bin_layout = layout;
    return PB_OK;
}

namespace {

// pb_des_score's work. keep_feats: copy the K feature ids into the context (stream-ordered,
// before pb_decide reads them), so that a caller of the per-phase C ABI may free or rewrite its
// buffer between pb_des_score and pb_decide; pb_grow_round passes false (the ids it scores
// stay put for the whole call, and a copy per depth would cost a launch).
int des_score(pb_ctx* c, const int32_t* hist_cnt, const float* hist_grad, const int32_t* feats,
              int32_t K, int32_t depth, int32_t max_nodes, const pb_split_params* p,
              pb_candidate* cand_all, void* stream, bool keep_feats) {
    if (!c || !hist_cnt || !hist_grad || !feats || !p)
        return fail(PB_ERR_INVALID, "pb_des_score: null argument");
    if (K < 1 || K > c->d.max_feats) return fail(PB_ERR_INVALID, "pb_des_score: K out of range");
    if (depth < 0 || depth >= c->d.max_depth) return fail(PB_ERR_RANGE, "pb_des_score: depth out of range");
    if (max_nodes < max_nodes_at(c, depth))
        return fail(PB_ERR_INVALID, "pb_des_score: max_nodes below the frontier bound of this depth");
    const int nb = c->d.max_bins;  // bins of the planes
    const int skip = p->skip_last_bin ? 1 : 0;
    if (skip && nb < 3)
        return fail(PB_ERR_INVALID, "pb_des_score: skip_last_bin needs a context of max_bins >= 3");
    const int T = thresholds_per_feature(c, p);
    const int full = std::max(1, nb - skip - 1);
    const int32_t* thr_tab = nullptr;
    if (p->k_cuts > 0 && p->k_cuts < full) {
        PB_HIP(pb::launch_kcuts(reinterpret_cast<const uint16_t*>(hist_cnt),
                                c->cnt32 ? reinterpret_cast<const uint32_t*>(hist_cnt) : nullptr,
                                hist_cnt + pb::plane_tot_off(c->d.num_eras, max_nodes, K, nb),
                                c->d.num_eras, max_nodes, K, nb - skip, skip, p->k_cuts,
                                p->cut_selection == 1 ? 1 : 0, c->st, depth, c->thr_tab,
                                (hipStream_t)stream),
               "kcuts launch");
        thr_tab = c->thr_tab;
    }
    const pb::ScoreShape sh = skip ? pb::score_shape_classic(K, T, c->d.num_eras)
                                   : pb::score_shape(K, T, c->d.num_eras, max_nodes_at(c, depth),
                                                     c->score_wgs);
    const int64_t grid = (int64_t)sh.ntiles * max_nodes_at(c, depth);
    if (grid > INT32_MAX) return fail(PB_ERR_UNSUPPORTED, "pb_des_score: grid too large");
    if (sh.ntiles * sh.wpt > c->wmax) return fail(PB_ERR_INVALID, "pb_des_score: candidate buffer too small");
    // the scorer addresses one chunk of eras' plane cells with 31-bit offsets
    if ((int64_t)(pb::kScoreChunkEras + 1) * max_nodes * K * std::max(1, nb - 1) >= (int64_t(1) << 31))
        return fail(PB_ERR_UNSUPPORTED, "pb_des_score: max_nodes x K x bins too large for one era chunk");
    pb::ScoreArgs a{};
    {
        const int64_t to = pb::plane_tot_off(c->d.num_eras, max_nodes, K, nb);
        a.cnt = reinterpret_cast<const uint16_t*>(hist_cnt);
        a.cnt32 = c->cnt32 ? reinterpret_cast<const uint32_t*>(hist_cnt) : nullptr;
        a.tot_cnt = hist_cnt + to;
        a.g = hist_grad;
        a.tot_g = hist_grad + to;
    }
    a.E = c->d.num_eras;
    a.U = max_nodes;
    a.K = K;
    a.nb = nb;
    a.T = T;
    a.feats = feats;
    a.thr_tab = thr_tab;
    a.lambda_l2 = (float)p->lambda_l2;
    a.lambda_dro = (float)p->lambda_dro;
    a.dir_w = (float)p->direction_weight;
    a.era_alpha = (float)p->era_alpha;
    a.msl = p->min_samples_leaf;
    a.st = c->st;
    a.depth = depth;
    a.cand_w = c->cand_w;
    a.cand_all = cand_all;
    a.ntot = c->ntot;
    a.fts = sh.fts;
    a.ntiles = sh.ntiles;
    a.ec = sh.ec;
    a.wpt = sh.wpt;
    a.rt = sh.rt;
    a.staged = c->score_staged;
    a.pc_classic = c->score_pc_classic;
    a.seq = c->seq;
    a.skip_last = skip;
    c->last_w = sh.ntiles * sh.wpt;
    c->last_K = K;
    c->last_T = T;
    c->last_feats = feats;
    c->last_thr_tab = thr_tab;
    PB_HIP(pb::launch_score(a, (int)grid, sh.lds_bytes, (hipStream_t)stream), "score launch");
    if (keep_feats) {
        PB_HIP(hipMemcpyAsync(c->feats_keep, feats, sizeof(int32_t) * K, hipMemcpyDeviceToDevice,
                              (hipStream_t)stream),
               "feature id copy");
        c->last_feats = c->feats_keep;
    }
    return PB_OK;
}

}  // namespace

int pb_des_score(pb_ctx* c, const int32_t* hist_cnt, const float* hist_grad, const int32_t* feats,
                 int32_t K, int32_t depth, int32_t max_nodes, const pb_split_params* p,
                 pb_candidate* cand_all, void* stream) {
    return des_score(c, hist_cnt, hist_grad, feats, K, depth, max_nodes, p, cand_all, stream, true);
}

int pb_decide(pb_ctx* c, int32_t depth, int32_t max_nodes, const pb_split_params* p,
              pb_decision* dec, float* values, void* stream) {
    if (!c || !p || !dec || !values) return fail(PB_ERR_INVALID, "pb_decide: null argument");
    if (depth < 0 || depth >= c->d.max_depth) return fail(PB_ERR_RANGE, "pb_decide: depth out of range");
    if (c->last_w <= 0) return fail(PB_ERR_INVALID, "pb_decide: call pb_des_score first");
    if (max_nodes < max_nodes_at(c, depth))
        return fail(PB_ERR_INVALID, "pb_decide: max_nodes below the frontier bound of this depth");
    pb::DecideCands dc;
    dc.cand_w = c->cand_w;
    dc.W = c->last_w;
    dc.seq = c->seq;
    dc.K = c->last_K;
    dc.T = c->last_T;
    dc.feats = c->last_feats;
    dc.thr_tab = c->last_thr_tab;
    PB_HIP(pb::launch_decide(dc, max_nodes, c->ntot, c->st, depth, p->min_samples_leaf, p->lambda_l2,
                             c->ids[depth & 1], c->ids[(depth + 1) & 1], c->rules, dec, values,
                             c->node_best, (hipStream_t)stream),
           "decide launch");
    return PB_OK;
}

int pb_partition(pb_ctx* c, const uint8_t* bins, int32_t depth, uint16_t* nid, uint16_t* tnode,
                 void* stream) {
    if (!c) return fail(PB_ERR_INVALID, "pb_partition: null argument");
    const int32_t nib = c->bin_layout;
    return partition(c, bins, nib ? c->d.ld / 2 : c->d.ld, nib, depth, nid, tnode, stream);
}

namespace {

// pb_round_end's work; with `header`, the kernel also writes the round header
int round_end(pb_ctx* c, const uint16_t* tnode, const float* values, int32_t pack_size, float lr,
              float* preds, pb_round_header* header, void* stream) {
    if (!c || !tnode || !values || !preds) return fail(PB_ERR_INVALID, "pb_round_end: null argument");
    if (pack_size < 1) return fail(PB_ERR_INVALID, "pb_round_end: pack_size must be >= 1");
    PB_HIP(pb::launch_round_end(tnode, values, pack_size, lr, preds, c->d.num_rows, c->st, header,
                                (hipStream_t)stream),
           "round_end launch");
    return PB_OK;
}

}  // namespace

int pb_round_end(pb_ctx* c, const uint16_t* tnode, const float* values, int32_t pack_size,
                 float lr, float* preds, void* stream) {
    return round_end(c, tnode, values, pack_size, lr, preds, nullptr, stream);
}

namespace {

// The segment-mode scorer of depth `depth` (pb::launch_seg_score) over the context's sorted rows,
// leaving what pb_decide reads as pb_des_score does.
int seg_score(pb_ctx* c, const uint8_t* bins, const int32_t* feats, int32_t K, int32_t depth, int32_t max_nodes,
              const pb_split_params* p, void* stream) {
    const int nb = c->d.max_bins;
    pb::SegScoreArgs a{};
    a.bins = bins;
    a.row = c->sb[c->seg_cur].row;
    a.ld = c->d.ld;
    a.g = c->sb[c->seg_cur].g;
    a.seg = c->seg[c->seg_cur];
    a.segw = c->ss.segw;
    a.sh_era = c->sh_era;
    a.feats = feats;
    a.K = K;
    a.E = c->d.num_eras;
    a.nb = nb;
    a.T = nb - 1;
    a.lambda_l2 = (float)p->lambda_l2;
    a.lambda_dro = (float)p->lambda_dro;
    a.dir_w = (float)p->direction_weight;
    a.era_alpha = (float)p->era_alpha;
    a.msl = p->min_samples_leaf;
    a.st = c->st;
    a.depth = depth;
    a.cand_w = c->cand_w;
    a.fts = pb::seg_score_fts(max_nodes, K);
    if (c->seg_ft > 0) a.fts = std::min<int32_t>(a.fts, c->seg_ft);  // PB_SEG_FT: at most this many
    a.ntiles = (K + a.fts - 1) / a.fts;
    a.wpt = std::min(4, (a.fts * a.T + pb::kWave - 1) / pb::kWave);
    a.seq = c->seq;
    a.ntot = c->ntot;
    a.rt = std::max(2, std::min<int32_t>(a.E + 1, 4096));
    a.tile_major = max_nodes >= c->seg_major_nodes ? 1 : 0;
    if (a.ntiles * a.wpt > c->wmax) return fail(PB_ERR_INVALID, "segment scorer: candidate buffer too small");
    c->last_w = a.ntiles * a.wpt;
    c->last_K = K;
    c->last_T = a.T;
    c->last_feats = feats;
    c->last_thr_tab = nullptr;
    PB_HIP(pb::launch_seg_score(a, max_nodes, (hipStream_t)stream), "segment scorer launch");
    return PB_OK;
}

}  // namespace

int pb_set_segment_mode(pb_ctx* c, int32_t enable, int32_t from_depth) {
    if (!c) return fail(PB_ERR_INVALID, "pb_set_segment_mode: null context");
    if (enable != 0 && enable != 1) return fail(PB_ERR_INVALID, "pb_set_segment_mode: enable must be 0 or 1");
    if (!enable) {
        c->seg_mode = false;
        return PB_OK;
    }
    if (c->max_era_rows > pb::kMaxEraRowsDirect)
        return fail(PB_ERR_UNSUPPORTED, "pb_set_segment_mode: an era holds more than 65535 rows");
    if (c->d.num_rows >= INT32_MAX || c->d.max_bins > 255)
        return fail(PB_ERR_UNSUPPORTED, "pb_set_segment_mode: too many rows or bins");
    const int64_t N = c->d.num_rows;
    const int32_t E = c->d.num_eras;
    const int32_t segw = c->umax + 1;
    const int64_t chunks = pb::seg_chunk_bound(N, E, segw);
    if (chunks >= INT32_MAX) return fail(PB_ERR_UNSUPPORTED, "pb_set_segment_mode: too many row chunks");
    int32_t from = from_depth;
    if (from < 0) {
        // the first depth whose planes would pass 1 GiB: below that, writing and reading the
        // planes costs less than the fused kernel's per-era histogram passes
        const int64_t cells = (int64_t)E * c->d.max_feats * std::max(1, c->d.max_bins - 1) * 6;
        from = c->d.max_depth;
        for (int dd = 0; dd < c->d.max_depth; ++dd)
            if ((int64_t)max_nodes_at(c, dd) * cells >= (int64_t(1) << 30)) {
                from = dd;
                break;
            }
    }
    int rc = PB_OK;
    if (!c->sb[0].row) {
        for (int i = 0; i < 2 && rc == PB_OK; ++i) {
            if ((rc = dev_alloc(&c->sb[i].g, (size_t)std::max<int64_t>(1, N), "alloc sorted rows")) ||
                (rc = dev_alloc(&c->sb[i].row, (size_t)std::max<int64_t>(1, N), "alloc sorted rows")) ||
                (rc = dev_alloc(&c->sb[i].tnode, (size_t)std::max<int64_t>(1, N), "alloc sorted rows")) ||
                (rc = dev_alloc(&c->seg[i], (size_t)E * segw, "alloc segments")))
                break;
        }
        if (rc == PB_OK) {
            if ((rc = dev_alloc(&c->ss.cp, (size_t)E * segw + 1, "alloc segment chunks")) ||
                (rc = dev_alloc(&c->ss.cnt_l, (size_t)chunks + 1, "alloc segment chunks")) ||
                (rc = dev_alloc(&c->ss.cnt_r, (size_t)chunks + 1, "alloc segment chunks")) ||
                (rc = dev_alloc(&c->ss.base, (size_t)E * segw * 2, "alloc segment chunks"))) {
            }
        }
        if (rc != PB_OK) {
            for (int i = 0; i < 2; ++i) {
                (void)hipFree(c->sb[i].g);
                (void)hipFree(c->sb[i].row);
                (void)hipFree(c->sb[i].tnode);
                (void)hipFree(c->seg[i]);
                c->sb[i] = pb::SegBuffers{};
                c->seg[i] = nullptr;
            }
            (void)hipFree(c->ss.cp);
            (void)hipFree(c->ss.cnt_l);
            (void)hipFree(c->ss.cnt_r);
            (void)hipFree(c->ss.base);
            c->ss = pb::SegState{};
            return rc;
        }
    }
    c->ss.N = N;
    c->ss.ld = c->d.ld;
    c->ss.E = E;
    c->ss.segw = segw;
    c->ss.era_off = c->era_off_dev;
    c->ss.st = c->st;
    c->ss.rules = c->rules;
    c->seg_from = std::min<int32_t>(from, c->d.max_depth);
    c->seg_ft = (int32_t)env_int("PB_SEG_FT", 0);
    // tile-major block order from this many frontier nodes on (PB_SEG_MAJOR)
    c->seg_major_nodes = (int32_t)std::max<long long>(1, env_int("PB_SEG_MAJOR", 32));
    if (c->seg_ft != 0 && c->seg_ft != 1 && c->seg_ft != 2 && c->seg_ft != 4)
        return fail(PB_ERR_INVALID, "pb_set_segment_mode: PB_SEG_FT must be 1, 2 or 4");
    c->seg_mode = true;
    return PB_OK;
}

int pb_grow_round(pb_ctx* c, const pb_fit_buffers* b, const int32_t* feats, int32_t K,
                  pb_decision* dec, pb_round_header* header, void* stream) {
    if (!c || !b || !feats || !dec || !header) return fail(PB_ERR_INVALID, "pb_grow_round: null argument");
    if (!b->bins_dev || !b->y_dev || !b->preds_dev || !b->grad_dev || !b->nid_dev || !b->tnode_dev ||
        !b->hist_cnt_dev || !b->hist_grad_dev || !b->values_dev)
        return fail(PB_ERR_INVALID, "pb_grow_round: null buffer");
    // the nibble copy, when bound, serves the histogram and partition reads
    const int32_t nib = b->bins4_dev ? 1 : 0;
    const uint8_t* bins = nib ? b->bins4_dev : b->bins_dev;
    const int64_t ld_bytes = nib ? c->d.ld / 2 : c->d.ld;
    if (nib && c->d.max_bins > 16)
        return fail(PB_ERR_INVALID, "pb_grow_round: the nibble bin layout needs max_bins <= 16");
    if (nib && (reinterpret_cast<uintptr_t>(b->bins4_dev) & 15))
        return fail(PB_ERR_INVALID, "pb_grow_round: bins4 must be 16-byte aligned");
    if (b->params.skip_last_bin)
        return fail(PB_ERR_UNSUPPORTED, "pb_grow_round: bins must lie below max_bins (skip_last_bin 0)");
    const bool seg = c->seg_mode;
    if (seg) {
        const int32_t full = std::max(1, c->d.max_bins - 1);
        if (b->params.k_cuts > 0 && b->params.k_cuts < full)
            return fail(PB_ERR_UNSUPPORTED, "pb_grow_round: segment mode scores every threshold (k_cuts 0)");
    }
    int rc = pb_round_begin(c, b->preds_dev, b->y_dev, b->grad_dev, b->nid_dev, b->tnode_dev, stream);
    if (rc) return rc;
    if (seg) {
        c->seg_cur = 0;
        pb::SegBuffers& cur = c->sb[0];
        PB_HIP(pb::launch_seg_begin(b->grad_dev, cur.row, cur.g, cur.tnode, c->d.num_rows, c->era_off_dev,
                                    c->d.num_eras, c->ss.segw, c->seg[0], (hipStream_t)stream),
               "segment round begin launch");
    }
    const int32_t fused_from = seg ? c->seg_from : c->d.max_depth;
    // the last partition can take the round end's work when its vector accesses are aligned
    const bool end_fusable = !(reinterpret_cast<uintptr_t>(b->preds_dev) & 15) &&
                             !(reinterpret_cast<uintptr_t>(b->nid_dev) & 15) &&
                             !(reinterpret_cast<uintptr_t>(b->tnode_dev) & 15) && b->pack_size >= 1 &&
                             c->d.num_rows <= c->rows_padded;
    for (int d = 0; d < c->d.max_depth; ++d) {
        const int32_t m = max_nodes_at(c, d);
        const int32_t* f = feats + (int64_t)d * K;
        std::array<hipEvent_t, 5> ev{};
        const bool prof = c->profile != 0;
        const int n_ev = c->profile == 2 ? 2 : 5;  // hist only: events 0 and 1
        if (prof) {
            for (int i = 0; i < n_ev; ++i) {
                hipEvent_t& e = ev[i];
                if (!c->ev_free.empty()) {
                    e = c->ev_free.back();
                    c->ev_free.pop_back();
                } else {
                    PB_HIP(hipEventCreate(&e), "profile event create");
                }
            }
            c->ev_pending.emplace_back(d, ev);
        }
        auto mark = [&](int i) -> int {
            if (prof && i < n_ev) PB_HIP(hipEventRecord(ev[i], (hipStream_t)stream), "profile event record");
            return PB_OK;
        };
        const bool fused = d >= fused_from;
        if ((rc = mark(0))) return rc;
        if (fused) {
            // one fused launch: its time is the histogram phase, the scorer phase is empty
            if ((rc = seg_score(c, b->bins_dev, f, K, d, m, &b->params, stream))) return rc;
            if ((rc = mark(1))) return rc;
        } else {
            if ((rc = hist_build(c, bins, ld_bytes, nib, b->grad_dev, b->nid_dev, f, K, d, m,
                                 b->hist_cnt_dev, b->hist_grad_dev, stream)))
                return rc;
            if ((rc = mark(1))) return rc;
            if ((rc = des_score(c, b->hist_cnt_dev, b->hist_grad_dev, f, K, d, m, &b->params, nullptr,
                                stream, false)))
                return rc;
        }
        if ((rc = mark(2))) return rc;
        if ((rc = pb_decide(c, d, m, &b->params, dec, b->values_dev, stream))) return rc;
        if ((rc = mark(3))) return rc;
        if (seg) {
            const bool last = d + 1 == c->d.max_depth;
            const int i = c->seg_cur;
            PB_HIP(pb::launch_seg_partition(c->ss, c->seg[i], c->seg[1 - i], c->sb[i], c->sb[1 - i], b->bins_dev,
                                            d, last, (hipStream_t)stream),
                   "segment partition launch");
            if (!last) c->seg_cur = 1 - i;
        }
        // the plane path's row ids: every depth without segments, else while a later depth's
        // histogram still reads them. Without segments the last depth's partition also does
        // the round end (each row's prediction from its final node, and the round header).
        if (!seg && d + 1 == c->d.max_depth && end_fusable) {
            PB_HIP(pb::launch_partition_end(bins, ld_bytes, nib, c->rows_padded, c->rules, c->st, d, b->nid_dev,
                                            b->tnode_dev, b->values_dev, b->pack_size, b->learning_rate,
                                            b->preds_dev, c->d.num_rows, header, (hipStream_t)stream),
                   "partition + round end launch");
        } else if ((!seg || d + 1 < fused_from) &&
                   (rc = partition(c, bins, ld_bytes, nib, d, b->nid_dev, b->tnode_dev, stream))) {
            return rc;
        }
        if ((rc = mark(4))) return rc;
    }
    if (!seg && end_fusable) return PB_OK;
    // the round-end kernel also writes the round's header (its first workgroup)
    if (seg) {
        const pb::SegBuffers& cur = c->sb[c->seg_cur];
        PB_HIP(pb::launch_seg_round_end(cur.tnode, cur.row, b->values_dev, b->pack_size, b->learning_rate,
                                        b->preds_dev, c->d.num_rows, c->st, header, (hipStream_t)stream),
               "segment round end launch");
        return PB_OK;
    }
    return round_end(c, b->tnode_dev, b->values_dev, b->pack_size, b->learning_rate, b->preds_dev, header,
                        stream);
}

int pb_select_subsets(const pb_round_header* prev_header, const int32_t* window, int32_t D,
                      int32_t K, int32_t* feats, void* stream) {
    if (!window || !feats) return fail(PB_ERR_INVALID, "pb_select_subsets: null argument");
    if (D < 1 || D > PB_MAX_DEPTH || K < 1) return fail(PB_ERR_INVALID, "pb_select_subsets: bad D or K");
    PB_HIP(pb::launch_select_subsets(prev_header, D, K, window, feats, (hipStream_t)stream),
           "select subsets launch");
    return PB_OK;
}

int pb_profile_enable(pb_ctx* c, int32_t enable) {
    if (!c) return fail(PB_ERR_INVALID, "pb_profile_enable: null context");
    if (enable < 0 || enable > 2) return fail(PB_ERR_INVALID, "pb_profile_enable: mode must be 0, 1 or 2");
    c->profile = enable;
    return PB_OK;
}

int pb_profile_read(pb_ctx* c, double* ms, int64_t* launches) {
    if (!c || !ms || !launches) return fail(PB_ERR_INVALID, "pb_profile_read: null argument");
    for (int i = 0; i < 4 * PB_MAX_DEPTH; ++i) {
        ms[i] = 0.0;
        launches[i] = 0;
    }
    int rc = PB_OK;
    for (auto& p : c->ev_pending) {
        const int d = p.first;
        auto& ev = p.second;
        const int n_ph = ev[4] ? 4 : 1;  // hist-only entries hold events 0 and 1
        if (rc == PB_OK) {
            hipError_t e = hipEventSynchronize(ev[n_ph]);
            if (e != hipSuccess) rc = hip_fail(e, "profile event sync");
        }
        for (int ph = 0; ph < n_ph && rc == PB_OK; ++ph) {
            float t = 0.f;
            hipError_t e = hipEventElapsedTime(&t, ev[ph], ev[ph + 1]);
            if (e != hipSuccess) {
                rc = hip_fail(e, "profile elapsed time");
                break;
            }
            ms[ph * PB_MAX_DEPTH + d] += t;
            launches[ph * PB_MAX_DEPTH + d] += 1;
        }
        for (hipEvent_t e : ev)
            if (e) c->ev_free.push_back(e);
    }
    c->ev_pending.clear();
    return rc;
}

int pb_frontier_set(pb_ctx* c, int32_t depth, int32_t num_active, const int32_t* node_ids_host,
                    int32_t tree_size, void* stream) {
    if (!c) return fail(PB_ERR_INVALID, "pb_frontier_set: null context");
    if (depth < 0 || depth >= c->d.max_depth) return fail(PB_ERR_RANGE, "pb_frontier_set: depth out of range");
    if (num_active < 0 || num_active > max_nodes_at(c, depth))
        return fail(PB_ERR_RANGE, "pb_frontier_set: num_active above the frontier bound of this depth");
    if (tree_size < 1 || tree_size > (1 << (c->d.max_depth + 1)))
        return fail(PB_ERR_RANGE, "pb_frontier_set: tree_size out of range");
    std::vector<int32_t> ids(std::max(num_active, 1));
    for (int i = 0; i < num_active; ++i) {
        ids[i] = node_ids_host ? node_ids_host[i] : i;
        if (ids[i] < 0 || ids[i] >= tree_size) return fail(PB_ERR_RANGE, "pb_frontier_set: node id out of range");
    }
    hipStream_t s = (hipStream_t)stream;
    PB_HIP(hipStreamSynchronize(s), "frontier_set sync");
    pb::Frontier f;
    PB_HIP(hipMemcpy(&f, c->st, sizeof(f), hipMemcpyDeviceToHost), "frontier_set read");
    f.u_active[depth] = num_active;
    for (int dd = depth + 1; dd <= PB_MAX_DEPTH; ++dd) f.u_active[dd] = 0;
    f.tree_size = tree_size;
    PB_HIP(hipMemcpy(c->st, &f, sizeof(f), hipMemcpyHostToDevice), "frontier_set write");
    if (num_active > 0)
        PB_HIP(hipMemcpy(c->ids[depth & 1], ids.data(), sizeof(int32_t) * num_active,
                         hipMemcpyHostToDevice),
               "frontier_set ids");
    return PB_OK;
}

int pb_frontier_counts(pb_ctx* c, int32_t* u_active_host, int32_t* tree_size_host, void* stream) {
    if (!c || !u_active_host || !tree_size_host)
        return fail(PB_ERR_INVALID, "pb_frontier_counts: null argument");
    pb::Frontier f;
    PB_HIP(hipMemcpyAsync(&f, c->st, sizeof(f), hipMemcpyDeviceToHost, (hipStream_t)stream),
           "frontier copy");
    PB_HIP(hipStreamSynchronize((hipStream_t)stream), "frontier sync");
    std::memcpy(u_active_host, f.u_active, sizeof(f.u_active));
    *tree_size_host = f.tree_size;
    return PB_OK;
}

int pb_predict_pack(const uint8_t* bins, int64_t N, int64_t ld, int32_t F, const int32_t* feature,
                    const int32_t* threshold, const int32_t* left_abs, const int32_t* right_abs,
                    const float* value, const uint8_t* is_leaf, const int32_t* offsets, int32_t B,
                    int32_t total_nodes, float tree_weight, float* out, int32_t* leaf,
                    void* stream) {
    if (N < 0 || ld < N || F < 1 || B < 0 || total_nodes < 0)
        return fail(PB_ERR_INVALID, "pb_predict_pack: bad shape");
    if (N == 0) return PB_OK;
    if (!bins || !feature || !threshold || !left_abs || !right_abs || !value || !is_leaf ||
        !offsets || !out)
        return fail(PB_ERR_INVALID, "pb_predict_pack: null argument");
    PB_HIP(pb::launch_predict_pack(bins, N, ld, F, feature, threshold, left_abs, right_abs, value,
                                   is_leaf, offsets, B, total_nodes, tree_weight, 0, out, leaf,
                                   (hipStream_t)stream),
           "predict_pack launch");
    return PB_OK;
}

int pb_quantile_edges(const float* sorted, int64_t n, int64_t ld, int32_t F, const double* q,
                      int32_t num_q, float* edges, int32_t edge_stride, void* stream) {
    if (!sorted || !q || !edges) return fail(PB_ERR_INVALID, "pb_quantile_edges: null argument");
    if (n < 0 || ld < n || F < 0 || num_q < 1 || num_q > 254 || edge_stride < F)
        return fail(PB_ERR_INVALID, "pb_quantile_edges: bad shape");
    if (F == 0) return PB_OK;
    PB_HIP(pb::launch_quantile_edges(sorted, n, ld, F, q, num_q, edges, edge_stride,
                                     (hipStream_t)stream),
           "quantile edges launch");
    return PB_OK;
}

int pb_apply_bins(const float* xt, int64_t n, int64_t ld_x, int32_t F, const float* edges,
                  int32_t num_edges, int32_t edge_stride, int32_t max_bins, const int64_t* perm,
                  uint8_t* bins, int64_t ld_out, void* stream) {
    if (!xt || !edges || !bins) return fail(PB_ERR_INVALID, "pb_apply_bins: null argument");
    if (n < 0 || ld_x < n || ld_out < n || F < 0 || num_edges < 1 || num_edges > 254 ||
        edge_stride < F || max_bins < 2 || max_bins > 255 || F > 65535)
        return fail(PB_ERR_INVALID, "pb_apply_bins: bad shape");
    if (n == 0 || F == 0) return PB_OK;
    PB_HIP(pb::launch_apply_bins(xt, n, ld_x, F, edges, num_edges, edge_stride, max_bins, perm, bins,
                                 ld_out, (hipStream_t)stream),
           "apply bins launch");
    return PB_OK;
}

int pb_pack_bins4(const uint8_t* bins, int64_t n, int64_t ld, int32_t F, uint8_t* out, void* stream) {
    if (!bins || !out) return fail(PB_ERR_INVALID, "pb_pack_bins4: null argument");
    if (ld < 0 || ld % 16 != 0 || F < 0) return fail(PB_ERR_INVALID, "pb_pack_bins4: ld must be a multiple of 16");
    if (n < 0 || n > ld) return fail(PB_ERR_INVALID, "pb_pack_bins4: n must lie in [0, ld]");
    if ((reinterpret_cast<uintptr_t>(bins) & 15) || (reinterpret_cast<uintptr_t>(out) & 7))
        return fail(PB_ERR_INVALID, "pb_pack_bins4: bins must be 16-byte and out 8-byte aligned");
    if (ld == 0 || F == 0) return PB_OK;
    PB_HIP(pb::launch_pack_bins4(bins, n, ld, F, out, (hipStream_t)stream), "pack bins launch");
    return PB_OK;
}

int pb_era_corr(const float* y, const float* preds, const int32_t* era_off, int32_t num_eras,
                double* era_corr, double* out, void* stream) {
    if (!y || !preds || !era_off || !era_corr || !out)
        return fail(PB_ERR_INVALID, "pb_era_corr: null argument");
    if (num_eras < 1) return fail(PB_ERR_INVALID, "pb_era_corr: num_eras must be >= 1");
    PB_HIP(pb::launch_era_corr(y, preds, era_off, num_eras, era_corr, out, (hipStream_t)stream),
           "era corr launch");
    return PB_OK;
}

int pb_predict_forest(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                      const int32_t* feature, const int32_t* threshold, const int32_t* left_abs,
                      const int32_t* right_abs, const float* value, const uint8_t* is_leaf,
                      const int32_t* offsets, int32_t T, int32_t total_nodes, float tree_weight,
                      float* out, void* stream) {
    if (N < 0 || ld < N || F < 1 || T < 0 || total_nodes < 0)
        return fail(PB_ERR_INVALID, "pb_predict_forest: bad shape");
    if (N == 0) return PB_OK;
    if (!bins || !feature || !threshold || !left_abs || !right_abs || !value || !is_leaf ||
        !offsets || !out)
        return fail(PB_ERR_INVALID, "pb_predict_forest: null argument");
    PB_HIP(pb::launch_predict_pack(bins, N, ld, F, feature, threshold, left_abs, right_abs, value,
                                   is_leaf, offsets, T, total_nodes, tree_weight, 1, out, nullptr,
                                   (hipStream_t)stream),
           "predict_forest launch");
    return PB_OK;
}

struct pb_forest {
    int4* rec = nullptr;       // one record per node
    int32_t* roots = nullptr;  // tree roots (node index)
    int32_t T = 0;
    int32_t total_nodes = 0;
    int32_t depth = 0;         // deepest leaf over all trees
    int32_t max_feature = -1;
    // every tree as a complete heap of `depth` levels (the tiled walk; null when the forest is
    // deeper than pb::kForestTileMaxDepth or its features do not fit a row tile)
    pb::ForestTile tile{};         // shape of the tiled walk's LDS tile
    uint32_t* heap_blocks = nullptr;  // tile.blocks x kForestBlockWords: per block of trees, the
                                      // packed records (pb::forest_tile_record), then leaf values
    int32_t* heap_id = nullptr;       // [T][2^depth] leaf node indices (absolute)
    int32_t* heap_first = nullptr;    // [heap_trees] first forest tree each heap tree stands for
    int32_t heap_trees = 0;           // distinct runs of consecutive identical trees
};

namespace {

void free_forest(pb_forest* fo) {
    if (!fo) return;
    (void)hipFree(fo->rec);
    (void)hipFree(fo->roots);
    (void)hipFree(fo->heap_blocks);
    (void)hipFree(fo->heap_id);
    (void)hipFree(fo->heap_first);
    delete fo;
}

// Heap form of one validated tree (root lo): a split at heap index h sends its children to
// 2h + 1 and 2h + 2; a leaf above the last level becomes always-left splits (threshold 255:
// every bin goes left) over its heap subtree, whose leaf slots all hold it.
void heap_tree(const pb::ForestTile& ft, int lo, int D, const std::vector<int32_t>& f, const std::vector<int32_t>& th,
               const std::vector<int32_t>& l, const std::vector<int32_t>& r, const std::vector<float>& v,
               const std::vector<uint8_t>& lf, uint32_t* rec, float* val, int32_t* id) {
    const int NI = (1 << D) - 1;
    std::vector<std::pair<int, int>> st{{lo, 0}};  // (node, heap index)
    while (!st.empty()) {
        const auto [n, h] = st.back();
        st.pop_back();
        if (!lf[n]) {
            rec[h] = pb::forest_tile_record(ft, f[n], th[n]);
            st.push_back({l[n], 2 * h + 1});
            st.push_back({r[n], 2 * h + 2});
            continue;
        }
        // the leaf's heap subtree: levels below h down to the leaf slots
        std::vector<int> lvl{h};
        while (!lvl.empty() && lvl[0] < NI) {
            std::vector<int> next;
            for (int x : lvl) {
                rec[x] = 255u << 24;  // offset 0 (feature 0 of the row), always left
                next.push_back(2 * x + 1);
                next.push_back(2 * x + 2);
            }
            lvl.swap(next);
        }
        for (int x : lvl) {
            val[x - NI] = v[n];
            id[x - NI] = n;
        }
    }
}

}  // namespace

int pb_forest_create(const int32_t* feature, const int32_t* threshold, const int32_t* left_abs,
                     const int32_t* right_abs, const float* value, const uint8_t* is_leaf,
                     const int32_t* offsets, int32_t T, int32_t total_nodes, pb_forest** out) {
    if (!out) return fail(PB_ERR_INVALID, "pb_forest_create: null output");
    *out = nullptr;
    if (T < 0 || total_nodes < 0) return fail(PB_ERR_INVALID, "pb_forest_create: bad shape");
    if (T > 0 && (!feature || !threshold || !left_abs || !right_abs || !value || !is_leaf || !offsets))
        return fail(PB_ERR_INVALID, "pb_forest_create: null argument");
    std::vector<int32_t> f(total_nodes), th(total_nodes), l(total_nodes), r(total_nodes), off(T + 1);
    std::vector<float> v(total_nodes);
    std::vector<uint8_t> lf(total_nodes);
    if (T > 0) {
        PB_HIP(hipMemcpy(off.data(), offsets, sizeof(int32_t) * (T + 1), hipMemcpyDeviceToHost), "forest copy");
        if (total_nodes > 0) {
            PB_HIP(hipMemcpy(f.data(), feature, 4 * (size_t)total_nodes, hipMemcpyDeviceToHost), "forest copy");
            PB_HIP(hipMemcpy(th.data(), threshold, 4 * (size_t)total_nodes, hipMemcpyDeviceToHost), "forest copy");
            PB_HIP(hipMemcpy(l.data(), left_abs, 4 * (size_t)total_nodes, hipMemcpyDeviceToHost), "forest copy");
            PB_HIP(hipMemcpy(r.data(), right_abs, 4 * (size_t)total_nodes, hipMemcpyDeviceToHost), "forest copy");
            PB_HIP(hipMemcpy(v.data(), value, 4 * (size_t)total_nodes, hipMemcpyDeviceToHost), "forest copy");
            PB_HIP(hipMemcpy(lf.data(), is_leaf, (size_t)total_nodes, hipMemcpyDeviceToHost), "forest copy");
        }
    }
    auto* fo = new pb_forest();
    fo->T = T;
    fo->total_nodes = total_nodes;
    std::vector<int4> rec(std::max(1, total_nodes));
    std::vector<int32_t> roots(std::max(1, T));
    std::vector<int32_t> depth(total_nodes, -1);
    for (int t = 0; t < T; ++t) {
        const int lo = off[t], hi = off[t + 1];
        if (lo < 0 || hi > total_nodes || hi <= lo) {
            free_forest(fo);
            return fail(PB_ERR_INVALID, "pb_forest_create: bad tree offsets");
        }
        roots[t] = lo;
        // breadth-first from the root: every reachable node once, children inside the tree
        std::vector<int32_t> q{lo};
        depth[lo] = 0;
        for (size_t k = 0; k < q.size(); ++k) {
            const int n = q[k];
            if (lf[n]) {
                rec[n] = make_int4((int)pb::kLeafFeatureBits, n, n, __builtin_bit_cast(int, v[n]));
                fo->depth = std::max(fo->depth, depth[n]);
                continue;
            }
            const int fe = f[n], tr = th[n], a = l[n], b = r[n];
            if (fe < 0 || fe >= (1 << 24) - 1 || tr < 0 || tr > 255 || a < lo || a >= hi || b < lo ||
                b >= hi || depth[a] >= 0 || depth[b] >= 0 || a == b) {
                free_forest(fo);
                return fail(PB_ERR_INVALID, "pb_forest_create: malformed tree (feature, threshold "
                                            "or child out of range, or a cycle)");
            }
            fo->max_feature = std::max(fo->max_feature, fe);
            rec[n] = make_int4((int)((uint32_t)fe | ((uint32_t)tr << 24)), a, b, 0);
            depth[a] = depth[b] = depth[n] + 1;
            q.push_back(a);
            q.push_back(b);
        }
    }
    if (hipMalloc(&fo->rec, sizeof(int4) * rec.size()) != hipSuccess ||
        hipMalloc(&fo->roots, sizeof(int32_t) * roots.size()) != hipSuccess) {
        free_forest(fo);
        return fail(PB_ERR_NOMEM, "pb_forest_create: device allocation failed");
    }
    hipError_t e1 = hipMemcpy(fo->rec, rec.data(), sizeof(int4) * rec.size(), hipMemcpyHostToDevice);
    hipError_t e2 = hipMemcpy(fo->roots, roots.data(), sizeof(int32_t) * roots.size(), hipMemcpyHostToDevice);
    if (e1 != hipSuccess || e2 != hipSuccess) {
        free_forest(fo);
        return hip_fail(e1 != hipSuccess ? e1 : e2, "forest upload");
    }
    // heap form for the tiled walk
    const int D = fo->depth;
    int32_t max_thr = 0;
    for (int t = 0; t < T; ++t)
        for (int n = off[t]; n < off[t + 1]; ++n)
            if (!lf[n] && depth[n] >= 0) max_thr = std::max(max_thr, th[n]);
    // Runs of consecutive identical trees (a fitted pack repeats one tree B times): the tiled
    // walk holds each run once, with its length, and counts its value that many times.
    auto same_tree = [&](int ta, int tb) {
        const int na = off[ta + 1] - off[ta];
        if (na != off[tb + 1] - off[tb]) return false;
        for (int k = 0; k < na; ++k) {
            const int x = off[ta] + k, y = off[tb] + k;
            if (lf[x] != lf[y] || __builtin_bit_cast(uint32_t, v[x]) != __builtin_bit_cast(uint32_t, v[y]))
                return false;
            if (!lf[x] && (f[x] != f[y] || th[x] != th[y] || l[x] - off[ta] != l[y] - off[tb] ||
                           r[x] - off[ta] != r[y] - off[tb]))
                return false;
        }
        return true;
    };
    std::vector<int32_t> first;  // first tree of each run
    std::vector<int32_t> count;  // its length
    for (int t = 0; t < T; ++t) {
        if (!first.empty() && same_tree(first.back(), t)) {
            ++count.back();
        } else {
            first.push_back(t);
            count.push_back(1);
        }
    }
    const int Td = (int)first.size();
    if (D <= pb::kForestTileMaxDepth) fo->tile = pb::forest_tile_shape(fo->max_feature + 1, max_thr, D, Td);
    if (T > 0 && D <= pb::kForestTileMaxDepth && pb::forest_tile_lds_bytes(fo->tile) <= pb::kForestTileMaxLds) {
        const size_t NL = (size_t)1 << D, TB = (size_t)fo->tile.tree_block;
        const size_t BW = pb::kForestBlockWords;
        // run k of block b at dwords b*BW + k*2NL: its length at dword 0 (a float), node i (from
        // 1) at dword i, leaves from NL; padding trees: length 0, always-left records and zero
        // leaf values
        std::vector<uint32_t> blk((size_t)fo->tile.blocks * BW, 0u);
        for (size_t x = 0; x < blk.size(); x += 2 * NL)
            std::fill(blk.begin() + x + 1, blk.begin() + x + NL, 255u << 24);
        std::vector<float> val(NL);
        std::vector<uint32_t> scratch(NL);
        std::vector<int32_t> hi((size_t)T * NL, -1);
        for (int k = 0; k < Td; ++k) {
            uint32_t* tree = blk.data() + (size_t)(k / TB) * BW + (size_t)(k % TB) * 2 * NL;
            tree[0] = __builtin_bit_cast(uint32_t, (float)count[k]);
            for (int c = 0; c < count[k]; ++c) {  // leaf node ids of every tree of the run
                const int t = first[k] + c;
                uint32_t* dst = c == 0 ? tree + 1 : scratch.data();
                heap_tree(fo->tile, off[t], D, f, th, l, r, v, lf, dst, val.data(), hi.data() + (size_t)t * NL);
                if (c == 0) std::memcpy(tree + NL, val.data(), sizeof(float) * NL);
            }
        }
        if (hipMalloc(&fo->heap_blocks, sizeof(uint32_t) * blk.size()) != hipSuccess ||
            hipMalloc(&fo->heap_id, sizeof(int32_t) * hi.size()) != hipSuccess ||
            hipMalloc(&fo->heap_first, sizeof(int32_t) * first.size()) != hipSuccess) {
            free_forest(fo);
            return fail(PB_ERR_NOMEM, "pb_forest_create: device allocation failed");
        }
        fo->heap_trees = Td;
        fo->tile.runs = Td < T ? 1 : 0;
        hipError_t e3 = hipMemcpy(fo->heap_blocks, blk.data(), sizeof(uint32_t) * blk.size(), hipMemcpyHostToDevice);
        if (e3 == hipSuccess) e3 = hipMemcpy(fo->heap_id, hi.data(), sizeof(int32_t) * hi.size(), hipMemcpyHostToDevice);
        if (e3 == hipSuccess)
            e3 = hipMemcpy(fo->heap_first, first.data(), sizeof(int32_t) * first.size(), hipMemcpyHostToDevice);
        if (e3 != hipSuccess) {
            free_forest(fo);
            return hip_fail(e3, "forest upload");
        }
    }
    *out = fo;
    return PB_OK;
}

int pb_forest_predict(const pb_forest* fo, const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                      float tree_weight, float* out, int32_t* leaf, void* stream) {
    if (!fo) return fail(PB_ERR_INVALID, "pb_forest_predict: null forest");
    if (N < 0 || ld < N || F < 1) return fail(PB_ERR_INVALID, "pb_forest_predict: bad shape");
    if (fo->max_feature >= F)
        return fail(PB_ERR_RANGE, "pb_forest_predict: the forest splits on a feature >= F");
    if (N == 0) return PB_OK;
    if (!bins || !out) return fail(PB_ERR_INVALID, "pb_forest_predict: null argument");
    if (fo->T == 0) {
        PB_HIP(hipMemsetAsync(out, 0, sizeof(float) * (size_t)N, (hipStream_t)stream), "zero predictions");
        return PB_OK;
    }
    // the tiled walk reads a tile's rows four at a time: row stride and columns 4-byte aligned
    if (fo->heap_blocks && ld % 4 == 0 && reinterpret_cast<uintptr_t>(bins) % 4 == 0 &&
        env_int("PB_FOREST_TILE", 1) != 0) {
        PB_HIP(pb::launch_forest_tile(bins, N, ld, fo->tile, fo->heap_blocks, fo->heap_id, fo->heap_first,
                                      fo->heap_trees, fo->depth, tree_weight, out, leaf, (hipStream_t)stream),
               "forest tile launch");
        return PB_OK;
    }
    static const int32_t group = (int32_t)env_int("PB_FOREST_GROUP", 8);
    static const int32_t max_grid = (int32_t)env_int("PB_FOREST_GRID", 0);
    PB_HIP(pb::launch_forest(bins, N, ld, fo->rec, fo->roots, fo->T, fo->depth, tree_weight, out, leaf,
                             group, max_grid, (hipStream_t)stream),
           "forest launch");
    return PB_OK;
}

int pb_forest_destroy(pb_forest* fo) {
    free_forest(fo);
    return PB_OK;
}

int pb_predict_bins(const uint8_t* bins, int64_t N, int64_t ld, int32_t F, const int32_t* feature,
                    const int32_t* threshold, const int32_t* left, const int32_t* right,
                    const float* value, const uint8_t* is_leaf, int32_t num_nodes, float* out,
                    void* stream) {
    if (N < 0 || ld < N || F < 1 || num_nodes < 0)
        return fail(PB_ERR_INVALID, "pb_predict_bins: bad shape");
    if (N == 0) return PB_OK;
    if (!bins || !feature || !threshold || !left || !right || !value || !is_leaf || !out)
        return fail(PB_ERR_INVALID, "pb_predict_bins: null argument");
    PB_HIP(pb::launch_predict_bins(bins, N, ld, F, feature, threshold, left, right, value, is_leaf,
                                   num_nodes, out, (hipStream_t)stream),
           "predict_bins launch");
    return PB_OK;
}

/* ---- row lists ---------------------------------------------------------------------- */

int64_t pb_rowlist_work_elems(int32_t num_nodes, int32_t num_eras) {
    if (num_nodes < 0 || num_eras < 0) return -1;
    return pb::rowlist_work_elems((int64_t)num_nodes * num_eras);
}

int pb_rowlist_partition(const uint8_t* bins, int64_t N, int64_t ld, int32_t F, const int32_t* rows,
                         int64_t R, const int32_t* node_row_splits, const int32_t* node_era_splits,
                         int32_t S, int32_t E, const int32_t* feat, const int32_t* thr,
                         int32_t* left_index, int32_t* right_index, int64_t capacity,
                         int32_t* left_splits, int32_t* right_splits, int32_t* work, void* stream) {
    if (S < 0 || E < 0 || N < 0 || R < 0 || F < 0 || capacity < 0)
        return fail(PB_ERR_INVALID, "pb_rowlist_partition: negative size");
    if (N > ld) return fail(PB_ERR_INVALID, "pb_rowlist_partition: N must be <= ld");
    if (R > INT32_MAX || capacity > INT32_MAX)
        return fail(PB_ERR_RANGE, "pb_rowlist_partition: row lists above 2^31 - 1 entries");
    if (S == 0) return PB_OK;
    if (!bins || (!rows && R > 0) || !node_row_splits || !node_era_splits || !feat || !thr ||
        (!left_index && capacity > 0) || (!right_index && capacity > 0) || !left_splits ||
        !right_splits || !work)
        return fail(PB_ERR_INVALID, "pb_rowlist_partition: null argument");
    PB_HIP(pb::launch_rowlist_partition(bins, N, ld, F, rows, R, node_row_splits, node_era_splits, S, E,
                                        feat, thr, left_index, right_index, capacity, left_splits,
                                        right_splits, work, (hipStream_t)stream),
           "rowlist partition launch");
    return PB_OK;
}

int64_t pb_rowlist_noalloc_max_segments(void) { return pb::rowlist_noalloc_max_segments(); }

int pb_rowlist_partition_noalloc(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                                 const int32_t* rows, int64_t R, const int32_t* node_row_splits,
                                 const int32_t* node_era_splits, int32_t S, int32_t E,
                                 const int32_t* feat, const int32_t* thr, int32_t* left_index,
                                 int32_t* right_index, int64_t capacity, int32_t* left_splits,
                                 int32_t* right_splits, int32_t* status, void* stream) {
    if (S < 0 || E < 0 || N < 0 || R < 0 || F < 0 || capacity < 0)
        return fail(PB_ERR_INVALID, "pb_rowlist_partition_noalloc: negative size");
    if (N > ld) return fail(PB_ERR_INVALID, "pb_rowlist_partition_noalloc: N must be <= ld");
    if (R > INT32_MAX || capacity > INT32_MAX)
        return fail(PB_ERR_RANGE, "pb_rowlist_partition_noalloc: row lists above 2^31 - 1 entries");
    const int64_t segments = (int64_t)S * E;
    const int64_t max_segments = pb::rowlist_noalloc_max_segments();
    if (segments > max_segments)
        return fail(PB_ERR_UNSUPPORTED,
                    "pb_rowlist_partition_noalloc: " + std::to_string(segments) +
                        " (node, era) segments exceed the static workspace (at most " +
                        std::to_string(max_segments) + "); use pb_rowlist_partition with a workspace");
    if (S == 0) return PB_OK;
    if (!bins || (!rows && R > 0) || !node_row_splits || !node_era_splits || !feat || !thr ||
        (!left_index && capacity > 0) || (!right_index && capacity > 0) || !left_splits ||
        !right_splits || !status)
        return fail(PB_ERR_INVALID, "pb_rowlist_partition_noalloc: null argument");
    PB_HIP(pb::launch_rowlist_partition_noalloc(bins, N, ld, F, rows, R, node_row_splits, node_era_splits,
                                                S, E, feat, thr, left_index, right_index, capacity,
                                                left_splits, right_splits, status, (hipStream_t)stream),
           "rowlist partition (no-alloc) launch");
    return PB_OK;
}

int pb_rowlist_gather(const uint8_t* bins, int64_t N, int64_t ld, int32_t F, const int32_t* feats,
                      int32_t K, const float* values, const int32_t* rows, int64_t R,
                      const int32_t* node_row_splits, const int32_t* node_era_splits,
                      int32_t node_begin, int32_t node_end, int32_t E, uint8_t* out_bins,
                      int64_t out_ld, float* out_values, uint16_t* out_slot, int32_t* era_off,
                      int32_t* work, void* stream) {
    if (N < 0 || R < 0 || F < 0 || K < 0 || E < 1 || out_ld < 0)
        return fail(PB_ERR_INVALID, "pb_rowlist_gather: negative size or no eras");
    if (N > ld) return fail(PB_ERR_INVALID, "pb_rowlist_gather: N must be <= ld");
    if (node_begin < 0 || node_end <= node_begin || node_end - node_begin >= PB_INACTIVE)
        return fail(PB_ERR_INVALID, "pb_rowlist_gather: node range must hold 1 .. 65534 nodes");
    if (R > INT32_MAX || out_ld > INT32_MAX)
        return fail(PB_ERR_RANGE, "pb_rowlist_gather: row lists above 2^31 - 1 entries");
    if (!bins || (!feats && K > 0) || (!values && R > 0) || (!rows && R > 0) || !node_row_splits ||
        !node_era_splits || (!out_bins && K > 0 && out_ld > 0) || (!out_values && out_ld > 0) ||
        (!out_slot && out_ld > 0) || !era_off || !work)
        return fail(PB_ERR_INVALID, "pb_rowlist_gather: null argument");
    PB_HIP(pb::launch_rowlist_gather(bins, N, ld, F, feats, K, values, rows, R, node_row_splits,
                                     node_era_splits, node_begin, node_end, E, out_bins, out_ld,
                                     out_values, out_slot, era_off, work, (hipStream_t)stream),
           "rowlist gather launch");
    return PB_OK;
}

int pb_best_thresholds(const pb_candidate* cand, int32_t M, int32_t K, int32_t T, float* scores,
                       int32_t* thresholds, float* left_grad, float* left_hess, int64_t* left_count,
                       void* stream) {
    if (M < 0 || K < 0 || T < 0) return fail(PB_ERR_INVALID, "pb_best_thresholds: negative size");
    if ((int64_t)M * K == 0) return PB_OK;
    if (!cand || !scores || !thresholds || !left_grad || !left_hess || !left_count)
        return fail(PB_ERR_INVALID, "pb_best_thresholds: null argument");
    PB_HIP(pb::launch_best_thresholds(cand, M, K, T, scores, thresholds, left_grad, left_hess, left_count,
                                      (hipStream_t)stream),
           "best thresholds launch");
    return PB_OK;
}

int pb_pick_sequential(const pb_candidate* cand, int32_t M, int32_t K, int32_t T, int32_t* band, pb_candidate* out,
                       void* stream) {
    if (M < 0 || K < 0 || T < 0) return fail(PB_ERR_INVALID, "pb_pick_sequential: negative size");
    if (M == 0) return PB_OK;
    if (!out || ((int64_t)K * T > 0 && (!cand || !band)))
        return fail(PB_ERR_INVALID, "pb_pick_sequential: null argument");
    PB_HIP(pb::launch_pick_sequential(cand, M, (int64_t)K * T, band, out, (hipStream_t)stream),
           "sequential pick launch");
    return PB_OK;
}

}  // extern "C"
