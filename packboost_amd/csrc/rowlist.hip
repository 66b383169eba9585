// Row-list entry points: the reference's CUDA backend hands its split finder and partition
// per-node, per-era row lists (rows_index with node_row_splits / node_era_splits,
// frontier_cuda.cu:576-716, 719-851). This file serves that interface on the device:
//
//  * partition (frontier_cuda.cu:719-851, frontier_cpu.cpp:446-497): every (node, era)
//    segment of the lists splits stably into its left rows (bin <= threshold) and right rows.
//    Left counts per segment (one wavefront per segment), an exclusive scan over the segments
//    in node-major order, then a stable scatter per segment (a ballot gives each row its rank
//    among the rows of its side that precede it).
//  * gather: the listed rows of a range of nodes, reordered era-major (era, then node, then
//    list order: the layout the histogram kernel reads), with their K sampled bins, values and
//    node slots, placed by a scan over the segment sizes in era-major order.
//  * best thresholds: per (node, feature) the CUDA split finder's sequential choice over
//    thresholds (frontier_cuda.cu:537-560) from the scorer's candidate records.
//
// Every read and write is bounds-checked: a segment outside the row list, a row id outside
// [0, N), a feature outside [0, F) or an output past its capacity sets a status word (the
// first entries of the workspace) instead of touching memory out of range.
#include <algorithm>

#include <mutex>

#include "pb_internal.h"

// Workspace of pb_rowlist_partition_noalloc: a fixed device array instead of caller or
// library allocations (for callers that cannot allocate device memory, e.g. under HIP graph
// capture). Every device the library runs on holds one copy until the process ends. Host code
// never passes `scratch` itself to a kernel (on the host it names a shadow variable, not
// device memory): pb::noalloc_scratch looks up each device's address once, with that device
// current, and launches take that address.
static __device__ __align__(256) int32_t scratch[pb::kNoAllocScratchInts];

namespace pb {

// Device address of `scratch` on the current device, looked up on the first call per device
// (hipGetSymbolAddress with that device current) and kept.
hipError_t noalloc_scratch(int32_t** out) {
    static std::mutex mu;
    static int32_t* addr[kNoAllocMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kNoAllocMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        addr[dev] = static_cast<int32_t*>(p);
    }
    *out = addr[dev];
    return hipSuccess;
}

namespace {

constexpr int kRlBlock = 256;
constexpr int kRlWaves = kRlBlock / kWave;
constexpr int kScanItems = 8;
constexpr int kScanTile = kRlBlock * kScanItems;  // pairs per scan tile

// Status words (the first kRlStatus entries of the workspace).
constexpr int kRlStatus = 4;
enum : int { kBadSegment = 0, kBadRow = 1, kBadFeature = 2, kOverflow = 3 };

__device__ __forceinline__ void raise_status(int32_t* status, int which) { status[which] = 1; }

// Segment (s, e) of the row lists: positions [lo, hi) of rows_index. An inconsistent segment
// (outside [0, R) or reversed) counts as empty and reports false.
__device__ __forceinline__ bool seg_range(const int32_t* nrs, const int32_t* nes, int32_t E, int64_t R,
                                          int32_t s, int32_t e, int64_t& lo, int64_t& hi) {
    const int64_t base = nrs[s];
    lo = base + nes[(int64_t)s * (E + 1) + e];
    hi = base + nes[(int64_t)s * (E + 1) + e + 1];
    if (lo < 0 || hi < lo || hi > R) {
        lo = hi = 0;
        return false;
    }
    return true;
}

__device__ __forceinline__ uint64_t lanes_below(int lane) {
    return lane == 0 ? 0ull : (~0ull >> (kWave - lane));
}

__global__ void rl_clear_kernel(int32_t* status) {
    if (threadIdx.x < kRlStatus) status[threadIdx.x] = 0;
}

// vals[2 seg] = left rows of segment seg = s * E + e, vals[2 seg + 1] = right rows.
__global__ __launch_bounds__(kRlBlock) void rl_count_kernel(
    const uint8_t* __restrict__ bins, int64_t N, int64_t ld, int32_t F, const int32_t* __restrict__ rows,
    int64_t R, const int32_t* nrs, const int32_t* nes, int32_t S, int32_t E, const int32_t* feat,
    const int32_t* thr, int32_t* vals, int32_t* status) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t n = (int64_t)S * E;
    for (int64_t seg = (int64_t)blockIdx.x * kRlWaves + threadIdx.x / kWave; seg < n;
         seg += (int64_t)gridDim.x * kRlWaves) {
        const int32_t s = (int32_t)(seg / E), e = (int32_t)(seg - (int64_t)s * E);
        int64_t lo, hi;
        if (!seg_range(nrs, nes, E, R, s, e, lo, hi) && lane == 0) raise_status(status, kBadSegment);
        const int32_t f = feat[s], t = thr[s];
        const bool fok = f >= 0 && f < F;
        if (!fok && lane == 0 && hi > lo) raise_status(status, kBadFeature);
        const uint8_t* col = bins + (fok ? (int64_t)f * ld : 0);
        int left = 0;
        bool bad = false;
        for (int64_t i = lo + lane; i < hi; i += kWave) {
            const int32_t r = rows[i];
            if (r < 0 || r >= N) {
                bad = true;
                continue;
            }
            left += fok && (int32_t)col[r] <= t;
        }
        if (bad) raise_status(status, kBadRow);
        for (int m = kWave / 2; m > 0; m >>= 1) left += __shfl_xor(left, m);
        if (lane == 0) {
            vals[2 * seg] = left;
            vals[2 * seg + 1] = (int32_t)(hi - lo) - left;
        }
    }
}

// Block-wide inclusive scan of pairs (kRlBlock threads). Returns this thread's inclusive value
// and the block total.
__device__ __forceinline__ int2 block_scan_pairs(int2 v, int2& total, int2* s_w) {
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    for (int m = 1; m < kWave; m <<= 1) {
        const int32_t y0 = __shfl_up(v.x, m), y1 = __shfl_up(v.y, m);
        if (lane >= m) {
            v.x += y0;
            v.y += y1;
        }
    }
    __syncthreads();
    if (lane == kWave - 1) s_w[wave] = v;
    __syncthreads();
    int2 before = make_int2(0, 0);
    total = make_int2(0, 0);
    for (int w = 0; w < kRlWaves; ++w) {
        if (w < wave) {
            before.x += s_w[w].x;
            before.y += s_w[w].y;
        }
        total.x += s_w[w].x;
        total.y += s_w[w].y;
    }
    return make_int2(v.x + before.x, v.y + before.y);
}

// Tile sums of the n pairs: tiles[2 t + c] = sum of vals[2 j + c] over tile t's pairs.
__global__ __launch_bounds__(kRlBlock) void rl_tile_sums_kernel(const int32_t* vals, int64_t n,
                                                             int32_t* tiles) {
    __shared__ int2 s_w[kRlWaves];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int2 acc = make_int2(0, 0);
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t j = base + k;
        if (j < n) {
            acc.x += vals[2 * j];
            acc.y += vals[2 * j + 1];
        }
    }
    int2 total;
    block_scan_pairs(acc, total, s_w);
    if (threadIdx.x == 0) {
        tiles[2 * blockIdx.x] = total.x;
        tiles[2 * blockIdx.x + 1] = total.y;
    }
}

// Exclusive scan of the nt tile sums in place, in one workgroup; tiles[2 nt + c] = the totals.
__global__ __launch_bounds__(kRlBlock) void rl_scan_tiles_kernel(int32_t* tiles, int64_t nt) {
    __shared__ int2 s_w[kRlWaves];
    int2 carry = make_int2(0, 0);
    for (int64_t b = 0; b < nt; b += kRlBlock) {
        const int64_t j = b + threadIdx.x;
        const int2 v = j < nt ? make_int2(tiles[2 * j], tiles[2 * j + 1]) : make_int2(0, 0);
        int2 total;
        const int2 inc = block_scan_pairs(v, total, s_w);
        if (j < nt) {
            tiles[2 * j] = carry.x + inc.x - v.x;
            tiles[2 * j + 1] = carry.y + inc.y - v.y;
        }
        carry.x += total.x;
        carry.y += total.y;
    }
    if (threadIdx.x == 0) {
        tiles[2 * nt] = carry.x;
        tiles[2 * nt + 1] = carry.y;
    }
}

// Exclusive scan of the pairs: scan[2 j + c] = sum_{i < j} vals[2 i + c]; scan[2 n + c] = the
// totals (copied from the scanned tiles by block 0).
__global__ __launch_bounds__(kRlBlock) void rl_tile_scan_kernel(const int32_t* vals, int64_t n,
                                                             const int32_t* tiles, int64_t nt,
                                                             int32_t* scan) {
    __shared__ int2 s_w[kRlWaves];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int2 v[kScanItems];
    int2 acc = make_int2(0, 0);
    for (int k = 0; k < kScanItems; ++k) {
        const int64_t j = base + k;
        v[k] = j < n ? make_int2(vals[2 * j], vals[2 * j + 1]) : make_int2(0, 0);
        acc.x += v[k].x;
        acc.y += v[k].y;
    }
    int2 total;
    const int2 inc = block_scan_pairs(acc, total, s_w);
    if (blockIdx.x < nt) {
        int2 run = make_int2(tiles[2 * blockIdx.x] + inc.x - acc.x, tiles[2 * blockIdx.x + 1] + inc.y - acc.y);
        for (int k = 0; k < kScanItems; ++k) {
            const int64_t j = base + k;
            if (j < n) {
                scan[2 * j] = run.x;
                scan[2 * j + 1] = run.y;
            }
            run.x += v[k].x;
            run.y += v[k].y;
        }
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        scan[2 * n] = tiles[2 * nt];
        scan[2 * n + 1] = tiles[2 * nt + 1];
    }
}

// [S][E+1] split offsets from the scan (node s's entries are scan pairs s*E .. s*E + E).
__global__ void rl_splits_kernel(const int32_t* scan, int32_t S, int32_t E, int32_t* left_splits,
                                 int32_t* right_splits) {
    const int64_t n = (int64_t)S * (E + 1);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t s = i / (E + 1), e = i - s * (E + 1);
        const int64_t j = s * E + e;
        left_splits[i] = scan[2 * j];
        right_splits[i] = scan[2 * j + 1];
    }
}

// Stable scatter of every segment's rows to its side, in list order (one wavefront per
// segment; the same left test as rl_count_kernel).
__global__ __launch_bounds__(kRlBlock) void rl_scatter_kernel(
    const uint8_t* __restrict__ bins, int64_t N, int64_t ld, int32_t F, const int32_t* __restrict__ rows,
    int64_t R, const int32_t* nrs, const int32_t* nes, int32_t S, int32_t E, const int32_t* feat,
    const int32_t* thr, const int32_t* scan, int32_t* left_out, int32_t* right_out, int64_t cap,
    int32_t* status) {
    const int lane = threadIdx.x & (kWave - 1);
    const uint64_t below = lanes_below(lane);
    const int64_t n = (int64_t)S * E;
    for (int64_t seg = (int64_t)blockIdx.x * kRlWaves + threadIdx.x / kWave; seg < n;
         seg += (int64_t)gridDim.x * kRlWaves) {
        const int32_t s = (int32_t)(seg / E), e = (int32_t)(seg - (int64_t)s * E);
        int64_t lo, hi;
        seg_range(nrs, nes, E, R, s, e, lo, hi);
        const int32_t f = feat[s], t = thr[s];
        const bool fok = f >= 0 && f < F;
        const uint8_t* col = bins + (fok ? (int64_t)f * ld : 0);
        int64_t lpos = scan[2 * seg], rpos = scan[2 * seg + 1];
        bool over = false;
        for (int64_t c = lo; c < hi; c += kWave) {
            const int64_t i = c + lane;
            const bool in = i < hi;
            const int32_t r = in ? rows[i] : -1;
            const bool left = in && fok && r >= 0 && r < N && (int32_t)col[r] <= t;
            const uint64_t bl = __ballot(left);
            const int lrank = __popcll(bl & below);
            const int n_in = (int)min<int64_t>(kWave, hi - c);
            if (in) {
                const int64_t p = left ? lpos + lrank : rpos + (lane - lrank);
                if (p >= 0 && p < cap)
                    (left ? left_out : right_out)[p] = r;
                else
                    over = true;
            }
            const int nl = __popcll(bl);
            lpos += nl;
            rpos += n_in - nl;
        }
        if (over) raise_status(status, kOverflow);
    }
}

// Era-major sizes of the segments of nodes [m0, m1): vals[2 j] = size of segment (m0 + sl, e)
// with j = e * (m1 - m0) + sl; vals[2 j + 1] = 0.
__global__ void rl_sizes_kernel(const int32_t* nrs, const int32_t* nes, int64_t R, int32_t m0, int32_t m1,
                                int32_t E, int32_t* vals, int32_t* status) {
    const int32_t Mc = m1 - m0;
    const int64_t n = (int64_t)Mc * E;
    for (int64_t j = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; j < n; j += (int64_t)gridDim.x * blockDim.x) {
        const int32_t e = (int32_t)(j / Mc), sl = (int32_t)(j - (int64_t)e * Mc);
        int64_t lo, hi;
        if (!seg_range(nrs, nes, E, R, m0 + sl, e, lo, hi)) raise_status(status, kBadSegment);
        vals[2 * j] = (int32_t)(hi - lo);
        vals[2 * j + 1] = 0;
    }
}

// One wavefront per segment: its rows to their era-major positions with K bins each.
__global__ __launch_bounds__(kRlBlock) void rl_gather_kernel(
    const uint8_t* __restrict__ bins, int64_t N, int64_t ld, int32_t F, const int32_t* feats, int32_t K,
    const float* __restrict__ values, const int32_t* __restrict__ rows, int64_t R, const int32_t* nrs,
    const int32_t* nes, int32_t m0, int32_t m1, int32_t E, const int32_t* scan, uint8_t* out_bins,
    int64_t out_ld, float* out_values, uint16_t* out_slot, int32_t* status) {
    const int lane = threadIdx.x & (kWave - 1);
    const int32_t Mc = m1 - m0;
    const int64_t n = (int64_t)Mc * E;
    bool bad_row = false, bad_feat = false, over = false;
    for (int64_t j = (int64_t)blockIdx.x * kRlWaves + threadIdx.x / kWave; j < n;
         j += (int64_t)gridDim.x * kRlWaves) {
        const int32_t e = (int32_t)(j / Mc), sl = (int32_t)(j - (int64_t)e * Mc);
        int64_t lo, hi;
        seg_range(nrs, nes, E, R, m0 + sl, e, lo, hi);
        const int64_t dst = scan[2 * j];
        for (int64_t i = lo + lane; i < hi; i += kWave) {
            const int64_t d = dst + (i - lo);
            if (d < 0 || d >= out_ld) {
                over = true;
                continue;
            }
            const int32_t r = rows[i];
            const bool rok = r >= 0 && r < N;
            bad_row |= !rok;
            out_values[d] = values[i];
            out_slot[d] = (uint16_t)sl;
            for (int k = 0; k < K; ++k) {
                const int32_t f = feats[k];
                const bool fok = f >= 0 && f < F;
                bad_feat |= !fok;
                out_bins[(int64_t)k * out_ld + d] = (rok && fok) ? bins[(int64_t)f * ld + r] : (uint8_t)0;
            }
        }
    }
    if (bad_row) raise_status(status, kBadRow);
    if (bad_feat) raise_status(status, kBadFeature);
    if (over) raise_status(status, kOverflow);
}

// era_off[e] = first era-major position of era e; era_off[E] = the row total.
__global__ void rl_era_off_kernel(const int32_t* scan, int32_t Mc, int32_t E, int32_t* era_off) {
    const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (e <= E) era_off[e] = scan[2 * e * Mc];
}

// Per (node, feature): frontier_cuda.cu:537-560's pick over the thresholds in their order
// (score within 1e-12 of the best: the larger left count, then the larger threshold wins; a
// non-finite best leaves threshold -1 and zero sums).
__global__ void rl_best_kernel(const pb_candidate* cand, int64_t MK, int32_t T, float* score, int32_t* thr,
                               float* left_grad, float* left_hess, int64_t* left_count) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= MK) return;
    float bs = -__builtin_inff(), blg = 0.0f;
    int32_t bt = -1;
    int64_t bl = 0;
    for (int t = 0; t < T; ++t) {
        const pb_candidate c = cand[i * T + t];
        if (!c.valid) continue;
        const float sc = c.score;
        const int64_t lc = c.left_total;
        bool better = sc > bs;
        if (!better && fabsf(sc - bs) <= 1e-12f) better = lc > bl || (lc == bl && c.threshold > bt);
        if (better) {
            bs = sc;
            bt = c.threshold;
            blg = c.left_grad;
            bl = lc;
        }
    }
    if (!(bs == bs) || isinf(bs)) {
        bt = -1;
        blg = 0.0f;
        bl = 0;
    }
    score[i] = bs;
    thr[i] = bt;
    left_grad[i] = blg;
    left_hess[i] = (float)bl;  // squared loss: hess == 1 per row
    left_count[i] = bl;
}

int grid_of(int64_t work, int64_t per_block, int64_t cap) {
    return (int)std::max<int64_t>(1, std::min<int64_t>((work + per_block - 1) / per_block, cap));
}

int64_t tiles_of(int64_t n) { return (n + kScanTile - 1) / kScanTile; }

// Exclusive scan of n pairs into scan[2n + 2]; tiles: [2 nt + 2] scratch.
void scan_pairs(const int32_t* vals, int64_t n, int32_t* tiles, int32_t* scan, hipStream_t s) {
    const int64_t nt = tiles_of(n);
    if (nt > 0)
        hipLaunchKernelGGL(rl_tile_sums_kernel, dim3((unsigned)nt), dim3(kRlBlock), 0, s, vals, n, tiles);
    hipLaunchKernelGGL(rl_scan_tiles_kernel, dim3(1), dim3(kRlBlock), 0, s, tiles, nt);
    hipLaunchKernelGGL(rl_tile_scan_kernel, dim3((unsigned)std::max<int64_t>(1, nt)), dim3(kRlBlock), 0, s,
                       vals, n, tiles, nt, scan);
}

}  // namespace

int64_t rowlist_work_elems(int64_t segments) {
    return kRlStatus + 2 * segments + (2 * segments + 2) + (2 * tiles_of(segments) + 2);
}

namespace {

void rowlist_partition_stages(const uint8_t* bins, int64_t N, int64_t ld, int32_t F, const int32_t* rows,
                              int64_t R, const int32_t* nrs, const int32_t* nes, int32_t S, int32_t E,
                              const int32_t* feat, const int32_t* thr, int32_t* left_out,
                              int32_t* right_out, int64_t cap, int32_t* left_splits,
                              int32_t* right_splits, int32_t* status, int32_t* rest, hipStream_t s) {
    const int64_t n = (int64_t)S * E;
    int32_t* vals = rest;               // [2n]
    int32_t* scan = vals + 2 * n;       // [2n + 2]
    int32_t* tiles = scan + 2 * n + 2;  // [2 nt + 2]
    const int g = grid_of(n, kRlWaves, 1 << 16);
    hipLaunchKernelGGL(rl_clear_kernel, dim3(1), dim3(kWave), 0, s, status);
    hipLaunchKernelGGL(rl_count_kernel, dim3(g), dim3(kRlBlock), 0, s, bins, N, ld, F, rows, R, nrs, nes,
                       S, E, feat, thr, vals, status);
    scan_pairs(vals, n, tiles, scan, s);
    hipLaunchKernelGGL(rl_splits_kernel, dim3(grid_of((int64_t)S * (E + 1), 256, 1 << 14)), dim3(256), 0, s,
                       scan, S, E, left_splits, right_splits);
    hipLaunchKernelGGL(rl_scatter_kernel, dim3(g), dim3(kRlBlock), 0, s, bins, N, ld, F, rows, R, nrs, nes,
                       S, E, feat, thr, scan, left_out, right_out, cap, status);
}

}  // namespace

hipError_t launch_rowlist_partition(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                                    const int32_t* rows, int64_t R, const int32_t* nrs,
                                    const int32_t* nes, int32_t S, int32_t E, const int32_t* feat,
                                    const int32_t* thr, int32_t* left_out, int32_t* right_out,
                                    int64_t cap, int32_t* left_splits, int32_t* right_splits,
                                    int32_t* work, hipStream_t s) {
    rowlist_partition_stages(bins, N, ld, F, rows, R, nrs, nes, S, E, feat, thr, left_out, right_out,
                             cap, left_splits, right_splits, work, work + kRlStatus, s);
    return hipGetLastError();
}

int64_t rowlist_noalloc_max_segments() {
    // largest n with rowlist_work_elems(n) - kRlStatus <= kNoAllocScratchInts
    int64_t lo = 0, hi = kNoAllocScratchInts;
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) / 2;
        if (rowlist_work_elems(mid) - kRlStatus <= kNoAllocScratchInts) lo = mid; else hi = mid - 1;
    }
    return lo;
}

hipError_t launch_rowlist_partition_noalloc(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                                            const int32_t* rows, int64_t R, const int32_t* nrs,
                                            const int32_t* nes, int32_t S, int32_t E,
                                            const int32_t* feat, const int32_t* thr, int32_t* left_out,
                                            int32_t* right_out, int64_t cap, int32_t* left_splits,
                                            int32_t* right_splits, int32_t* status, hipStream_t s) {
    int32_t* rest = nullptr;
    hipError_t e = noalloc_scratch(&rest);
    if (e != hipSuccess) return e;
    rowlist_partition_stages(bins, N, ld, F, rows, R, nrs, nes, S, E, feat, thr, left_out, right_out,
                             cap, left_splits, right_splits, status, rest, s);
    return hipGetLastError();
}

hipError_t launch_rowlist_gather(const uint8_t* bins, int64_t N, int64_t ld, int32_t F,
                                 const int32_t* feats, int32_t K, const float* values,
                                 const int32_t* rows, int64_t R, const int32_t* nrs,
                                 const int32_t* nes, int32_t m0, int32_t m1, int32_t E,
                                 uint8_t* out_bins, int64_t out_ld, float* out_values,
                                 uint16_t* out_slot, int32_t* era_off, int32_t* work, hipStream_t s) {
    const int32_t Mc = m1 - m0;
    const int64_t n = (int64_t)Mc * E;
    int32_t* status = work;
    int32_t* vals = status + kRlStatus;
    int32_t* scan = vals + 2 * n;
    int32_t* tiles = scan + 2 * n + 2;
    hipLaunchKernelGGL(rl_clear_kernel, dim3(1), dim3(kWave), 0, s, status);
    hipLaunchKernelGGL(rl_sizes_kernel, dim3(grid_of(n, 256, 1 << 14)), dim3(256), 0, s, nrs, nes, R, m0, m1,
                       E, vals, status);
    scan_pairs(vals, n, tiles, scan, s);
    hipLaunchKernelGGL(rl_gather_kernel, dim3(grid_of(n, kRlWaves, 1 << 16)), dim3(kRlBlock), 0, s, bins, N,
                       ld, F, feats, K, values, rows, R, nrs, nes, m0, m1, E, scan, out_bins, out_ld,
                       out_values, out_slot, status);
    hipLaunchKernelGGL(rl_era_off_kernel, dim3(grid_of((int64_t)E + 1, 256, 1 << 14)), dim3(256), 0, s, scan,
                       Mc, E, era_off);
    return hipGetLastError();
}

hipError_t launch_best_thresholds(const pb_candidate* cand, int32_t M, int32_t K, int32_t T,
                                  float* score, int32_t* thr, float* left_grad, float* left_hess,
                                  int64_t* left_count, hipStream_t s) {
    const int64_t n = (int64_t)M * K;
    hipLaunchKernelGGL(rl_best_kernel, dim3(grid_of(n, 256, 1 << 24)), dim3(256), 0, s, cand, n, T, score,
                       thr, left_grad, left_hess, left_count);
    return hipGetLastError();
}

}  // namespace pb
