// frnn_internal.hpp -- host-side declarations shared by the engine and the kernel files.
#pragma once

#include <hip/hip_runtime.h>

#include "frnn_mi355x.h"

namespace frnn {

// Padded AoS row length (floats).  It is also the dimension the MFMA search is
// instantiated for; padding coordinates are zero in every row, which leaves
// both the MFMA dot products and the exact fp32 distances unchanged.
__host__ __device__ inline int aos_stride(int D) {
    return D <= 4 ? 4 : D <= 8 ? 8 : D <= 12 ? 12 : D <= 16 ? 16 : D <= 32 ? 32 : D <= 64 ? 64 : 128;
}

// Per-query candidate list entries: K kept after a compaction, room for a full
// 64-entry recheck batch and at least 64 more arrivals between compactions.
// At most 256, the largest register sort of the search kernel.
inline int list_capacity(int K) { return K + 128; }

int scan_partials_count(int n);

// ---- within-cell refinement -------------------------------------------------
// Cells holding at least kBigCell points are ordered internally by a 2-D
// sub-bin key on the projections onto the two principal directions of the
// non-grid coordinates (one direction when only one non-grid coordinate
// exists), kSubBins sub-bins per big cell.  The search then restricts each big
// cell to the sub-bins that intersect its queries' windows.
constexpr int kBigCell = 256;
constexpr int kSubBins = 1024;
constexpr int kStatBlocks = 64;        // point slices per coordinate (statistics)
constexpr int kMaxTerms = FRNN_REFINE_TERMS;
constexpr int kMaxPairs = kMaxTerms * (kMaxTerms + 1) / 2;   // covariance entries
constexpr int kCovBlocks = 512;         // sampled 256-point tiles (covariance)

struct RefineInfo {
    int L;              // refinement directions (0 = none)
    int nb1, nb2;       // sub-bins per direction, nb1 * nb2 == kSubBins
    int terms;          // coordinates per projection
    float lo0, lo1;     // bin origin per direction
    float inv0, inv1;   // bins per unit per direction
    float margin;       // bound on the projection rounding of any finite point
    int pad[7];
    int coord[kMaxTerms];
    float mean[kMaxTerms];
    float w0[kMaxTerms], w1[kMaxTerms];
};
static_assert(sizeof(RefineInfo) == sizeof(frnn_refine_info_t), "RefineInfo mirrors frnn_refine_info_t");

struct RefineLayout {
    size_t info, bidx, subcnt, substart, scanpart, cov, subkey, total;   // byte offsets
    int max_big;        // upper bound on cells with >= kBigCell points
    int nsub;           // max_big * kSubBins + 1 scanned entries
};

// Per-coordinate statistics of the input (fp64 accumulation): the mean is the
// centre of the MFMA filter rows, variance and range choose and scale the
// refinement axes.
struct DimStat { float mean, var, lo, hi; };
struct StatsLayout { size_t dims, part, total; };
StatsLayout stats_layout(int D);
int launch_point_stats(const float* pts, int N, int D, void* stats_ws, hipStream_t s);

// Number of refinement axes the plan allows (0 for brute force and full-D grids).
inline int refine_axes(const frnn_plan_t& p, int D) {
    if (p.path != FRNN_PATH_GRID_FIRST) return 0;
    const int extra = D - p.grid_dim;
    return extra <= 0 ? 0 : (extra >= 2 ? 2 : 1);
}
RefineLayout refine_layout(int N, int D, long long cells);
int launch_refine(const float* pts, int N, int D, int g, long long cells, const int* cell_of, const int* cnt,
                  int* rank, const void* stats_ws, void* ws, hipStream_t s);

// Launchers return 0, 1 (bad argument), 2 (size limit) or 3 (HIP launch error;
// the error code is kept for last_launch_error()).
int launch_result();
hipError_t last_launch_error();

int launch_fill_i32(int* p, long long n, int v, hipStream_t s);
int launch_bin_count(const float* pts, int N, int g, int res, float inv_cell, int* cell_of, int* rank,
                     int* cnt, hipStream_t s);
// flag_min > 0 scans (in[i] >= flag_min) instead of in[i]
int launch_exclusive_scan(const int* in, int n, int* out, int* partials, hipStream_t s, int flag_min = 0);
// refine_ws: workspace of launch_refine, or nullptr when the plan has no refinement.
// stats_ws/frows/fnorm: when given, also write the centred filter rows
// fl(x - mean) (stride aos_stride(D)) and their squared norms.
int launch_reorder(const float* pts, int N, int D, const int* cell_of, const int* rank, const int* start,
                   const int* cnt, const void* refine_ws, long long cells, int* sorted_idx, int* inv,
                   float* aos, const void* stats_ws, float* frows, float* fnorm, hipStream_t s);
int launch_transpose(const float* pts, int N, int D, float* aos, const void* stats_ws, float* frows,
                     float* fnorm, hipStream_t s);
int launch_unpermute(const unsigned long long* lists, int cap, const int* inv, int N, int K, int* idxs,
                     float* dists, hipStream_t s);
int launch_search(const float* aos, const float* frows, const float* fnorm, const int* sorted_idx,
                  const int* start, const void* refine_ws, int N, int D, int K, const frnn_plan_t& plan,
                  unsigned long long* lists, int cap, unsigned long long* counters, hipStream_t s);

}  // namespace frnn
