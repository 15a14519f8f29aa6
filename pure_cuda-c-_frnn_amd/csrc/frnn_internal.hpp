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

// Per-query candidate list entries: 256 for every K.  The search keeps a
// histogram of each list's keys by distance and lowers the query's threshold
// as soon as K keys lie below a bucket edge, so a list fills up slowly; with
// 255 usable entries most lists never need a compaction before the final
// selection (a sort of at most 128 keys after dropping the keys above the
// threshold).
inline int list_capacity(int /*K*/) { return 256; }

int scan_partials_count(int n);

// ---- grid frame ---------------------------------------------------------------
// First-coordinate plans grid the data on its principal directions (Frame).
constexpr int kStatBlocks = 64;        // point slices per coordinate (statistics)
constexpr int kMaxTerms = FRNN_FRAME_TERMS;
constexpr int kMaxPairs = kMaxTerms * (kMaxTerms + 1) / 2;   // covariance entries
constexpr int kCovBlocks = 512;         // sampled 256-point tiles (covariance)
constexpr int kFrameGrid = FRNN_FRAME_DIRS;   // grid directions of a frame

struct Frame {
    int g, cells, terms;                // grid directions, cells, projection terms
    int projected;                      // 0: raw first coordinates (infinite input)
    int fine0;                          // cells of axis 0 per cell edge h
    int res[kFrameGrid];
    int stride[kFrameGrid];
    float lo[kFrameGrid];
    float h, inv_h, margin, slack;
    float h0, inv_h0;                   // axis 0's cell edge h / fine0 and fl(1/h0)
    float sigma[kFrameGrid];
    int coord[kMaxTerms];
    float mean[kMaxTerms];
    float dir[kFrameGrid][kMaxTerms];
};
static_assert(sizeof(Frame) == sizeof(frnn_frame_t), "Frame mirrors frnn_frame_t");

struct FrameLayout {
    size_t frame, cov, covsum, total;   // byte offsets
};

// Per-coordinate statistics of the input (fp64 accumulation): the mean is the
// centre of the MFMA filter rows and of the projections, variance and range
// choose and bound the projection terms.
struct DimStat { float mean, var, lo, hi; };
struct StatsLayout { size_t dims, part, total; };
StatsLayout stats_layout(int D);
int launch_point_stats(const float* pts, int N, int D, void* stats_ws, hipStream_t s);

// Grid plans with at most kFrameGrid axes bin through a frame (Frame): a
// first-coordinate plan with D > g on its principal directions (projected
// frame), every other one on the plan's own raw cells (raw frame).  A
// frame's axis 0 has kFine0 cells per cell edge h: points are ordered by
// their coordinate on it inside every row of cells, so a chunk of queries
// covers a short stretch of its row and the search streams only the stretch
// of each neighbouring row within reach of the chunk (all other grid axes keep
// cells of edge h, so the rows, and the query runs sharing one, stay as long).
constexpr int kFine0 = 8;
inline bool has_projected_frame(const frnn_plan_t& p, int D) {
    return p.path == FRNN_PATH_GRID_FIRST && D > p.grid_dim;
}
inline bool has_frame(const frnn_plan_t& p, int D) {
    return has_projected_frame(p, D) || ((p.path == FRNN_PATH_GRID_FULL || p.path == FRNN_PATH_GRID_FIRST) &&
                                         p.grid_dim >= 1 && p.grid_dim <= kFrameGrid);
}
// Cells (count array length - 1) of a grid plan: res^g without a frame; a
// projected frame's capacity kFine0 x max(min(max(N, 4096), 1M), res^g) (its
// raw-coordinate fallback uses res^g); kFine0 x res^g for a raw frame.
inline long long grid_cells(int N, int D, const frnn_plan_t& p) {
    if (has_projected_frame(p, D)) {
        long long c = N < 4096 ? 4096 : N;
        c = c < FRNN_MAX_CELLS ? c : FRNN_MAX_CELLS;
        return (c > p.cells ? c : p.cells) * kFine0;
    }
    if (has_frame(p, D)) return p.cells * kFine0;
    return p.cells;
}
FrameLayout frame_layout();

// The grid the device pipeline bins on.  Raw grids (raw frames, or no frame
// above kFrameGrid axes) cover the reference's [0, 1] domain with
// res = ceil(1/r) cells of edge r per axis.
// When 1/r lies just above an integer, the last layer of cells,
// [(res-1) r, 1], is a sliver: its rows hold a few points spread along the
// whole row, and every such row becomes a segment of the search that streams
// three full neighbouring rows.  Binning clamps into the edge cells, which
// every pruning test treats as unbounded outward, so merging a sliver
// thinner than half a cell into the layer before it (res - 1 cells per axis,
// the last one wider than r) keeps every pair within the radius in adjacent
// cells.  Plans with a projected frame and all other grids are returned
// unchanged.
inline frnn_plan_t binning_plan(const frnn_plan_t& p, int D) {
    if ((p.path != FRNN_PATH_GRID_FULL && p.path != FRNN_PATH_GRID_FIRST) || has_projected_frame(p, D) ||
        p.res < 4)
        return p;
    const double r = p.cell_size;
    if ((double)(p.res - 1) * r < 1.0 - 0.5 * r) return p;
    frnn_plan_t q = p;
    q.res = p.res - 1;
    long long c = 1;
    for (int d = 0; d < p.grid_dim; ++d) c *= q.res;
    q.cells = c;
    return q;
}
// Frame of a grid plan with at most kFrameGrid axes: for a projected frame
// the terms, sampled covariance, principal directions and grid geometry
// (needs the point statistics); for a raw frame the plan's own cells.
int launch_frame(const float* pts, int N, int D, const frnn_plan_t& plan, long long cells,
                 const void* stats_ws, void* ws, hipStream_t s);

// Launchers return 0, 1 (bad argument), 2 (size limit) or 3 (HIP launch error;
// the error code is kept for last_launch_error()).
int launch_result();
hipError_t last_launch_error();

int launch_fill_i32(int* p, long long n, int v, hipStream_t s);
// frame_ws: bin on the frame's grid directions (first-coordinate plans; cell
// ids are kept below `cells`, the count array's length - 1); nullptr: raw
// coordinates
int launch_bin_count(const float* pts, int N, int g, int res, float inv_cell, const void* frame_ws,
                     int cells, int* cell_of, int* rank, int* cnt, hipStream_t s);
int launch_exclusive_scan(const int* in, int n, int* out, int* partials, hipStream_t s);
// The engine's scan of its count array: over min(n, *bound + 1) entries when
// bound (a device int, the frame's cell count) is given, else n; the counts
// are zeroed as they are read, so the array is clean for the next binning.
int launch_count_scan(int* cnt, int n, const int* bound, int* out, int* partials, hipStream_t s);
// The same scan with its partial sums in a file-scope device scratch array
// (no workspace argument, no allocation); n <= scan_noalloc_max().  Returns
// 0, 2 (n too large), 3 (launch error) or 4 (the scratch's device address
// could not be looked up: scan_noalloc_error()).
int launch_exclusive_scan_noalloc(const int* in, int n, int* out, hipStream_t s);
int scan_noalloc_max();
hipError_t scan_noalloc_error();
// With frows (which needs stats_ws) the centred filter rows fl(x - mean) are
// written too.
int launch_reorder(const float* pts, int N, int D, const int* cell_of, const int* rank, const int* start,
                   int* sorted_idx, int* inv, float* aos, const void* stats_ws, float* frows, hipStream_t s);
int launch_transpose(const float* pts, int N, int D, float* aos, const void* stats_ws, float* frows,
                     hipStream_t s);
// Wide rows (padded length >= 64) stream precomputed centred filter rows;
// narrower rows are centred in registers as they are loaded.
inline bool uses_filter_rows(int D) { return aos_stride(D) >= 64; }
int launch_unpermute(const unsigned long long* lists, int cap, const int* inv, int N, int K, int* idxs,
                     float* dists, hipStream_t s);
// stats_ws: the point statistics (the per-coordinate means centre the MFMA
// filter operands).
// Queries distinct from the points, in search order: AoS rows (stride
// aos_stride(D)), centred rows (wide rows only), search position -> original
// query and original query -> cell id on the points' grid (grid paths).
struct QuerySet {
    const float* aos;
    const float* frows;
    const int* sorted_idx;
    const int* cell_of;
    int M;
};
// queries == nullptr: every point is a query (the all-points search).
// ranges: brute force on wide rows may split the points into that many
// ranges (search_ranges), whose per-range lists lie at rows r * M + query of
// `lists` (ranges * M rows) and are merged into rows 0 .. M-1; 1 for callers
// whose lists hold M rows.
int launch_search(const float* aos, const float* frows, const void* stats_ws, const int* sorted_idx,
                  const int* cell_of,
                  const int* start, const void* frame_ws, int N, int D, int K, const frnn_plan_t& plan,
                  unsigned long long* lists, int cap, unsigned long long* counters, unsigned* status,
                  hipStream_t s, const QuerySet* queries = nullptr, int ranges = 1);
// Point ranges the engine gives brute force on wide rows (1 for other plans).
int search_ranges(const frnn_plan_t& plan, int D, int N, int M);

}  // namespace frnn
