/*
 * frnn_mi355x.h -- C ABI of the MI355X (gfx950) fixed-radius nearest-neighbour engine.
 *
 * Plain C types only: device pointers are raw addresses, streams are hipStream_t
 * passed as void*.  Every entry point returns an frnn_status (0 = success) and
 * validates its arguments on the host before any HIP call.
 *
 * Reference interfaces replaced (paths under the reference tree):
 *   engine entry points    python_interface/frnn_engine.h:9-55 and
 *                          python_interface/nanobind_module.cu:8-21 (FRNNEngine)
 *   kernel launch seam     python_interface/frnn_engine.cu:9-20 (extern "C" run_*)
 *
 * Layouts (same as the reference):
 *   input   SoA fp32, p[d*N + i]                       (frnn_engine.h:21-26)
 *   output  SoA, idx[k*N + i] int32, dist[k*N + i] fp32 squared L2
 *                                                      (find_nbrs.cu:206-213)
 * Semantics: every point is a query; the neighbours of query i are the (up to)
 * K points j with fl32 squared distance d2 < fl32(radius*radius), the K
 * smallest in (d2, j) order, written in ascending order; unused slots hold
 * (d2 = r2, idx = -1).
 */
#ifndef FRNN_MI355X_H
#define FRNN_MI355X_H

#ifdef __cplusplus
extern "C" {
#endif

#define FRNN_MAX_K 128           /* grid.h:59 MAX_K_CAPACITY */
#define FRNN_MAX_DIM 128         /* grid.h:60 MAX_DIM_SUPPORTED */
#define FRNN_MAX_CELLS 1000000   /* frnn_engine.cu:35 */

enum frnn_status {
    FRNN_OK = 0,
    FRNN_ERR_INVALID_ARGUMENT = 1, /* N, dim, K, radius or a pointer out of range */
    FRNN_ERR_CAPACITY = 2,         /* N above the engine's max_points, or sizes too large */
    FRNN_ERR_HIP = 3,              /* a HIP runtime call or kernel launch failed */
    FRNN_ERR_NO_DEVICE = 4,        /* no HIP device visible */
    FRNN_ERR_STATE = 5             /* e.g. get_results before any search */
};

enum frnn_path {
    FRNN_PATH_EMPTY = -1,          /* N == 0: nothing to do */
    FRNN_PATH_BRUTEFORCE = 0,      /* frnn_engine.cu:224-225 / :156,228 fallback */
    FRNN_PATH_GRID_FULL = 1,       /* full-D uniform grid, frnn_engine.cu:230-245 */
    FRNN_PATH_GRID_FIRST = 2       /* first-coordinate grid, frnn_engine.cu:64-102 */
};

/* Result of the reference's auto-dispatch (frnn_engine.cu:201-246, :64-86). */
typedef struct frnn_plan {
    int path;          /* enum frnn_path */
    int grid_dim;      /* g: number of gridded coordinates (0 for brute force) */
    int res;           /* cells per gridded axis */
    int rev_order;     /* 1: D=3 grid distance order fma(dx,dx,fma(dy,dy,dz*dz)) */
    long long cells;   /* res^g */
    float r2;          /* fl32(radius * radius) */
    float cell_size;   /* cell edge = radius (frnn_engine.cu:206) */
    float inv_cell;    /* fl32(1 / radius) */
} frnn_plan_t;

typedef struct frnn_engine frnn_engine_t;

/* Per-coordinate input statistics; a statistics workspace starts with
 * FRNN_MAX_DIM of them.  mean is the centre of the MFMA filter operands (0 if
 * not finite), var/lo/hi choose the frame's terms and bound its projections. */
typedef struct frnn_dim_stat {
    float mean, var, lo, hi;
} frnn_dim_stat_t;

/* Grid frame of grid plans with at most 4 grid axes (no reference
 * counterpart); a frame workspace starts with it.  First-coordinate plans with
 * dim > grid_dim get a projected frame, every other such grid plan a raw frame
 * (projected == 0: the plan's own cells on the first grid_dim coordinates,
 * axis 0 split fine0 ways).  The result does not depend on the grid: every point
 * within the radius of a query lies in the query's 3^g cell shell of any grid
 * whose cells are at least the radius wide (plus rounding slack), so the engine
 * grids the data along its own principal directions instead of the first g
 * coordinates, which shrinks the shells of low-rank data several-fold.
 *
 * Projection of point x onto direction k (0 <= k < grid_dim):
 *   s = 0;  s = fmaf(dir[k][t], fl(x[coord[t]] - mean[t]), s)  for t = 0..terms-1
 * (sequential fp32 fma chain; the weights of each direction have norm < 1 and the
 * directions are orthonormal up to a 2^-18 shrink); margin bounds |computed -
 * exact projection| over every finite input point.  Cell coordinate
 * c_k = clamp(floor((s_k - lo[k]) * inv_h), 0, res[k] - 1) (inv_h0 for k = 0)
 * and cell id sum_k c_k * stride[k].  Direction 0 has fine0 cells per cell edge
 * h, so the points of a row of cells (fixed c_1..c_{g-1}) are ordered by their
 * projection on it.  projected == 0 (raw frames, and projected frames on
 * infinite input) bins the first grid_dim raw coordinates with the plan's cell
 * size and resolution (axis 0 still split fine0 ways). */
#define FRNN_FRAME_TERMS 32
#define FRNN_FRAME_DIRS 4
typedef struct frnn_frame {
    int grid_dim;          /* gridded directions g */
    int cells;             /* prod res[k] */
    int terms;             /* coordinates per projection, <= FRNN_FRAME_TERMS */
    int projected;         /* 1: principal directions; 0: raw first coordinates */
    int fine0;             /* cells of direction 0 per cell edge h (its cells are h / fine0 wide) */
    int res[FRNN_FRAME_DIRS];      /* cells per grid direction */
    int stride[FRNN_FRAME_DIRS];   /* cell-id stride per grid direction, stride[0] == 1 */
    float lo[FRNN_FRAME_DIRS];     /* grid origin per direction */
    float h, inv_h;        /* cell edge and fl(1/h) */
    float margin;          /* projection rounding bound */
    float slack;           /* binning rounding bound on a cell boundary */
    float h0, inv_h0;      /* direction 0's cell edge h / fine0 and fl(1/h0) */
    float sigma[FRNN_FRAME_DIRS];  /* standard deviation of the projections per direction */
    int coord[FRNN_FRAME_TERMS];               /* term coordinates, highest variance first */
    float mean[FRNN_FRAME_TERMS];              /* term centres (the point-statistics means) */
    float dir[FRNN_FRAME_DIRS][FRNN_FRAME_TERMS];   /* grid directions */
} frnn_frame_t;

/* ---- host-only helpers (no HIP call) ------------------------------------ */

const char* frnn_status_string(int status);
/* Message of the last failure on the calling thread ("" if none). */
const char* frnn_last_error(void);
int frnn_version(void);

/* Argument checks the reference never made (grid.h:59-60 documents K, D <= 128;
 * C9 of the reference contract): 0 < N <= max_points, 1 <= dim <= 128,
 * 1 <= K <= 128, radius finite and > 0.  max_points <= 0 skips the N check. */
int frnn_validate(int max_points, int N, int dim, int K, float radius);

/* The reference dispatch rules, integer-exact (frnn_engine.cu:201-246, :64-86). */
int frnn_make_plan(int N, int dim, int K, float radius, frnn_plan_t* out);

/* Workspace geometry used by the launch seam below. */
int frnn_aos_stride(int dim);                 /* padded AoS row length in floats */
int frnn_list_capacity(int K);                /* per-query candidate list entries */
int frnn_scan_partials_count(int n);          /* ints of scratch for frnn_launch_exclusive_scan */

/* ---- engine (replaces FRNNEngine, frnn_engine.h:9-55) -------------------- */

/* FRNNEngine::FRNNEngine(int max_points), frnn_engine.cu:23-46 */
int frnn_engine_create(int max_points, frnn_engine_t** out);
/* FRNNEngine::~FRNNEngine, frnn_engine.cu:48-55 */
int frnn_engine_destroy(frnn_engine_t* engine);
int frnn_engine_max_points(const frnn_engine_t* engine, int* out);

/* FRNNEngine::search_gpu, frnn_engine.cu:195-250.  d_points_soa is borrowed for
 * the call; *d_idxs / *d_dists receive engine-owned device buffers (SoA
 * [k*N+i]) valid until the next search or destroy.  Synchronous. */
int frnn_engine_search_gpu(frnn_engine_t* engine, const float* d_points_soa, int N, int dim,
                           int K, float radius, int** d_idxs, float** d_dists);

/* Queries distinct from the points: the two-array form of the reference's
 * kernels (run_find_nbrs with d_points1 != d_points2, find_nbrs.cu:562-567;
 * run_bruteforce with p1 != p2, no_grid_frnn.cu:273-276), which its engine
 * only ever calls with the same array.  The plan and the grid are the N
 * points' (frnn_make_plan(N, ...)); every query is binned with the same
 * parameters.  d_queries_soa is SoA [d*M + j], M <= max_points; outputs are
 * engine-owned SoA [k*M + j] with indices into the points, valid until the
 * next search.  N == 0 gives padding rows.  Synchronous. */
int frnn_engine_search_gpu_queries(frnn_engine_t* engine, const float* d_points_soa, int N,
                                   const float* d_queries_soa, int M, int dim, int K, float radius,
                                   int** d_idxs, float** d_dists);

/* Grid reuse across calls (no reference counterpart at the engine level:
 * its kernels take a prebuilt grid, find_nbrs.cu:562-567, but its engine
 * rebuilds on every call).  frnn_engine_build plans, bins and reorders the N
 * points into engine-owned buffers (the input may be freed afterwards);
 * frnn_engine_query then searches M query points against that grid, any
 * number of times, with the K and radius of the build.  search_gpu,
 * search_gpu_queries and search replace the built grid with their own, which
 * frnn_engine_query reuses as well.  Outputs as frnn_engine_search_gpu_queries.
 * frnn_engine_query before any build returns FRNN_ERR_STATE. */
int frnn_engine_build(frnn_engine_t* engine, const float* d_points_soa, int N, int dim, int K,
                      float radius);
int frnn_engine_query(frnn_engine_t* engine, const float* d_queries_soa, int M, int** d_idxs,
                      float** d_dists);

/* FRNNEngine::search, frnn_engine.cu:104-193.  Host AoS points [i*dim + d] with
 * n_values = max_points * dim; N is max_points as in the reference
 * (frnn_engine.cu:108-109).  Outputs are host AoS [i*K + k], n_values/dim*K each. */
int frnn_engine_search(frnn_engine_t* engine, const float* h_points_aos, long long n_values,
                       int K, float radius, int* h_idxs_aos, float* h_dists_aos);

/* FRNNEngine::get_results, frnn_engine.cu:252-258: copies N*K entries of the
 * last search_gpu output device->host, SoA order [k*N+i], no un-transpose. */
int frnn_engine_get_results(frnn_engine_t* engine, int N, int K, int* h_idxs_soa,
                            float* h_dists_soa);

/* Stream for all engine work (default: the null stream, as the reference). */
int frnn_engine_set_stream(frnn_engine_t* engine, void* hip_stream);

/* Plan used by the last search. */
int frnn_engine_last_plan(const frnn_engine_t* engine, frnn_plan_t* out);

/* Profiling (replaces the reference's FRNN_REPORT_OCCUPANCY diagnostics,
 * find_nbrs.cu:355-382).  flags: FRNN_PROFILE_EVENTS records per-stage HIP
 * events; FRNN_PROFILE_SEARCH_EVENTS records only the two around the
 * neighbour search (stage 6; the others read 0), which keeps the event
 * overhead out of timed calls; FRNN_PROFILE_COUNTERS runs the counting build
 * of the search kernel and reads its work counters back after each search
 * (0: none).  Stages:
 * 0 zero-fill, 1 point statistics, 2 grid frame, 3 bin+count, 4 scan,
 * 5 reorder/transpose (and, for separate queries, their binning, scan and
 * reorder), 6 neighbour search, 7 unpermute.  After frnn_engine_query, stages
 * 0-4 read 0 (they belong to the build) and stage 5 is the queries' own
 * binning, scan and reorder. */
#define FRNN_NUM_STAGES 8
#define FRNN_PROFILE_EVENTS 1
#define FRNN_PROFILE_COUNTERS 2
#define FRNN_PROFILE_SEARCH_EVENTS 4
int frnn_engine_set_profiling(frnn_engine_t* engine, int flags);
int frnn_engine_stage_times(const frnn_engine_t* engine, float* ms, int n);
/* Work counters of the last search run with FRNN_PROFILE_COUNTERS:
 * [0] shell candidates (sum over queries of the points in their 3^g cells,
 * or N per query for brute force), [1] pairs passing the MFMA filter,
 * [2] pairs accepted after the exact check, [3] query-candidate pairs
 * streamed through the MFMA filter (after the window and AABB pruning).
 * Such a search also fails with FRNN_ERR_HIP if the kernel's internal
 * capacity guards ever fired. */
#define FRNN_NUM_COUNTERS 4
int frnn_engine_counters(const frnn_engine_t* engine, long long* out, int n);
/* Count-array work of the last build (no reference counterpart: the figures
 * behind the build's HBM accounting): out[0] = entries zero-filled (0 when
 * the previous call's count scan had left the array zero), out[1] = entries
 * the count scan covered (a frame's cells + 1, read back from the device
 * only while FRNN_PROFILE_EVENTS is set; otherwise the plan's capacity + 1;
 * 0 without a grid). */
int frnn_engine_count_work(const frnn_engine_t* engine, long long* out, int n);

/* ---- kernel launch seam (replaces run_*, frnn_engine.cu:9-20) ------------ */
/* All pointers are device pointers; launches are asynchronous on `stream`. */

/* Cell count a plan's grid uses: res^g without a frame (more than 4 grid
 * axes); fine0 * res^g with fine0 = 8 for a raw frame; for first-coordinate
 * plans with dim > grid_dim (projected frame) the frame's capacity
 * fine0 * max(min(max(N, 4096), FRNN_MAX_CELLS), res^g) (the frame picks its
 * resolution to fit).  At most 8 * FRNN_MAX_CELLS.
 * Count arrays hold cells + 1 ints. */
long long frnn_grid_cells(int N, int dim, const frnn_plan_t* plan);

/* run_insert_points (insert_points.cu:45-88,167-174): zero d_cnt[0..cells],
 * bin every point (without d_frame_ws: the first grid_dim coordinates, clamped
 * to [0,res-1]; with a frame: its grid directions), d_cell_of[i] = cell id,
 * d_rank[i] = arrival slot in its cell, d_cnt[c] = occupancy. */
int frnn_launch_bin_count(const float* d_points_soa, int N, int grid_dim, int res,
                          float inv_cell, long long cells, const void* d_frame_ws, int* d_cell_of,
                          int* d_rank, int* d_cnt, void* stream);

/* thrust::exclusive_scan (frnn_engine.cu:91-94): d_out[i] = sum_{j<i} d_in[j]
 * for i < n.  d_partials holds frnn_scan_partials_count(n) ints. */
int frnn_launch_exclusive_scan(const int* d_in, int n, int* d_out, int* d_partials,
                               void* stream);

/* No counterpart in the reference: frnn_launch_exclusive_scan without the
 * d_partials workspace, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  It calls no allocating routine: the per-tile partial sums live
 * in a fixed 16 KB device array inside the library (one per device, kept
 * until the process ends).  n <= FRNN_SCAN_NOALLOC_MAX_N, else
 * FRNN_ERR_CAPACITY.  All calls on one device share that array, so calls that
 * overlap on a device (concurrent streams or threads) race; calls in sequence
 * on one stream are safe.  Results equal frnn_launch_exclusive_scan's. */
#define FRNN_SCAN_NOALLOC_MAX_N 16777216
int frnn_launch_exclusive_scan_noalloc(const int* d_in, int n, int* d_out, void* stream);

/* Per-coordinate statistics of the input (no reference counterpart): mean,
 * variance, minimum and maximum of every coordinate, accumulated in fp64 in a
 * fixed order.  Needs frnn_stats_workspace_bytes(dim) bytes at d_stats_ws. */
long long frnn_stats_workspace_bytes(int dim);
int frnn_launch_point_stats(const float* d_points_soa, int N, int dim, void* d_stats_ws, void* stream);

/* Grid frame of grid plans with at most 4 grid axes (no reference
 * counterpart; frnn_frame_t).  frnn_frame_workspace_bytes() bytes at
 * d_frame_ws (0: the plan has no frame).  frnn_launch_frame writes the frame:
 * for first-coordinate plans with dim > grid_dim the principal directions of
 * the up to 32 highest-variance coordinates from a sampled covariance (needs
 * the point statistics), otherwise the raw frame (d_stats_ws may be NULL);
 * run it before binning. */
long long frnn_frame_workspace_bytes(int N, int dim, const frnn_plan_t* plan);
int frnn_launch_frame(const float* d_points_soa, int N, int dim, const frnn_plan_t* plan,
                      const void* d_stats_ws, void* d_frame_ws, void* stream);

/* run_counting_sort / run_counting_sort_aos3 (insert_points.cu:142-164,205-226):
 * pos = d_start[cell] + rank; d_sorted_idx[pos] = i; d_inv[i] = pos; AoS row
 * pos of d_sorted_aos (stride frnn_aos_stride(dim), zero padded) = point i.
 * With d_frows (needs d_stats_ws), row pos of d_frows also gets the centred
 * row fl(x - mean), which the search streams when frnn_uses_filter_rows(dim).
 * d_stats_ws and d_frows may be NULL. */
int frnn_launch_reorder(const float* d_points_soa, int N, int dim, const int* d_cell_of,
                        const int* d_rank, const int* d_start, int* d_sorted_idx, int* d_inv,
                        float* d_sorted_aos, const void* d_stats_ws, float* d_frows, void* stream);

/* Brute-force input staging: AoS copy of the SoA points in original order,
 * plus the centred rows as frnn_launch_reorder when d_frows is given. */
int frnn_launch_transpose(const float* d_points_soa, int N, int dim, float* d_aos,
                          const void* d_stats_ws, float* d_frows, void* stream);

/* 1 when the search streams precomputed centred filter rows for this dim
 * (padded rows of 64 floats or more), 0 when it centres rows in registers. */
int frnn_uses_filter_rows(int dim);

/* run_find_nbrs / run_find_nbrs_griddim / run_find_nbrs_aos3 / run_bruteforce
 * (find_nbrs.cu:525-633, no_grid_frnn.cu:273-326): neighbour search over the
 * plan's path.  The MFMA filter works on rows centred on the means of
 * d_stats_ws (frnn_launch_point_stats): d_frows (required when
 * frnn_uses_filter_rows(dim), ignored otherwise) or the AoS rows centred as
 * they are loaded; exact distances use the raw AoS rows.  Grid paths read the
 * cell-sorted AoS points, d_sorted_idx, d_cell_of (cell id per original
 * point), d_start (frnn_grid_cells + 1 exclusive offsets) and, for
 * first-coordinate plans, the frame workspace; brute force reads the
 * transposed AoS points and ignores them.
 *
 * queries == NULL: every point is a query (the engine's all-points search,
 * run_find_nbrs(d_points, d_points, ...) as frnn_engine.cu:241-245 calls it).
 * Otherwise the M queries of *queries are searched against the N points: the
 * two-array form run_find_nbrs(d_points1 = queries, d_points2 = points, ...)
 * (find_nbrs.cu:562-567; run_find_nbrs_griddim :597-633) and
 * run_bruteforce(d_p1, d_p2, P1, P2, ...) (no_grid_frnn.cu:273-276).
 *
 * Results: for search position s (sorted position of the point, or of the
 * query), entries d_lists[s*list_cap + k], k < K, hold ascending keys
 * (bits(d2) << 32 | idx) with padding (bits(r2) << 32 | 0xffffffff).
 * list_cap >= K; below frnn_list_capacity(K) a list can overflow, and then
 * *d_status (a device-visible word the caller zeroes; may be NULL) is set to 1
 * and the lists are not valid.  d_counters (5 u64: the FRNN_NUM_COUNTERS work
 * counters and a capacity-guard counter; may be NULL) runs the counting build
 * of the kernel and accumulates the counters. */
typedef struct frnn_queries {
    int M;                      /* number of queries */
    const float* d_aos;         /* [M x frnn_aos_stride(dim)] rows in search order: frnn_launch_reorder
                                   of the queries binned on the points' grid, or frnn_launch_transpose
                                   for brute force */
    const float* d_frows;       /* their centred rows (when frnn_uses_filter_rows(dim)), centred on the
                                   points' statistics */
    const int* d_sorted_idx;    /* search position -> original query index (grid paths) */
    const int* d_cell_of;       /* original query index -> cell id on the points' grid (grid paths) */
} frnn_queries_t;
int frnn_launch_find_nbrs(const float* d_aos, const float* d_frows, const void* d_stats_ws,
                          const int* d_sorted_idx, const int* d_cell_of, const int* d_start,
                          const void* d_frame_ws, int N, int dim, int K, const frnn_plan_t* plan,
                          const frnn_queries_t* queries, unsigned long long* d_lists, int list_cap,
                          unsigned long long* d_counters, unsigned int* d_status, void* stream);

/* run_scatter_to_orig (find_nbrs.cu:505-535): output row of original query i is
 * list row d_inv[i] (identity when d_inv is NULL); writes SoA [k*N+i]. */
int frnn_launch_unpermute(const unsigned long long* d_lists, int list_cap, const int* d_inv,
                          int N, int K, int* d_idxs, float* d_dists, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FRNN_MI355X_H */
