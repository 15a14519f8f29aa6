// engine.cpp -- host side of the MI355X FRNN engine behind the C ABI of
// include/frnn_mi355x.h.
//
// Replaces python_interface/frnn_engine.{h,cu}: workspace ownership
// (frnn_engine.cu:23-55), auto-dispatch (frnn_engine.cu:201-246, 64-86), the
// grid build / search / scatter pipeline (frnn_engine.cu:64-102, 224-246) and
// the host path search()/get_results() (frnn_engine.cu:104-193, 252-258).
//
// Differences by design: arguments are validated before any HIP call and a
// status is returned instead of silently overflowing; every kernel is launched
// on one stream (the null stream unless the caller sets one) and the call
// synchronises that stream once at the end; the dim- and K-dependent
// workspaces are sized on first use instead of for a fixed D <= 32
// (frnn_engine.cu:26-28).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "frnn_internal.hpp"
#include "frnn_mi355x.h"

namespace {

// public counters plus the kernel's internal capacity-guard counter
constexpr int kCounterSlots = FRNN_NUM_COUNTERS + 1;

thread_local std::string g_last_error;

int fail(int status, const char* what) {
    g_last_error = what;
    return status;
}

int hip_fail(hipError_t e, const char* what) {
    g_last_error = std::string(what) + ": " + hipGetErrorString(e);
    return FRNN_ERR_HIP;
}

#define HIP_TRY(call, what)                          \
    do {                                             \
        hipError_t e_ = (call);                      \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

#define ST_TRY(call)                \
    do {                            \
        int s_ = (call);            \
        if (s_ != FRNN_OK) return s_; \
    } while (0)

int launch_status(int rc, const char* what) {
    if (rc == 0) return FRNN_OK;
    if (rc == 3) return hip_fail(frnn::last_launch_error(), what);
    return fail(rc == 2 ? FRNN_ERR_CAPACITY : FRNN_ERR_INVALID_ARGUMENT, what);
}

long long ipow_sat(long long b, int e, long long cap) {
    long long v = 1;
    for (int i = 0; i < e; ++i) {
        if (v > cap / (b > 0 ? b : 1)) return cap + 1;
        v *= b;
    }
    return v;
}

template <typename T>
int grow(T** p, size_t* have, size_t need_elems, const char* what) {
    const size_t need = need_elems * sizeof(T);
    if (*have >= need && *p) return FRNN_OK;
    if (*p) {
        (void)hipFree(*p);
        *p = nullptr;
        *have = 0;
    }
    HIP_TRY(hipMalloc((void**)p, need), what);
    *have = need;
    return FRNN_OK;
}

}  // namespace

// The points' side of a search, kept in the engine for the queries that
// follow (this call's, or later frnn_engine_query calls): the plans, the
// grid geometry and the filter rows.
struct BuiltGrid {
    bool valid = false;
    frnn_plan_t ref_plan{}, plan{};
    int N = 0, dim = 0, K = 0, ds = 0, cap = 0;
    float radius = 0.0f;
    bool grid = false;
    long long cells = 0;
    const void* frame = nullptr;
    float* frows = nullptr;
};

struct frnn_engine {
    int max_p = 0;
    hipStream_t stream = nullptr;
    int* cell_of = nullptr;
    int* rank = nullptr;
    int* sorted_idx = nullptr;
    int* inv = nullptr;
    int* cnt = nullptr;
    // leading entries of cnt known to be zero: a build fills only past them;
    // the count scan zeroes what the binning wrote, so every call after the
    // first skips the fill
    long long cnt_zero = 0;
    long long last_fill = 0;      // entries the last build zero-filled
    long long last_scan = 0;      // entries its count scan covered (read back when profiling)
    int* start = nullptr;
    int* partials = nullptr;
    unsigned long long* counters = nullptr;
    // status word of the search kernel's capacity guards, in pinned host
    // memory (the kernel writes it only when a guard fires; read after the
    // call's stream synchronisation, no copy)
    unsigned* status_host = nullptr;
    unsigned* status_dev = nullptr;
    int* out_idx = nullptr;
    float* out_dist = nullptr;
    float* aos = nullptr;
    size_t aos_bytes = 0;
    void* frame_ws = nullptr;     // grid frame and its covariance scratch
    size_t frame_bytes = 0;
    void* stats_ws = nullptr;     // per-coordinate statistics (filter centre, frame terms)
    float* frows = nullptr;       // centred filter rows (wide rows only), stride aos_stride(dim)
    size_t frows_bytes = 0;
    size_t stats_bytes = 0;
    unsigned long long* lists = nullptr;
    size_t lists_bytes = 0;
    float* h2d_points = nullptr;  // search() staging (frnn_engine.cu:27 d_points)
    size_t h2d_bytes = 0;
    // separate queries (search_gpu_queries): binned on the points' grid and
    // reordered into their own search order; allocated on first use
    int* q_cell_of = nullptr;
    int* q_rank = nullptr;
    int* q_sorted_idx = nullptr;
    int* q_inv = nullptr;
    size_t q_cell_bytes = 0, q_rank_bytes = 0, q_sorted_bytes = 0, q_inv_bytes = 0;
    int* q_start = nullptr;
    size_t q_start_bytes = 0;
    float* q_aos = nullptr;
    size_t q_aos_bytes = 0;
    float* q_frows = nullptr;
    size_t q_frows_bytes = 0;
    frnn_plan_t last_plan{};
    bool has_result = false;
    int last_N = 0, last_K = 0;
    bool profiling = false;   // per-stage HIP events
    bool search_events = false;   // HIP events around the search kernel only
    bool counting = false;    // work counters (the counting search kernel)
    hipEvent_t ev[FRNN_NUM_STAGES + 1] = {};
    bool ev_recorded[FRNN_NUM_STAGES + 1] = {};   // recorded since the last build
    float stage_ms[FRNN_NUM_STAGES] = {};
    long long ctr[FRNN_NUM_COUNTERS] = {};
    BuiltGrid built;          // the points' grid of the last build
};

namespace {

unsigned float_bits(float f) {
    unsigned u;
    std::memcpy(&u, &f, sizeof(u));
    return u;
}

void release(frnn_engine* e) {
    void* bufs[] = {e->cell_of, e->rank, e->sorted_idx, e->inv, e->cnt, e->start, e->partials,
                    e->counters, e->out_idx, e->out_dist, e->aos, e->lists, e->h2d_points,
                    e->frame_ws, e->stats_ws, e->frows, e->q_cell_of, e->q_rank, e->q_sorted_idx,
                    e->q_inv, e->q_start, e->q_aos, e->q_frows};
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (e->status_host) (void)hipHostFree(e->status_host);
    for (auto& ev : e->ev)
        if (ev) (void)hipEventDestroy(ev);
}

// Stage events: every call records the stages it runs; stage_times() reads
// the ones of the last call that ran the search.
int mark_stage(frnn_engine* e, int i) {
    if (e->profiling || (e->search_events && (i == 6 || i == 7))) {
        HIP_TRY(hipEventRecord(e->ev[i], e->stream), "event record");
        e->ev_recorded[i] = true;
    }
    return FRNN_OK;
}

// Makes the first n count entries zero (a fill past the known-zero prefix)
// and marks them dirty for the binning that follows.
int clean_counts(frnn_engine* e, long long n) {
    if (e->cnt_zero < n) {
        ST_TRY(launch_status(frnn::launch_fill_i32(e->cnt, n, 0, e->stream), "zero-fill cells"));
        e->last_fill = n;
        e->cnt_zero = n;
    }
    e->cnt_zero = 0;   // until the count scan below has zeroed what binning wrote
    return FRNN_OK;
}

// Exclusive scan of the counts into out, over the frame's cells + 1 when a
// frame holds them (its cell count is on the device), else cells + 1; the
// scan zeroes the counts it reads, and binning wrote no others.
int count_scan(frnn_engine* e, long long cells, const void* frame, int* out) {
    const int* bound = frame ? reinterpret_cast<const int*>(static_cast<const char*>(frame) +
                                                            offsetof(frnn::Frame, cells))
                             : nullptr;
    ST_TRY(launch_status(frnn::launch_count_scan(e->cnt, (int)cells + 1, bound, out, e->partials, e->stream),
                         "scan launch"));
    e->cnt_zero = cells + 1;
    e->last_scan = cells + 1;
    if (bound && e->profiling)
        HIP_TRY(hipMemcpyAsync(e->status_host + 4, bound, sizeof(int), hipMemcpyDeviceToHost, e->stream),
                "reading the frame's cell count");
    else
        e->status_host[4] = (unsigned)cells;
    return FRNN_OK;
}

// Stages 0-5 on the N points (SoA device input): plan, statistics, frame,
// bin + count, scan, reorder (or the brute-force AoS copy).
int build_points(frnn_engine* e, BuiltGrid& b, const float* d_pts, int N, int dim, int K, float radius) {
    b.valid = false;
    for (bool& r : e->ev_recorded) r = false;
    ST_TRY(frnn_make_plan(N, dim, K, radius, &b.ref_plan));
    e->last_plan = b.ref_plan;
    // the grid the kernels bin and search on (the reference's, with a
    // sliver of a last cell layer merged)
    b.plan = frnn::binning_plan(b.ref_plan, dim);
    b.N = N;
    b.dim = dim;
    b.K = K;
    b.radius = radius;
    b.ds = frnn::aos_stride(dim);
    b.cap = frnn::list_capacity(K);
    if (b.plan.path == FRNN_PATH_EMPTY) {
        b.valid = true;
        return FRNN_OK;
    }
    const int ds = b.ds;
    const frnn_plan_t& plan = b.plan;
    ST_TRY(grow(&e->aos, &e->aos_bytes, (size_t)N * ds, "allocating AoS point rows"));
    ST_TRY(grow((char**)&e->stats_ws, &e->stats_bytes, frnn::stats_layout(dim).total, "allocating statistics"));
    b.frows = nullptr;
    if (frnn::uses_filter_rows(dim)) {
        ST_TRY(grow(&e->frows, &e->frows_bytes, (size_t)N * ds, "allocating filter rows"));
        b.frows = e->frows;
    }
    float* const frows = b.frows;
    hipStream_t s = e->stream;
    b.grid = plan.path != FRNN_PATH_BRUTEFORCE;
    const bool grid = b.grid;
    const bool framed = grid && frnn::has_frame(plan, dim);
    b.cells = grid ? frnn::grid_cells(N, dim, plan) : 0;
    const long long cells = b.cells;
    b.frame = nullptr;
    if (framed) {
        ST_TRY(grow((char**)&e->frame_ws, &e->frame_bytes, frnn::frame_layout().total,
                    "allocating the grid frame"));
        b.frame = e->frame_ws;
    }
    const void* const frame = b.frame;
    ST_TRY(mark_stage(e, 0));
    // stage 0: zero-fill the counts (frnn_engine.cu:89-90), unless the last
    // count scan left them zero
    e->last_fill = 0;
    e->last_scan = 0;
    if (grid) ST_TRY(clean_counts(e, cells + 1));
    ST_TRY(mark_stage(e, 1));
    // stage 1: per-coordinate statistics (filter centre, frame terms)
    ST_TRY(launch_status(frnn::launch_point_stats(d_pts, N, dim, e->stats_ws, s), "statistics launch"));
    ST_TRY(mark_stage(e, 2));
    // stage 2: grid frame (projected, or raw)
    if (framed)
        ST_TRY(launch_status(frnn::launch_frame(d_pts, N, dim, plan, cells, e->stats_ws, e->frame_ws, s),
                             "frame launch"));
    ST_TRY(mark_stage(e, 3));
    // stage 3: bin + count (run_insert_points, frnn_engine.cu:159-160)
    if (grid)
        ST_TRY(launch_status(frnn::launch_bin_count(d_pts, N, plan.grid_dim, plan.res, plan.inv_cell, frame,
                                                    (int)cells, e->cell_of, e->rank, e->cnt, s),
                             "bin/count launch"));
    ST_TRY(mark_stage(e, 4));
    // stage 4: exclusive scan of the counts (thrust::exclusive_scan, frnn_engine.cu:91-94)
    if (grid) ST_TRY(count_scan(e, cells, frame, e->start));
    ST_TRY(mark_stage(e, 5));
    // stage 5: reorder into cell order (CountingSort{ND,AoS3}Kernel) or, for
    // brute force, the AoS copy
    if (grid)
        ST_TRY(launch_status(frnn::launch_reorder(d_pts, N, dim, e->cell_of, e->rank, e->start, e->sorted_idx,
                                                  e->inv, e->aos, e->stats_ws, frows, s),
                             "reorder launch"));
    else
        ST_TRY(launch_status(frnn::launch_transpose(d_pts, N, dim, e->aos, e->stats_ws, frows, s),
                             "transpose launch"));
    b.valid = true;
    return FRNN_OK;
}

// Stages 6-7 against a built grid: every point as a query (sep false), or
// the M queries d_q (SoA [d*M + j]), first binned on the points' grid and
// reordered into their own search order (part of stage 5).
// own_prep: a call that only queries a grid built earlier (frnn_engine_query):
// its stage 5 is the queries' own binning, scan and reorder, and stages 0-4
// (the build's) read 0.
int run_queries(frnn_engine* e, const BuiltGrid& b, bool sep, const float* d_q, int M, bool own_prep = false) {
    const int Mq = sep ? M : b.N;   // queries = result rows
    const int K = b.K;
    e->has_result = false;
    hipStream_t s = e->stream;
    if (Mq == 0) {
        e->has_result = true;
        e->last_N = 0;
        e->last_K = K;
        return FRNN_OK;
    }
    if (b.plan.path == FRNN_PATH_EMPTY) {
        // no points: every query row is padding (r2, -1)
        ST_TRY(launch_status(frnn::launch_fill_i32(e->out_idx, (long long)Mq * K, -1, s), "padding"));
        ST_TRY(launch_status(frnn::launch_fill_i32(reinterpret_cast<int*>(e->out_dist), (long long)Mq * K,
                                                   (int)float_bits(b.ref_plan.r2), s),
                             "padding"));
        HIP_TRY(hipStreamSynchronize(s), "padding");
        e->has_result = true;
        e->last_N = Mq;
        e->last_K = K;
        return FRNN_OK;
    }
    const frnn_plan_t& plan = b.plan;
    const int dim = b.dim, ds = b.ds, cap = b.cap;
    const bool grid = b.grid;
    const long long cells = b.cells;
    const void* frame = b.frame;
    float* const frows = b.frows;
    // brute force on wide rows may split the points into ranges, each with
    // its own lists (merged into the first Mq rows)
    const int ranges = frnn::search_ranges(plan, dim, b.N, Mq);
    ST_TRY(grow(&e->lists, &e->lists_bytes, (size_t)Mq * cap * ranges, "allocating candidate lists"));
    if (e->counting)
        ST_TRY(launch_status(frnn::launch_fill_i32((int*)e->counters, 2 * kCounterSlots, 0, s),
                             "clearing counters"));
    // separate queries: binned on the points' grid (the count array is free
    // again after the points' scan), scanned and reordered into their own
    // search order, or transposed for brute force; their filter rows are
    // centred on the points' mean, as the points' are
    frnn::QuerySet qs{};
    // this call's search and unpermute stages record afresh
    for (int i = 6; i <= FRNN_NUM_STAGES; ++i) e->ev_recorded[i] = false;
    if (own_prep) {
        for (int i = 0; i <= 5; ++i) e->ev_recorded[i] = false;
        ST_TRY(mark_stage(e, 5));
    }
    if (sep) {
        ST_TRY(grow(&e->q_aos, &e->q_aos_bytes, (size_t)M * ds, "allocating query rows"));
        float* q_frows = nullptr;
        if (frows) {
            ST_TRY(grow(&e->q_frows, &e->q_frows_bytes, (size_t)M * ds, "allocating query filter rows"));
            q_frows = e->q_frows;
        }
        if (grid) {
            ST_TRY(grow(&e->q_cell_of, &e->q_cell_bytes, (size_t)M, "allocating query cells"));
            ST_TRY(grow(&e->q_rank, &e->q_rank_bytes, (size_t)M, "allocating query ranks"));
            ST_TRY(grow(&e->q_sorted_idx, &e->q_sorted_bytes, (size_t)M, "allocating query order"));
            ST_TRY(grow(&e->q_inv, &e->q_inv_bytes, (size_t)M, "allocating query positions"));
            ST_TRY(grow(&e->q_start, &e->q_start_bytes, (size_t)cells + 1, "allocating query cell starts"));
            ST_TRY(clean_counts(e, cells + 1));
            ST_TRY(launch_status(frnn::launch_bin_count(d_q, M, plan.grid_dim, plan.res, plan.inv_cell, frame,
                                                        (int)cells, e->q_cell_of, e->q_rank, e->cnt, s),
                                 "query bin/count launch"));
            ST_TRY(count_scan(e, cells, frame, e->q_start));
            ST_TRY(launch_status(frnn::launch_reorder(d_q, M, dim, e->q_cell_of, e->q_rank, e->q_start,
                                                      e->q_sorted_idx, e->q_inv, e->q_aos, e->stats_ws, q_frows,
                                                      s),
                                 "query reorder launch"));
        } else {
            ST_TRY(launch_status(frnn::launch_transpose(d_q, M, dim, e->q_aos, e->stats_ws, q_frows, s),
                                 "query transpose launch"));
        }
        qs = frnn::QuerySet{e->q_aos, q_frows, grid ? e->q_sorted_idx : nullptr, grid ? e->q_cell_of : nullptr, M};
    }
    ST_TRY(mark_stage(e, 6));
    // stage 6: neighbour search
    __atomic_store_n(e->status_host, 0u, __ATOMIC_SEQ_CST);
    ST_TRY(launch_status(frnn::launch_search(e->aos, frows, e->stats_ws, grid ? e->sorted_idx : nullptr,
                                             grid ? e->cell_of : nullptr, grid ? e->start : nullptr, frame,
                                             b.N, dim, K, plan, e->lists, cap,
                                             e->counting ? e->counters : nullptr, e->status_dev, s,
                                             sep ? &qs : nullptr, ranges),
                         "search launch"));
    ST_TRY(mark_stage(e, 7));
    // stage 7: results to the original query order (ScatterToOrigKernel)
    const int* qinv = grid ? (sep ? e->q_inv : e->inv) : nullptr;
    ST_TRY(launch_status(frnn::launch_unpermute(e->lists, cap, qinv, Mq, K, e->out_idx, e->out_dist, s),
                         "unpermute launch"));
    ST_TRY(mark_stage(e, 8));
    HIP_TRY(hipStreamSynchronize(s), "search pipeline");
    if (__atomic_load_n(e->status_host, __ATOMIC_SEQ_CST) != 0)
        return fail(FRNN_ERR_HIP, "internal list/queue capacity overflow in the search kernel");
    if (e->profiling || e->search_events)
        for (int i = 0; i < FRNN_NUM_STAGES; ++i) {
            // stages the build ran without profiling read as 0
            e->stage_ms[i] = 0.0f;
            if (e->ev_recorded[i] && e->ev_recorded[i + 1])
                HIP_TRY(hipEventElapsedTime(&e->stage_ms[i], e->ev[i], e->ev[i + 1]), "event timing");
        }
    if (e->counting) {
        unsigned long long c[kCounterSlots];
        HIP_TRY(hipMemcpy(c, e->counters, sizeof(c), hipMemcpyDeviceToHost), "reading counters");
        for (int i = 0; i < FRNN_NUM_COUNTERS; ++i) e->ctr[i] = (long long)c[i];
        if (c[FRNN_NUM_COUNTERS] != 0)
            return fail(FRNN_ERR_HIP, "internal list/queue capacity overflow in the search kernel");
    }
    e->has_result = true;
    e->last_N = Mq;
    e->last_K = K;
    return FRNN_OK;
}

// The whole device pipeline: build the N points' grid, then search every
// point (sep false) or the M queries d_q against it.
int run_pipeline(frnn_engine* e, const float* d_pts, int N, int dim, int K, float radius, bool sep = false,
                 const float* d_q = nullptr, int M = 0) {
    e->has_result = false;
    ST_TRY(build_points(e, e->built, d_pts, N, dim, K, radius));
    return run_queries(e, e->built, sep, d_q, M);
}

}  // namespace

extern "C" {

const char* frnn_status_string(int status) {
    switch (status) {
        case FRNN_OK: return "ok";
        case FRNN_ERR_INVALID_ARGUMENT: return "invalid argument";
        case FRNN_ERR_CAPACITY: return "capacity exceeded";
        case FRNN_ERR_HIP: return "HIP runtime error";
        case FRNN_ERR_NO_DEVICE: return "no HIP device";
        case FRNN_ERR_STATE: return "invalid engine state";
        default: return "unknown status";
    }
}

const char* frnn_last_error(void) { return g_last_error.c_str(); }

int frnn_version(void) { return 1; }

int frnn_validate(int max_points, int N, int dim, int K, float radius) {
    if (N < 0) return fail(FRNN_ERR_INVALID_ARGUMENT, "N must be >= 0");
    if (max_points > 0 && N > max_points) return fail(FRNN_ERR_CAPACITY, "N exceeds max_points");
    if (dim < 1 || dim > FRNN_MAX_DIM) return fail(FRNN_ERR_INVALID_ARGUMENT, "dim must be in [1, 128]");
    if (K < 1 || K > FRNN_MAX_K) return fail(FRNN_ERR_INVALID_ARGUMENT, "K must be in [1, 128]");
    if (!(radius > 0.0f) || !std::isfinite(radius))
        return fail(FRNN_ERR_INVALID_ARGUMENT, "radius must be finite and > 0");
    return FRNN_OK;
}

int frnn_make_plan(int N, int dim, int K, float radius, frnn_plan_t* out) {
    if (!out) return fail(FRNN_ERR_INVALID_ARGUMENT, "null plan pointer");
    ST_TRY(frnn_validate(0, N, dim, K, radius));
    frnn_plan_t p{};
    p.r2 = radius * radius;
    p.cell_size = radius;
    p.inv_cell = 1.0f / radius;
    if (N == 0) {
        p.path = FRNN_PATH_EMPTY;
        *out = p;
        return FRNN_OK;
    }
    // frnn_engine.cu:201-213: res = ceil((max-min)/cell) in fp32, cells = res^dim in double
    const float cr = std::ceil((1.0f - 0.0f) / radius);
    const int res = cr >= 1073741824.0f ? 1073741824 : (int)cr;
    const double total_d = std::pow((double)res, dim);
    const bool feasible = total_d <= 1000000.0;
    const long long total = feasible ? (long long)total_d : 0;
    // frnn_engine.cu:215-219: small-problem brute-force rule
    const long long kBF = 2000000LL;
    const long long sel = std::max(1LL, (long long)(K + 7) / 8);
    const long long db = ((long long)N * dim > kBF) ? (kBF + 1LL) : (long long)N * dim;
    const bool use_bf = (db <= kBF / sel) && ((long long)N <= kBF / (db * sel));
    const long long shell = ipow_sat(3, dim, (long long)4e18);
    if (use_bf) {
        p.path = FRNN_PATH_BRUTEFORCE;
    } else if (res <= 1 || !feasible || shell >= total) {
        // frnn_engine.cu:64-86: grid on the first g coordinates, else brute force
        const int g = (dim > 4) ? 4 : std::min(dim, 3);
        const int r2res = std::max(res, 2);
        const double tc = std::pow((double)r2res, g);
        const long long gshell = ipow_sat(3, g, (long long)4e18);
        if (tc > 1000000.0 || gshell >= (long long)tc) {
            p.path = FRNN_PATH_BRUTEFORCE;
        } else {
            p.path = FRNN_PATH_GRID_FIRST;
            p.grid_dim = g;
            p.res = r2res;
            p.cells = (long long)tc;
        }
    } else {
        p.path = FRNN_PATH_GRID_FULL;
        p.grid_dim = dim;
        p.res = res;
        p.cells = total;
        p.rev_order = (dim == 3) ? 1 : 0;   // find_nbrs.cu:474-477 (D=3 AoS path)
    }
    *out = p;
    return FRNN_OK;
}

int frnn_aos_stride(int dim) { return (dim < 1 || dim > FRNN_MAX_DIM) ? -1 : frnn::aos_stride(dim); }
int frnn_list_capacity(int K) { return (K < 1 || K > FRNN_MAX_K) ? -1 : frnn::list_capacity(K); }
int frnn_scan_partials_count(int n) { return n < 0 ? -1 : frnn::scan_partials_count(n); }

int frnn_engine_create(int max_points, frnn_engine_t** out) {
    if (!out) return fail(FRNN_ERR_INVALID_ARGUMENT, "null engine pointer");
    *out = nullptr;
    if (max_points < 1) return fail(FRNN_ERR_INVALID_ARGUMENT, "max_points must be >= 1");
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
        (void)hipGetLastError();
        return fail(FRNN_ERR_NO_DEVICE, "no HIP device visible");
    }
    frnn_engine* e = new frnn_engine();
    e->max_p = max_points;
    const size_t P = (size_t)max_points;
    // count arrays hold a frame's cells (kFine0 x the raw cap) + 1
    const size_t C = (size_t)frnn::kFine0 * FRNN_MAX_CELLS + 1;
    hipError_t err = hipSuccess;
    auto alloc = [&](void** p, size_t bytes) {
        if (err == hipSuccess) err = hipMalloc(p, bytes);
    };
    alloc((void**)&e->cell_of, P * sizeof(int));
    alloc((void**)&e->rank, P * sizeof(int));
    alloc((void**)&e->sorted_idx, P * sizeof(int));
    alloc((void**)&e->inv, P * sizeof(int));
    alloc((void**)&e->cnt, C * sizeof(int));
    alloc((void**)&e->start, C * sizeof(int));
    alloc((void**)&e->partials, (size_t)frnn::scan_partials_count((int)C) * sizeof(int));
    alloc((void**)&e->counters, kCounterSlots * sizeof(unsigned long long));
    if (err == hipSuccess) err = hipHostMalloc((void**)&e->status_host, 64, hipHostMallocDefault);
    if (err == hipSuccess) err = hipHostGetDevicePointer((void**)&e->status_dev, e->status_host, 0);
    if (err == hipSuccess) *e->status_host = 0u;
    // engine-owned outputs sized max_points*128 as the reference (frnn_engine.cu:39-40)
    alloc((void**)&e->out_idx, P * FRNN_MAX_K * sizeof(int));
    alloc((void**)&e->out_dist, P * FRNN_MAX_K * sizeof(float));
    for (auto& ev : e->ev)
        if (err == hipSuccess) err = hipEventCreate(&ev);
    if (err != hipSuccess) {
        int st = hip_fail(err, "allocating engine workspace");
        release(e);
        delete e;
        return st;
    }
    *out = e;
    return FRNN_OK;
}

int frnn_engine_destroy(frnn_engine_t* e) {
    if (!e) return fail(FRNN_ERR_INVALID_ARGUMENT, "null engine");
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    else (void)hipDeviceSynchronize();
    release(e);
    delete e;
    return FRNN_OK;
}

int frnn_engine_max_points(const frnn_engine_t* e, int* out) {
    if (!e || !out) return fail(FRNN_ERR_INVALID_ARGUMENT, "null pointer");
    *out = e->max_p;
    return FRNN_OK;
}

int frnn_engine_set_stream(frnn_engine_t* e, void* stream) {
    if (!e) return fail(FRNN_ERR_INVALID_ARGUMENT, "null engine");
    e->stream = (hipStream_t)stream;
    return FRNN_OK;
}

int frnn_engine_search_gpu(frnn_engine_t* e, const float* d_pts, int N, int dim, int K, float radius,
                           int** d_idxs, float** d_dists) {
    if (!e) return fail(FRNN_ERR_INVALID_ARGUMENT, "null engine");
    ST_TRY(frnn_validate(e->max_p, N, dim, K, radius));
    if (!d_pts && N > 0) return fail(FRNN_ERR_INVALID_ARGUMENT, "null device points");
    ST_TRY(run_pipeline(e, d_pts, N, dim, K, radius));
    if (d_idxs) *d_idxs = e->out_idx;
    if (d_dists) *d_dists = e->out_dist;
    return FRNN_OK;
}

int frnn_engine_search_gpu_queries(frnn_engine_t* e, const float* d_pts, int N, const float* d_queries, int M,
                                   int dim, int K, float radius, int** d_idxs, float** d_dists) {
    if (!e) return fail(FRNN_ERR_INVALID_ARGUMENT, "null engine");
    ST_TRY(frnn_validate(e->max_p, N, dim, K, radius));
    if (M < 0) return fail(FRNN_ERR_INVALID_ARGUMENT, "M must be >= 0");
    if (M > e->max_p) return fail(FRNN_ERR_CAPACITY, "M exceeds max_points");
    if ((!d_pts && N > 0) || (!d_queries && M > 0)) return fail(FRNN_ERR_INVALID_ARGUMENT, "null device pointer");
    ST_TRY(run_pipeline(e, d_pts, N, dim, K, radius, true, d_queries, M));
    if (d_idxs) *d_idxs = e->out_idx;
    if (d_dists) *d_dists = e->out_dist;
    return FRNN_OK;
}

int frnn_engine_build(frnn_engine_t* e, const float* d_pts, int N, int dim, int K, float radius) {
    if (!e) return fail(FRNN_ERR_INVALID_ARGUMENT, "null engine");
    ST_TRY(frnn_validate(e->max_p, N, dim, K, radius));
    if (!d_pts && N > 0) return fail(FRNN_ERR_INVALID_ARGUMENT, "null device points");
    e->has_result = false;
    ST_TRY(build_points(e, e->built, d_pts, N, dim, K, radius));
    // the points' data now live in the engine's own buffers
    HIP_TRY(hipStreamSynchronize(e->stream), "grid build");
    return FRNN_OK;
}

int frnn_engine_query(frnn_engine_t* e, const float* d_queries, int M, int** d_idxs, float** d_dists) {
    if (!e) return fail(FRNN_ERR_INVALID_ARGUMENT, "null engine");
    if (!e->built.valid) return fail(FRNN_ERR_STATE, "query called before a grid was built");
    if (M < 0) return fail(FRNN_ERR_INVALID_ARGUMENT, "M must be >= 0");
    if (M > e->max_p) return fail(FRNN_ERR_CAPACITY, "M exceeds max_points");
    if (!d_queries && M > 0) return fail(FRNN_ERR_INVALID_ARGUMENT, "null device queries");
    e->last_plan = e->built.ref_plan;
    ST_TRY(run_queries(e, e->built, true, d_queries, M, true));
    if (d_idxs) *d_idxs = e->out_idx;
    if (d_dists) *d_dists = e->out_dist;
    return FRNN_OK;
}

int frnn_engine_search(frnn_engine_t* e, const float* h_pts, long long n_values, int K, float radius,
                       int* h_idxs, float* h_dists) {
    if (!e) return fail(FRNN_ERR_INVALID_ARGUMENT, "null engine");
    if (!h_pts || !h_idxs || !h_dists) return fail(FRNN_ERR_INVALID_ARGUMENT, "null host pointer");
    // frnn_engine.cu:108-109: dim = size / max_points, N = max_points
    if (n_values <= 0 || n_values % e->max_p != 0)
        return fail(FRNN_ERR_INVALID_ARGUMENT, "len(points) must be a positive multiple of max_points");
    const long long dimll = n_values / e->max_p;
    if (dimll > FRNN_MAX_DIM) return fail(FRNN_ERR_INVALID_ARGUMENT, "dim must be in [1, 128]");
    const int dim = (int)dimll;
    const int N = e->max_p;
    ST_TRY(frnn_validate(e->max_p, N, dim, K, radius));
    // AoS -> SoA on the host, then H2D (frnn_engine.cu:113-117)
    std::vector<float> soa((size_t)N * dim);
    for (int i = 0; i < N; ++i)
        for (int d = 0; d < dim; ++d) soa[(size_t)d * N + i] = h_pts[(size_t)i * dim + d];
    ST_TRY(grow(&e->h2d_points, &e->h2d_bytes, soa.size(), "allocating staging points"));
    HIP_TRY(hipMemcpyAsync(e->h2d_points, soa.data(), soa.size() * sizeof(float), hipMemcpyHostToDevice,
                           e->stream),
            "copying points to device");
    ST_TRY(run_pipeline(e, e->h2d_points, N, dim, K, radius));
    // D2H and SoA -> AoS (frnn_engine.cu:179-191)
    std::vector<int> ti((size_t)N * K);
    std::vector<float> td((size_t)N * K);
    HIP_TRY(hipMemcpy(ti.data(), e->out_idx, ti.size() * sizeof(int), hipMemcpyDeviceToHost),
            "copying indices to host");
    HIP_TRY(hipMemcpy(td.data(), e->out_dist, td.size() * sizeof(float), hipMemcpyDeviceToHost),
            "copying distances to host");
    for (int k = 0; k < K; ++k)
        for (int i = 0; i < N; ++i) {
            h_idxs[(size_t)i * K + k] = ti[(size_t)k * N + i];
            h_dists[(size_t)i * K + k] = td[(size_t)k * N + i];
        }
    return FRNN_OK;
}

int frnn_engine_get_results(frnn_engine_t* e, int N, int K, int* h_idxs, float* h_dists) {
    if (!e) return fail(FRNN_ERR_INVALID_ARGUMENT, "null engine");
    if (!e->has_result) return fail(FRNN_ERR_STATE, "get_results called before search_gpu");
    if (N < 0 || K < 0) return fail(FRNN_ERR_INVALID_ARGUMENT, "N and K must be >= 0");
    const size_t n = (size_t)N * (size_t)K;
    if (n > (size_t)e->max_p * FRNN_MAX_K) return fail(FRNN_ERR_CAPACITY, "N*K exceeds the output buffers");
    if (n == 0) return FRNN_OK;
    if (!h_idxs || !h_dists) return fail(FRNN_ERR_INVALID_ARGUMENT, "null host pointer");
    HIP_TRY(hipMemcpy(h_idxs, e->out_idx, n * sizeof(int), hipMemcpyDeviceToHost), "copying indices");
    HIP_TRY(hipMemcpy(h_dists, e->out_dist, n * sizeof(float), hipMemcpyDeviceToHost), "copying distances");
    return FRNN_OK;
}

int frnn_engine_last_plan(const frnn_engine_t* e, frnn_plan_t* out) {
    if (!e || !out) return fail(FRNN_ERR_INVALID_ARGUMENT, "null pointer");
    *out = e->last_plan;
    return FRNN_OK;
}

int frnn_engine_set_profiling(frnn_engine_t* e, int flags) {
    if (!e) return fail(FRNN_ERR_INVALID_ARGUMENT, "null engine");
    if (flags & ~(FRNN_PROFILE_EVENTS | FRNN_PROFILE_COUNTERS | FRNN_PROFILE_SEARCH_EVENTS))
        return fail(FRNN_ERR_INVALID_ARGUMENT, "unknown profiling flags");
    e->profiling = (flags & FRNN_PROFILE_EVENTS) != 0;
    e->search_events = (flags & FRNN_PROFILE_SEARCH_EVENTS) != 0;
    e->counting = (flags & FRNN_PROFILE_COUNTERS) != 0;
    return FRNN_OK;
}

int frnn_engine_stage_times(const frnn_engine_t* e, float* ms, int n) {
    if (!e || !ms) return fail(FRNN_ERR_INVALID_ARGUMENT, "null pointer");
    for (int i = 0; i < n && i < FRNN_NUM_STAGES; ++i) ms[i] = e->stage_ms[i];
    return FRNN_OK;
}

int frnn_engine_counters(const frnn_engine_t* e, long long* out, int n) {
    if (!e || !out) return fail(FRNN_ERR_INVALID_ARGUMENT, "null pointer");
    for (int i = 0; i < n && i < FRNN_NUM_COUNTERS; ++i) out[i] = e->ctr[i];
    return FRNN_OK;
}

int frnn_engine_count_work(const frnn_engine_t* e, long long* out, int n) {
    if (!e || !out) return fail(FRNN_ERR_INVALID_ARGUMENT, "null pointer");
    const long long w[2] = {e->last_fill, e->last_scan > 0 ? (long long)e->status_host[4] + 1 : 0};
    for (int i = 0; i < n && i < 2; ++i) out[i] = w[i];
    return FRNN_OK;
}

// ---- kernel launch seam ----------------------------------------------------

long long frnn_grid_cells(int N, int dim, const frnn_plan_t* plan) {
    if (!plan || N < 0 || dim < 1 || dim > FRNN_MAX_DIM) return -1;
    if (plan->path != FRNN_PATH_GRID_FIRST && plan->path != FRNN_PATH_GRID_FULL) return 0;
    return frnn::grid_cells(N, dim, *plan);
}

int frnn_launch_bin_count(const float* d_pts, int N, int grid_dim, int res, float inv_cell, long long cells,
                          const void* d_frame_ws, int* d_cell_of, int* d_rank, int* d_cnt, void* stream) {
    if (N < 0 || grid_dim < 1 || grid_dim > 9 || res < 1 || cells < 1 ||
        cells > (d_frame_ws ? (long long)frnn::kFine0 * FRNN_MAX_CELLS : FRNN_MAX_CELLS))
        return fail(FRNN_ERR_INVALID_ARGUMENT, "bad bin/count geometry");
    if (!d_frame_ws && ipow_sat(res, grid_dim, (long long)4e18) != cells)
        return fail(FRNN_ERR_INVALID_ARGUMENT, "cells must equal res^grid_dim");
    if (d_frame_ws && grid_dim > 4) return fail(FRNN_ERR_INVALID_ARGUMENT, "a frame has at most 4 grid axes");
    if (N > 0 && (!d_pts || !d_cell_of || !d_rank || !d_cnt))
        return fail(FRNN_ERR_INVALID_ARGUMENT, "null device pointer");
    hipStream_t s = (hipStream_t)stream;
    ST_TRY(launch_status(frnn::launch_fill_i32(d_cnt, cells + 1, 0, s), "zero-fill cells"));
    return launch_status(frnn::launch_bin_count(d_pts, N, grid_dim, res, inv_cell, d_frame_ws, (int)cells,
                                                d_cell_of, d_rank, d_cnt, s),
                         "bin/count launch");
}

int frnn_launch_exclusive_scan(const int* d_in, int n, int* d_out, int* d_partials, void* stream) {
    if (n < 0) return fail(FRNN_ERR_INVALID_ARGUMENT, "n must be >= 0");
    if (n > 0 && (!d_in || !d_out || !d_partials)) return fail(FRNN_ERR_INVALID_ARGUMENT, "null device pointer");
    return launch_status(frnn::launch_exclusive_scan(d_in, n, d_out, d_partials, (hipStream_t)stream),
                         "scan launch");
}

int frnn_launch_exclusive_scan_noalloc(const int* d_in, int n, int* d_out, void* stream) {
    if (n < 0) return fail(FRNN_ERR_INVALID_ARGUMENT, "n must be >= 0");
    if (n > frnn::scan_noalloc_max())
        return fail(FRNN_ERR_CAPACITY, "n exceeds FRNN_SCAN_NOALLOC_MAX_N (16777216 = 4096 tiles of 4096 ints; "
                                       "the partial sums live in a fixed 16 KB device scratch)");
    if (n > 0 && (!d_in || !d_out)) return fail(FRNN_ERR_INVALID_ARGUMENT, "null device pointer");
    const int rc = frnn::launch_exclusive_scan_noalloc(d_in, n, d_out, (hipStream_t)stream);
    if (rc == 4) return hip_fail(frnn::scan_noalloc_error(), "looking up the scan scratch's device address");
    return launch_status(rc, "allocation-free scan launch");
}

long long frnn_stats_workspace_bytes(int dim) {
    if (dim < 1 || dim > FRNN_MAX_DIM) return -1;
    return (long long)frnn::stats_layout(dim).total;
}

int frnn_launch_point_stats(const float* d_pts, int N, int dim, void* d_stats_ws, void* stream) {
    if (N < 0 || dim < 1 || dim > FRNN_MAX_DIM) return fail(FRNN_ERR_INVALID_ARGUMENT, "bad N or dim");
    if (N > 0 && (!d_pts || !d_stats_ws)) return fail(FRNN_ERR_INVALID_ARGUMENT, "null device pointer");
    return launch_status(frnn::launch_point_stats(d_pts, N, dim, d_stats_ws, (hipStream_t)stream),
                         "statistics launch");
}

long long frnn_frame_workspace_bytes(int N, int dim, const frnn_plan_t* plan) {
    if (!plan || N < 0 || dim < 1 || dim > FRNN_MAX_DIM) return -1;
    if (N == 0 || !frnn::has_frame(*plan, dim)) return 0;
    return (long long)frnn::frame_layout().total;
}

static int check_frame_plan(int N, int dim, const frnn_plan_t* plan) {
    if (!plan || N < 0 || dim < 1 || dim > FRNN_MAX_DIM) return fail(FRNN_ERR_INVALID_ARGUMENT, "bad N, dim or plan");
    if (!frnn::has_frame(*plan, dim)) return fail(FRNN_ERR_INVALID_ARGUMENT, "the plan has no frame");
    if (plan->grid_dim < 1 || plan->grid_dim > 4 || plan->res < 1 || plan->cells < 1 ||
        plan->cells > FRNN_MAX_CELLS || ipow_sat(plan->res, plan->grid_dim, (long long)4e18) != plan->cells)
        return fail(FRNN_ERR_INVALID_ARGUMENT, "inconsistent grid plan");
    return FRNN_OK;
}

int frnn_launch_frame(const float* d_pts, int N, int dim, const frnn_plan_t* plan, const void* d_stats_ws,
                      void* d_frame_ws, void* stream) {
    ST_TRY(check_frame_plan(N, dim, plan));
    if (N == 0) return FRNN_OK;
    if (!d_pts || !d_frame_ws || (frnn::has_projected_frame(*plan, dim) && !d_stats_ws))
        return fail(FRNN_ERR_INVALID_ARGUMENT, "null device pointer");
    return launch_status(frnn::launch_frame(d_pts, N, dim, *plan, frnn::grid_cells(N, dim, *plan), d_stats_ws,
                                            d_frame_ws, (hipStream_t)stream),
                         "frame launch");
}

int frnn_uses_filter_rows(int dim) {
    if (dim < 1 || dim > FRNN_MAX_DIM) return -1;
    return frnn::uses_filter_rows(dim) ? 1 : 0;
}

int frnn_launch_reorder(const float* d_pts, int N, int dim, const int* d_cell_of, const int* d_rank,
                        const int* d_start, int* d_sorted_idx, int* d_inv, float* d_sorted_aos,
                        const void* d_stats_ws, float* d_frows, void* stream) {
    if (N < 0 || dim < 1 || dim > FRNN_MAX_DIM) return fail(FRNN_ERR_INVALID_ARGUMENT, "bad N or dim");
    if (N > 0 && (!d_pts || !d_cell_of || !d_rank || !d_start || !d_sorted_idx || !d_inv || !d_sorted_aos))
        return fail(FRNN_ERR_INVALID_ARGUMENT, "null device pointer");
    if (d_frows && !d_stats_ws) return fail(FRNN_ERR_INVALID_ARGUMENT, "filter rows need the statistics");
    return launch_status(frnn::launch_reorder(d_pts, N, dim, d_cell_of, d_rank, d_start, d_sorted_idx, d_inv,
                                              d_sorted_aos, d_stats_ws, d_frows, (hipStream_t)stream),
                         "reorder launch");
}

int frnn_launch_transpose(const float* d_pts, int N, int dim, float* d_aos, const void* d_stats_ws,
                          float* d_frows, void* stream) {
    if (N < 0 || dim < 1 || dim > FRNN_MAX_DIM) return fail(FRNN_ERR_INVALID_ARGUMENT, "bad N or dim");
    if (N > 0 && (!d_pts || !d_aos)) return fail(FRNN_ERR_INVALID_ARGUMENT, "null device pointer");
    if (d_frows && !d_stats_ws) return fail(FRNN_ERR_INVALID_ARGUMENT, "filter rows need the statistics");
    return launch_status(frnn::launch_transpose(d_pts, N, dim, d_aos, d_stats_ws, d_frows, (hipStream_t)stream),
                         "transpose launch");
}

int frnn_launch_find_nbrs(const float* d_aos, const float* d_frows, const void* d_stats_ws,
                          const int* d_sorted_idx, const int* d_cell_of, const int* d_start,
                          const void* d_frame_ws, int N, int dim, int K, const frnn_plan_t* plan,
                          const frnn_queries_t* queries, unsigned long long* d_lists, int list_cap,
                          unsigned long long* d_counters, unsigned int* d_status, void* stream) {
    if (!plan) return fail(FRNN_ERR_INVALID_ARGUMENT, "null plan");
    ST_TRY(frnn_validate(0, N, dim, K, plan->cell_size));
    if (queries && queries->M < 0) return fail(FRNN_ERR_INVALID_ARGUMENT, "queries->M must be >= 0");
    if (plan->path == FRNN_PATH_EMPTY || N == 0 || (queries && queries->M == 0)) return FRNN_OK;
    if (list_cap < K) return fail(FRNN_ERR_INVALID_ARGUMENT, "list_cap must be >= K");
    const bool grid = plan->path != FRNN_PATH_BRUTEFORCE;
    if (!d_aos || !d_stats_ws || !d_lists || (grid && (!d_sorted_idx || !d_cell_of || !d_start)))
        return fail(FRNN_ERR_INVALID_ARGUMENT, "null device pointer");
    if (frnn::uses_filter_rows(dim) && !d_frows)
        return fail(FRNN_ERR_INVALID_ARGUMENT, "this dimension needs the centred filter rows");
    if (queries && (!queries->d_aos || (grid && (!queries->d_sorted_idx || !queries->d_cell_of)) ||
                    (frnn::uses_filter_rows(dim) && !queries->d_frows)))
        return fail(FRNN_ERR_INVALID_ARGUMENT, "null query pointer");
    if (grid && (plan->grid_dim < 1 || plan->grid_dim > 9 || plan->grid_dim > dim || plan->res < 1 ||
                 ipow_sat(plan->res, plan->grid_dim, (long long)4e18) != plan->cells ||
                 plan->cells > FRNN_MAX_CELLS))
        return fail(FRNN_ERR_INVALID_ARGUMENT, "inconsistent grid plan");
    if (plan->rev_order && (!grid || dim != 3)) return fail(FRNN_ERR_INVALID_ARGUMENT, "reversed order is D=3 grid only");
    if (d_frame_ws && !frnn::has_frame(*plan, dim))
        return fail(FRNN_ERR_INVALID_ARGUMENT, "a frame given for a plan without one");
    frnn::QuerySet qs{};
    if (queries)
        qs = frnn::QuerySet{queries->d_aos, queries->d_frows, grid ? queries->d_sorted_idx : nullptr,
                            grid ? queries->d_cell_of : nullptr, queries->M};
    return launch_status(frnn::launch_search(d_aos, d_frows, d_stats_ws, d_sorted_idx, d_cell_of, d_start,
                                             d_frame_ws, N, dim, K, *plan, d_lists, list_cap, d_counters,
                                             d_status, (hipStream_t)stream, queries ? &qs : nullptr),
                         "search launch");
}

int frnn_launch_unpermute(const unsigned long long* d_lists, int list_cap, const int* d_inv, int N, int K,
                          int* d_idxs, float* d_dists, void* stream) {
    if (N < 0 || K < 1 || K > FRNN_MAX_K || list_cap < K)
        return fail(FRNN_ERR_INVALID_ARGUMENT, "bad N, K or list_cap");
    if (N > 0 && (!d_lists || !d_idxs || !d_dists)) return fail(FRNN_ERR_INVALID_ARGUMENT, "null device pointer");
    return launch_status(frnn::launch_unpermute(d_lists, list_cap, d_inv, N, K, d_idxs, d_dists,
                                                (hipStream_t)stream),
                         "unpermute launch");
}

}  // extern "C"
