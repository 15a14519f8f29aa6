// frnn_oracle.cpp -- CPU restatement of the reference FRNN algorithm.
//
// TEST INFRASTRUCTURE ONLY.  This file is the parity oracle and the CPU
// baseline ("port") for bench.py.  Only tests/, __graft_entry__.smoke() and
// bench.py's cpu_baseline leg may load it; the product library never does.
//
// What it restates (reference = /root/reference):
//   * dispatch          python_interface/frnn_engine.cu:201-246 and :64-86
//   * binning / hash    frnn/csrc/grid/insert_points.cu:64-80, grid.h:73-81
//   * 3^g cell shell    frnn/csrc/grid/find_nbrs.cu:167-187 (full-D grid),
//                       :288-304 (first-coordinate grid), :439-465 (D=3 grid)
//   * distance order    find_nbrs.cu:474-477 (D=3 grid: fma(dx,dx,fma(dy,dy,dz*dz)))
//                       find_nbrs.cu:194-199, :335-340 (sequential fma d=0..D-1)
//   * in-radius test    strict d2 < r2 with r2 = fl(radius*radius)
//                       (find_nbrs.cu:550,571,603; no_grid_frnn.cu:195,329)
//   * padding           (dist=r2, idx=-1)  (find_nbrs.cu:136-143; no_grid_frnn.cu:169)
//
// Deliberate semantic choices shared with the HIP engine (documented there too):
//   * binned coordinates are clamped to [0,res-1] for every point (the
//     reference drops out-of-domain points from the database, insert_points.cu:74-87,
//     and leaves their output rows undefined);
//   * the K results of a query are the K smallest (d2, idx) pairs in lexicographic
//     order, written in ascending order (the reference keeps heap order and breaks
//     ties by atomic arrival order, find_nbrs.cu:77-97, insert_points.cu:158);
//   * brute force uses the sequential-fma order (the reference's float4 grouping
//     at no_grid_frnn.cu:84-106 leaves contraction to the compiler).
//
// Build: see oracle/Makefile (g++ -O3 -mfma -fopenmp -ffp-contract=off).

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>
#include <omp.h>

namespace {

enum Path { PATH_EMPTY = -1, PATH_BF = 0, PATH_GRID_FULL = 1, PATH_GRID_FIRST = 2 };

struct Plan {
    int path;
    int g;          // grid dims (0 for brute force)
    int res;        // cells per grid axis
    long long cells;
    int rev;        // 1 -> D=3 grid order fma(dx,dx,fma(dy,dy,dz*dz))
    float r2;
    float inv_cell;
};

long long ipow_sat(long long b, int e, long long cap) {
    long long v = 1;
    for (int i = 0; i < e; ++i) {
        if (v > cap / (b > 0 ? b : 1)) return cap + 1;
        v *= b;
    }
    return v;
}

// frnn_engine.cu:201-246 (search_gpu) and :64-86 (run_firstd_search).
Plan make_plan(int N, int D, int K, float radius) {
    Plan p{};
    p.r2 = radius * radius;
    if (N <= 0) { p.path = PATH_EMPTY; return p; }
    const float cs = radius;
    const float cr = std::ceil((1.0f - 0.0f) / cs);
    const int res = cr >= 1073741824.0f ? 1073741824 : (int)cr;   // avoid int overflow at tiny radii
    const double total_d = std::pow((double)res, D);
    const bool feasible = total_d <= 1000000.0;
    const long long total = feasible ? (long long)total_d : 0;

    const long long kBF = 2000000LL;
    const long long sel = std::max(1LL, (long long)(K + 7) / 8);
    const long long db = ((long long)N * D > kBF) ? (kBF + 1LL) : (long long)N * D;
    const bool use_bf = (db <= kBF / sel) && ((long long)N <= kBF / (db * sel));
    const long long shell = ipow_sat(3, D, (long long)4e18);

    if (use_bf) { p.path = PATH_BF; return p; }
    if (res <= 1 || !feasible || shell >= total) {
        const int g = (D > 4) ? 4 : std::min(D, 3);
        const int r2res = std::max(res, 2);
        const double tc = std::pow((double)r2res, g);
        if (tc > 1000000.0) { p.path = PATH_BF; return p; }
        const long long gshell = ipow_sat(3, g, (long long)4e18);
        if (gshell >= (long long)tc) { p.path = PATH_BF; return p; }
        p.path = PATH_GRID_FIRST; p.g = g; p.res = r2res; p.cells = (long long)tc;
        p.inv_cell = 1.0f / cs; p.rev = 0;
        return p;
    }
    p.path = PATH_GRID_FULL; p.g = D; p.res = res; p.cells = total;
    p.inv_cell = 1.0f / cs; p.rev = (D == 3) ? 1 : 0;
    return p;
}

inline int bin_coord(float x, float inv_cell, int res) {
    // insert_points.cu:72 floorf((pos - min_val) * inv_cell) with min_val = 0,
    // clamped to [0,res-1] (the reference drops points outside instead).
    float t = x * inv_cell;
    float f = std::floor(t);
    f = std::fmax(f, 0.0f);              // NaN -> 0
    f = std::fmin(f, (float)(res - 1));
    return (int)f;
}

inline float dist2_fwd(const float* q, const float* p, int D) {
    float acc = 0.0f;
    for (int d = 0; d < D; ++d) {
        float diff = q[d] - p[d];
        acc = std::fma(diff, diff, acc);
    }
    return acc;
}

inline float dist2_rev(const float* q, const float* p, int D) {
    float acc = 0.0f;
    for (int d = D - 1; d >= 0; --d) {
        float diff = q[d] - p[d];
        acc = std::fma(diff, diff, acc);
    }
    return acc;
}

struct Cand { float d2; int idx; };
inline bool cand_less(const Cand& a, const Cand& b) {
    return a.d2 < b.d2 || (a.d2 == b.d2 && a.idx < b.idx);
}

struct Grid {
    std::vector<int> cell_of;   // per original point
    std::vector<int> start;     // cells+1 exclusive scan
    std::vector<int> order;     // sorted position -> original index (stable)
    std::vector<float> aos;     // AoS coords in original order [i*D + d]
};

void build_grid(const float* soa, int N, const Plan& p, Grid& G) {
    G.cell_of.assign(N, 0);
    G.start.assign((size_t)p.cells + 1, 0);
    for (int i = 0; i < N; ++i) {
        long long h = 0, s = 1;
        for (int d = 0; d < p.g; ++d) {
            h += (long long)bin_coord(soa[(size_t)d * N + i], p.inv_cell, p.res) * s;
            s *= p.res;
        }
        G.cell_of[i] = (int)h;
        G.start[h + 1]++;
    }
    for (long long c = 0; c < p.cells; ++c) G.start[c + 1] += G.start[c];
    std::vector<int> fill(G.start.begin(), G.start.end() - 1);
    G.order.assign(N, 0);
    for (int i = 0; i < N; ++i) G.order[fill[G.cell_of[i]]++] = i;
}

void to_aos(const float* soa, int N, int D, std::vector<float>& aos) {
    aos.assign((size_t)N * D, 0.0f);
    for (int d = 0; d < D; ++d)
        for (int i = 0; i < N; ++i) aos[(size_t)i * D + d] = soa[(size_t)d * N + i];
}

void finish_row(std::vector<Cand>& c, int K, float r2, int* idx_row, float* dist_row, int stride) {
    const size_t keep = std::min((size_t)K, c.size());
    std::partial_sort(c.begin(), c.begin() + keep, c.end(), cand_less);
    for (int k = 0; k < K; ++k) {
        if ((size_t)k < keep) { idx_row[(size_t)k * stride] = c[k].idx; dist_row[(size_t)k * stride] = c[k].d2; }
        else { idx_row[(size_t)k * stride] = -1; dist_row[(size_t)k * stride] = r2; }
    }
}

void query_bf(const std::vector<float>& aos, int N, int D, const float* q, float r2, std::vector<Cand>& c) {
    c.clear();
    for (int j = 0; j < N; ++j) {
        float e = dist2_fwd(q, &aos[(size_t)j * D], D);
        if (e < r2) c.push_back({e, j});
    }
}

void query_grid(const std::vector<float>& aos, int D, const Plan& p, const Grid& G, const float* q,
                std::vector<Cand>& c) {
    int qc[16];
    for (int d = 0; d < p.g; ++d) qc[d] = bin_coord(q[d], p.inv_cell, p.res);
    long long nshell = 1;
    for (int d = 0; d < p.g; ++d) nshell *= 3;
    c.clear();
    for (long long t = 0; t < nshell; ++t) {
        long long tmp = t, h = 0, s = 1;
        bool ok = true;
        for (int d = 0; d < p.g; ++d) {
            int cc = qc[d] + (int)(tmp % 3) - 1;
            tmp /= 3;
            if (cc < 0 || cc >= p.res) { ok = false; break; }
            h += (long long)cc * s;
            s *= p.res;
        }
        if (!ok) continue;
        for (int sp = G.start[h]; sp < G.start[h + 1]; ++sp) {
            const int j = G.order[sp];
            const float* pt = &aos[(size_t)j * D];
            float e = p.rev ? dist2_rev(q, pt, D) : dist2_fwd(q, pt, D);
            if (e < p.r2) c.push_back({e, j});
        }
    }
}

}  // namespace

extern "C" {

// plan_out[6] = {path, grid_dim, res, cells, rev, 0}
int oracle_plan(int N, int D, int K, float radius, long long* plan_out) {
    Plan p = make_plan(N, D, K, radius);
    plan_out[0] = p.path; plan_out[1] = p.g; plan_out[2] = p.res;
    plan_out[3] = p.cells; plan_out[4] = p.rev; plan_out[5] = 0;
    return 0;
}

// Clamped cell id of every point for a grid on the first `g` coordinates.
void oracle_bin(const float* soa, int N, int g, int res, float inv_cell, int* cell_out) {
    for (int i = 0; i < N; ++i) {
        long long h = 0, s = 1;
        for (int d = 0; d < g; ++d) {
            h += (long long)bin_coord(soa[(size_t)d * N + i], inv_cell, res) * s;
            s *= res;
        }
        cell_out[i] = (int)h;
    }
}

// order: 0 = sequential fma d=0..D-1, 1 = reversed (the D=3 grid order)
float oracle_dist2(const float* q, const float* p, int D, int order) {
    return order ? dist2_rev(q, p, D) : dist2_fwd(q, p, D);
}

// Full search with the reference dispatch (force_path < 0) or a forced path
// (0 = brute force with the fwd order, 1/2 = the planned grid; forcing a grid
// on a brute-force plan is an error).
// query_ids == NULL: all N queries, output SoA [k*N + i] (the engine layout).
// query_ids != NULL: nq selected queries, output rows [j*K + k].
// timings (may be NULL): [0] = build seconds, [1] = search seconds.
int oracle_search(const float* soa, int N, int D, int K, float radius, int force_path,
                  int nthreads, const int* query_ids, int nq,
                  int* idx_out, float* dist_out, double* timings) {
    if (N <= 0 || D <= 0 || K <= 0) return 1;
    Plan p = make_plan(N, D, K, radius);
    if (force_path == PATH_BF) { p.path = PATH_BF; p.rev = 0; }
    else if (force_path > 0 && p.path == PATH_BF) return 2;
    if (nthreads > 0) omp_set_num_threads(nthreads);

    auto t0 = std::chrono::steady_clock::now();
    std::vector<float> aos;
    to_aos(soa, N, D, aos);
    Grid G;
    if (p.path != PATH_BF) build_grid(soa, N, p, G);
    auto t1 = std::chrono::steady_clock::now();

    const bool all = (query_ids == nullptr);
    const int Q = all ? N : nq;
#pragma omp parallel
    {
        std::vector<Cand> c;
#pragma omp for schedule(dynamic, 16)
        for (int j = 0; j < Q; ++j) {
            const int qi = all ? j : query_ids[j];
            const float* q = &aos[(size_t)qi * D];
            if (p.path == PATH_BF) query_bf(aos, N, D, q, p.r2, c);
            else query_grid(aos, D, p, G, q, c);
            if (all) finish_row(c, K, p.r2, idx_out + qi, dist_out + qi, N);
            else finish_row(c, K, p.r2, idx_out + (size_t)j * K, dist_out + (size_t)j * K, 1);
        }
    }
    auto t2 = std::chrono::steady_clock::now();
    if (timings) {
        timings[0] = std::chrono::duration<double>(t1 - t0).count();
        timings[1] = std::chrono::duration<double>(t2 - t1).count();
    }
    return 0;
}

// Queries distinct from the points: the reference kernels' two-array form
// (run_find_nbrs with d_points1 != d_points2, find_nbrs.cu:562-567;
// run_bruteforce with p1 != p2, no_grid_frnn.cu:273-276).  The plan and the
// grid are the points' own (N points); every query is binned with the same
// parameters and scans its 3^g shell of the points' grid, or all N points on
// a brute-force plan.  Output rows [j*K + k] for the M queries.
int oracle_search_queries(const float* soa_p, int N, const float* soa_q, int M, int D, int K, float radius,
                          int force_path, int nthreads, int* idx_out, float* dist_out) {
    if (N <= 0 || M < 0 || D <= 0 || K <= 0) return 1;
    Plan p = make_plan(N, D, K, radius);
    if (force_path == PATH_BF) { p.path = PATH_BF; p.rev = 0; }
    else if (force_path > 0 && p.path == PATH_BF) return 2;
    if (nthreads > 0) omp_set_num_threads(nthreads);
    std::vector<float> aos, qaos;
    to_aos(soa_p, N, D, aos);
    to_aos(soa_q, M, D, qaos);
    Grid G;
    if (p.path != PATH_BF) build_grid(soa_p, N, p, G);
#pragma omp parallel
    {
        std::vector<Cand> c;
#pragma omp for schedule(dynamic, 16)
        for (int j = 0; j < M; ++j) {
            const float* q = &qaos[(size_t)j * D];
            if (p.path == PATH_BF) query_bf(aos, N, D, q, p.r2, c);
            else query_grid(aos, D, p, G, q, c);
            finish_row(c, K, p.r2, idx_out + (size_t)j * K, dist_out + (size_t)j * K, 1);
        }
    }
    return 0;
}

// Number of shell candidates (points in the 3^g cells around each query, no
// pruning) summed over the given queries; the work measure used for the grid
// search roofline.  Returns -1 for brute-force plans.
long long oracle_shell_candidates(const float* soa, int N, int D, int K, float radius,
                                  const int* query_ids, int nq) {
    Plan p = make_plan(N, D, K, radius);
    if (p.path == PATH_BF || p.path == PATH_EMPTY) return -1;
    Grid G;
    build_grid(soa, N, p, G);
    long long total = 0;
    const bool all = (query_ids == nullptr);
    const int Q = all ? N : nq;
    long long nshell = 1;
    for (int d = 0; d < p.g; ++d) nshell *= 3;
#pragma omp parallel for reduction(+ : total) schedule(dynamic, 256)
    for (int j = 0; j < Q; ++j) {
        const int qi = all ? j : query_ids[j];
        int qc[16];
        for (int d = 0; d < p.g; ++d) qc[d] = bin_coord(soa[(size_t)d * N + qi], p.inv_cell, p.res);
        for (long long t = 0; t < nshell; ++t) {
            long long tmp = t, h = 0, s = 1;
            bool ok = true;
            for (int d = 0; d < p.g; ++d) {
                int cc = qc[d] + (int)(tmp % 3) - 1;
                tmp /= 3;
                if (cc < 0 || cc >= p.res) { ok = false; break; }
                h += (long long)cc * s;
                s *= p.res;
            }
            if (ok) total += G.start[h + 1] - G.start[h];
        }
    }
    return total;
}

}  // extern "C"
