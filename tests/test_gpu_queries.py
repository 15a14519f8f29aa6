"""Separate queries through the engine (GPU): M query points against N points,
the reference kernels' two-array form (find_nbrs.cu:562-567,
no_grid_frnn.cu:273-276), compared bit-exactly with the oracle's
search_queries on every path."""
import numpy as np
import pytest

import frnn_cuda
import frnn_oracle as O
import frnn_workloads as W
from gpu_util import assert_rows_equal, device_soa, log
from test_oracle_pins import CASES, separate_queries, unit_cloud

pytestmark = pytest.mark.gpu


def engine_search_queries(P, Q, K, radius, engine=None):
    """search_gpu_queries on AoS P[N, D] and Q[M, D]; returns ([M, K] idx, [M, K] dist, plan)."""
    P = np.asarray(P, dtype=np.float32)
    Q = np.asarray(Q, dtype=np.float32)
    N, D = P.shape
    M = Q.shape[0]
    eng = engine or frnn_cuda.FRNNEngine(max_points=max(N, M, 1))
    dp = device_soa(P)
    dq = device_soa(Q) if M else dp
    eng.search_gpu_queries(dp.data_ptr(), N, dq.data_ptr(), M, D, K, radius)
    idx, dist = eng.get_results_numpy(M, K)
    plan = eng.last_plan()
    if engine is None:
        eng.close()
    return idx.reshape(K, M).T.copy(), dist.reshape(K, M).T.copy(), plan


@pytest.mark.parametrize("label,D,k,N,r,K,path", CASES)
def test_queries_match_oracle(label, D, k, N, r, K, path):
    X = unit_cloud(N, D, k, 11)
    X[7] = X[3]
    Q = separate_queries(X, 700, 5)
    log(f"queries {label}: N={N} M={len(Q)} D={D} K={K} r={r}")
    gi, gd, plan = engine_search_queries(X, Q, K, r)
    assert plan["path"] == path
    ri, rd = O.search_queries(X, Q, K, r)
    assert_rows_equal(gi, gd, ri, rd, f"queries {label}")


@pytest.mark.parametrize("M", [1, 31, 33, 5000])
def test_query_counts_and_reuse(M):
    # fewer and more queries than points, on one engine reused across calls
    X = unit_cloud(3000, 12, 3, 21)
    eng = frnn_cuda.FRNNEngine(max_points=5000)
    Q = separate_queries(X, M, 6) if M > 1 else X[:1] + np.float32(0.001)
    log(f"query counts M={M}")
    for K, r in ((16, 0.1), (32, 0.15)):
        gi, gd, _ = engine_search_queries(X, Q, K, r, engine=eng)
        ri, rd = O.search_queries(X, Q, K, r)
        assert_rows_equal(gi, gd, ri, rd, f"M={M} K={K}")
    eng.close()


def test_queries_equal_to_points_give_the_all_points_rows():
    X = unit_cloud(4000, 16, 4, 22)
    gi, gd, _ = engine_search_queries(X, X, 32, 0.2)
    eng = frnn_cuda.FRNNEngine(max_points=4000)
    d = device_soa(X)
    eng.search_gpu(d.data_ptr(), 4000, 16, 32, 0.2)
    ai, ad = eng.get_results_numpy(4000, 32)
    eng.close()
    assert np.array_equal(gi, ai.reshape(32, 4000).T)
    assert np.array_equal(gd.view(np.uint32), ad.reshape(32, 4000).T.view(np.uint32))


def test_empty_query_and_point_sets():
    X = unit_cloud(500, 3, 3, 23)
    eng = frnn_cuda.FRNNEngine(max_points=500)
    dp = device_soa(X)
    # no queries (also with a null query pointer): nothing to return, and no
    # all-points search in their place
    eng.search_gpu_queries(dp.data_ptr(), 500, dp.data_ptr(), 0, 3, 8, 0.1)
    assert eng.get_results_numpy(0, 8)[0].size == 0
    Q = separate_queries(X, 500, 11)
    dq = device_soa(Q)
    eng.search_gpu_queries(dp.data_ptr(), 500, dq.data_ptr(), 500, 3, 8, 0.1)
    before = eng.get_results_numpy(500, 8)
    eng.search_gpu_queries(dp.data_ptr(), 500, 0, 0, 3, 8, 0.1)
    eng.query(0, 0)
    after = eng.get_results_numpy(500, 8)          # the output buffers, untouched
    assert np.array_equal(before[0], after[0]) and np.array_equal(before[1], after[1])
    # no points: every query row is padding (r2, -1)
    eng.search_gpu_queries(dp.data_ptr(), 0, dp.data_ptr(), 500, 3, 8, 0.1)
    idx, dist = eng.get_results_numpy(500, 8)
    assert np.all(idx == -1) and np.all(dist == np.float32(np.float32(0.1) * np.float32(0.1)))
    with pytest.raises(ValueError, match="max_points"):
        eng.search_gpu_queries(dp.data_ptr(), 500, dp.data_ptr(), 501, 3, 8, 0.1)
    eng.close()


def test_metric_points_with_separate_queries_sampled():
    # the headline point set with 20 000 queries near its points
    w = W.config("metric")
    rs = np.random.RandomState(77)
    Q = w.X[rs.randint(0, w.N, 20000)] + (0.003 * rs.standard_normal((20000, 16))).astype(np.float32)
    log(f"metric points N={w.N} with M={len(Q)} separate queries")
    gi, gd, plan = engine_search_queries(w.X, Q, w.K, w.radius)
    assert plan["path"] == "grid_first"
    sel = np.sort(np.random.RandomState(3).choice(len(Q), 400, replace=False))
    ri, rd = O.search_queries(w.X, Q[sel], w.K, w.radius)
    assert_rows_equal(gi[sel], gd[sel], ri, rd, "metric queries sampled")


@pytest.mark.parametrize("label,D,k,N,r,K,path", [c for c in CASES if c[0] in
                                                  ("full_d3_rev", "first_d16", "full_d5", "bf_d16")])
def test_grid_reuse_across_query_sets(label, D, k, N, r, K, path):
    """build() once, then query() several query sets against the same grid;
    the input points are overwritten after the build (the grid owns a copy)."""
    X = unit_cloud(N, D, k, 11)
    eng = frnn_cuda.FRNNEngine(max_points=2000)
    dp = device_soa(X)
    eng.build(dp.data_ptr(), N, D, K, r)
    dp.fill_(float("nan"))
    assert eng.last_plan()["path"] == path
    for seed, M in ((5, 700), (6, 1), (7, 2000), (8, 0)):
        Q = separate_queries(X, M, seed) if M > 1 else X[:M] + np.float32(0.001)
        log(f"reuse {label}: query set M={M}")
        dq = device_soa(Q) if M else device_soa(X[:1])
        eng.query(dq.data_ptr(), M)
        gi, gd = eng.get_results_numpy(M, K)
        ri, rd = O.search_queries(X, Q, K, r)
        assert_rows_equal(gi.reshape(K, M).T, gd.reshape(K, M).T, ri, rd, f"reuse {label} M={M}")
    eng.close()


def test_query_before_build_and_after_search():
    X = unit_cloud(1500, 12, 3, 24)
    eng = frnn_cuda.FRNNEngine(max_points=1500)
    d = device_soa(X)
    with pytest.raises(frnn_cuda.FRNNError, match="before a grid was built"):
        eng.query(d.data_ptr(), 10)
    # an all-points search leaves its grid for query() to reuse
    eng.search_gpu(d.data_ptr(), 1500, 12, 16, 0.1)
    Q = separate_queries(X, 300, 9)
    dq = device_soa(Q)
    eng.query(dq.data_ptr(), 300)
    gi, gd = eng.get_results_numpy(300, 16)
    ri, rd = O.search_queries(X, Q, 16, 0.1)
    assert_rows_equal(gi.reshape(16, 300).T, gd.reshape(16, 300).T, ri, rd, "query after search_gpu")
    eng.close()


@pytest.mark.parametrize("name,M,nq", [("C2", 50_000, 600), ("C5", 3_000, 100)])
def test_full_size_points_with_separate_queries(name, M, nq):
    """Separate queries against full-size BASELINE point sets: the raw-frame
    D=3 grid with the reversed distance order (C2) and D=128 brute force (C5);
    sampled rows against the oracle over all points."""
    w = W.config(name)
    rs = np.random.RandomState(78)
    spread = 0.3 * w.radius / np.sqrt(w.D)        # offsets of norm ~0.3 r
    Q = (w.X[rs.randint(0, w.N, M)] + spread * rs.standard_normal((M, w.D))).astype(np.float32)
    log(f"full-size {name}: N={w.N} points, M={M} separate queries")
    gi, gd, plan = engine_search_queries(w.X, Q, w.K, w.radius)
    assert plan["path"] == ("grid_full" if name == "C2" else "bruteforce")
    sel = np.sort(rs.choice(M, nq, replace=False))
    ri, rd = O.search_queries(w.X, Q[sel], w.K, w.radius)
    assert_rows_equal(gi[sel], gd[sel], ri, rd, f"{name} separate queries sampled")
    assert (gi[sel] >= 0).sum(1).mean() > 1


def test_profiling_enabled_between_build_and_query():
    # a build without profiling, then a profiled query: the build's stages
    # read as 0, the query's search stage is timed, counters are kept
    X = unit_cloud(3000, 16, 4, 25)
    eng = frnn_cuda.FRNNEngine(max_points=3000)
    d = device_soa(X)
    eng.build(d.data_ptr(), 3000, 16, 32, 0.2)
    eng.set_profiling(True, counters=True)
    Q = separate_queries(X, 1000, 10)
    dq = device_soa(Q)
    eng.query(dq.data_ptr(), 1000)
    st = eng.stage_times()
    assert st["bin_count"] == 0 and st["search"] > 0 and st["unpermute"] > 0
    # stage 5 of a query() call is the queries' own binning, scan and reorder
    assert st["reorder"] > 0
    assert eng.counters()["accepted"] > 0
    # a profiled build, then a query: the query's stage times cover only its
    # own work (the build's stages read 0 after it)
    eng.build(d.data_ptr(), 3000, 16, 32, 0.2)
    eng.query(dq.data_ptr(), 1000)
    st = eng.stage_times()
    assert st["zero_fill"] == 0 and st["stats"] == 0 and st["scan"] == 0
    assert st["reorder"] > 0 and st["search"] > 0
    gi, gd = eng.get_results_numpy(1000, 32)
    ri, rd = O.search_queries(X, Q, 32, 0.2)
    assert_rows_equal(gi.reshape(32, 1000).T, gd.reshape(32, 1000).T, ri, rd, "profiled query")
    eng.close()


@pytest.mark.parametrize("D,k,N,r", [(12, 3, 20000, 0.1), (16, 4, 30000, 0.12)])
def test_queries_outside_the_points_range_on_a_projected_frame(D, k, N, r):
    """Queries beyond the points' bounding box, each at fp32 d2 = r2 - 2 .. r2 + 1
    ulps (reference order) from a boundary point.  The frame's projection
    margin is bounded on the points (R = the points' spread); such a query's
    projection error exceeds it by at most (T+2) u |q - p| for a neighbour p,
    which the cell edge's r 2^-12 and the window's relative slack absorb."""
    from test_gpu_margins import _partner_at, _ulps
    rs = np.random.RandomState(D)
    X = unit_cloud(N, D, k, 31)
    r2 = np.float32(np.float32(r) * np.float32(r))
    # boundary points: the extremes of each coordinate; each query steps out
    # of the points' box past its point's extreme coordinate
    far, Q = [], []
    for j in range(24):
        d = j % D
        sign = 1.0 if (j // D) % 2 == 0 else -1.0
        p = int(np.argmax(sign * X[:, d]))
        e = np.zeros(D)
        e[d] = sign
        t = _ulps(r2, (-2, -1, 0, 1)[j % 4])
        far.append(p)
        Q.append(_partner_at(X[p], t, 2e-6, rs, direction=e))
    Q = np.array(Q, np.float32)
    lo, hi = X.min(0), X.max(0)
    assert np.all(np.any((Q < lo) | (Q > hi), axis=1)), "every query lies outside the points' box"
    log(f"outside queries D={D} N={N} M={len(Q)} r={r}")
    gi, gd, plan = engine_search_queries(X, Q, 16, r)
    assert plan["path"] == "grid_first"
    ri, rd = O.search_queries(X, Q, 16, r)
    assert_rows_equal(gi, gd, ri, rd, f"outside D={D}")
    for j, p in enumerate(far):
        assert (p in gi[j]) == (j % 4 < 2)


@pytest.mark.parametrize("D,N,r,K", [(64, 20000, 0.2, 32), (128, 12000, 0.2, 64)])
def test_queries_on_wide_row_grids(D, N, r, K):
    # first-coordinate grids with 64- and 128-float rows: the queries' own
    # centred filter rows, binned and reordered on the points' grid
    X = unit_cloud(N, D, 4, 9)
    Q = separate_queries(X, 3000, 6)
    assert O.plan(N, D, K, r)["path"] == "grid_first"
    log(f"queries on a wide-row grid: N={N} M={len(Q)} D={D} K={K} r={r}")
    gi, gd, plan = engine_search_queries(X, Q, K, r)
    assert plan["path"] == "grid_first"
    ri, rd = O.search_queries(X, Q, K, r)
    assert_rows_equal(gi, gd, ri, rd, f"queries wide grid D={D}")
