"""End-to-end parity of the HIP engine with the CPU oracle (GPU).

Bar: bit-exact neighbour indices, counts and distances on every compared row
(rows are the K smallest (d2, idx) keys in ascending order, padded (r2, -1)).
Full-size BASELINE configs are checked on sampled queries against the oracle
run over the full database, plus size-independent row properties; C1, C2 and
C3 on every row at full size, the metric workload on every row at 300 000
points.
"""
import glob
import os

import numpy as np
import pytest

import frnn_cuda
import frnn_oracle as O
import frnn_workloads as W
from conftest import ROOT
from gpu_util import assert_rows_equal, device_soa, engine_search, log, torch
from test_oracle_pins import CASES, unit_cloud

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("label,D,k,N,r,K,path", CASES)
def test_paths_match_oracle(label, D, k, N, r, K, path):
    X = unit_cloud(N, D, k, 11)
    X[7] = X[3]
    log(f"case {label}: N={N} D={D} K={K} r={r}")
    gi, gd, plan = engine_search(X, K, r)
    assert plan["path"] == path
    ri, rd = O.search(X, K, r)
    assert_rows_equal(gi, gd, ri, rd, label)


EDGE = [
    # label, D, k, N, radius, K
    ("n1", 3, 3, 1, 0.1, 4),
    ("n31", 16, 4, 31, 0.4, 8),
    ("n33_k1", 12, 3, 33, 0.5, 1),
    ("k128_grid", 16, 4, 3000, 0.2, 128),
    ("k128_bf", 32, 4, 2000, 0.6, 128),
    ("k_gt_n", 3, 3, 40, 0.5, 64),
    ("d20_pad", 20, 4, 2500, 0.6, 16),
    ("d64", 64, 4, 2000, 0.6, 32),
    ("d128", 128, 4, 1500, 0.8, 128),
    ("d9_full", 9, 9, 4000, 0.25, 16),
]


@pytest.mark.parametrize("label,D,k,N,r,K", EDGE)
def test_edge_shapes(label, D, k, N, r, K):
    X = unit_cloud(N, D, k, 5)
    log(f"edge {label}: N={N} D={D} K={K} r={r} plan={O.plan(N, D, K, r)['path']}")
    gi, gd, _ = engine_search(X, K, r)
    ri, rd = O.search(X, K, r)
    assert_rows_equal(gi, gd, ri, rd, label)


def test_duplicates_and_ties():
    rs = np.random.RandomState(3)
    base = rs.rand(300, 3).astype(np.float32)
    X = np.concatenate([base] * 6 + [base[:50] + np.float32(0.01)])   # many exact ties in d2
    log("ties: N=%d" % len(X))
    for K in (4, 16, 32):
        gi, gd, _ = engine_search(X, K, 0.05)
        ri, rd = O.search(X, K, 0.05)
        assert_rows_equal(gi, gd, ri, rd, f"ties K={K}")


# The final selection (K <= 64) takes one of four forms by the number of list
# keys at or below the query's threshold: <= 64 (one sort register), 65-80 (a
# second register of <= 16 keys sorted by the network's first four levels),
# 81-128 (a second full register), > 128 (the general filter-and-merge path).
# Clusters of exact duplicates put that many keys at d2 = 0 (all in the lowest
# histogram bucket, ties broken by index) in every member's list, so each size
# below lands in a chosen form; no list is compacted before the end (sizes <
# 255 - 64).  Jittered copies beside them give distinct small distances.
FINAL_SIZES = (40, 64, 66, 75, 80, 81, 100, 128, 129, 150, 180)


@pytest.mark.parametrize("D,k,r", [(3, 3, 0.05), (16, 4, 0.2)])
@pytest.mark.parametrize("K", [32, 48, 64])
def test_final_selection_forms(D, k, r, K):
    rs = np.random.RandomState(40 + D + K)
    X = [unit_cloud(20000, D, k, 21)]
    for j, size in enumerate(FINAL_SIZES):
        c = X[0][rs.randint(0, 20000)]
        dup = np.repeat(c[None, :], size, axis=0)
        if j % 2:   # half of the clusters: jittered copies (distinct d2 far below r2)
            dup = dup + (1e-4 * r) * rs.standard_normal(dup.shape).astype(np.float32)
        X.append(dup.astype(np.float32))
    X = np.concatenate(X)
    log(f"final selection forms: N={len(X)} D={D} K={K} r={r} plan={O.plan(len(X), D, K, r)['path']}")
    gi, gd, plan = engine_search(X, K, r)
    assert plan["path"] != "bruteforce"
    ri, rd = O.search(X, K, r)
    assert_rows_equal(gi, gd, ri, rd, f"final forms D={D} K={K}")


def test_out_of_domain_points_are_clamped_not_dropped():
    rs = np.random.RandomState(4)
    X = rs.uniform(-0.3, 1.3, (5000, 3)).astype(np.float32)
    X[:20] = 1.0                     # closed upper cell (x == 1.0 at r = 0.01 -> cell res)
    X[20:40] = -0.0
    for r, K in ((0.05, 16), (0.01, 8)):
        log(f"out-of-domain r={r}")
        gi, gd, plan = engine_search(X, K, r)
        assert plan["path"] == "grid_full"
        ri, rd = O.search(X, K, r)
        assert_rows_equal(gi, gd, ri, rd, f"ood r={r}")
        bi, bd = O.search(X, K, r, force_path=0)
        same = np.all(np.sort(ri, 1) == np.sort(bi, 1), axis=1)
        assert same.mean() > 0.999   # grid shell == brute force except fp-order ties at r


@pytest.mark.parametrize("D,r", [(3, 0.02629), (2, 0.0101), (3, 0.05)])
def test_sliver_last_cell_layer(D, r):
    # 1/r just above an integer: the last cell layer [(res-1) r, 1] is a
    # sliver that the device grid merges into the layer before it (r = 0.05:
    # no sliver, the reference's grid unchanged); points at x == 1.0 and past
    # the domain exercise the merged, unbounded edge cells
    rs = np.random.RandomState(5)
    X = rs.rand(20000, D).astype(np.float32)
    X[:50, 0] = 1.0
    X[50:100] = rs.uniform(0.97, 1.03, (50, D)).astype(np.float32)
    log(f"sliver D={D} r={r}")
    gi, gd, plan = engine_search(X, 16, r)
    assert plan["path"] == "grid_full"
    ri, rd = O.search(X, 16, r)
    assert_rows_equal(gi, gd, ri, rd, f"sliver D={D} r={r}")


def test_reference_sweep_cell_sampled():
    # a cell of the reference's own published sweep (its generator, radius
    # and K = 16), sampled rows against the oracle over the full database
    w = W.config("refD16N200000")
    log(f"reference sweep cell: N={w.N} D={w.D} K={w.K} r={w.radius}")
    gi, gd, plan = engine_search(w.X, w.K, w.radius)
    assert plan["path"] == "grid_first"
    q = _sample_queries(w.N, 1000)
    ri, rd = O.search(w.X, w.K, w.radius, query_ids=q)
    assert_rows_equal(gi[q], gd[q], ri, rd, "refD16N200000 sampled")


@pytest.mark.parametrize("D,N,r,K", [(3, 200_000, 0.004, 32), (2, 60_000, 0.0005, 16)])
def test_bruteforce_rows_of_4_at_scale(D, N, r, K):
    # radii below the grid's cell limit send D <= 4 to brute force (rows of 4
    # floats): a dense cluster gives the lists K-deep neighbourhoods, and a
    # run of duplicates gives exact ties; more chunks than fit the device at
    # once, every row against the oracle
    rs = np.random.RandomState(8 + D)
    X = (0.5 + 0.01 * rs.randn(N, D)).astype(np.float32)
    X[100:140] = X[0]
    log(f"bruteforce rows of 4: N={N} D={D} K={K} r={r}")
    gi, gd, plan = engine_search(X, K, r)
    assert plan["path"] == "bruteforce"
    ri, rd = O.search(X, K, r)
    assert_rows_equal(gi, gd, ri, rd, f"bruteforce D={D} N={N}")
    assert (ri >= 0).sum(1).mean() > K / 2


@pytest.mark.parametrize("D,k,N,r,K,path", [(5, 5, 100_000, 0.1, 16, "grid_full"),
                                             (8, 3, 100_000, 0.05, 32, "grid_first"),
                                             (7, 3, 150_000, 0.05, 16, "grid_first"),
                                             (24, 3, 60_000, 0.1, 32, "grid_first"),
                                             (32, 4, 60_000, 0.15, 16, "grid_first"),
                                             (48, 3, 40_000, 0.15, 16, "grid_first"),
                                             (64, 4, 40_000, 0.2, 32, "grid_first")])
def test_rows_of_8_to_64_at_scale(D, k, N, r, K, path):
    # rows padded to 8 floats (D = 5..8) on a full-D grid and on projected
    # frames, rows of 32 and 64 floats (D = 17..64) on projected frames,
    # every row against the oracle
    X = unit_cloud(N, D, k, 13)
    X[7] = X[3]
    log(f"rows at scale: N={N} D={D} K={K} r={r} {path}")
    gi, gd, plan = engine_search(X, K, r)
    assert plan["path"] == path
    ri, rd = O.search(X, K, r)
    assert_rows_equal(gi, gd, ri, rd, f"rows at scale D={D} N={N}")


def test_nan_points_have_no_neighbours():
    rs = np.random.RandomState(6)
    X = rs.rand(2000, 16).astype(np.float32)
    X[5, 3] = np.nan
    X[9, :] = np.nan
    gi, gd, _ = engine_search(X, 8, 0.6)
    ri, rd = O.search(X, 8, 0.6)
    assert_rows_equal(gi, gd, ri, rd, "nan")
    assert np.all(gi[5] == -1) and not np.any(gi == 5)


def _degenerate(kind):
    rs = np.random.RandomState(17)
    if kind == "identical":                 # one point repeated: every projection equal
        X = np.full((3000, 12), 0.37, np.float32)
        X[:5] += np.float32(0.01) * np.arange(5, dtype=np.float32)[:, None]
        return X, 16, 0.1
    if kind == "line":                      # rank 1: one principal direction carries all spread
        u = rs.randn(12)
        u /= np.linalg.norm(u)
        t = rs.rand(5000)
        return (0.5 + 0.4 * (t[:, None] - 0.5) * u[None, :]).astype(np.float32), 16, 0.1
    if kind == "two_clusters":              # far apart relative to r: empty middle cells
        c = np.where(rs.rand(20000) < 0.5, 0.25, 0.75)[:, None]
        return (c + 0.008 * rs.randn(20000, 16)).astype(np.float32), 16, 0.05
    if kind == "slab":                      # all spread on one coordinate, many points per fine cell
        X = (1e-4 * rs.rand(20000, 8)).astype(np.float32)
        X[:, 0] = rs.rand(20000).astype(np.float32)
        return X, 16, 0.05
    if kind == "gauss6":                    # full-rank data: every frame axis carries spread
        return (0.5 + 0.1 * rs.randn(50000, 6)).astype(np.float32), 32, 0.09
    raise ValueError(kind)


@pytest.mark.parametrize("kind", ["identical", "line", "two_clusters", "slab", "gauss6"])
def test_degenerate_frame_geometries(kind):
    """Frames on inputs whose principal directions or spread degenerate: the
    fine axis-0 windows and the frame geometry must still return the oracle's
    rows on every query."""
    X, K, r = _degenerate(kind)
    log(f"degenerate frame {kind}: N={len(X)} D={X.shape[1]} K={K} r={r}")
    gi, gd, plan = engine_search(X, K, r)
    assert plan["path"] == "grid_first"
    ri, rd = O.search(X, K, r)
    assert_rows_equal(gi, gd, ri, rd, f"degenerate {kind}")


def test_huge_radius_everything_in_range():
    rs = np.random.RandomState(8)
    X = rs.rand(700, 5).astype(np.float32)
    gi, gd, _ = engine_search(X, 16, 50.0)
    ri, rd = O.search(X, 16, 50.0)
    assert_rows_equal(gi, gd, ri, rd, "huge r")
    assert np.all(gi >= 0)


def test_large_coordinates_overflow_filter():
    # |x|^2 overflows fp32 in the MFMA filter; such pairs must still be re-evaluated exactly
    rs = np.random.RandomState(9)
    X = (rs.rand(600, 4) * 1e4).astype(np.float32)
    X[:100] = (1e19 + rs.rand(100, 4) * 1e13).astype(np.float32)
    gi, gd, _ = engine_search(X, 8, 3e13)
    ri, rd = O.search(X, 8, 3e13)
    assert_rows_equal(gi, gd, ri, rd, "large coords")


def test_engine_reuse_and_api():
    """One engine, several calls with different N/D/K (buffers grow and are reused);
    search() host path, get_results() SoA order and search_gpu pointers."""
    eng = frnn_cuda.FRNNEngine(max_points=6000)
    for (N, D, k, r, K) in ((6000, 16, 4, 0.2, 32), (1000, 3, 3, 0.1, 8), (5000, 12, 3, 0.1, 64),
                            (6000, 3, 3, 0.05, 16)):
        X = unit_cloud(N, D, k, N)
        gi, gd, _ = engine_search(X, K, r, engine=eng)
        ri, rd = O.search(X, K, r)
        assert_rows_equal(gi, gd, ri, rd, f"reuse N={N} D={D}")
    X = unit_cloud(6000, 3, 3, 1)
    idx_l, dist_l = eng.search(X.reshape(-1).tolist(), 16, 0.05)          # host AoS path
    ri, rd = O.search(X, 16, 0.05)
    assert idx_l == ri.reshape(-1).tolist()
    assert np.array_equal(np.asarray(dist_l, np.float32), rd.reshape(-1))
    t = torch()
    d = device_soa(X)
    pi, pd = eng.search_gpu(d.data_ptr(), 6000, 3, 16, 0.05)
    assert pi and pd
    gi_l, gd_l = eng.get_results(6000, 16)                                 # SoA lists
    assert gi_l == ri.T.reshape(-1).tolist()
    with pytest.raises(ValueError):
        eng.search_gpu(d.data_ptr(), 7000, 3, 16, 0.05)                    # N > max_points
    with pytest.raises(ValueError):
        eng.search_gpu(d.data_ptr(), 6000, 3, 0, 0.05)
    with pytest.raises(ValueError):
        eng.search([0.0] * 7, 4, 0.1)
    eng.close()
    t.cuda.synchronize()


def test_profiling_counters_and_stage_times():
    # raw grid: the shell counter equals the oracle's 3^D shell count
    X = unit_cloud(20000, 3, 3, 2)
    eng = frnn_cuda.FRNNEngine(max_points=20000)
    eng.set_profiling(True)
    d = device_soa(X)
    eng.search_gpu(d.data_ptr(), 20000, 3, 32, 0.05)
    assert eng.last_plan()["path"] == "grid_full"
    st = eng.stage_times()
    c = eng.counters()
    assert set(st) == set(frnn_cuda.STAGE_NAMES)
    assert st["search"] > 0 and all(v >= 0 for v in st.values())
    assert c["shell_candidates"] == O.shell_candidates(X, 32, 0.05)
    assert c["filter_hits"] >= c["accepted"] > 0
    # framed first-coordinate grid: the frame stage runs; the shell is the
    # frame's 3^g cells, and every accepted pair lies in it, was streamed and
    # passed the filter
    X = unit_cloud(20000, 16, 4, 2)
    d = device_soa(X)
    eng.search_gpu(d.data_ptr(), 20000, 16, 32, 0.15)
    assert eng.last_plan()["path"] == "grid_first"
    st = eng.stage_times()
    c = eng.counters()
    assert st["frame"] > 0
    assert c["shell_candidates"] >= c["accepted"]
    assert c["streamed_pairs"] >= c["filter_hits"] >= c["accepted"] > 0
    # events around the search kernel only: every other stage reads 0, also
    # after calls that recorded all of them
    eng.set_profiling(True, counters=False, search_only=True)
    for _ in range(2):
        eng.search_gpu(d.data_ptr(), 20000, 16, 32, 0.15)
        st = eng.stage_times()
        assert st["search"] > 0
        assert all(v == 0 for k, v in st.items() if k != "search"), st
    gi, gd = eng.get_results_numpy(20000, 32)
    ri, rd = O.search(X, 32, 0.15)
    assert_rows_equal(gi.reshape(32, 20000).T, gd.reshape(32, 20000).T, ri, rd, "search-only events")
    eng.close()


def test_count_array_reuse_across_grids():
    # the count scan zeroes the counts it reads, so only the first build on an
    # engine fills the array; grids of different sizes and kinds in turn on
    # one engine (projected frame, raw frame, a larger projected frame, the
    # first again) must each match the oracle
    eng = frnn_cuda.FRNNEngine(max_points=30000)
    cases = [(unit_cloud(20000, 16, 4, 31), 32, 0.15), (unit_cloud(30000, 3, 3, 32), 16, 0.03),
             (unit_cloud(30000, 12, 3, 33), 32, 0.1), (unit_cloud(20000, 16, 4, 31), 32, 0.15)]
    eng.set_profiling(True, counters=False)
    for j, (X, K, r) in enumerate(cases):
        N, D = X.shape
        d = device_soa(X)
        eng.search_gpu(d.data_ptr(), N, D, K, r)
        cw = eng.count_work()
        log(f"count reuse {j}: D={D} N={N} plan={eng.last_plan()['path']} {cw}")
        assert eng.last_plan()["path"] != "bruteforce"
        assert cw["scanned"] >= 2
        if j == 0:
            assert cw["zero_filled"] >= cw["scanned"]
        gi, gd = eng.get_results_numpy(N, K)
        ri, rd = O.search(X, K, r)
        assert_rows_equal(gi.reshape(K, N).T, gd.reshape(K, N).T, ri, rd, f"count reuse {j}")
    # the same grid again: nothing left to fill
    eng.search_gpu(d.data_ptr(), N, D, K, r)
    assert eng.count_work()["zero_filled"] == 0
    eng.close()


@pytest.mark.parametrize("bad", ["nan", "inf"])
def test_nonfinite_points_on_a_framed_grid(bad):
    # NaN: projections of such points are NaN (binned to cell 0, never within
    # the radius); inf: the frame falls back to the raw first coordinates
    X = unit_cloud(20000, 12, 3, 21)
    X[5, 3] = np.nan if bad == "nan" else np.inf
    X[9, :] = np.nan if bad == "nan" else -np.inf
    X[11, 0] = np.nan if bad == "nan" else np.inf
    log(f"non-finite {bad} on grid_first D=12")
    gi, gd, plan = engine_search(X, 32, 0.1)
    assert plan["path"] == "grid_first"
    ri, rd = O.search(X, 32, 0.1)
    assert_rows_equal(gi, gd, ri, rd, bad)
    assert np.all(gi[9] == -1) and not np.any(gi == 9)


def _golden_files():
    return sorted(glob.glob(os.path.join(ROOT, "tests", "golden", "*.npz")))


@pytest.mark.parametrize("path", _golden_files(), ids=lambda p: os.path.basename(p))
def test_golden_fixtures(path):
    z = np.load(path)
    X, K, r = z["X"], int(z["K"]), float(z["radius"])
    log(f"golden {os.path.basename(path)}")
    gi, gd, plan = engine_search(X, K, r)
    assert plan["path"] == str(z["path"])
    assert_rows_equal(gi, gd, z["idx"], z["dist"], os.path.basename(path))


def _sample_queries(N, n, seed=1234):
    rs = np.random.RandomState(seed)
    return np.sort(rs.choice(N, size=min(n, N), replace=False)).astype(np.int32)


def _row_properties(gi, gd, r2, N):
    valid = gi >= 0
    assert np.all(gi < N)
    assert np.all(gd[valid] < r2)
    assert np.all(gd[~valid] == r2)
    # valid entries first, ascending (d2, idx)
    assert np.all(valid[:, :-1] | ~valid[:, 1:])
    d0, d1 = gd[:, :-1], gd[:, 1:]
    i0, i1 = gi[:, :-1], gi[:, 1:]
    both = valid[:, :-1] & valid[:, 1:]
    assert np.all(~both | (d0 < d1) | ((d0 == d1) & (i0 < i1)))


@pytest.mark.parametrize("name,nq", [("C1", 2000), ("C2", 1000), ("C3", 400), ("metric", 400),
                                     ("C4", 300), ("C5", 200)])
def test_baseline_configs_full_size(name, nq):
    w = W.config(name)
    log(f"full-size {name}: N={w.N} D={w.D} K={w.K} r={w.radius:.6f}")
    gi, gd, plan = engine_search(w.X, w.K, w.radius)
    r2 = np.float32(np.float32(w.radius) * np.float32(w.radius))
    _row_properties(gi, gd, r2, w.N)
    # every point finds itself (d2 = 0 < r2)
    assert np.all(gd[:, 0] == 0)
    q = _sample_queries(w.N, nq)
    ri, rd = O.search(w.X, w.K, w.radius, query_ids=q)
    assert_rows_equal(gi[q], gd[q], ri, rd, f"{name} sampled")
    log(f"  path={plan['path']} mean neighbours={(gi >= 0).sum(1).mean():.1f}")


@pytest.mark.parametrize("name", ["C1", "C2"])
def test_baseline_configs_all_rows(name):
    """Every row of the full-size C1 and C2 searches against the oracle run
    over the full database (all 200 000 / 1 000 000 queries)."""
    w = W.config(name)
    log(f"all rows {name}: N={w.N} D={w.D} K={w.K} r={w.radius:.6f}")
    gi, gd, plan = engine_search(w.X, w.K, w.radius)
    assert plan["path"] == "grid_full"
    ri, rd = O.search(w.X, w.K, w.radius)
    assert_rows_equal(gi, gd, ri, rd, f"{name} all rows")


@pytest.mark.parametrize("name,N", [("metric", 300_000), ("C3", 500_000)])
def test_framed_configs_all_rows(name, N):
    """Every row of the projected-frame searches (rows of 16 and 12 floats):
    C3 at full size and the metric workload at 300 000 points (its radius
    follows N), against the oracle's first-coordinate grid over the full
    database."""
    w = W.config(name, N=N)
    log(f"all rows {name}: N={w.N} D={w.D} K={w.K} r={w.radius:.6f}")
    gi, gd, plan = engine_search(w.X, w.K, w.radius)
    assert plan["path"] == "grid_first"
    ri, rd = O.search(w.X, w.K, w.radius)
    assert_rows_equal(gi, gd, ri, rd, f"{name} N={N} all rows")


@pytest.mark.parametrize("D,k,N,r,K", [(64, 4, 1500, 0.6, 32), (128, 4, 1200, 0.8, 128), (40, 4, 1000, 0.5, 16)])
def test_host_search_wide_rows(D, k, N, r, K):
    """The host path search() at D > 32, where the reference's staging buffer
    (d_points, sized for 32 coordinates: frnn_engine.cu:26-28, written at
    :113-117) overflows; here the staging grows with D."""
    X = unit_cloud(N, D, k, 61)
    eng = frnn_cuda.FRNNEngine(max_points=N)
    log(f"host search D={D} N={N} K={K} r={r}")
    idx, dist = eng.search_numpy(X.reshape(-1), K, r)
    eng.close()
    ri, rd = O.search(X, K, r)
    assert_rows_equal(idx, dist, ri, rd, f"host search D={D}")


def test_concurrent_calls_on_one_engine_are_serialised():
    """Python threads sharing one engine: every call runs whole (the binding
    serialises them; the reference's binding held the GIL), so each thread's
    host-path results match the oracle for its own input."""
    import threading
    eng = frnn_cuda.FRNNEngine(max_points=8000)
    inputs = [(unit_cloud(8000, 3, 3, 70 + i), 16, 0.05 + 0.01 * i) for i in range(4)]
    refs = [O.search(X, K, r) for X, K, r in inputs]
    errors = []

    def worker(i):
        X, K, r = inputs[i]
        try:
            for _ in range(3):
                idx, dist = eng.search_numpy(X.reshape(-1), K, r)
                assert_rows_equal(idx, dist, refs[i][0], refs[i][1], f"thread {i}")
        except Exception as e:          # reported by the main thread
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    eng.close()
    assert not errors, errors[0]


WIDE_GRIDS = [
    # label, D, N, radius, K: first-coordinate grids whose padded rows are 64 or
    # 128 floats (centred filter rows, queued exact rechecks, the tile loop
    # without the next-tile prefetch)
    ("first_d40", 40, 20000, 0.2, 16),
    ("first_d64", 64, 20000, 0.2, 32),
    ("first_d100", 100, 20000, 0.2, 16),
    ("first_d128", 128, 12000, 0.2, 64),
]


@pytest.mark.parametrize("label,D,N,r,K", WIDE_GRIDS)
def test_wide_rows_on_grids(label, D, N, r, K):
    X = unit_cloud(N, D, 4, 9)
    X[11] = X[5]
    assert O.plan(N, D, K, r)["path"] == "grid_first"
    log(f"wide grid {label}: N={N} D={D} K={K} r={r}")
    gi, gd, plan = engine_search(X, K, r)
    assert plan["path"] == "grid_first"
    ri, rd = O.search(X, K, r)
    assert_rows_equal(gi, gd, ri, rd, label)
