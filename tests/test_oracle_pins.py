"""Pins for the CPU oracle (oracle/frnn_oracle.cpp) -- CPU only.

The reference ships no golden vectors for this path (its only correctness
check, Tests/scripts/validate_correctness.py, is a float64 tolerance-band
property test), so the oracle is pinned by:
  * exact rational arithmetic for the fp32 fma emulation (oracle/exact_fp32.py),
    which in turn pins the oracle's fp32 distance orders;
  * closed-form binning and a hand-derived dispatch table;
  * an independent numpy brute force (exact_fp32.brute_force) for every path;
  * the reference's own float64 tolerance-band criterion (validate_correctness.py:99-139).
"""
from fractions import Fraction

import numpy as np
import pytest

import exact_fp32 as E
import frnn_oracle as O


def _round_f32(x: Fraction) -> np.float32:
    """Round an exact rational to fp32, round-to-nearest-even (incl. subnormals, overflow)."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    # 2^e <= a < 2^(e+1)
    q = max(e, -126) - 23                       # quantum of the fp32 grid at this binade
    scaled = a / Fraction(2) ** q
    n = scaled.numerator // scaled.denominator
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    val = Fraction(n) * Fraction(2) ** q
    if val >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    return np.float32(sign * float(val))


def test_round_f32_helper_matches_numpy_cast():
    rs = np.random.RandomState(7)
    x = rs.standard_normal(2000) * 10.0 ** rs.randint(-40, 38, 2000)
    for v in x:
        assert _round_f32(Fraction(float(v))) == np.float32(v)


def test_fma32_exact_on_random_and_cancellation():
    rs = np.random.RandomState(1)
    a = rs.standard_normal(3000).astype(np.float32)
    b = (rs.standard_normal(3000) * 10.0 ** rs.randint(-8, 8, 3000)).astype(np.float32)
    c = -(a.astype(np.float64) * b.astype(np.float64) * (1 + rs.standard_normal(3000) * 1e-6)).astype(np.float32)
    got = E.fma32(a, b, c)
    for i in range(len(a)):
        want = _round_f32(Fraction(float(a[i])) * Fraction(float(b[i])) + Fraction(float(c[i])))
        assert got[i] == want, (a[i], b[i], c[i])


def test_fma32_double_rounding_hazard():
    # a*b = 2^-24 (1 - 2^-46); a*b + c lies just below the fp32 midpoint between
    # 1+2^-23 (odd) and 1+2^-22, and the float64 sum lands exactly on it.  A plain
    # float64->fp32 cast rounds to even (up); the correct fma rounds down.
    a = np.float32(2.0 ** -24 * (1 + 2.0 ** -23))
    b = np.float32(1 - 2.0 ** -23)
    c = np.float32(1 + 2.0 ** -23)
    naive = np.float32(np.float64(a) * np.float64(b) + np.float64(c))
    assert naive == np.float32(1 + 2.0 ** -22)
    assert E.fma32(a, b, c) == c
    want = _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))
    assert want == c


@pytest.mark.parametrize("order", [0, 1])
def test_oracle_dist2_equals_exact_emulation(order):
    rs = np.random.RandomState(2 + order)
    for D in (1, 2, 3, 5, 12, 16, 33):
        q = rs.rand(400, D).astype(np.float32)
        p = (q + rs.standard_normal((400, D)).astype(np.float32) * np.float32(1e-3)).astype(np.float32)
        want = E.dist2(q, p, order)
        got = np.array([O.dist2(q[i], p[i], order) for i in range(400)], dtype=np.float32)
        assert np.array_equal(got, want)


def test_distance_orders_differ_somewhere():
    # The two orders are distinct functions: a dropped/reordered term would be caught.
    rs = np.random.RandomState(5)
    q = rs.rand(20000, 3).astype(np.float32)
    p = rs.rand(20000, 3).astype(np.float32)
    assert np.any(E.dist2(q, p, 0) != E.dist2(q, p, 1))


def test_dist2_special_values():
    q = np.array([[0.0, 0.0, 0.0], [1e-30, 0, 0], [np.nan, 0, 0], [np.inf, 0, 0], [3e19, 0, 0]], np.float32)
    p = np.array([[0.0, 0.0, 0.0], [0, 0, 0], [0, 0, 0], [0, 0, 0], [0, 0, 0]], np.float32)
    for order in (0, 1):
        e = E.dist2(q, p, order)
        o = np.array([O.dist2(q[i], p[i], order) for i in range(len(q))], np.float32)
        assert e[0] == 0 and e[1] == 0          # 1e-60 underflows below the fp32 subnormal range
        assert np.isnan(e[2]) and np.isnan(o[2])
        assert np.isinf(e[3]) and np.isinf(o[3]) and np.isinf(e[4])
        np.testing.assert_array_equal(e[[0, 1, 3, 4]], o[[0, 1, 3, 4]])


def test_binning_closed_form():
    rs = np.random.RandomState(3)
    res, r = 27, np.float32(0.037923)
    inv = np.float32(1.0) / r
    X = np.concatenate([rs.rand(3000, 4), rs.uniform(-0.5, 1.5, (500, 4)),
                        np.array([[0.0, 1.0, -0.0, np.nan], [1e30, -1e30, 0.5, 1.0]])]).astype(np.float32)
    X[:50, 0] = (np.arange(50, dtype=np.float32) * r).astype(np.float32)   # on cell edges
    got = O.bin_cells(X, 4, res, inv)
    coords = np.floor(X * inv)
    coords = np.where(np.isnan(coords), 0, coords)
    coords = np.clip(coords, 0, res - 1).astype(np.int64)
    want = coords[:, 0] + res * (coords[:, 1] + res * (coords[:, 2] + res * coords[:, 3]))
    assert np.array_equal(got, want.astype(np.int32))


# (N, D, K, radius) -> expected plan, derived by hand from frnn_engine.cu:201-246, 64-86.
DISPATCH_TABLE = [
    ((500, 3, 16, 0.1), ("bruteforce", 0, 0)),        # sel=2, db=1500: 500 <= 2e6/3000
    ((1000, 3, 16, 0.1), ("grid_full", 3, 10)),       # 1000 > 333; res 10, 27 < 1000
    ((1000, 3, 16, 0.34), ("bruteforce", 0, 0)),      # res 3: 27 >= 27; first-coord 27 >= 27
    ((100000, 12, 32, 0.0345), ("grid_first", 4, 29)),
    ((100000, 16, 64, 0.03), ("bruteforce", 0, 0)),   # res 34: 34^4 > 1e6
    ((100000, 4, 8, 0.02), ("grid_first", 3, 50)),    # 50^4 > 1e6, g = min(4,3) = 3
    ((100000, 2, 8, 0.001), ("grid_full", 2, 1000)),  # exactly 1e6 cells
    ((100000, 2, 8, 0.0009), ("bruteforce", 0, 0)),   # 1112^2 > 1e6 for both grids
    ((200000, 128, 128, 12.96), ("bruteforce", 0, 0)),  # res 1 -> res' 2, 81 >= 16
    ((100000, 6, 16, 0.1), ("grid_full", 6, 10)),     # 10^6 <= 1e6
    ((100000, 7, 16, 0.1), ("grid_first", 4, 10)),    # 10^7 > 1e6
    ((100000, 1, 4, 0.5), ("bruteforce", 0, 0)),      # res 2: 3 >= 2 twice
    ((100000, 1, 4, 0.2), ("grid_full", 1, 5)),
    ((1000, 16, 128, 0.5), ("bruteforce", 0, 0)),     # sel 16: 1000 > 7; then 81 >= 16
    ((60, 16, 64, 0.05), ("bruteforce", 0, 0)),       # sel 8, db 960: 60 <= 260
    ((3000000, 3, 16, 0.03), ("grid_full", 3, 34)),   # N*D > 2e6 saturates db
]


@pytest.mark.parametrize("args,want", DISPATCH_TABLE)
def test_oracle_dispatch_table(args, want):
    p = O.plan(*args)
    assert (p["path"], p["grid_dim"], p["res"]) == want
    if want[0] != "bruteforce":
        assert p["cells"] == want[2] ** want[1]
        assert p["rev_order"] == int(want[0] == "grid_full" and args[1] == 3)


def test_oracle_plan_empty():
    assert O.plan(0, 3, 4, 0.1)["path"] == "empty"


def unit_cloud(N, D, k, seed):
    """Points in [0,1]^D on a k-dimensional random affine subspace plus small noise."""
    rs = np.random.RandomState(seed)
    if k >= D:
        return rs.rand(N, D).astype(np.float32)
    A, _ = np.linalg.qr(rs.standard_normal((D, k)))
    X = rs.rand(N, k) @ A.T + 0.01 * rs.standard_normal((N, D))
    X = (X - X.min()) / ((X.max() - X.min()) * (1 + 1e-6))
    return X.astype(np.float32)


CASES = [
    # (label, D, k, N, radius, K, expected path)
    ("full_d1", 1, 1, 1500, 0.002, 4, "grid_full"),
    ("full_d2", 2, 2, 1500, 0.03, 8, "grid_full"),
    ("full_d3_rev", 3, 3, 1500, 0.08, 16, "grid_full"),
    ("full_d4", 4, 4, 1500, 0.15, 16, "grid_full"),
    ("full_d5", 5, 5, 1200, 0.3, 16, "grid_full"),
    ("first_d8", 8, 2, 1500, 0.1, 16, "grid_first"),
    ("first_d12", 12, 3, 1500, 0.1, 32, "grid_first"),
    ("first_d16", 16, 4, 1500, 0.2, 64, "grid_first"),
    ("bf_tiny_d3", 3, 3, 500, 0.1, 16, "bruteforce"),
    ("bf_d16", 16, 4, 600, 0.5, 64, "bruteforce"),      # res 2: first-coord 81 >= 16
    ("bf_tiny_d16", 16, 4, 120, 0.3, 64, "bruteforce"), # N^2*16*8 <= 2e6
    ("bf_d40", 40, 3, 300, 0.6, 8, "bruteforce"),       # res 2: first-coord rejected
]


@pytest.mark.parametrize("label,D,k,N,r,K,path", CASES)
def test_oracle_matches_exact_bruteforce(label, D, k, N, r, K, path):
    X = unit_cloud(N, D, k, 11)
    X[7] = X[3]                                           # exact duplicate -> tie on idx
    p = O.plan(N, D, K, r)
    assert p["path"] == path
    gi, gd = O.search(X, K, r)
    ni, nd = E.brute_force(X, K, r, order=p["rev_order"])
    assert np.array_equal(gi, ni), label
    assert np.array_equal(gd, nd), label
    bi, bd = O.search(X, K, r, force_path=0)              # brute force: fwd order
    fi, fd = E.brute_force(X, K, r, order=0)
    assert np.array_equal(bi, fi) and np.array_equal(bd, fd), label


def separate_queries(X, M, seed):
    """Queries for a point set X: fresh points from a nearby cloud, exact
    copies of some points (d2 = 0 matches), and a few outside [0, 1]."""
    rs = np.random.RandomState(seed)
    N, D = X.shape
    Q = X[rs.randint(0, N, M)] + (0.02 * rs.standard_normal((M, D))).astype(np.float32)
    Q[: M // 8] = X[rs.randint(0, N, M // 8)]
    Q[M // 8: M // 8 + 3] += np.float32(1.5)
    return Q.astype(np.float32)


@pytest.mark.parametrize("label,D,k,N,r,K,path", CASES)
def test_oracle_queries_match_exact_bruteforce(label, D, k, N, r, K, path):
    # queries distinct from the points: the points' plan and grid, each query
    # binned with the same parameters (clamped), against an exhaustive search
    X = unit_cloud(N, D, k, 11)
    Q = separate_queries(X, 300, 5)
    p = O.plan(N, D, K, r)
    assert p["path"] == path
    gi, gd = O.search_queries(X, Q, K, r)
    ni, nd = E.brute_force(X, K, r, order=p["rev_order"], Q=Q)
    assert np.array_equal(gi, ni), label
    assert np.array_equal(gd, nd), label
    # the all-points search is the special case Q = X
    si, sd = O.search_queries(X, X, K, r)
    ai, ad = O.search(X, K, r)
    assert np.array_equal(si, ai) and np.array_equal(sd, ad), label


def test_oracle_paths_cover_grid_first():
    X = unit_cloud(20000, 12, 3, 12)
    assert O.plan(20000, 12, 32, 0.1)["path"] == "grid_first"
    q = np.arange(0, 20000, 97)
    gi, gd = O.search(X, 32, 0.1, query_ids=q)
    assert (gi >= 0).sum(1).mean() > 5
    bi, bd = O.search(X, 32, 0.1, force_path=0, query_ids=q)
    assert np.array_equal(gi, bi) and np.array_equal(gd, bd)


def test_oracle_float64_band_criterion():
    """validate_correctness.py:99-139: against float64 truth, returned neighbours
    must be inside r (up to a TAU band) and the K-nearest distances must agree
    except within the band."""
    rs = np.random.RandomState(13)
    TAU, RTOL, ATOL = 1e-4, 1e-3, 1e-6
    for D, r, K in ((3, 0.06, 16), (12, 0.45, 16), (16, 0.6, 16)):
        X = rs.rand(3000, D).astype(np.float32)
        qs = rs.choice(3000, 300, replace=False)
        idx, dist = O.search(X, K, r, query_ids=qs)
        P = X.astype(np.float64)
        d2 = ((P[qs][:, None, :] - P[None, :, :]) ** 2).sum(-1)
        r2_lo, r2_hi = r * r * (1 - TAU), r * r * (1 + TAU)
        for row, q in enumerate(qs):
            mine = idx[row][idx[row] >= 0]
            assert np.all(d2[row][mine] <= r2_hi)
            truth = np.sort(d2[row][d2[row] <= r2_hi])[:K]
            got = np.sort(dist[row][idx[row] >= 0].astype(np.float64))
            n = min(len(truth), len(got))
            bad = ~np.isclose(truth[:n], got[:n], rtol=RTOL, atol=ATOL)
            assert not np.any(truth[:n][bad] < r2_lo) and not np.any(got[:n][bad] < r2_lo)
            assert all(x >= r2_lo for x in list(truth[n:]) + list(got[n:]))


def test_oracle_padding_and_self():
    X = np.array([[0.1, 0.1, 0.1], [0.9, 0.9, 0.9], [0.11, 0.1, 0.1]], np.float32)
    idx, dist = O.search(X, 4, 0.05)
    r2 = np.float32(np.float32(0.05) * np.float32(0.05))
    assert list(idx[0]) == [0, 2, -1, -1] and list(idx[1]) == [1, -1, -1, -1]
    assert dist[0][0] == 0 and np.all(dist[1][1:] == r2)


@pytest.mark.parametrize("D,k,N,r,K", [(3, 3, 3000, 0.08, 16), (2, 2, 2500, 0.05, 8), (12, 3, 4000, 0.2, 32),
                                       (5, 5, 2000, 0.3, 16)])
def test_oracle_shell_candidates_closed_form(D, k, N, r, K):
    """oracle_shell_candidates (the reference's unpruned 3^g shell size per
    query, find_nbrs.cu:167-187 / :288-304) against a numpy count: clamped
    cells of every point on the plan's grid, a bincount, and for every query
    the sum of the counts of its in-range neighbouring cells."""
    X = unit_cloud(N, D, k, 5)
    X[:40, 0] = 1.0                                    # closed upper cell
    p = O.plan(N, D, K, r)
    assert p["path"] in ("grid_full", "grid_first")
    g, res = p["grid_dim"], p["res"]
    inv = np.float32(1.0) / np.float32(r)
    coords = np.clip(np.floor(X[:, :g] * inv), 0, res - 1).astype(np.int64)
    cell = (coords * (res ** np.arange(g))[None, :]).sum(1)
    cnt = np.bincount(cell, minlength=res ** g)
    total = 0
    offsets = np.array(np.meshgrid(*[[-1, 0, 1]] * g, indexing="ij")).reshape(g, -1).T
    for o in offsets:
        nb = coords + o[None, :]
        ok = np.all((nb >= 0) & (nb < res), axis=1)
        total += int(cnt[(nb[ok] * (res ** np.arange(g))[None, :]).sum(1)].sum())
    assert O.shell_candidates(X, K, r) == total
    q = np.array([0, 5, 17, N - 1], dtype=np.int32)
    sub = 0
    for o in offsets:
        nb = coords[q] + o[None, :]
        ok = np.all((nb >= 0) & (nb < res), axis=1)
        sub += int(cnt[(nb[ok] * (res ** np.arange(g))[None, :]).sum(1)].sum())
    assert O.shell_candidates(X, K, r, query_ids=q) == sub
