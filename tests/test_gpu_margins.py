"""Where the MFMA filter's rounding margin is tightest (GPU).

The search decides hits with fp32 MFMA values F = |p'|^2 + |q'|^2 - 2 p'.q' of
rows centred on the input mean; F's rounding error grows with |p'|^2 + |q'|^2,
and only the margin (norm_scale, thr_rel) keeps a true neighbour from being
dropped.  These cases put query/neighbour pairs far from the data mean, so the
three terms are large and cancel, at squared distances a few fp32 ulps around
r^2 (strict d2 < r2: find_nbrs.cu:200,341, no_grid_frnn.cu:163) and around a
query's K-th distance (the running threshold of its list).  Every pair's fp32
distance in the reference order is constructed exactly (oracle/exact_fp32.py
emulates the sequential fma chain), so each expected membership is known
independently of the oracle, and the rows are also compared bit for bit with
the oracle.
"""
import numpy as np
import pytest

import exact_fp32 as E
import frnn_oracle as O
from gpu_util import assert_rows_equal, engine_search, log

pytestmark = pytest.mark.gpu


def _ulps(x, k):
    """x moved by k fp32 ulps (k may be negative)."""
    x = np.float32(x)
    for _ in range(abs(k)):
        x = np.nextafter(x, np.float32(np.inf) if k > 0 else np.float32(-np.inf))
    return np.float32(x)


def _partner_at(q, target, scale, rs, tries=200, direction=None):
    """A point p with fp32 dist2(q, p) == target exactly (reference order),
    found by sampling directions (around `direction` if given) and squared
    lengths around `target`."""
    D = q.shape[0]
    for _ in range(tries):
        u = rs.standard_normal((4096, D))
        if direction is not None:
            u = 0.4 * u / np.sqrt(D) + np.asarray(direction, np.float64)[None, :]
        u /= np.linalg.norm(u, axis=1, keepdims=True)
        # lengths spread over a few hundred ulps of sqrt(target)
        L = np.sqrt(np.float64(target)) * (1.0 + scale * rs.uniform(-1.0, 1.0, (4096, 1)))
        P = (q[None, :].astype(np.float64) + u * L).astype(np.float32)
        d2 = E.dist2(q[None, :], P, 0)
        hit = np.nonzero(d2 == np.float32(target))[0]
        if len(hit):
            return P[hit[0]]
    raise AssertionError(f"no partner found at {target}")


def _far_pairs(D, r, offset, ks, rs):
    """Pairs (q, p) far from the origin-centred background, at fp32 squared
    distances r2 + k ulps for k in ks.  Pairs sit 20 r apart from each other."""
    r2 = np.float32(np.float32(r) * np.float32(r))
    rows, expect = [], []
    for j, k in enumerate(ks):
        q = np.full(D, np.float32(offset), np.float32)
        q[j % D] += np.float32(20.0 * r * (1 + j // D))
        q = q + (rs.uniform(-0.25, 0.25, D) * r).astype(np.float32)
        t = _ulps(r2, k)
        p = _partner_at(q, t, 2e-6, rs)
        assert E.dist2(q[None], p[None], 0)[0] == t
        rows += [q, p]
        expect.append((k < 0))                 # strict d2 < r2
    return np.array(rows, np.float32), np.array(expect)


@pytest.mark.parametrize("D,N,offset,r,K,path", [
    (128, 1500, 400.0, 12.9, 16, "bruteforce"),    # C5-like rows, brute force, DS = 128
    (16, 6000, 60.0, 0.1, 16, "grid_first"),       # framed first-coordinate grid, DS = 16
    (32, 3000, 80.0, 0.35, 16, "bruteforce"),      # DS = 32, tile-exact brute force
])
def test_pairs_far_from_the_mean_at_r2(D, N, offset, r, K, path):
    rs = np.random.RandomState(D + N)
    ks = [-3, -2, -1, 0, 1, 2] * 4
    pairs, expect = _far_pairs(D, r, offset, ks, rs)
    bg = (rs.rand(N, D) if path == "grid_first" else rs.standard_normal((N, D))).astype(np.float32)
    X = np.concatenate([bg, pairs])
    log(f"far pairs D={D} N={len(X)} offset={offset} r={r} K={K}")
    gi, gd, plan = engine_search(X, K, r)
    assert plan["path"] == path
    ri, rd = O.search(X, K, r)
    assert_rows_equal(gi, gd, ri, rd, f"far pairs D={D}")
    # the constructed partner is found exactly when its d2 is below r2
    for j, e in enumerate(expect):
        qi, pi = N + 2 * j, N + 2 * j + 1
        assert (pi in gi[qi]) == bool(e), (j, ks[j])
        assert (qi in gi[pi]) == bool(e), (j, ks[j])


@pytest.mark.parametrize("D,N,offset,r,path", [
    (128, 1500, 300.0, 12.9, "bruteforce"),
    (16, 6000, 50.0, 0.1, "grid_first"),
])
def test_kth_threshold_ties_far_from_the_mean(D, N, offset, r, path):
    """A query with K + 4 neighbours whose distances straddle its K-th key by
    single ulps (and repeat it, so the index breaks the tie): the running
    threshold (histogram edges and exact compactions) must keep exactly the
    K smallest (d2, idx) keys."""
    rs = np.random.RandomState(7 + D)
    K = 16
    r2 = np.float32(np.float32(r) * np.float32(r))
    q = np.full(D, np.float32(offset), np.float32) + (rs.uniform(-0.2, 0.2, D) * r).astype(np.float32)
    kth = _ulps(np.float32(0.7) * r2, 0)
    # K - 3 neighbours well inside, then the boundary group around the K-th key
    inner = [np.float32(v) for v in np.linspace(0.05, 0.6, K - 3) * r2]
    edge = [_ulps(kth, -1), kth, kth, kth, _ulps(kth, 1), _ulps(kth, 1), _ulps(kth, 2)]
    pts = [_partner_at(q, t, 2e-6, rs) for t in inner + edge]
    bg = (rs.rand(N, D) if path == "grid_first" else rs.standard_normal((N, D))).astype(np.float32)
    X = np.concatenate([bg, q[None], np.array(pts, np.float32)])
    log(f"K-th ties D={D} N={len(X)} r={r}")
    gi, gd, plan = engine_search(X, K, r)
    assert plan["path"] == path
    ri, rd = O.search(X, K, r)
    assert_rows_equal(gi, gd, ri, rd, f"kth ties D={D}")
    row = gi[N]
    # the query itself (d2 = 0), the K - 3 inner points, the one an ulp below
    # the K-th key and the first of the three copies at it (lowest index wins)
    first = N + 1
    want = [N] + list(range(first, first + K - 3)) + [first + K - 3, first + K - 2]
    assert list(row) == want
    assert gd[N][K - 1] == kth and gd[N][K - 2] == _ulps(kth, -1)
