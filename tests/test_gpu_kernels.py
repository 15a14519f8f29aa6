"""Per-kernel parity of the grid build through the C-ABI launch seam (GPU).

bin/count  vs the oracle's clamped binning and numpy bincount
scan       vs numpy cumsum (exclusive)
reorder    permutation / cell-order / row-copy invariants
"""
import ctypes

import numpy as np
import pytest

import exact_fp32 as E
import frnn_cuda
import frnn_oracle as O
import frnn_workloads as W
from gpu_util import device_soa, log, torch, vp

pytestmark = pytest.mark.gpu


def _build(X, g, res, inv):
    t = torch()
    N = X.shape[0]
    cells = res ** g
    L = frnn_cuda._load()
    d = device_soa(X)
    cell_of = t.empty(N, dtype=t.int32, device="cuda:0")
    rank = t.empty(N, dtype=t.int32, device="cuda:0")
    cnt = t.full((cells + 1,), -7, dtype=t.int32, device="cuda:0")
    rc = L.frnn_launch_bin_count(vp(d), N, g, res, ctypes.c_float(inv), cells, vp(cell_of), vp(rank),
                                 vp(cnt), None)
    assert rc == 0
    start = t.empty(cells + 1, dtype=t.int32, device="cuda:0")
    part = t.empty(frnn_cuda.scan_partials_count(cells + 1), dtype=t.int32, device="cuda:0")
    assert L.frnn_launch_exclusive_scan(vp(cnt), cells + 1, vp(start), vp(part), None) == 0
    D = X.shape[1]
    ds = frnn_cuda.aos_stride(D)
    sidx = t.empty(N, dtype=t.int32, device="cuda:0")
    inv_p = t.empty(N, dtype=t.int32, device="cuda:0")
    aos = t.full((N * ds,), float("nan"), dtype=t.float32, device="cuda:0")
    assert L.frnn_launch_reorder(vp(d), N, D, vp(cell_of), vp(rank), vp(start), vp(cnt), None, cells,
                                 vp(sidx), vp(inv_p), vp(aos), None, None, None, None) == 0
    t.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in dict(cell_of=cell_of, rank=rank, cnt=cnt, start=start,
                                                  sidx=sidx, inv=inv_p, aos=aos).items()}


@pytest.mark.parametrize("name,N", [("C1", 200_000), ("C2", 300_000), ("metric", 200_000)])
def test_build_pipeline_parity(name, N):
    w = W.config(name, N=N)
    p = O.plan(1_000_000 if name != "C1" else N, w.D, w.K, w.radius)  # full-size grid geometry
    g, res = p["grid_dim"], p["res"]
    inv = np.float32(1.0) / np.float32(w.radius)
    log(f"build parity {name} N={N} g={g} res={res}")
    out = _build(w.X, g, res, float(inv))
    cells = res ** g
    want_cells = O.bin_cells(w.X, g, res, inv)
    assert np.array_equal(out["cell_of"], want_cells)
    cnt = np.bincount(want_cells, minlength=cells + 1)
    assert np.array_equal(out["cnt"], cnt)
    # ranks: within each cell, a permutation of 0..count-1
    order = np.lexsort((out["rank"], want_cells))
    c_sorted = want_cells[order]
    first = np.searchsorted(c_sorted, c_sorted, side="left")
    assert np.array_equal(out["rank"][order], np.arange(N) - first)
    start = np.concatenate([[0], np.cumsum(cnt)[:-1]])
    assert np.array_equal(out["start"], start)
    sidx, inv_p = out["sidx"], out["inv"]
    assert np.array_equal(np.sort(sidx), np.arange(N))
    assert np.array_equal(sidx[inv_p], np.arange(N))
    assert np.all(np.diff(want_cells[sidx]) >= 0)
    ds = frnn_cuda.aos_stride(w.D)
    rows = out["aos"].reshape(N, ds)
    assert np.array_equal(rows[:, :w.D], w.X[sidx])
    assert np.all(rows[:, w.D:] == 0)


@pytest.mark.parametrize("n", [1, 2, 4095, 4096, 4097, 100_003, 1_000_001, 4096 * 4096])
def test_exclusive_scan(n):
    t = torch()
    rs = np.random.RandomState(n % 1000)
    a = rs.randint(0, 64, n).astype(np.int32)
    if n > 1:
        a[-1] = 0
    d_in = t.from_numpy(a).to("cuda:0")
    d_out = t.full((n,), -1, dtype=t.int32, device="cuda:0")
    part = t.empty(frnn_cuda.scan_partials_count(n), dtype=t.int32, device="cuda:0")
    log(f"scan n={n}")
    assert frnn_cuda._load().frnn_launch_exclusive_scan(vp(d_in), n, vp(d_out), vp(part), None) == 0
    t.cuda.synchronize()
    want = np.concatenate([[0], np.cumsum(a.astype(np.int64))[:-1]])
    assert np.array_equal(d_out.cpu().numpy().astype(np.int64), want)


def test_scan_rejects_oversize():
    t = torch()
    assert frnn_cuda._load().frnn_launch_exclusive_scan(None, 4096 * 4096 + 1, None, None, None) == 1
    n = 4096 * 4096 + 1
    d = t.zeros(n, dtype=t.int32, device="cuda:0")
    part = t.empty(frnn_cuda.scan_partials_count(n), dtype=t.int32, device="cuda:0")
    assert frnn_cuda._load().frnn_launch_exclusive_scan(vp(d), n, vp(d), vp(part), None) == 2


def test_bin_count_out_of_domain_and_nan():
    X = np.array([[-5.0, 0.5], [0.5, 7.0], [1.0, 1.0], [np.nan, 0.2], [0.0, -0.0], [0.9999, 0.25]],
                 np.float32)
    res, inv = 4, float(np.float32(1.0) / np.float32(0.25))
    out = _build(X, 2, res, inv)
    assert np.array_equal(out["cell_of"], O.bin_cells(X, 2, res, np.float32(inv)))
    assert list(out["cell_of"][:3]) == [0 + 4 * 2, 2 + 4 * 3, 3 + 4 * 3]


def _sub_bins(x, lo, inv, nb):
    t = (x.astype(np.float32) - np.float32(lo)).astype(np.float32) * np.float32(inv)
    f = np.fmin(np.fmax(np.floor(t.astype(np.float32)), np.float32(0)), np.float32(nb - 1))
    return f.astype(np.int64)


def _project(X, ri):
    """The refinement projections in fp32: s = fma(w[t], fl(x[coord[t]] - mean[t]), s)."""
    s0 = np.zeros(len(X), np.float32)
    s1 = np.zeros(len(X), np.float32)
    for t in range(ri.terms):
        y = (X[:, ri.coord[t]] - np.float32(ri.mean[t])).astype(np.float32)
        s0 = E.fma32(np.float32(ri.w0[t]), y, s0)
        s1 = E.fma32(np.float32(ri.w1[t]), y, s1)
    return s0, s1


@pytest.mark.parametrize("name,N", [("metric", 300_000), ("C3", 300_000)])
def test_refinement_orders_big_cells(name, N):
    """Within-cell refinement: the projection descriptor (terms, weights, margin,
    bin geometry), the sub-bin order inside big cells, and the usual permutation /
    cell-order / row-copy invariants of the reorder."""
    t = torch()
    w = W.config(name, N=N)
    plan = frnn_cuda._plan_struct(N, w.D, w.K, w.radius)
    assert plan.path == 2 and plan.grid_dim == 4
    g, res, cells = plan.grid_dim, plan.res, plan.cells
    L = frnn_cuda._load()
    log(f"refinement {name} N={N} res={res}")
    d = device_soa(w.X)
    cell_of = t.empty(N, dtype=t.int32, device="cuda:0")
    rank = t.empty(N, dtype=t.int32, device="cuda:0")
    cnt = t.empty(cells + 1, dtype=t.int32, device="cuda:0")
    assert L.frnn_launch_bin_count(vp(d), N, g, res, ctypes.c_float(plan.inv_cell), cells, vp(cell_of),
                                   vp(rank), vp(cnt), None) == 0
    start = t.empty(cells + 1, dtype=t.int32, device="cuda:0")
    part = t.empty(frnn_cuda.scan_partials_count(cells + 1), dtype=t.int32, device="cuda:0")
    assert L.frnn_launch_exclusive_scan(vp(cnt), cells + 1, vp(start), vp(part), None) == 0
    sws = t.zeros(L.frnn_stats_workspace_bytes(w.D), dtype=t.uint8, device="cuda:0")
    assert L.frnn_launch_point_stats(vp(d), N, w.D, vp(sws), None) == 0
    wsb = L.frnn_refine_workspace_bytes(N, w.D, ctypes.byref(plan))
    assert wsb > 0
    ws = t.zeros(wsb, dtype=t.uint8, device="cuda:0")
    assert L.frnn_launch_refine(vp(d), N, w.D, ctypes.byref(plan), vp(cell_of), vp(cnt), vp(rank),
                                vp(sws), vp(ws), None) == 0
    ds = frnn_cuda.aos_stride(w.D)
    sidx = t.empty(N, dtype=t.int32, device="cuda:0")
    inv_p = t.empty(N, dtype=t.int32, device="cuda:0")
    aos = t.empty(N * ds, dtype=t.float32, device="cuda:0")
    frows = t.empty(N * ds, dtype=t.float32, device="cuda:0")
    fnorm = t.empty(N, dtype=t.float32, device="cuda:0")
    assert L.frnn_launch_reorder(vp(d), N, w.D, vp(cell_of), vp(rank), vp(start), vp(cnt), vp(ws), cells,
                                 vp(sidx), vp(inv_p), vp(aos), vp(sws), vp(frows), vp(fnorm), None) == 0
    t.cuda.synchronize()
    ri = frnn_cuda.RefineInfo.from_workspace(ws[:1024].cpu().numpy())
    stats = sws[:16 * w.D].cpu().numpy().view(np.float32).reshape(w.D, 4)
    mean, var, lo, hi = (stats[:, k] for k in range(4))
    T = min(w.D - g, 32)
    assert ri.axes == 2 and ri.bins0 * ri.bins1 == 1024 and ri.terms == T
    # terms: the highest-variance non-grid coordinates, lower index on ties
    order = g + np.argsort(-var[g:], kind="stable")
    coord = np.array(ri.coord[:T])
    assert np.array_equal(coord, order[:T])
    assert np.array_equal(np.array(ri.mean[:T], np.float32), mean[coord])
    W0 = np.array(ri.w0[:T], np.float64)
    W1 = np.array(ri.w1[:T], np.float64)
    assert np.linalg.norm(W0) < 1 and np.linalg.norm(W1) < 1
    assert abs(np.linalg.norm(W0) - 1) < 1e-5 and abs(np.linalg.norm(W1) - 1) < 1e-5 and abs(W0 @ W1) < 1e-5
    # the directions capture (nearly) the variance of the top-2 principal
    # subspace of the terms; the subspace itself is ill-defined when the second
    # and third eigenvalues nearly tie (C3), and only pruning depends on it
    Y = (w.X[:, coord] - mean[coord]).astype(np.float64)
    C = Y.T @ Y / N
    ev = np.linalg.eigvalsh(C)[::-1]
    captured = W0 @ C @ W0 + W1 @ C @ W1
    assert captured >= 0.97 * (ev[0] + ev[1]), (captured, ev[:3])
    # bins span +-2.5 standard deviations of each projection (the library
    # estimates the covariance from a sample of >= 128K points: 3% tolerance)
    for wk, lok, invk, nbk in ((W0, ri.lo0, ri.inv0, ri.bins0), (W1, ri.lo1, ri.inv1, ri.bins1)):
        sg = np.sqrt(wk @ C @ wk)
        assert abs(lok + 2.5 * sg) <= 0.03 * 2.5 * sg and abs(invk * 5 * sg / nbk - 1) <= 0.03
        assert lok == np.float32(lok) and abs(invk * (-2 * lok) / nbk - 1) < 1e-5
    # margin >= (T + 2) u |x - mean| over the input
    R = np.sqrt(np.sum(np.maximum(hi[coord].astype(np.float64) - mean[coord], mean[coord] - lo[coord].astype(np.float64)) ** 2))
    assert ri.margin >= (T + 2) * 2.0 ** -24 * R
    assert ri.margin <= 1.01 * (T + 2) * 2.0 ** -24 * R
    # the window bound: pairs within the radius project within r(1 + 2^-15) + 2 margin
    s0, s1 = _project(w.X, ri)
    rs = np.random.RandomState(5)
    r = float(np.float32(w.radius))
    r2 = np.float32(np.float32(w.radius) ** 2)
    X64 = w.X.astype(np.float64)
    n2 = np.sum(X64 ** 2, 1)
    dmax = 0.0
    for qb in np.array_split(rs.randint(0, N, 400), 8):
        near = (n2[None, :] + n2[qb, None] - 2 * X64[qb] @ X64.T) <= (1.01 * r) ** 2
        qq, pp = np.nonzero(near)
        qq = qb[qq]
        inside = E.dist2(w.X[qq], w.X[pp], 0) < r2
        qq, pp = qq[inside], pp[inside]
        for s in (s0, s1):
            dmax = max(dmax, float(np.max(np.abs(s[pp].astype(np.float64) - s[qq]))))
    assert 0 < dmax <= r * (1 + 2.0 ** -15) + 2 * ri.margin
    # reorder invariants
    sidx, inv_p = sidx.cpu().numpy(), inv_p.cpu().numpy()
    cnt = cnt.cpu().numpy()[:cells]
    cells_of = O.bin_cells(w.X, g, res, np.float32(plan.inv_cell))
    assert np.array_equal(np.sort(sidx), np.arange(N))
    assert np.array_equal(sidx[inv_p], np.arange(N))
    cs = cells_of[sidx]
    assert np.all(np.diff(cs) >= 0)
    rows = aos.cpu().numpy().reshape(N, ds)
    assert np.array_equal(rows[:, :w.D], w.X[sidx])
    key = _sub_bins(s0[sidx], ri.lo0, ri.inv0, ri.bins0) * ri.bins1 + _sub_bins(s1[sidx], ri.lo1, ri.inv1, ri.bins1)
    # filter rows: fl(x - mean) and their sequential-fma squared norms
    fr = frows.cpu().numpy().reshape(N, ds)
    assert np.array_equal(fr[:, :w.D], (w.X[sidx] - mean[None, :]).astype(np.float32))
    assert np.all(fr[:, w.D:] == 0)
    assert np.array_equal(fnorm.cpu().numpy(), E.dist2(fr, np.zeros_like(fr), 0))
    big = cnt[cs] >= 256
    assert big.mean() > 0.5                      # most points live in refined cells here
    same_cell = np.concatenate([[False], cs[1:] == cs[:-1]])
    step = np.concatenate([[0], np.diff(key)])
    assert np.all(step[same_cell & big] >= 0)
    # the keys are not all equal: the refinement splits the big cells
    assert len(np.unique(key[big])) > 256


def test_point_stats():
    t = torch()
    rs = np.random.RandomState(2)
    X = (rs.standard_normal((100_003, 7)) * [1, 2, 3, 0.5, 10, 1e-3, 4] + [0, 1, -2, 5, 0, 1e3, 0]).astype(np.float32)
    X[5, 3] = np.nan                              # NaN column: mean falls back to 0, variance -1
    d = device_soa(X)
    L = frnn_cuda._load()
    sws = t.zeros(L.frnn_stats_workspace_bytes(7), dtype=t.uint8, device="cuda:0")
    assert L.frnn_launch_point_stats(vp(d), len(X), 7, vp(sws), None) == 0
    t.cuda.synchronize()
    st = sws[:16 * 7].cpu().numpy().view(np.float32).reshape(7, 4)
    X64 = X.astype(np.float64)
    for dd in range(7):
        if dd == 3:
            assert st[dd, 0] == 0 and st[dd, 1] == -1
            continue
        assert abs(st[dd, 0] - X64[:, dd].mean()) <= 1e-6 * (1 + abs(X64[:, dd].mean()))
        assert abs(st[dd, 1] - X64[:, dd].var()) <= 1e-5 * X64[:, dd].var()
        assert st[dd, 2] == X[:, dd].min() and st[dd, 3] == X[:, dd].max()
