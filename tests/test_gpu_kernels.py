"""Per-kernel parity of the grid build through the C-ABI launch seam (GPU).

bin/count  vs the oracle's clamped binning and numpy bincount
scan       vs numpy cumsum (exclusive)
reorder    permutation / cell-order / row-copy invariants
frame      descriptor, binning recomputed in exact fp32 (fine axis 0), the
           3^g shell guarantee on sampled pairs
"""
import ctypes

import numpy as np
import pytest

import exact_fp32 as E
import frnn_cuda
import frnn_oracle as O
import frnn_workloads as W
from gpu_util import assert_rows_equal, device_soa, log, torch, vp

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
    rc = L.frnn_launch_bin_count(vp(d), N, g, res, ctypes.c_float(inv), cells, None, vp(cell_of),
                                 vp(rank), vp(cnt), None)
    assert rc == 0
    start = t.empty(cells + 1, dtype=t.int32, device="cuda:0")
    part = t.empty(frnn_cuda.scan_partials_count(cells + 1), dtype=t.int32, device="cuda:0")
    assert L.frnn_launch_exclusive_scan(vp(cnt), cells + 1, vp(start), vp(part), None) == 0
    D = X.shape[1]
    ds = frnn_cuda.aos_stride(D)
    sidx = t.empty(N, dtype=t.int32, device="cuda:0")
    inv_p = t.empty(N, dtype=t.int32, device="cuda:0")
    aos = t.full((N * ds,), float("nan"), dtype=t.float32, device="cuda:0")
    assert L.frnn_launch_reorder(vp(d), N, D, vp(cell_of), vp(rank), vp(start), vp(sidx), vp(inv_p), vp(aos),
                                 None, None, None) == 0
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


@pytest.mark.parametrize("n,off_in,off_out", [(4097, 1, 0), (100_003, 0, 3), (9, 2, 2), (1_000_001, 3, 1)])
def test_exclusive_scan_unaligned(n, off_in, off_out):
    """Arrays that are not 16-byte aligned (offset by whole ints) take the
    per-int path; lengths that are not multiples of 4 exercise the tails."""
    t = torch()
    rs = np.random.RandomState(n % 997)
    a = rs.randint(0, 64, n).astype(np.int32)
    buf_in = t.full((n + 4,), 12345, dtype=t.int32, device="cuda:0")
    buf_in[off_in:off_in + n] = t.from_numpy(a).to("cuda:0")
    buf_out = t.full((n + 4,), -1, dtype=t.int32, device="cuda:0")
    part = t.empty(frnn_cuda.scan_partials_count(n), dtype=t.int32, device="cuda:0")
    log(f"scan unaligned n={n} off_in={off_in} off_out={off_out}")
    assert frnn_cuda._load().frnn_launch_exclusive_scan(vp(buf_in[off_in:]), n, vp(buf_out[off_out:]),
                                                        vp(part), None) == 0
    t.cuda.synchronize()
    got = buf_out.cpu().numpy()
    want = np.concatenate([[0], np.cumsum(a.astype(np.int64))[:-1]])
    assert np.array_equal(got[off_out:off_out + n].astype(np.int64), want)
    assert np.all(got[:off_out] == -1) and np.all(got[off_out + n:] == -1)


@pytest.mark.parametrize("off", [0, 1, 2, 3])
def test_bin_count_zero_fills_unaligned_counts(off):
    """bin/count zero-fills its count array itself (garbage before, guards
    around it untouched), also when the array is not 16-byte aligned."""
    t = torch()
    rs = np.random.RandomState(7 + off)
    N, res = 5000, 37
    X = rs.rand(N, 2).astype(np.float32)
    inv = float(np.float32(1.0) / np.float32(1.0 / res))
    cells = res * res
    d = device_soa(X)
    buf = t.full((cells + 1 + 8,), -7, dtype=t.int32, device="cuda:0")
    cell_of = t.empty(N, dtype=t.int32, device="cuda:0")
    rank = t.empty(N, dtype=t.int32, device="cuda:0")
    log(f"bin/count unaligned counts off={off}")
    assert frnn_cuda._load().frnn_launch_bin_count(vp(d), N, 2, res, ctypes.c_float(inv), cells, None,
                                                   vp(cell_of), vp(rank), vp(buf[off:]), None) == 0
    t.cuda.synchronize()
    got = buf.cpu().numpy()
    want = np.bincount(O.bin_cells(X, 2, res, np.float32(inv)), minlength=cells + 1)
    assert np.array_equal(got[off:off + cells + 1], want)
    assert np.all(got[:off] == -7) and np.all(got[off + cells + 1:] == -7)


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


def _project(X, fi, slots):
    """Frame projections in fp32: s = fma(dir[k][t], fl(x[coord[t]] - mean[t]), s) over the terms."""
    out = []
    for k in slots:
        s = np.zeros(len(X), np.float32)
        for t in range(fi.terms):
            y = (X[:, fi.coord[t]] - np.float32(fi.mean[t])).astype(np.float32)
            s = E.fma32(np.float32(fi.dir[k][t]), y, s)
        out.append(s)
    return out


def _frame_build(X, K, radius):
    """stats -> frame -> bin/count -> scan -> reorder through the seam, as the engine runs them."""
    t = torch()
    N, D = X.shape
    plan = frnn_cuda._plan_struct(N, D, K, radius)
    L = frnn_cuda._load()
    cells = L.frnn_grid_cells(N, D, ctypes.byref(plan))
    d = device_soa(X)
    sws = t.zeros(L.frnn_stats_workspace_bytes(D), dtype=t.uint8, device="cuda:0")
    assert L.frnn_launch_point_stats(vp(d), N, D, vp(sws), None) == 0
    wsb = L.frnn_frame_workspace_bytes(N, D, ctypes.byref(plan))
    assert wsb > 0
    ws = t.zeros(wsb, dtype=t.uint8, device="cuda:0")
    assert L.frnn_launch_frame(vp(d), N, D, ctypes.byref(plan), vp(sws), vp(ws), None) == 0
    cell_of = t.empty(N, dtype=t.int32, device="cuda:0")
    rank = t.empty(N, dtype=t.int32, device="cuda:0")
    cnt = t.empty(cells + 1, dtype=t.int32, device="cuda:0")
    assert L.frnn_launch_bin_count(vp(d), N, plan.grid_dim, plan.res, ctypes.c_float(plan.inv_cell), cells,
                                   vp(ws), vp(cell_of), vp(rank), vp(cnt), None) == 0
    start = t.empty(cells + 1, dtype=t.int32, device="cuda:0")
    part = t.empty(frnn_cuda.scan_partials_count(cells + 1), dtype=t.int32, device="cuda:0")
    assert L.frnn_launch_exclusive_scan(vp(cnt), cells + 1, vp(start), vp(part), None) == 0
    ds = frnn_cuda.aos_stride(D)
    sidx = t.empty(N, dtype=t.int32, device="cuda:0")
    inv_p = t.empty(N, dtype=t.int32, device="cuda:0")
    aos = t.empty(N * ds, dtype=t.float32, device="cuda:0")
    frows = t.empty(N * ds, dtype=t.float32, device="cuda:0")
    assert L.frnn_launch_reorder(vp(d), N, D, vp(cell_of), vp(rank), vp(start), vp(sidx), vp(inv_p), vp(aos),
                                 vp(sws), vp(frows), None) == 0
    t.cuda.synchronize()
    out = {k: v.cpu().numpy() for k, v in dict(cell_of=cell_of, rank=rank, cnt=cnt, start=start, sidx=sidx,
                                                 inv=inv_p, aos=aos, frows=frows).items()}
    out["frame"] = frnn_cuda.FrameInfo.from_workspace(ws[:4096].cpu().numpy())
    out["stats"] = sws[:16 * D].cpu().numpy().view(np.float32).reshape(D, 4)
    out["plan"], out["cells"] = plan, cells
    return out


def _near_pairs(X, radius, nq=400, seed=5):
    """(q, p) pairs with exact fp32 distance < r2, for nq random queries."""
    N = len(X)
    rs = np.random.RandomState(seed)
    r = float(np.float32(radius))
    r2 = np.float32(np.float32(radius) ** 2)
    X64 = X.astype(np.float64)
    n2 = np.sum(X64 ** 2, 1)
    Q, P = [], []
    for qb in np.array_split(rs.randint(0, N, nq), 8):
        near = (n2[None, :] + n2[qb, None] - 2 * X64[qb] @ X64.T) <= (1.01 * r) ** 2
        qq, pp = np.nonzero(near)
        qq = qb[qq]
        inside = E.dist2(X[qq], X[pp], 0) < r2
        Q.append(qq[inside])
        P.append(pp[inside])
    return np.concatenate(Q), np.concatenate(P)


@pytest.mark.parametrize("name,N", [("metric", 300_000), ("C3", 300_000)])
def test_frame_grid(name, N):
    """The grid frame of first-coordinate plans: descriptor (terms, directions,
    margin, geometry with a fine axis 0), the binning recomputed in exact fp32,
    the guarantee that pairs within the radius fall in neighbouring cells of
    edge h and the reorder invariants."""
    w = W.config(name, N=N)
    log(f"frame {name} N={N}")
    out = _frame_build(w.X, w.K, w.radius)
    fi, plan, cap = out["frame"], out["plan"], out["cells"]
    g = plan.grid_dim
    assert plan.path == 2 and g == 4 and fi.grid_dim == g and fi.projected == 1
    st = out["stats"]
    mean, var, lo, hi = (st[:, k] for k in range(4))
    T = min(w.D, 32)
    assert fi.terms == T
    # terms: the highest-variance coordinates, lower index on ties
    coord = np.array(fi.coord[:T])
    assert np.array_equal(coord, np.argsort(-var, kind="stable")[:T])
    assert np.array_equal(np.array(fi.mean[:T], np.float32), mean[coord])
    # directions: orthonormal up to the 1 - 2^-18 shrink; the grid block has
    # spectral norm < 1, so projected gaps lower-bound distances
    dirs = fi.directions()[:, :T].astype(np.float64)
    slots = list(range(g))
    Wm = dirs[slots]
    G = Wm @ Wm.T
    assert np.all(np.abs(np.diag(G) - 1) < 1e-5) and np.all(np.diag(G) < 1)
    assert np.max(np.abs(G - np.diag(np.diag(G)))) < 1e-5
    assert np.linalg.norm(dirs[:g], 2) < 1
    # the directions capture (nearly) the variance of the leading principal
    # subspace (covariance from a sample of >= 128K points: 3% tolerance)
    Y = (w.X[:, coord] - mean[coord]).astype(np.float64)
    C = Y.T @ Y / N
    ev = np.linalg.eigvalsh(C)[::-1]
    captured = sum(wk @ C @ wk for wk in Wm)
    assert captured >= 0.97 * ev[:len(slots)].sum(), (captured, ev[:len(slots) + 1])
    for k in slots:
        sg = np.sqrt(dirs[k] @ C @ dirs[k])
        assert abs(fi.sigma[k] / sg - 1) <= 0.03
    # margin >= (T + 2) u |x - mean| over the input
    R = np.sqrt(np.sum(np.maximum(hi[coord].astype(np.float64) - mean[coord],
                                  mean[coord] - lo[coord].astype(np.float64)) ** 2))
    u = 2.0 ** -24
    assert (T + 2) * u * R <= fi.margin <= 1.01 * (T + 2) * u * R
    # geometry: cell edge >= r (1 + 2^-12) + 2 margin + 2 slack, binning
    # reciprocal rounded down, grid within the capacity;
    # axis 0 split into fine0 cells of edge h / fine0 (exact scalings)
    r = float(np.float32(w.radius))
    h0 = r * (1 + 2.0 ** -12) + 2 * fi.margin
    smax = max(fi.sigma[k] for k in range(g))
    assert fi.slack >= 2.0 ** -18 * (4 * smax + h0)
    assert fi.h >= h0 + 2 * fi.slack and float(fi.inv_h) * float(fi.h) <= 1.0
    F = fi.fine0
    assert F == 8 and np.float32(fi.h0) * F == np.float32(fi.h) and np.float32(fi.inv_h0) == np.float32(fi.inv_h) * F
    res = np.array(fi.res[:g])
    assert res[0] % F == 0
    assert np.all(res >= 1) and fi.cells == np.prod(res) <= cap
    assert list(fi.stride[:g]) == [int(np.prod(res[:d])) for d in range(g)]
    # cells per axis: max(1, floor(8 sigma / h)); split axes centred on the mean
    for d in range(g):
        coarse = fi.res[d] // (F if d == 0 else 1)
        m = max(1, int(np.floor(8.0 * np.float64(fi.sigma[d]) / np.float64(fi.h))))
        assert coarse in (m, m + 1)      # the kernel divides by h before its fp32 round-up
        if coarse >= 2:
            assert fi.lo[d] == np.float32(-0.5 * coarse * np.float64(np.float32(fi.h)))
    # binning, recomputed in exact fp32
    S = _project(w.X, fi, slots)
    cc = np.stack([_sub_bins(S[d], fi.lo[d], fi.inv_h0 if d == 0 else fi.inv_h, fi.res[d]) for d in range(g)], 1)
    cell_of = cc @ np.array(fi.stride[:g])
    assert np.array_equal(out["cell_of"], cell_of)
    cnt = np.bincount(cell_of, minlength=cap + 1)
    assert np.array_equal(out["cnt"], cnt)
    # the shell guarantee: pairs within the radius sit in neighbouring cells of
    # edge h (axis 0: fine cell // fine0, the same as binning with inv_h), and
    # their projections differ by at most r (1 + 2^-15) + 2 margin
    qq, pp = _near_pairs(w.X, w.radius)
    assert len(qq) > 1000
    coarse = cc.copy()
    coarse[:, 0] //= F
    assert np.array_equal(coarse[:, 0], _sub_bins(S[0], fi.lo[0], fi.inv_h, fi.res[0] // F))
    assert np.max(np.abs(coarse[qq] - coarse[pp])) <= 1
    for s in S:
        assert np.max(np.abs(s[pp].astype(np.float64) - s[qq])) <= r * (1 + 2.0 ** -15) + 2 * fi.margin
    # reorder invariants
    sidx, inv_p = out["sidx"], out["inv"]
    assert np.array_equal(np.sort(sidx), np.arange(N))
    assert np.array_equal(sidx[inv_p], np.arange(N))
    cs = cell_of[sidx]
    assert np.all(np.diff(cs) >= 0)
    ds = frnn_cuda.aos_stride(w.D)
    assert np.array_equal(out["aos"].reshape(N, ds)[:, :w.D], w.X[sidx])
    # centred filter rows: fl(x - mean), zero padded
    fr = out["frows"].reshape(N, ds)
    assert np.array_equal(fr[:, :w.D], (w.X[sidx] - mean[None, :]).astype(np.float32))
    assert np.all(fr[:, w.D:] == 0)
    log(f"  res={list(res)} h/r={fi.h / r:.3f} cells={fi.cells}")


@pytest.mark.parametrize("D,r", [(3, 0.1), (2, 0.02), (4, 0.25)])
def test_raw_frame_on_full_grid(D, r):
    """Full-D grids with at most 4 axes bin through a raw frame: the plan's
    own cells on the raw coordinates, axis 0 split 8 ways (fine cell // 8 is
    the reference's cell coordinate)."""
    rs = np.random.RandomState(40 + D)
    X = rs.rand(100_000, D).astype(np.float32)
    X[:3] = np.float32(1.0)                       # x = 1.0 clamps into the last cell
    out = _frame_build(X, 16, r)
    fi, plan = out["frame"], out["plan"]
    g, F = plan.grid_dim, fi.fine0
    assert plan.path == 1 and g == D and fi.projected == 0 and fi.terms == 0 and F == 8
    assert fi.cells == F * plan.cells == out["cells"]
    assert list(fi.res[:g]) == [F * plan.res] + [plan.res] * (g - 1)
    assert np.float32(fi.h) == np.float32(plan.cell_size) and np.float32(fi.inv_h0) == np.float32(plan.inv_cell) * F
    fine_x = np.clip(np.floor(X[:, 0] * np.float32(plan.inv_cell * F)), 0, F * plan.res - 1).astype(np.int64)
    ref = O.bin_cells(X, g, plan.res, np.float32(plan.inv_cell))
    assert np.array_equal(fine_x // F, ref % plan.res)
    assert np.array_equal(out["cell_of"], fine_x + F * plan.res * (ref // plan.res))


def test_frame_falls_back_to_raw_coordinates_on_infinite_input():
    """An infinite coordinate makes the projection bound infinite: the frame
    then bins the raw first g coordinates on the plan's own grid."""
    rs = np.random.RandomState(12)
    X = rs.rand(20000, 12).astype(np.float32)
    X[17, 2] = np.inf
    out = _frame_build(X, 16, 0.1)
    fi, plan = out["frame"], out["plan"]
    assert plan.path == 2 and fi.projected == 0
    g, F = plan.grid_dim, fi.fine0
    assert fi.cells == F * plan.cells and list(fi.res[:g]) == [F * plan.res] + [plan.res] * (g - 1)
    # the plan's cells, axis 0 split F ways: fine x, then the reference's hash
    # of the other coordinates
    fine_x = np.clip(np.floor(X[:, 0] * np.float32(plan.inv_cell * F)), 0, F * plan.res - 1).astype(np.int64)
    ref = O.bin_cells(X, g, plan.res, np.float32(plan.inv_cell))
    want = fine_x + F * plan.res * (ref // plan.res)
    assert np.array_equal(out["cell_of"], want)


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


@pytest.mark.parametrize("framed", [True, False])
def test_seam_search_first_coordinate_plan(framed):
    """The whole search through the launch seam on a first-coordinate plan,
    with the frame and without it (raw first coordinates, as the reference
    bins them): both give the oracle's rows."""
    t = torch()
    rs = np.random.RandomState(31)
    N, D, K, r = 30000, 12, 32, 0.1
    X = rs.rand(N, D).astype(np.float32)
    plan = frnn_cuda._plan_struct(N, D, K, r)
    assert plan.path == 2
    L = frnn_cuda._load()
    ws_bytes = L.frnn_frame_workspace_bytes(N, D, ctypes.byref(plan))
    assert ws_bytes > 0
    d = device_soa(X)
    cells = L.frnn_grid_cells(N, D, ctypes.byref(plan)) if framed else plan.cells
    sws = t.zeros(L.frnn_stats_workspace_bytes(D), dtype=t.uint8, device="cuda:0")
    assert L.frnn_launch_point_stats(vp(d), N, D, vp(sws), None) == 0
    ws = None
    if framed:
        ws = t.zeros(ws_bytes, dtype=t.uint8, device="cuda:0")
        assert L.frnn_launch_frame(vp(d), N, D, ctypes.byref(plan), vp(sws), vp(ws), None) == 0
    cell_of = t.empty(N, dtype=t.int32, device="cuda:0")
    rank = t.empty(N, dtype=t.int32, device="cuda:0")
    cnt = t.empty(cells + 1, dtype=t.int32, device="cuda:0")
    assert L.frnn_launch_bin_count(vp(d), N, plan.grid_dim, plan.res, ctypes.c_float(plan.inv_cell), cells,
                                   vp(ws), vp(cell_of), vp(rank), vp(cnt), None) == 0
    start = t.empty(cells + 1, dtype=t.int32, device="cuda:0")
    part = t.empty(frnn_cuda.scan_partials_count(cells + 1), dtype=t.int32, device="cuda:0")
    assert L.frnn_launch_exclusive_scan(vp(cnt), cells + 1, vp(start), vp(part), None) == 0
    ds = frnn_cuda.aos_stride(D)
    sidx = t.empty(N, dtype=t.int32, device="cuda:0")
    inv_p = t.empty(N, dtype=t.int32, device="cuda:0")
    aos = t.empty(N * ds, dtype=t.float32, device="cuda:0")
    assert L.frnn_uses_filter_rows(D) == 0
    assert L.frnn_launch_reorder(vp(d), N, D, vp(cell_of), vp(rank), vp(start), vp(sidx), vp(inv_p), vp(aos),
                                 None, None, None) == 0
    cap = frnn_cuda.list_capacity(K)
    lists = t.empty(N * cap, dtype=t.int64, device="cuda:0")
    assert L.frnn_launch_find_nbrs(vp(aos), None, vp(sws), vp(sidx), vp(cell_of), vp(start), vp(ws),
                                   N, D, K, ctypes.byref(plan), None, vp(lists), cap, None, None, None) == 0
    idx = t.empty(K * N, dtype=t.int32, device="cuda:0")
    dist = t.empty(K * N, dtype=t.float32, device="cuda:0")
    assert L.frnn_launch_unpermute(vp(lists), cap, vp(inv_p), N, K, vp(idx), vp(dist), None) == 0
    t.cuda.synchronize()
    gi = idx.cpu().numpy().reshape(K, N).T
    gd = dist.cpu().numpy().reshape(K, N).T
    ri, rd = O.search(X, K, r)
    assert_rows_equal(gi, gd, ri, rd, f"seam framed={framed}")
