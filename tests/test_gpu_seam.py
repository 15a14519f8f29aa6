"""The kernel launch seam end to end (GPU): the whole pipeline driven through
the C ABI's frnn_launch_* entry points, with the queries given as the second
array (frnn_queries_t), as the reference's run_find_nbrs(d_points1 = queries,
d_points2 = points, ...) (find_nbrs.cu:562-567) and run_bruteforce(d_p1,
d_p2, P1, P2, ...) (no_grid_frnn.cu:273-276) take them; and the capacity
guard's status word, forced from the host with a list too short for a round.
"""
import ctypes

import numpy as np
import pytest

import frnn_cuda
import frnn_oracle as O
from gpu_util import assert_rows_equal, device_soa, log, torch, vp
from test_oracle_pins import separate_queries, unit_cloud

pytestmark = pytest.mark.gpu


def _dev(n, dtype):
    t = torch()
    return t.empty(max(int(n), 1), dtype=dtype, device="cuda:0")


def _grid_side(L, d, N, D, plan, sws, fws):
    """bin/count + scan + reorder of N rows (points or queries) on the plan's
    grid (the frame workspace fws is the points')."""
    t = torch()
    cells = L.frnn_grid_cells(N, D, ctypes.byref(plan)) if fws is not None else plan.cells
    cell_of, rank = _dev(N, t.int32), _dev(N, t.int32)
    cnt = _dev(cells + 1, t.int32)
    assert L.frnn_launch_bin_count(vp(d), N, plan.grid_dim, plan.res, ctypes.c_float(plan.inv_cell), cells,
                                   vp(fws), vp(cell_of), vp(rank), vp(cnt), None) == 0
    start = _dev(cells + 1, t.int32)
    part = _dev(frnn_cuda.scan_partials_count(cells + 1), t.int32)
    assert L.frnn_launch_exclusive_scan(vp(cnt), cells + 1, vp(start), vp(part), None) == 0
    ds = frnn_cuda.aos_stride(D)
    sidx, inv = _dev(N, t.int32), _dev(N, t.int32)
    aos = _dev(N * ds, t.float32)
    frows = _dev(N * ds, t.float32) if L.frnn_uses_filter_rows(D) else None
    assert L.frnn_launch_reorder(vp(d), N, D, vp(cell_of), vp(rank), vp(start), vp(sidx), vp(inv), vp(aos),
                                 vp(sws), vp(frows), None) == 0
    return dict(cell_of=cell_of, start=start, sidx=sidx, inv=inv, aos=aos, frows=frows, keep=(cnt, part))


def _bf_side(L, d, N, D, sws):
    t = torch()
    ds = frnn_cuda.aos_stride(D)
    aos = _dev(N * ds, t.float32)
    frows = _dev(N * ds, t.float32) if L.frnn_uses_filter_rows(D) else None
    assert L.frnn_launch_transpose(vp(d), N, D, vp(aos), vp(sws), vp(frows), None) == 0
    return dict(cell_of=None, start=None, sidx=None, inv=None, aos=aos, frows=frows)


def seam_search(P, Q, K, r, list_cap=None):
    """M queries Q against N points P through the launch seam.  Returns
    ([M, K] idx, [M, K] dist, status word, plan path)."""
    t = torch()
    L = frnn_cuda._load()
    N, D = P.shape
    M = Q.shape[0]
    plan = frnn_cuda._plan_struct(N, D, K, r)
    dp, dq = device_soa(P), device_soa(Q)
    sws = _dev(L.frnn_stats_workspace_bytes(D), t.uint8)
    assert L.frnn_launch_point_stats(vp(dp), N, D, vp(sws), None) == 0
    bf = plan.path == 0
    fws = None
    if not bf:
        fb = L.frnn_frame_workspace_bytes(N, D, ctypes.byref(plan))
        if fb > 0:
            fws = _dev(fb, t.uint8)
            assert L.frnn_launch_frame(vp(dp), N, D, ctypes.byref(plan), vp(sws), vp(fws), None) == 0
    pts = _bf_side(L, dp, N, D, sws) if bf else _grid_side(L, dp, N, D, plan, sws, fws)
    qs = _bf_side(L, dq, M, D, sws) if bf else _grid_side(L, dq, M, D, plan, sws, fws)
    queries = frnn_cuda.Queries(M, qs["aos"].data_ptr(), qs["frows"].data_ptr() if qs["frows"] is not None else None,
                                qs["sidx"].data_ptr() if not bf else None,
                                qs["cell_of"].data_ptr() if not bf else None)
    cap = list_cap or frnn_cuda.list_capacity(K)
    lists = _dev(M * cap, t.int64)
    status = t.zeros(1, dtype=t.int32, device="cuda:0")
    rc = L.frnn_launch_find_nbrs(vp(pts["aos"]), vp(pts["frows"]), vp(sws), vp(pts["sidx"]), vp(pts["cell_of"]),
                                 vp(pts["start"]), vp(fws), N, D, K, ctypes.byref(plan), ctypes.byref(queries),
                                 vp(lists), cap, None, vp(status), None)
    assert rc == 0, L.frnn_last_error()
    idx, dist = _dev(K * M, t.int32), _dev(K * M, t.float32)
    assert L.frnn_launch_unpermute(vp(lists), cap, vp(qs["inv"]), M, K, vp(idx), vp(dist), None) == 0
    t.cuda.synchronize()
    gi = idx.cpu().numpy()[:K * M].reshape(K, M).T
    gd = dist.cpu().numpy()[:K * M].reshape(K, M).T
    return gi, gd, int(status.item()), frnn_cuda.PATH_NAMES[plan.path]


@pytest.mark.parametrize("label,D,k,N,M,r,K,path", [
    ("framed_first_d12", 12, 3, 30000, 7000, 0.1, 32, "grid_first"),
    ("raw_full_d3", 3, 3, 20000, 5000, 0.05, 16, "grid_full"),
    ("bf_d64_filter_rows", 64, 4, 3000, 900, 0.6, 32, "bruteforce"),
    ("bf_d16", 16, 4, 2000, 700, 0.4, 16, "bruteforce"),
])
def test_seam_two_array_form(label, D, k, N, M, r, K, path):
    X = unit_cloud(N, D, k, 41)
    Q = separate_queries(X, M, 9)
    log(f"seam two-array {label}: N={N} M={M} D={D} K={K} r={r}")
    gi, gd, st, p = seam_search(X, Q, K, r)
    assert p == path and st == 0
    ri, rd = O.search_queries(X, Q, K, r)
    assert_rows_equal(gi, gd, ri, rd, f"seam {label}")


def test_short_lists_that_still_fit_are_exact():
    # list_cap between K and the default: compactions are more frequent, and
    # no round overflows (cap - 64 >= K + 32 leaves room after each one)
    X = unit_cloud(20000, 3, 3, 43)
    Q = separate_queries(X, 4000, 10)
    gi, gd, st, _ = seam_search(X, Q, 16, 0.08, list_cap=128)
    assert st == 0
    ri, rd = O.search_queries(X, Q, 16, 0.08)
    assert_rows_equal(gi, gd, ri, rd, "cap 128")


@pytest.mark.parametrize("D,r", [(3, 0.1), (64, 0.9)])
def test_list_overflow_sets_the_status_word(D, r):
    """A list of exactly K entries cannot hold a round of new keys: the
    kernel's capacity guard drops them (no write past the list) and sets the
    caller's status word; the kernel still runs to completion."""
    X = unit_cloud(6000 if D == 3 else 2000, D, 3 if D == 3 else 4, 44)
    Q = X[:1500].copy()
    log(f"forced overflow D={D}")
    _, _, st, _ = seam_search(X, Q, 8, r, list_cap=8)
    assert st == 1
