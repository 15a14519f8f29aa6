"""The allocation-free scan (frnn_launch_exclusive_scan_noalloc) against the
scan with a caller workspace (frnn_launch_exclusive_scan), through the C ABI
(GPU).  Two calls in a row, the second on a smaller input, so the shared
device scratch holds the first call's partial sums when the second runs; and
the size limit is rejected before any launch."""
import ctypes

import numpy as np
import pytest

import frnn_cuda
from gpu_util import log, torch, vp

pytestmark = pytest.mark.gpu

MAX_N = 16_777_216


def _scan_both(x):
    t = torch()
    L = frnn_cuda._load()
    n = len(x)
    d_in = t.from_numpy(x).to("cuda:0")
    ref = t.full((n,), -1, dtype=t.int32, device="cuda:0")
    out = t.full((n,), -2, dtype=t.int32, device="cuda:0")
    part = t.empty(frnn_cuda.scan_partials_count(n), dtype=t.int32, device="cuda:0")
    assert L.frnn_launch_exclusive_scan(vp(d_in), n, vp(ref), vp(part), None) == 0
    assert L.frnn_launch_exclusive_scan_noalloc(vp(d_in), n, vp(out), None) == 0
    t.cuda.synchronize()
    return ref.cpu().numpy(), out.cpu().numpy()


@pytest.mark.parametrize("sizes", [(5_000_011, 40_961), (MAX_N, 4097)])
def test_noalloc_scan_matches_the_workspace_scan(sizes):
    rs = np.random.RandomState(len(sizes) + sizes[0] % 97)
    for n in sizes:
        x = rs.randint(0, 7, n).astype(np.int32)
        log(f"noalloc scan n={n}")
        ref, out = _scan_both(x)
        assert np.array_equal(out, ref)
        want = np.concatenate([[0], np.cumsum(x, dtype=np.int64)[:-1]])
        assert np.array_equal(out.astype(np.int64), want)


def test_noalloc_scan_limits():
    L = frnn_cuda._load()
    t = torch()
    d = t.zeros(4, dtype=t.int32, device="cuda:0")
    assert L.frnn_launch_exclusive_scan_noalloc(vp(d), MAX_N + 1, vp(d), None) == 2    # capacity
    assert b"16777216" in L.frnn_last_error()
    assert L.frnn_launch_exclusive_scan_noalloc(vp(d), -1, vp(d), None) == 1
    assert L.frnn_launch_exclusive_scan_noalloc(None, 5, vp(d), None) == 1
    assert L.frnn_launch_exclusive_scan_noalloc(None, 0, None, None) == 0            # empty: no launch
