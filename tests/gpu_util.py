"""Helpers for the GPU tests: device buffers come from torch (plumbing only);
every computation runs in libfrnn_mi355x.so through the C ABI."""
import ctypes
import sys

import numpy as np

import frnn_cuda


def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need a visible MI355X"
    return t


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def device_soa(X):
    t = torch()
    d = t.from_numpy(np.ascontiguousarray(np.asarray(X, dtype=np.float32).T)).to("cuda:0")
    t.cuda.synchronize()
    return d


def vp(tensor_or_none):
    return None if tensor_or_none is None else ctypes.c_void_p(tensor_or_none.data_ptr())


def engine_search(X, K, radius, engine=None):
    """Run search_gpu on AoS X[N, D]; returns ([N, K] idx, [N, K] dist, plan)."""
    X = np.asarray(X, dtype=np.float32)
    N, D = X.shape
    eng = engine or frnn_cuda.FRNNEngine(max_points=max(N, 1))
    d = device_soa(X)
    eng.search_gpu(d.data_ptr(), N, D, K, radius)
    idx, dist = eng.get_results_numpy(N, K)
    plan = eng.last_plan()
    if engine is None:
        eng.close()
    return idx.reshape(K, N).T.copy(), dist.reshape(K, N).T.copy(), plan


def assert_rows_equal(gi, gd, ri, rd, label=""):
    """Bit-exact index sets, counts and distances (rows are ascending (d2, idx))."""
    assert gi.shape == ri.shape, label
    bad = np.nonzero(~(np.all(gi == ri, axis=1) & np.all(gd.view(np.uint32) == rd.view(np.uint32), axis=1)))[0]
    if len(bad):
        r = bad[0]
        raise AssertionError(f"{label}: {len(bad)} rows differ; first row {r}:\n gpu idx {gi[r][:12]}\n ref idx "
                             f"{ri[r][:12]}\n gpu d2 {gd[r][:6]}\n ref d2 {rd[r][:6]}")
