"""ctypes wrapper of the C++ CPU oracle -- TEST INFRASTRUCTURE ONLY.

Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
the checker; the product (the HIP engine) never imports it.  See
oracle/frnn_oracle.cpp for the reference lines each function restates.
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_frnn.so")
_lib = None

PATH_NAMES = {-1: "empty", 0: "bruteforce", 1: "grid_full", 2: "grid_first"}


def build(force=False):
    """Compile liboracle_frnn.so with the committed Makefile."""
    cmd = ["make", "-C", _HERE] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i32, f32, i64 = ctypes.c_int, ctypes.c_float, ctypes.c_longlong
        vp = ctypes.c_void_p
        L.oracle_plan.argtypes = [i32, i32, i32, f32, vp]
        L.oracle_plan.restype = i32
        L.oracle_bin.argtypes = [vp, i32, i32, i32, f32, vp]
        L.oracle_bin.restype = None
        L.oracle_dist2.argtypes = [vp, vp, i32, i32]
        L.oracle_dist2.restype = f32
        L.oracle_search.argtypes = [vp, i32, i32, i32, f32, i32, i32, vp, i32, vp, vp, vp]
        L.oracle_search.restype = i32
        L.oracle_search_queries.argtypes = [vp, i32, vp, i32, i32, i32, f32, i32, i32, vp, vp]
        L.oracle_search_queries.restype = i32
        L.oracle_shell_candidates.argtypes = [vp, i32, i32, i32, f32, vp, i32]
        L.oracle_shell_candidates.restype = i64
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def plan(N, D, K, radius):
    out = np.zeros(6, dtype=np.int64)
    lib().oracle_plan(int(N), int(D), int(K), float(radius), _ptr(out))
    return {"path": PATH_NAMES[int(out[0])], "grid_dim": int(out[1]), "res": int(out[2]),
            "cells": int(out[3]), "rev_order": int(out[4])}


def bin_cells(X, g, res, inv_cell):
    """Clamped cell ids of AoS points X[N, D] on a grid over the first g coords."""
    X = np.asarray(X, dtype=np.float32)
    soa = np.ascontiguousarray(X.T)
    out = np.empty(X.shape[0], dtype=np.int32)
    lib().oracle_bin(_ptr(soa), X.shape[0], int(g), int(res), float(inv_cell), _ptr(out))
    return out


def dist2(q, p, order=0):
    q = np.ascontiguousarray(q, dtype=np.float32)
    p = np.ascontiguousarray(p, dtype=np.float32)
    return np.float32(lib().oracle_dist2(_ptr(q), _ptr(p), q.shape[0], int(order)))


def search(X, K, radius, force_path=-1, nthreads=0, query_ids=None, timings=None):
    """Oracle FRNN on AoS X[N, D].

    Returns (idx, dist) as [Q, K] arrays (Q = N, or len(query_ids)), rows in
    ascending (d2, idx) order, padding (r2, -1).  ``timings``, if a list, gets
    [build_s, search_s] appended.
    """
    X = np.asarray(X, dtype=np.float32)
    N, D = X.shape
    soa = np.ascontiguousarray(X.T)
    t = np.zeros(2, dtype=np.float64)
    if query_ids is None:
        idx = np.empty((K, N), dtype=np.int32)
        dist = np.empty((K, N), dtype=np.float32)
        rc = lib().oracle_search(_ptr(soa), N, D, int(K), float(radius), int(force_path),
                                 int(nthreads), None, 0, _ptr(idx), _ptr(dist), _ptr(t))
        idx, dist = idx.T.copy(), dist.T.copy()
    else:
        q = np.ascontiguousarray(query_ids, dtype=np.int32)
        idx = np.empty((len(q), K), dtype=np.int32)
        dist = np.empty((len(q), K), dtype=np.float32)
        rc = lib().oracle_search(_ptr(soa), N, D, int(K), float(radius), int(force_path),
                                 int(nthreads), _ptr(q), len(q), _ptr(idx), _ptr(dist), _ptr(t))
    if rc != 0:
        raise ValueError(f"oracle_search failed with code {rc}")
    if timings is not None:
        timings.extend([float(t[0]), float(t[1])])
    return idx, dist


def search_queries(P, Q, K, radius, force_path=-1, nthreads=0):
    """Oracle FRNN of the queries Q[M, D] against the points P[N, D] (the
    reference kernels' two-array form; plan and grid are the points').

    Returns (idx, dist) as [M, K] arrays, rows in ascending (d2, idx) order,
    padding (r2, -1); indices refer to rows of P.
    """
    P = np.asarray(P, dtype=np.float32)
    Q = np.asarray(Q, dtype=np.float32)
    N, D = P.shape
    M = Q.shape[0]
    assert Q.shape[1] == D
    sp = np.ascontiguousarray(P.T)
    sq = np.ascontiguousarray(Q.T) if M else np.zeros((D, 1), np.float32)
    idx = np.empty((M, K), dtype=np.int32)
    dist = np.empty((M, K), dtype=np.float32)
    rc = lib().oracle_search_queries(_ptr(sp), N, _ptr(sq), M, D, int(K), float(radius), int(force_path),
                                     int(nthreads), _ptr(idx), _ptr(dist))
    if rc != 0:
        raise ValueError(f"oracle_search_queries failed with code {rc}")
    return idx, dist


def shell_candidates(X, K, radius, query_ids=None):
    X = np.asarray(X, dtype=np.float32)
    soa = np.ascontiguousarray(X.T)
    if query_ids is None:
        return int(lib().oracle_shell_candidates(_ptr(soa), X.shape[0], X.shape[1], int(K),
                                                 float(radius), None, 0))
    q = np.ascontiguousarray(query_ids, dtype=np.int32)
    return int(lib().oracle_shell_candidates(_ptr(soa), X.shape[0], X.shape[1], int(K),
                                             float(radius), _ptr(q), len(q)))
