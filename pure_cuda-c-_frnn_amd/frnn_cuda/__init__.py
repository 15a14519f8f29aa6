"""frnn_cuda -- drop-in Python module for the reference FRNN engine, backed by
the MI355X (gfx950) library libfrnn_mi355x.so through its C ABI
(include/frnn_mi355x.h).

Same module name, class, methods, argument names and result shapes as the
reference's nanobind binding (python_interface/nanobind_module.cu:8-21):

    engine = frnn_cuda.FRNNEngine(max_points=N)
    idxs, dists = engine.search(points, K, radius)           # host AoS in/out (lists)
    d_idx, d_dist = engine.search_gpu(dev_ptr, N, dim, K, radius)  # SoA device ptrs
    idxs, dists = engine.get_results(N, K)                   # SoA lists of the last search_gpu

Errors the reference never reported (its launch wrappers return void) raise
ValueError for bad arguments and RuntimeError for device failures.  There is
no CPU fallback: without the built library or a visible GPU the calls raise.

Threading: ctypes releases the GIL around every library call, so each engine
serialises its own calls with a lock; calls on one engine from several Python
threads run one at a time, as they did under the reference's binding, which
holds the GIL (nanobind_module.cu:11-19).  Separate engines run concurrently.
"""
import ctypes
import functools
import os
import threading

import numpy as np

__all__ = ["FRNNEngine", "plan", "FRNNError", "LIB_PATH", "MAX_K", "MAX_DIM", "MAX_CELLS"]

MAX_K = 128
MAX_DIM = 128
MAX_CELLS = 1_000_000
NUM_STAGES = 8
NUM_COUNTERS = 4
PROFILE_EVENTS, PROFILE_COUNTERS, PROFILE_SEARCH_EVENTS = 1, 2, 4
STAGE_NAMES = ("zero_fill", "stats", "frame", "bin_count", "scan", "reorder", "search", "unpermute")
PATH_NAMES = {-1: "empty", 0: "bruteforce", 1: "grid_full", 2: "grid_first"}

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libfrnn_mi355x.so")

_OK, _INVALID, _CAPACITY, _HIP, _NODEV, _STATE = range(6)


class FRNNError(RuntimeError):
    """A device-side failure reported by the engine."""


class _Plan(ctypes.Structure):
    _fields_ = [("path", ctypes.c_int), ("grid_dim", ctypes.c_int), ("res", ctypes.c_int),
                ("rev_order", ctypes.c_int), ("cells", ctypes.c_longlong), ("r2", ctypes.c_float),
                ("cell_size", ctypes.c_float), ("inv_cell", ctypes.c_float)]

    def as_dict(self):
        return {"path": PATH_NAMES.get(self.path, str(self.path)), "grid_dim": self.grid_dim,
                "res": self.res, "rev_order": self.rev_order, "cells": self.cells,
                "r2": self.r2, "cell_size": self.cell_size, "inv_cell": self.inv_cell}


class Queries(ctypes.Structure):
    """frnn_queries_t: M separate queries for frnn_launch_find_nbrs (device pointers)."""
    _fields_ = [("M", ctypes.c_int), ("d_aos", ctypes.c_void_p), ("d_frows", ctypes.c_void_p),
                ("d_sorted_idx", ctypes.c_void_p), ("d_cell_of", ctypes.c_void_p)]


FRAME_TERMS = 32
FRAME_DIRS = 4


class FrameInfo(ctypes.Structure):
    """frnn_frame_t: the descriptor at the start of a frame workspace."""
    _fields_ = [("grid_dim", ctypes.c_int), ("cells", ctypes.c_int), ("terms", ctypes.c_int),
                ("projected", ctypes.c_int), ("fine0", ctypes.c_int),
                ("res", ctypes.c_int * FRAME_DIRS), ("stride", ctypes.c_int * FRAME_DIRS),
                ("lo", ctypes.c_float * FRAME_DIRS), ("h", ctypes.c_float), ("inv_h", ctypes.c_float),
                ("margin", ctypes.c_float), ("slack", ctypes.c_float),
                ("h0", ctypes.c_float), ("inv_h0", ctypes.c_float), ("sigma", ctypes.c_float * FRAME_DIRS),
                ("coord", ctypes.c_int * FRAME_TERMS), ("mean", ctypes.c_float * FRAME_TERMS),
                ("dir", (ctypes.c_float * FRAME_TERMS) * FRAME_DIRS)]

    @classmethod
    def from_workspace(cls, head):
        """Decode from the first bytes of a frame workspace (bytes or uint8 array)."""
        return cls.from_buffer_copy(bytes(np.asarray(head, dtype=np.uint8)[:ctypes.sizeof(cls)]))

    def directions(self):
        """(4, 32) float32 array of direction weights over the term coordinates."""
        return np.array([[self.dir[k][t] for t in range(FRAME_TERMS)] for k in range(FRAME_DIRS)],
                        dtype=np.float32)


_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build() or "
                          f"make -C {_PKG_DIR}")
    L = ctypes.CDLL(LIB_PATH)
    i32, f32, i64, vp = ctypes.c_int, ctypes.c_float, ctypes.c_longlong, ctypes.c_void_p
    pi32 = ctypes.POINTER(ctypes.c_int)
    sig = {
        "frnn_status_string": ([i32], ctypes.c_char_p),
        "frnn_last_error": ([], ctypes.c_char_p),
        "frnn_version": ([], i32),
        "frnn_validate": ([i32, i32, i32, i32, f32], i32),
        "frnn_make_plan": ([i32, i32, i32, f32, ctypes.POINTER(_Plan)], i32),
        "frnn_aos_stride": ([i32], i32),
        "frnn_list_capacity": ([i32], i32),
        "frnn_scan_partials_count": ([i32], i32),
        "frnn_engine_create": ([i32, ctypes.POINTER(vp)], i32),
        "frnn_engine_destroy": ([vp], i32),
        "frnn_engine_max_points": ([vp, pi32], i32),
        "frnn_engine_search_gpu": ([vp, vp, i32, i32, i32, f32, ctypes.POINTER(vp),
                                    ctypes.POINTER(vp)], i32),
        "frnn_engine_search_gpu_queries": ([vp, vp, i32, vp, i32, i32, i32, f32, ctypes.POINTER(vp),
                                            ctypes.POINTER(vp)], i32),
        "frnn_engine_build": ([vp, vp, i32, i32, i32, f32], i32),
        "frnn_engine_query": ([vp, vp, i32, ctypes.POINTER(vp), ctypes.POINTER(vp)], i32),
        "frnn_engine_search": ([vp, vp, i64, i32, f32, vp, vp], i32),
        "frnn_engine_get_results": ([vp, i32, i32, vp, vp], i32),
        "frnn_engine_set_stream": ([vp, vp], i32),
        "frnn_engine_last_plan": ([vp, ctypes.POINTER(_Plan)], i32),
        "frnn_engine_set_profiling": ([vp, i32], i32),
        "frnn_engine_stage_times": ([vp, vp, i32], i32),
        "frnn_engine_counters": ([vp, vp, i32], i32),
        "frnn_engine_count_work": ([vp, vp, i32], i32),
        "frnn_grid_cells": ([i32, i32, ctypes.POINTER(_Plan)], i64),
        "frnn_launch_bin_count": ([vp, i32, i32, i32, f32, i64, vp, vp, vp, vp, vp], i32),
        "frnn_launch_exclusive_scan": ([vp, i32, vp, vp, vp], i32),
        "frnn_launch_exclusive_scan_noalloc": ([vp, i32, vp, vp], i32),
        "frnn_stats_workspace_bytes": ([i32], i64),
        "frnn_launch_point_stats": ([vp, i32, i32, vp, vp], i32),
        "frnn_frame_workspace_bytes": ([i32, i32, ctypes.POINTER(_Plan)], i64),
        "frnn_launch_frame": ([vp, i32, i32, ctypes.POINTER(_Plan), vp, vp, vp], i32),
        "frnn_launch_reorder": ([vp, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp], i32),
        "frnn_launch_transpose": ([vp, i32, i32, vp, vp, vp, vp], i32),
        "frnn_uses_filter_rows": ([i32], i32),
        "frnn_launch_find_nbrs": ([vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, ctypes.POINTER(_Plan),
                                   ctypes.POINTER(Queries), vp, i32, vp, vp, vp], i32),
        "frnn_launch_unpermute": ([vp, i32, vp, i32, i32, vp, vp, vp], i32),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    _lib = L
    return L


def _check(status, what=""):
    if status == _OK:
        return
    L = _load()
    msg = L.frnn_last_error().decode() or L.frnn_status_string(status).decode()
    text = f"{what}: {msg}" if what else msg
    if status in (_INVALID, _CAPACITY):
        raise ValueError(text)
    raise FRNNError(text)


def plan(N, dim, K, radius):
    """The reference's auto-dispatch decision for (N, dim, K, radius) as a dict."""
    return _plan_struct(N, dim, K, radius).as_dict()


def _plan_struct(N, dim, K, radius):
    p = _Plan()
    _check(_load().frnn_make_plan(int(N), int(dim), int(K), float(radius), ctypes.byref(p)), "plan")
    return p


def frame_workspace_bytes(N, dim, K, radius):
    """Bytes of the grid-frame workspace for this problem (0: the plan has no frame)."""
    return int(_load().frnn_frame_workspace_bytes(int(N), int(dim),
                                                  ctypes.byref(_plan_struct(N, dim, K, radius))))


def grid_cells(N, dim, K, radius):
    """Cells of the problem's grid (count arrays hold one more); 0 for brute force."""
    return int(_load().frnn_grid_cells(int(N), int(dim), ctypes.byref(_plan_struct(N, dim, K, radius))))


def aos_stride(dim):
    return _load().frnn_aos_stride(int(dim))


def list_capacity(K):
    return _load().frnn_list_capacity(int(K))


def scan_partials_count(n):
    return _load().frnn_scan_partials_count(int(n))


def _serialised(method):
    """Run an engine method under the engine's lock (the engine's device
    buffers, built grid and results are shared state)."""
    @functools.wraps(method)
    def call(self, *args, **kwargs):
        with self._lock:
            return method(self, *args, **kwargs)
    return call


class FRNNEngine:
    """N-dimensional fixed-radius K-nearest search engine (reference: frnn_engine.h:9-55)."""

    def __init__(self, max_points):
        self._lock = threading.RLock()
        L = _load()
        h = ctypes.c_void_p()
        _check(L.frnn_engine_create(int(max_points), ctypes.byref(h)), "FRNNEngine")
        self._h = h
        self.max_points = int(max_points)

    # -- reference API ----------------------------------------------------------
    def search(self, points, K, radius):
        """Host path: flat AoS points (len = max_points * dim) -> (idxs, dists) flat
        AoS lists [i*K + k] (frnn_engine.cu:104-193)."""
        idx, dist = self.search_numpy(points, K, radius)
        return idx.reshape(-1).tolist(), dist.reshape(-1).tolist()

    @_serialised
    def search_gpu(self, dev_ptr, N, dim, K, radius):
        """Device path: SoA fp32 device pointer p[d*N + i] -> (d_idxs_ptr, d_dists_ptr),
        engine-owned SoA [k*N + i] buffers valid until the next call (frnn_engine.cu:195-250)."""
        di, dd = ctypes.c_void_p(), ctypes.c_void_p()
        _check(_load().frnn_engine_search_gpu(self._handle(), ctypes.c_void_p(int(dev_ptr)),
                                              int(N), int(dim), int(K), float(radius),
                                              ctypes.byref(di), ctypes.byref(dd)), "search_gpu")
        return int(di.value or 0), int(dd.value or 0)

    @_serialised
    def search_gpu_queries(self, points_ptr, N, queries_ptr, M, dim, K, radius):
        """Separate queries: SoA fp32 device pointers to N points p[d*N + i] and M
        queries q[d*M + j] -> (d_idxs_ptr, d_dists_ptr), engine-owned SoA
        [k*M + j] buffers of indices into the points (the reference kernels'
        two-array form, find_nbrs.cu:562-567, no_grid_frnn.cu:273-276)."""
        di, dd = ctypes.c_void_p(), ctypes.c_void_p()
        _check(_load().frnn_engine_search_gpu_queries(self._handle(), ctypes.c_void_p(int(points_ptr)), int(N),
                                                      ctypes.c_void_p(int(queries_ptr)), int(M), int(dim),
                                                      int(K), float(radius), ctypes.byref(di), ctypes.byref(dd)),
               "search_gpu_queries")
        return int(di.value or 0), int(dd.value or 0)

    @_serialised
    def build(self, points_ptr, N, dim, K, radius):
        """Build the grid of N points (SoA fp32 device pointer p[d*N + i]) once,
        for any number of query() calls with this K and radius."""
        _check(_load().frnn_engine_build(self._handle(), ctypes.c_void_p(int(points_ptr)), int(N), int(dim),
                                         int(K), float(radius)), "build")

    @_serialised
    def query(self, queries_ptr, M):
        """Search M queries (SoA fp32 device pointer q[d*M + j]) against the last
        built grid -> (d_idxs_ptr, d_dists_ptr), SoA [k*M + j]."""
        di, dd = ctypes.c_void_p(), ctypes.c_void_p()
        _check(_load().frnn_engine_query(self._handle(), ctypes.c_void_p(int(queries_ptr)), int(M),
                                         ctypes.byref(di), ctypes.byref(dd)), "query")
        return int(di.value or 0), int(dd.value or 0)

    def get_results(self, N, K):
        """D2H copy of the last search_gpu output, SoA order [k*N + i], as lists
        (frnn_engine.cu:252-258)."""
        idx, dist = self.get_results_numpy(N, K)
        return idx.tolist(), dist.tolist()

    # -- numpy conveniences (same semantics, no list conversion) -----------------
    @_serialised
    def search_numpy(self, points, K, radius):
        """Host path returning ([max_points, K] int32, [max_points, K] float32)."""
        pts = np.ascontiguousarray(np.asarray(points, dtype=np.float32).reshape(-1))
        n = pts.size
        if n == 0 or n % self.max_points:
            raise ValueError("len(points) must be a positive multiple of max_points")
        K = int(K)
        if not 1 <= K <= MAX_K:
            raise ValueError("K must be in [1, 128]")
        idx = np.empty((self.max_points, K), dtype=np.int32)
        dist = np.empty((self.max_points, K), dtype=np.float32)
        _check(_load().frnn_engine_search(self._handle(), pts.ctypes.data_as(ctypes.c_void_p),
                                          n, K, float(radius),
                                          idx.ctypes.data_as(ctypes.c_void_p),
                                          dist.ctypes.data_as(ctypes.c_void_p)), "search")
        return idx, dist

    @_serialised
    def get_results_numpy(self, N, K):
        n = int(N) * int(K)
        idx = np.empty(max(n, 0), dtype=np.int32)
        dist = np.empty(max(n, 0), dtype=np.float32)
        _check(_load().frnn_engine_get_results(self._handle(), int(N), int(K),
                                               idx.ctypes.data_as(ctypes.c_void_p),
                                               dist.ctypes.data_as(ctypes.c_void_p)), "get_results")
        return idx, dist

    # -- engine controls ----------------------------------------------------------
    @_serialised
    def set_stream(self, stream):
        """Launch on a HIP stream (int handle, e.g. torch.cuda.current_stream().cuda_stream)."""
        _check(_load().frnn_engine_set_stream(self._handle(), ctypes.c_void_p(int(stream or 0))),
               "set_stream")

    @_serialised
    def last_plan(self):
        p = _Plan()
        _check(_load().frnn_engine_last_plan(self._handle(), ctypes.byref(p)), "last_plan")
        return p.as_dict()

    @_serialised
    def set_profiling(self, enable=True, counters=True, search_only=False):
        """enable: per-stage HIP event times (stage_times()); counters: also run
        the counting build of the search kernel (counters()); search_only:
        events around the search kernel only (the other stages read 0), which
        keeps the event overhead out of timed calls."""
        ev = PROFILE_SEARCH_EVENTS if search_only else PROFILE_EVENTS
        flags = (ev | (PROFILE_COUNTERS if counters else 0)) if enable else 0
        _check(_load().frnn_engine_set_profiling(self._handle(), flags), "set_profiling")

    @_serialised
    def stage_times(self):
        """Per-stage milliseconds of the last profiled search (HIP events)."""
        ms = np.zeros(NUM_STAGES, dtype=np.float32)
        _check(_load().frnn_engine_stage_times(self._handle(), ms.ctypes.data_as(ctypes.c_void_p),
                                               NUM_STAGES), "stage_times")
        return dict(zip(STAGE_NAMES, (float(x) for x in ms)))

    @_serialised
    def counters(self):
        c = np.zeros(NUM_COUNTERS, dtype=np.int64)
        _check(_load().frnn_engine_counters(self._handle(), c.ctypes.data_as(ctypes.c_void_p),
                                            NUM_COUNTERS), "counters")
        return {"shell_candidates": int(c[0]), "filter_hits": int(c[1]), "accepted": int(c[2]),
                "streamed_pairs": int(c[3])}

    @_serialised
    def count_work(self):
        """Count-array entries the last build zero-filled and scanned (the scan's
        extent is a frame's actual cells + 1 when profiling events are on)."""
        c = np.zeros(2, dtype=np.int64)
        _check(_load().frnn_engine_count_work(self._handle(), c.ctypes.data_as(ctypes.c_void_p), 2),
               "count_work")
        return {"zero_filled": int(c[0]), "scanned": int(c[1])}

    @_serialised
    def close(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            _load().frnn_engine_destroy(h)
        self._h = None

    def _handle(self):
        if getattr(self, "_h", None) is None or not self._h.value:
            raise ValueError("engine is closed")
        return self._h

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
