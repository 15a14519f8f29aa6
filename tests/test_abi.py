"""C-ABI and host-logic tests that need no GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

import frnn_cuda
import frnn_oracle as O
from conftest import ROOT, gpu_visible
from test_oracle_pins import DISPATCH_TABLE

HEADER = os.path.join(ROOT, "include", "frnn_mi355x.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(frnn_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(frnn_cuda.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_declared_symbols():
    L = frnn_cuda._load()
    for n in declared_functions():
        assert getattr(L, n).restype is not None or n == "frnn_status_string"


@pytest.mark.parametrize("args,want", DISPATCH_TABLE)
def test_plan_matches_dispatch_table(args, want):
    p = frnn_cuda.plan(*args)
    assert (p["path"], p["grid_dim"], p["res"]) == want


def test_plan_matches_oracle_on_random_inputs():
    rs = np.random.RandomState(21)
    for _ in range(3000):
        N = int(rs.choice([1, 7, 100, 577, 578, 5000, 100000, 2000000]))
        D = int(rs.randint(1, 129))
        K = int(rs.randint(1, 129))
        r = float(np.float32(10.0 ** rs.uniform(-3.5, 1.2)))
        a, b = frnn_cuda.plan(N, D, K, r), O.plan(N, D, K, r)
        for key in ("path", "grid_dim", "res", "cells", "rev_order"):
            assert a[key] == b[key], (N, D, K, r, key, a, b)
        assert a["r2"] == np.float32(np.float32(r) * np.float32(r))


@pytest.mark.parametrize("args,status", [
    ((10, 5, 3, 4, 0.1), 0),
    ((10, 11, 3, 4, 0.1), 2),       # N > max_points
    ((10, -1, 3, 4, 0.1), 1),
    ((10, 5, 0, 4, 0.1), 1),
    ((10, 5, 129, 4, 0.1), 1),
    ((10, 5, 3, 0, 0.1), 1),
    ((10, 5, 3, 129, 0.1), 1),
    ((10, 5, 3, 4, 0.0), 1),
    ((10, 5, 3, 4, -0.1), 1),
    ((10, 5, 3, 4, float("nan")), 1),
    ((10, 5, 3, 4, float("inf")), 1),
    ((0, 5, 3, 4, 0.1), 0),          # max_points <= 0 skips the N check
])
def test_validate_statuses(args, status):
    assert frnn_cuda._load().frnn_validate(*args) == status


def test_plan_errors_raise_value_error():
    with pytest.raises(ValueError):
        frnn_cuda.plan(10, 3, 0, 0.1)
    with pytest.raises(ValueError):
        frnn_cuda.plan(10, 200, 4, 0.1)


def test_geometry_helpers():
    assert [frnn_cuda.aos_stride(d) for d in (1, 3, 4, 5, 12, 16, 17, 33, 128)] == \
        [4, 4, 4, 8, 12, 16, 32, 64, 128]
    assert frnn_cuda.aos_stride(0) == -1 and frnn_cuda.aos_stride(129) == -1
    assert [frnn_cuda.list_capacity(k) for k in (1, 32, 64, 65, 128)] == [256] * 5
    assert frnn_cuda.list_capacity(0) == -1
    assert frnn_cuda.scan_partials_count(1_000_001) == 246


def test_status_strings():
    L = frnn_cuda._load()
    assert L.frnn_status_string(0) == b"ok"
    assert L.frnn_status_string(4) == b"no HIP device"
    assert L.frnn_version() >= 1


def test_launch_seam_rejects_bad_geometry_without_touching_the_device():
    L = frnn_cuda._load()
    # cells != res^g, grid_dim out of range, null pointers: all rejected on the host
    assert L.frnn_launch_bin_count(None, 10, 2, 4, 1.0, 15, None, None, None, None, None) == 1
    assert L.frnn_launch_bin_count(None, 10, 0, 4, 1.0, 1, None, None, None, None, None) == 1
    assert L.frnn_launch_bin_count(None, 10, 2, 4, 1.0, 16, None, None, None, None, None) == 1
    # a frame grid has at most 4 axes and a cell count within the cap
    ws = ctypes.c_void_p(1)
    assert L.frnn_launch_bin_count(None, 10, 5, 4, 1.0, 100, ws, None, None, None, None) == 1
    assert L.frnn_launch_bin_count(None, 10, 4, 4, 1.0, 1_000_001, ws, None, None, None, None) == 1
    assert L.frnn_launch_exclusive_scan(None, 5, None, None, None) == 1
    assert L.frnn_launch_unpermute(None, 10, None, 5, 20, None, None, None) == 1
    p = frnn_cuda._Plan()
    assert L.frnn_make_plan(100000, 12, 32, ctypes.c_float(0.0345), ctypes.byref(p)) == 0
    assert L.frnn_launch_frame(None, 10, 12, ctypes.byref(p), None, None, None) == 1   # null pointers
    p.cells = 5
    assert L.frnn_launch_find_nbrs(None, None, None, None, None, None, None, 100000, 12, 32, ctypes.byref(p),
                                   None, None, 128, None, None, None) == 1
    assert L.frnn_launch_frame(None, 10, 12, ctypes.byref(p), None, None, None) == 1   # inconsistent plan
    q = frnn_cuda._Plan()
    assert L.frnn_make_plan(100000, 3, 16, ctypes.c_float(0.1), ctypes.byref(q)) == 0
    assert L.frnn_launch_frame(None, 10, 3, ctypes.byref(q), None, None, None) == 1     # raw frame, null pointers
    assert L.frnn_launch_reorder(None, 10, 3, None, None, None, None, None, None, None, None, None) == 1
    assert L.frnn_launch_transpose(None, 10, 3, None, None, None, None) == 1
    # wide rows stream precomputed centred rows; narrower ones centre in registers
    assert [L.frnn_uses_filter_rows(d) for d in (0, 3, 16, 32, 33, 64, 128, 129)] == [-1, 0, 0, 0, 1, 1, 1, -1]
    assert L.frnn_launch_point_stats(None, 10, 3, None, None) == 1
    assert L.frnn_stats_workspace_bytes(0) == -1 and L.frnn_stats_workspace_bytes(16) > 0


def test_frame_workspace_sizes():
    # a frame for every grid plan with at most 4 grid axes: projected for
    # first-coordinate plans with dim > grid_dim, raw otherwise
    assert frnn_cuda.frame_workspace_bytes(100000, 12, 32, 0.0345) > 0     # grid_first g=4
    assert frnn_cuda.frame_workspace_bytes(100000, 3, 16, 0.1) > 0         # full-D grid g=3 (raw)
    assert frnn_cuda.frame_workspace_bytes(200000, 128, 128, 12.96) == 0   # brute force
    assert frnn_cuda.frame_workspace_bytes(100000, 4, 8, 0.02) > 0         # grid_first g=3
    p = frnn_cuda.plan(200000, 6, 8, 0.2)                                  # full-D grid g=6
    assert p["path"] == "grid_full" and p["grid_dim"] == 6
    assert frnn_cuda.frame_workspace_bytes(200000, 6, 8, 0.2) == 0


def test_grid_cells():
    # a raw frame has 8 (its fine axis-0 cells per cell edge) x res^g cells,
    # a projected frame's capacity is 8 x clamp(N, 4096, 1M), at least
    # 8 x res^g; grids above 4 axes (no frame) use res^g
    F = 8
    p = frnn_cuda.plan(100000, 3, 16, 0.1)
    assert frnn_cuda.grid_cells(100000, 3, 16, 0.1) == F * p["cells"]
    assert frnn_cuda.grid_cells(200000, 6, 8, 0.2) == frnn_cuda.plan(200000, 6, 8, 0.2)["cells"]
    assert frnn_cuda.grid_cells(200000, 128, 128, 12.96) == 0
    assert frnn_cuda.grid_cells(100000, 12, 32, 0.0345) == F * max(100000, frnn_cuda.plan(100000, 12, 32, 0.0345)["cells"])
    assert frnn_cuda.grid_cells(100000, 12, 32, 0.2) == F * 100000
    assert frnn_cuda.grid_cells(1000, 12, 32, 0.0345) == F * max(4096, frnn_cuda.plan(1000, 12, 32, 0.0345)["cells"])
    assert frnn_cuda.grid_cells(3_000_000, 12, 32, 0.0345) == F * 1_000_000


@pytest.mark.skipif(gpu_visible(), reason="checks the no-device error path")
def test_engine_without_device_raises():
    with pytest.raises(frnn_cuda.FRNNError, match="no HIP device"):
        frnn_cuda.FRNNEngine(max_points=16)


def test_engine_rejects_bad_max_points():
    with pytest.raises(ValueError):
        frnn_cuda.FRNNEngine(max_points=0)


def test_frame_struct_layout_matches_header(tmp_path):
    # the ctypes mirror of frnn_frame_t against the C compiler's layout
    src = tmp_path / "frame_layout.c"
    src.write_text('#include <stddef.h>\n#include <stdio.h>\n#include "frnn_mi355x.h"\n'
                   'int main(void) { printf("%zu %zu %zu %zu %zu", sizeof(frnn_frame_t), '
                   'offsetof(frnn_frame_t, h), offsetof(frnn_frame_t, sigma), '
                   'offsetof(frnn_frame_t, coord), offsetof(frnn_frame_t, dir)); return 0; }\n')
    exe = tmp_path / "frame_layout"
    import subprocess
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True,
                                          text=True).stdout.split()]
    F = frnn_cuda.FrameInfo
    assert got == [ctypes.sizeof(F), F.h.offset, F.sigma.offset, F.coord.offset, F.dir.offset]
