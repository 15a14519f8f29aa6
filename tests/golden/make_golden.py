"""Writes the golden fixtures tests/golden/*.npz (inputs + expected outputs).

The reference holds no golden vectors for this path, so these are produced by
the CPU oracle (oracle/frnn_oracle.cpp) after it passed the pins in
tests/test_oracle_pins.py; they freeze that behaviour for regression tests of
the oracle (CPU) and of the HIP engine (GPU).  One fixture per dispatch path.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "oracle"), os.path.join(ROOT, "pure_cuda-c-_frnn_amd")]

import frnn_oracle as O  # noqa: E402
import frnn_workloads as W  # noqa: E402


def fixtures():
    yield "uniform_d3_grid_full", W.uniform(1200, 3, 0.08, 16)
    yield "gmm_d3_closed_cell", W.gmm(1200, 3, 16, 0.02, 0.05, 16)
    yield "lowrank_d12_grid_first", W.lowrank(1200, 12, 3, 0.01, 1.2, 32)
    yield "lowrank_d16_grid_first", W.lowrank(1200, 16, 4, 0.01, 1.5, 32)
    yield "gauss_d128_bruteforce", W.gaussian_highd(600, 128, 32, pct=1.0)
    yield "uniform_d5_grid_full", W.uniform(1200, 5, 0.3, 16)
    yield "uniform_d1_grid_full", W.uniform(2000, 1, 0.004, 4)


def main():
    for name, w in fixtures():
        p = O.plan(w.N, w.D, w.K, w.radius)
        idx, dist = O.search(w.X, w.K, w.radius)
        out = os.path.join(HERE, name + ".npz")
        np.savez_compressed(out, X=w.X, K=np.int32(w.K), radius=np.float64(w.radius),
                            path=np.str_(p["path"]), idx=idx, dist=dist)
        print(f"{name}: path={p['path']} N={w.N} D={w.D} K={w.K} "
              f"mean neighbours={(idx >= 0).sum(1).mean():.2f} -> {os.path.getsize(out)} B")


if __name__ == "__main__":
    main()
