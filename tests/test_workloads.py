"""Synthetic workload recipes -- CPU only, reduced sizes."""
import numpy as np

import frnn_oracle as O
import frnn_workloads as W


def test_uniform_and_gmm_recipes():
    w = W.config("C1", N=5000)
    assert w.X.shape == (5000, 3) and w.X.dtype == np.float32 and w.K == 16
    assert 0 <= w.X.min() and w.X.max() < 1
    g = W.config("C2", N=20000)
    assert g.K == 32 and g.radius == 0.01
    assert g.X.min() >= 0 and g.X.max() <= 1 and np.any(g.X == 1.0)   # closed upper cell


def test_lowrank_normalisation_preserves_distances():
    w = W.lowrank(3000, 16, 4, 0.01, 0.3, 64)
    s = w.notes["scale"]
    assert w.X.min() >= 0 and w.X.max() < 1
    rs = np.random.RandomState(1234)
    Z = rs.standard_normal((3000, 4))
    A, _ = np.linalg.qr(rs.standard_normal((16, 4)))
    X = Z @ A.T + 0.01 * rs.standard_normal((3000, 16))
    d_raw = np.linalg.norm(X[0] - X[1])
    d_n = np.linalg.norm(w.X[0].astype(np.float64) - w.X[1])
    assert abs(d_raw / s - d_n) < 1e-5
    assert abs(w.radius - 0.3 / s) < 1e-12


def test_config_dispatch_paths():
    # full sizes only through the plan (no data generated)
    assert O.plan(200_000, 3, 16, 0.03)["path"] == "grid_full"
    assert O.plan(1_000_000, 3, 32, 0.01)["cells"] == 1_000_000
    for name, N in (("C3", 500_000), ("C4", 1_500_000), ("metric", 1_000_000)):
        w = W.config(name, N=20000)      # same normalisation recipe, smaller N
        p = O.plan(N, w.D, w.K, w.radius)
        assert p["path"] == "grid_first" and p["grid_dim"] == 4


def test_c5_radius_percentile():
    w = W.gaussian_highd(20000, 128, 128)
    assert 12.0 < w.radius < 14.0
    assert O.plan(200_000, 128, 128, w.radius)["path"] == "bruteforce"


def test_reference_sweep_generator_reproduces_published_radii():
    # The reference calibrated each published cell's radius on its own
    # generator's data (Tests/scripts/benchmark_vs_libfrnn.py:94-133); the
    # restated generator and calibration give the same radii to the printed
    # digits, so the bench's refD<D>N<N> cells run the reference's workloads.
    for D, N in ((16, 200_000), (12, 200_000), (3, 200_000)):
        r = W.calibrate_radius(W.ref_lowrank_points(N, D))
        published = W.REF_SWEEP[(D, N)][0]
        assert round(r, 5 if D == 3 else 6) == published, (D, N, r, published)
    w = W.config("refD16N200000")
    assert w.K == 16 and w.radius == 0.075802 and w.notes["a100_ms"] > 0
    assert O.plan(1_000_000, 16, 16, W.REF_SWEEP[(16, 1_000_000)][0])["path"] == "grid_first"
