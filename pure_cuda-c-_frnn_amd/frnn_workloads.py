"""Synthetic point clouds for the all-points FRNN benchmark configurations.

Seed 1234 with numpy RandomState, as the reference harness uses
(Tests/scripts/benchmark_vs_libfrnn.py:40).  Each recipe returns a Workload
with AoS fp32 points X[N, D], the search radius and K.

The low-rank recipes are normalised isotropically, x' = (x - min) / s with
s = (max - min) * (1 + 1e-6) over all coordinates, and the radius is scaled by
the same s.  That keeps every point inside the reference's [0, 1] grid domain
(frnn_engine.cu:73-80) while preserving all pairwise distance ratios; the
reference's own harness min-max normalises per column instead
(validate_correctness.py:55-64), which would change the distances.
"""
from dataclasses import dataclass, field

import numpy as np

SEED = 1234


@dataclass
class Workload:
    name: str
    X: np.ndarray          # [N, D] float32, AoS
    radius: float
    K: int
    notes: dict = field(default_factory=dict)

    @property
    def N(self):
        return self.X.shape[0]

    @property
    def D(self):
        return self.X.shape[1]

    def soa(self):
        """SoA layout p[d*N + i] expected by search_gpu (frnn_engine.h:21-26)."""
        return np.ascontiguousarray(self.X.T)


def uniform(N, D=3, radius=0.03, K=16, seed=SEED):
    """C1: i.i.d. uniform in [0,1)^D."""
    rs = np.random.RandomState(seed)
    X = rs.rand(N, D).astype(np.float32)
    return Workload(f"uniform_D{D}_N{N}", X, float(radius), K)


def gmm(N, D=3, centers=64, sigma=0.02, radius=0.01, K=32, seed=SEED):
    """C2: isotropic Gaussian mixture, centres uniform in [0,1]^D, clipped to [0,1].

    Not normalised, so coordinates equal to 1.0 occur and land in the closed
    upper cell."""
    rs = np.random.RandomState(seed)
    C = rs.rand(centers, D)
    lab = rs.randint(0, centers, N)
    X = np.clip(C[lab] + sigma * rs.standard_normal((N, D)), 0.0, 1.0).astype(np.float32)
    return Workload(f"gmm_D{D}_N{N}", X, float(radius), K, {"centers": centers, "sigma": sigma})


def lowrank(N, D, k, sigma, radius, K, seed=SEED):
    """C3/C4/metric: X = Z A^T + eps, Z ~ N(0,1)^{N x k}, A (D x k) orthonormal
    from QR of a seeded Gaussian, eps ~ N(0, sigma^2); isotropic normalisation."""
    rs = np.random.RandomState(seed)
    Z = rs.standard_normal((N, k))
    A, _ = np.linalg.qr(rs.standard_normal((D, k)))
    X = Z @ A.T + sigma * rs.standard_normal((N, D))
    mn, mx = float(X.min()), float(X.max())
    s = (mx - mn) * (1.0 + 1e-6)
    Xn = ((X - mn) / s).astype(np.float32)
    return Workload(f"lowrank_D{D}_k{k}_N{N}", Xn, float(radius / s), K,
                    {"raw_radius": radius, "scale": s, "intrinsic": k, "sigma": sigma})


def gaussian_highd(N, D=128, K=128, pairs=10_000, pct=0.1, seed=SEED):
    """C5: i.i.d. N(0,1)^D; r = the pct-th percentile of `pairs` seeded pair distances."""
    rs = np.random.RandomState(seed)
    X = rs.standard_normal((N, D)).astype(np.float32)
    i = rs.randint(0, N, pairs)
    j = rs.randint(0, N, pairs)
    d = np.sqrt(((X[i].astype(np.float64) - X[j].astype(np.float64)) ** 2).sum(1))
    r = float(np.percentile(d, pct))
    return Workload(f"gauss_D{D}_N{N}", X, r, K, {"pairs": pairs, "percentile": pct})


def config(name, N=None):
    """BASELINE.json configurations by name ('C1'..'C5', 'metric'), optional N override."""
    if name == "C1":
        return uniform(N or 200_000, 3, 0.03, 16)
    if name == "C2":
        return gmm(N or 1_000_000, 3, 64, 0.02, 0.01, 32)
    if name == "C3":
        return lowrank(N or 500_000, 12, 3, 0.01, 0.25, 32)
    if name == "C4":
        return lowrank(N or 1_500_000, 16, 4, 0.01, 0.3, 64)
    if name == "metric":
        return lowrank(N or 1_000_000, 16, 4, 0.01, 0.3, 64)
    if name == "C5":
        return gaussian_highd(N or 200_000, 128, 128)
    raise KeyError(name)


CONFIGS = ("C1", "C2", "C3", "C4", "metric", "C5")
