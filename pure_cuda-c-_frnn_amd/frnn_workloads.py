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


# The reference's own published sweep (NVIDIA A100, K=16, low-rank intrinsic 3,
# noise 0.02, per-column min-max normalisation, radius calibrated to ~16
# neighbours): (D, N) -> (radius, A100 search_gpu median ms).  Sources:
# Tests/json_results/requested_new_cells.partial.json:2-11 (D3 all N, D12
# N750K/1.25M/1.5M, D16 N750K), vs_libfrnn_results.before_requested_sweep.json
# :2-48 (D12 N200K/500K/1M, D16 N200K/500K/1M), requested_remaining_d16.json
# :2-17 (D16 N1.25M/1.5M).
REF_SWEEP = {
    (3, 200_000): (0.02629, 0.8798484923318028),
    (3, 500_000): (0.01934, 3.186592541169375),
    (3, 750_000): (0.01684, 5.293745547533035),
    (3, 1_000_000): (0.01521, 7.279802463017404),
    (3, 1_250_000): (0.01431, 9.438642533496022),
    (3, 1_500_000): (0.01345, 11.439650494139642),
    (12, 200_000): (0.053695, 7.3781710234470665),
    (12, 500_000): (0.049318, 23.22301553795114),
    (12, 750_000): (0.04992, 60.99493900546804),
    (12, 1_000_000): (0.039409, 59.32024650974199),
    (12, 1_250_000): (0.03673, 78.37455556727946),
    (12, 1_500_000): (0.04346, 240.20811956143007),
    (16, 200_000): (0.075802, 20.085041061975062),
    (16, 500_000): (0.057647, 43.707173492293805),
    (16, 750_000): (0.04788, 47.09805402671918),
    (16, 1_000_000): (0.048421, 98.8155270460993),
    (16, 1_250_000): (0.05034, 175.28476048028097),
    (16, 1_500_000): (0.049079, 198.13100999454036),
}
REF_K = 16


def ref_lowrank_points(N, D, intrinsic=3, noise=0.02, seed=SEED):
    """The reference harness's low-rank cloud (Tests/scripts/
    benchmark_vs_libfrnn.py:94-107, DIST=lowrank): core ~ U[0,1)^{N x k},
    embed ~ N(0,1)^{k x D}, Q from QR of an N(0,1)^{D x D} draw, points =
    core.embed.Q + noise.N(0,1), then per-column min-max normalisation into
    [0, 1] -- the same RandomState draws in the same order.  An intrinsic
    dimension of at least D gives i.i.d. uniform points, as there (:100-101)."""
    rng = np.random.RandomState(seed)
    if intrinsic <= 0 or intrinsic >= D:
        return rng.rand(N, D).astype(np.float32)
    core = rng.rand(N, intrinsic)
    embed = rng.standard_normal((intrinsic, D))
    Q, _ = np.linalg.qr(rng.standard_normal((D, D)))
    pts = (core @ embed) @ Q + noise * rng.standard_normal((N, D))
    mn, mx = pts.min(0, keepdims=True), pts.max(0, keepdims=True)
    return ((pts - mn) / np.maximum(mx - mn, 1e-9)).astype(np.float32)


def calibrate_radius(pts, target=REF_K, sample=256, lo=1e-4, hi=2.0, iters=20):
    """The reference's radius calibration (benchmark_vs_libfrnn.py:110-133):
    bisection on the radius until `sample` seeded queries average `target`
    points with d2 <= r^2 (self included), rounded to 6 decimals."""
    rng = np.random.RandomState(0)
    qi = rng.choice(len(pts), size=min(sample, len(pts)), replace=False)
    d2 = np.empty((len(qi), len(pts)), dtype=np.float32)
    for i, q in enumerate(pts[qi]):
        diff = pts - q
        d2[i] = (diff * diff).sum(axis=1)
    want = target * len(qi)
    for _ in range(iters):
        mid = 0.5 * (lo + hi)
        if int((d2 <= mid * mid).sum()) < want:
            lo = mid
        else:
            hi = mid
    return round(0.5 * (lo + hi), 6)


def ref_sweep(D, N):
    """One cell of the reference's published K=16 sweep, at its published radius."""
    r, ms = REF_SWEEP[(D, N)]
    return Workload(f"ref_lowrank_D{D}_N{N}_K16", ref_lowrank_points(N, D), r, REF_K,
                    {"a100_ms": ms, "source": "reference published sweep (A100)"})


def config(name, N=None):
    """BASELINE.json configurations by name ('C1'..'C5', 'metric'), optional N
    override; 'refD<D>N<N>' is a cell of the reference's published K=16 sweep."""
    if name.startswith("refD"):
        d, n = name[4:].split("N")
        return ref_sweep(int(d), int(n))
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
