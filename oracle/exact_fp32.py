"""Exact fp32 arithmetic emulated in numpy float64 -- TEST INFRASTRUCTURE ONLY.

This module is an independent pin for the C++ oracle (oracle/frnn_oracle.cpp):
it re-derives the reference's fp32 distance orders and the brute-force
selection without sharing any code with the oracle or with the HIP engine.

* ``fma32(a, b, c)`` is a correctly rounded fp32 fused multiply-add built from
  first principles: the fp32 product a*b is exact in float64 (24+24 bits), the
  float64 sum is made exact with Knuth's TwoSum, and the one double-rounding
  hazard (a float64 sum that lands exactly on an fp32 midpoint) is resolved
  from the sign of the TwoSum error term.
* ``dist2(q, p, order)`` follows the reference's fp32 orders:
  order 0 = sequential ``fmaf(diff, diff, d2)`` over d = 0..D-1
  (frnn/csrc/grid/find_nbrs.cu:194-199 and :335-340),
  order 1 = ``fmaf(dx,dx,fmaf(dy,dy,dz*dz))`` generalised as the reversed
  sequence (find_nbrs.cu:474-477).
* ``brute_force`` selects, per query, the K smallest (d2, idx) among points
  with d2 < fl32(r*r), padding with (r2, -1)
  (no_grid_frnn.cu:163-176, find_nbrs.cu:136-143).
"""
import numpy as np


def fma32(a, b, c):
    """Correctly rounded fp32 fma of numpy float32 arrays (round-to-nearest-even)."""
    a64 = np.asarray(a, dtype=np.float32).astype(np.float64)
    b64 = np.asarray(b, dtype=np.float32).astype(np.float64)
    c64 = np.asarray(c, dtype=np.float32).astype(np.float64)
    p = a64 * b64                      # exact: 48-bit significand product
    s = p + c64                        # float64 rounding
    bp = s - c64                       # Knuth TwoSum: s + e == c + p exactly
    ap = s - bp
    e = (c64 - ap) + (p - bp)
    with np.errstate(over="ignore", invalid="ignore"):
        r = s.astype(np.float32)
        r64 = r.astype(np.float64)
        # neighbour of r on the other side of s
        toward = np.where(s > r64, np.float32(np.inf), np.float32(-np.inf)).astype(np.float32)
        other = np.nextafter(r, toward)
        mid = (r64 + other.astype(np.float64)) * 0.5
    on_mid = (r64 != s) & (s == mid) & (e != 0) & np.isfinite(s)
    if np.any(on_mid):
        # s sits exactly on the fp32 midpoint; the exact value is above s when
        # e > 0 and below when e < 0, so round to the neighbour on that side.
        hi = np.maximum(r, other)
        lo = np.minimum(r, other)
        fixed = np.where(e > 0, hi, lo)
        r = np.where(on_mid, fixed, r)
    # exact ties (e == 0 and s on a midpoint) were already rounded to even by the cast
    return r.astype(np.float32)


def dist2(q, p, order=0):
    """fp32 squared distance between rows q[..., D] and p[..., D] (broadcasting)."""
    q = np.asarray(q, dtype=np.float32)
    p = np.asarray(p, dtype=np.float32)
    D = q.shape[-1]
    dims = range(D - 1, -1, -1) if order == 1 else range(D)
    acc = None
    for d in dims:
        diff = (q[..., d] - p[..., d]).astype(np.float32)
        if acc is None:
            acc = np.zeros(np.broadcast(q[..., d], p[..., d]).shape, dtype=np.float32)
        acc = fma32(diff, diff, acc)
    return acc


def brute_force(X, K, radius, order=0, Q=None):
    """FRNN on AoS X[N, D] (fp32) by exhaustive search: all points as queries,
    or the separate queries Q[M, D] against the points of X.

    Returns (idx[M, K] int32, dist[M, K] float32) with rows in ascending
    (d2, idx) order and (r2, -1) padding.  Quadratic memory: small N only.
    """
    X = np.asarray(X, dtype=np.float32)
    Q = X if Q is None else np.asarray(Q, dtype=np.float32)
    N, M = X.shape[0], Q.shape[0]
    r2 = np.float32(np.float32(radius) * np.float32(radius))
    E = dist2(Q[:, None, :], X[None, :, :], order)          # [M, N]
    idx = np.full((M, K), -1, dtype=np.int32)
    dist = np.full((M, K), r2, dtype=np.float32)
    cols = np.arange(N)
    for i in range(M):
        row = E[i]
        m = row < r2
        cand = cols[m]
        d = row[m]
        o = np.lexsort((cand, d))[:K]
        idx[i, :len(o)] = cand[o]
        dist[i, :len(o)] = d[o]
    return idx, dist
