"""float64 CPU restatement of the rotation calibration math (TEST INFRASTRUCTURE, never
product): the checker of the GPU calibration kernels (oscar_new_amd/calibration.py).

Reference: oscar_ascend/calibration_kernels.py (Gram sums 14-70, attention weights 73-126,
normalize 129-156, cyclic Jacobi 159-249, U H Pbr 270-284) and the CPU oracles of
tests/test_calibration_math.py:6-92.

Pinned in tests/test_calibration.py: the butterflies against the recursive Sylvester
matrix; the bit-reversed scatter against the explicit permutation-matrix product and a
hand-worked D = 4 case; the round-robin schedule against "every pair exactly once per
sweep"; the Jacobi eigenpairs against torch.linalg.eigh (LAPACK) and by reconstruction; the
streaming weighted covariance against the reference test's one-shot normalization.
"""

from __future__ import annotations

import math

import torch

__all__ = [
    "gram", "key_weights", "query_covariance", "WeightedCovariance", "round_pairs",
    "jacobi_eigh", "eigenpairs", "hadamard_rows", "bit_reverse", "compose_rotation",
]


def gram(x, weights=None):
    """sum over rows (token, head) of w x x^T, float64 (calibration_kernels.py:14-56)."""
    flat = x.reshape(-1, x.shape[-1]).double()
    w = torch.ones(flat.shape[0], dtype=torch.float64) if weights is None else weights.double()
    return flat.T @ (flat * w[:, None])


def query_covariance(q):
    """Per-layer query covariance over tokens and query heads: q [T, Hq, D]."""
    flat = q.reshape(-1, q.shape[-1]).double()
    return flat.T @ flat / flat.shape[0]


def key_weights(k, qcov):
    """Attention weight of each key row, max(k_t^T C_q k_t, 0) (calibration_kernels.py:93-99)."""
    k = k.reshape(-1, k.shape[-1]).double()
    return ((k @ qcov.double()) * k).sum(-1).clamp_min(0.0)


class WeightedCovariance:
    """Streaming sum_t w_t x_t x_t^T / sum_t w_t over chunks of rows x [T, D] and weights [T]."""

    def __init__(self, dim):
        self.total = torch.zeros((dim, dim), dtype=torch.float64)
        self.weight = 0.0

    def update(self, rows, weights=None):
        self.total += gram(rows, weights)
        self.weight += float(rows.shape[0] if weights is None else weights.double().sum())

    def finalize(self):
        if not self.weight > 0:
            raise RuntimeError("No calibration tokens were observed")
        return self.total / self.weight


def round_pairs(dim, r):
    """The disjoint (p, q) pairs of round r of the round-robin schedule
    (calibration_kernels.py:170-174): (dim - 1, r), then ((r + j) mod (dim - 1),
    (r - j) mod (dim - 1)) for j = 1 .. dim/2 - 1."""
    j = torch.arange(dim // 2)
    p = torch.where(j == 0, dim - 1, (r + j) % (dim - 1))
    q = torch.where(j == 0, r, (r - j + dim - 1) % (dim - 1))
    return p, q


def jacobi_eigh(covariance, sweeps=10):
    """Cyclic two-sided Jacobi in float64 (calibration_kernels.py:159-249): per round, the
    rotation angle of each pair from the current A, then A <- J^T (A J) and U <- U J.
    Returns (U with columns sorted by ascending eigenvalue, eigenvalues ascending)."""
    a = (covariance.double() + covariance.double().T) / 2
    dim = a.shape[0]
    u = torch.eye(dim, dtype=torch.float64)
    for _ in range(sweeps):
        for r in range(dim - 1):
            p, q = round_pairs(dim, r)
            app, aqq, apq = a[p, p], a[q, q], a[p, q]
            delta = (aqq - app) / 2
            sign = torch.where(delta >= 0, 1.0, -1.0)
            t = sign * apq / (delta.abs() + (delta * delta + apq * apq).sqrt()).clamp_min(1e-30)
            t = torch.where(apq.abs() > 1e-8 * (app.abs() + aqq.abs()) + 1e-20, t, 0.0)
            c = 1 / (1 + t * t).sqrt()
            s = t * c
            b = a.clone()
            b[:, p], b[:, q] = a[:, p] * c - a[:, q] * s, a[:, p] * s + a[:, q] * c
            nu = u.clone()
            nu[:, p], nu[:, q] = u[:, p] * c - u[:, q] * s, u[:, p] * s + u[:, q] * c
            a = b.clone()
            a[p], a[q] = c[:, None] * b[p] - s[:, None] * b[q], s[:, None] * b[p] + c[:, None] * b[q]
            u = nu
    values = a.diag()
    order = values.argsort(stable=True)
    return u[:, order], values[order]


def eigenpairs(covariance):
    """Eigenvalues ascending and matching eigenvectors (columns) by LAPACK (torch.linalg.eigh)."""
    values, vectors = torch.linalg.eigh(covariance.double())
    order = values.argsort()
    return vectors[:, order], values[order]


def hadamard_rows(x):
    """Rows of ``x`` [.., D] times the orthonormal Sylvester Hadamard matrix H_D (butterflies
    over bits 0, 1, ..., log2 D - 1, as calibration_kernels.py:273-275)."""
    y = x.clone()
    dim = y.shape[-1]
    if dim & (dim - 1):
        raise ValueError("Hadamard size must be a power of two")
    idx = torch.arange(dim)
    for bit in range(dim.bit_length() - 1):
        partner = y[..., idx ^ (1 << bit)]
        low = (idx & (1 << bit)) == 0
        y = torch.where(low, y + partner, partner - y)
    return y / math.sqrt(dim)


def bit_reverse(i, bits):
    return int(f"{i:0{bits}b}"[::-1], 2)


def compose_rotation(u_ascending):
    """R = U H Pbr for eigenvectors sorted by ascending eigenvalue (columns of ``u``):
    element i of each row of U H lands in column bit_reverse(D - 1 - i)
    (calibration_kernels.py:276-284)."""
    dim = u_ascending.shape[-1]
    bits = dim.bit_length() - 1
    y = hadamard_rows(u_ascending)
    dest = torch.tensor([bit_reverse(dim - 1 - i, bits) for i in range(dim)])
    r = torch.empty_like(y)
    r[..., dest] = y
    return r
