"""Calibration math of the K/V rotations (reference calibration_kernels.py:250-327 and
tests/test_calibration_math.py): the attention-weighted covariances, their eigenvectors and
the rotation R = U H Pbr.

* Covariances (test_calibration_math.py:70-91): K uses the query covariance as is; V is
  weighted per token by w_t = k_t^T C_q k_t, accumulated in chunks as
  sum_t w_t v_t v_t^T / sum_t w_t (``WeightedCovariance``), equal to the one-shot form.
* Eigenvectors: ``torch.linalg.eigh`` (LAPACK / rocSOLVER) replaces the reference's cyclic
  Jacobi sweeps on the NPU; the eigenpairs are sorted ascending as the reference sorts them.
  Calibration runs once per model, off the decode path.
* Composition (calibration_kernels.py:270-284): each row of U goes through the in-place
  Walsh-Hadamard butterfly, scaled by 1/sqrt(D), and element i lands in column
  bit_reverse(D - 1 - i) (the descending-eigenvalue bit-reversal permutation Pbr).
"""

from __future__ import annotations

import math

import torch


def hadamard_rows(x):
    """Rows of ``x`` [.., D] times the orthonormal Sylvester Hadamard matrix H_D (butterflies)."""
    y = x.clone()
    dim = y.shape[-1]
    if dim & (dim - 1):
        raise ValueError("Hadamard size must be a power of two")
    idx = torch.arange(dim, device=y.device)
    for bit in range(dim.bit_length() - 1):
        partner = y[..., idx ^ (1 << bit)]
        low = (idx & (1 << bit)) == 0
        y = torch.where(low, y + partner, partner - y)
    return y / math.sqrt(dim)


def bit_reverse(i, bits):
    return int(f"{i:0{bits}b}"[::-1], 2)


def compose_rotation(u_ascending):
    """R = U H Pbr for eigenvectors sorted by ascending eigenvalue (columns of ``u``)."""
    dim = u_ascending.shape[-1]
    bits = dim.bit_length() - 1
    y = hadamard_rows(u_ascending)
    dest = torch.tensor([bit_reverse(dim - 1 - i, bits) for i in range(dim)], device=y.device)
    r = torch.empty_like(y)
    r[..., dest] = y
    return r


def eigenpairs(covariance):
    """Eigenvalues ascending and matching eigenvectors (columns) of a symmetric matrix."""
    values, vectors = torch.linalg.eigh(covariance.double())
    order = values.argsort()
    return vectors[:, order], values[order]


def calibrated_rotation(covariance):
    """The rotation of one covariance, its eigenvalues and the reconstruction residual."""
    if not torch.isfinite(covariance).all():
        raise RuntimeError("Nonfinite calibration covariance; rotations not published")
    u, values = eigenpairs(covariance)
    rotation = compose_rotation(u)
    residual = (u @ torch.diag(values) @ u.T - covariance.double()).abs().max().item()
    return rotation.float(), values.float(), residual


class WeightedCovariance:
    """Streaming sum_t w_t x_t x_t^T / sum_t w_t over chunks of rows x [T, D] and weights [T]."""

    def __init__(self, dim, device="cpu"):
        self.total = torch.zeros((dim, dim), dtype=torch.float64, device=device)
        self.weight = 0.0

    def update(self, rows, weights=None):
        rows = rows.double()
        w = torch.ones(rows.shape[0], dtype=torch.float64, device=rows.device) if weights is None \
            else weights.double()
        self.total += rows.T @ (rows * w[:, None])
        self.weight += float(w.sum())

    def finalize(self):
        if not self.weight > 0:
            raise RuntimeError("No calibration tokens were observed")
        return self.total / self.weight


def query_covariance(q):
    """Per-layer query covariance over tokens and query heads: q [T, Hq, D]."""
    flat = q.reshape(-1, q.shape[-1]).double()
    return flat.T @ flat / flat.shape[0]


def key_weights(k, qcov):
    """Attention weight of each key row, w_t = k_t^T C_q k_t (k [T, D])."""
    k = k.double()
    return (k @ qcov * k).sum(-1)
