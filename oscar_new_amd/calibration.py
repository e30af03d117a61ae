"""Calibration math of the K/V rotations on the GPU (reference
``oscar_ascend/calibration_kernels.py``): streamed covariance sums, the attention weights of
the V covariance, normalization, and the batched Jacobi eigensolver that turns each
covariance into the rotation R = U H Pbr.

Startup-only work: the decode path only applies the resulting matrices. Every function runs
the HIP library (``csrc/calibrate.hip``); there is no CPU path. The covariance objectives:
K uses the query covariance C_q as is; V is weighted per token by w_t = max(k_t^T C_q k_t, 0),
accumulated as sum_t w_t v_t v_t^T and divided by sum_t w_t.
"""

from __future__ import annotations

import math

import torch

from . import _ext
from .kernels import _device_check, _ptr, _stream

__all__ = ["accumulate_gram", "sst_weights", "normalize", "calibrated_rotations"]

DIM = 256


def _input_flag(t, name):
    if t.dtype == torch.bfloat16:
        return 0
    if t.dtype == torch.float32:
        return 1
    raise ValueError(f"{name} must be bfloat16 or float32, got {t.dtype}")


def _fp32_matrix(t, name, shape):
    if t.dtype != torch.float32 or tuple(t.shape) != tuple(shape) or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous float32 tensor of shape {tuple(shape)}")


def accumulate_gram(x, covariance, weights=None):
    """covariance += sum over rows (token, head) of w x x^T (calibration_kernels.py:59-70).

    ``x``: [n, heads, dim] bf16 or fp32 (any strides); ``covariance``: fp32 [dim, dim],
    updated in place; ``weights``: optional fp32 [n * heads] (row token * heads + head).
    """
    _device_check(x, covariance, weights)
    n, heads, dim = x.shape
    flag = _input_flag(x, "x")
    _fp32_matrix(covariance, "covariance", (dim, dim))
    if weights is not None and (weights.dtype != torch.float32 or weights.numel() != n * heads
                                or not weights.is_contiguous()):
        raise ValueError("weights must be a contiguous float32 tensor with one value per row")
    _ext.check(
        _ext.library().oscar_accumulate_gram(
            _ptr(x), flag, n, heads, dim, *x.stride(), _ptr(weights), _ptr(covariance),
            _stream(x)),
        "accumulate_gram",
    )
    return covariance


def sst_weights(key, q_covariance, total_weight):
    """Per-token weights max(k^T C_q k, 0) of the keys of one KV head, and
    ``total_weight += their sum`` (calibration_kernels.py:109-126).

    ``key``: [n, 1, 256] bf16 or fp32; ``q_covariance``: fp32 [256, 256]; ``total_weight``:
    fp32 scalar tensor on the device. Returns fp32 [n].
    """
    _device_check(key, q_covariance, total_weight)
    n, heads, dim = key.shape
    if heads != 1:
        raise ValueError(f"sst_weights takes the keys of one KV head ([n, 1, {DIM}]); got "
                         f"{heads} heads")
    if dim != DIM:
        raise ValueError(f"the calibration weights are built for head_dim {DIM}, got {dim}")
    flag = _input_flag(key, "key")
    _fp32_matrix(q_covariance, "q_covariance", (DIM, DIM))
    if total_weight.dtype != torch.float32 or total_weight.numel() != 1:
        raise ValueError("total_weight must be a float32 scalar tensor")
    weights = torch.empty(n, dtype=torch.float32, device=key.device)
    _ext.check(
        _ext.library().oscar_sst_weights(
            _ptr(key), flag, n, dim, key.stride(0), key.stride(2), _ptr(q_covariance),
            _ptr(weights), _ptr(total_weight), _stream(key)),
        "sst_weights",
    )
    return weights


def normalize(x, denominator):
    """x / max(denominator, 1e-30) (calibration_kernels.py:145-156); ``denominator`` is a
    number or an fp32 scalar tensor on the device (read there, no host sync)."""
    _device_check(x)
    if x.dtype != torch.float32 or not x.is_contiguous():
        raise ValueError("normalize takes a contiguous float32 tensor")
    out = torch.empty_like(x)
    if isinstance(denominator, torch.Tensor):
        _device_check(denominator)
        if denominator.dtype != torch.float32 or denominator.numel() != 1:
            raise ValueError("a tensor denominator must be a float32 scalar")
        den, value = _ptr(denominator), 1.0
    else:
        den, value = None, float(denominator)
    _ext.check(
        _ext.library().oscar_normalize(_ptr(x), x.numel(), den, value, _ptr(out), _stream(x)),
        "normalize",
    )
    return out


def calibrated_rotations(covariances, max_sweeps=12, tolerance=1e-6):
    """Batched eigen-decomposition and R = U H Pbr (calibration_kernels.py:287-327).

    ``covariances``: fp32 [batch, 256, 256] on the device. Returns ``(rotations fp32 [batch,
    256, 256], eigenvalues fp32 [batch, 256] ascending, {"sweeps", "relative_off_diagonal"})``.
    All sweeps run on the device; only the per-matrix (sweeps, residual) pairs are read back
    at the end. Raises RuntimeError for a non-finite covariance or when the residual is not
    below ``tolerance`` after ``max_sweeps`` sweeps (nothing is returned then).
    """
    _device_check(covariances)
    if covariances.dim() != 3 or covariances.dtype != torch.float32:
        raise ValueError("covariances must be float32 [batch, 256, 256]")
    batch, dim, last = covariances.shape
    if dim != DIM or last != DIM:
        raise ValueError(f"the eigensolver is built for {DIM} x {DIM} covariances, got "
                         f"{dim} x {last}")
    if not 1 <= max_sweeps <= 64:
        raise ValueError("max_sweeps must be in [1, 64]")
    lib = _ext.library()
    cov = covariances.contiguous()
    size = lib.oscar_calibration_workspace_bytes(batch, max_sweeps)
    workspace = torch.empty(size, dtype=torch.uint8, device=cov.device)
    rotations = torch.empty_like(cov)
    eigenvalues = torch.empty((batch, DIM), dtype=torch.float32, device=cov.device)
    info = torch.empty((batch, 2), dtype=torch.float32, device=cov.device)
    _ext.check(
        lib.oscar_calibrated_rotations(_ptr(cov), batch, dim, max_sweeps, float(tolerance),
                                       _ptr(workspace), size, _ptr(rotations),
                                       _ptr(eigenvalues), _ptr(info), _stream(cov)),
        "calibrated_rotations",
    )
    done = info.cpu()
    residual = float(done[:, 1].max())
    sweeps = int(done[:, 0].max())
    if not math.isfinite(residual):
        raise RuntimeError("calibration covariance holds NaN or infinite values; no rotation "
                           "is produced")
    if not residual < tolerance:
        raise RuntimeError(f"Jacobi sweeps stopped at relative off-diagonal {residual:.3e} "
                           f"(tolerance {tolerance:g}) after {sweeps} sweeps; no rotation is "
                           "produced")
    return rotations, eigenvalues, {"sweeps": sweeps, "relative_off_diagonal": residual}
