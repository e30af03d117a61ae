"""GPU calibration math (csrc/calibrate.hip via oscar_new_amd.calibration) against float64
references, as the reference's hardware tests check it (tests/test_npu_calibration.py:18-57):

* streamed covariances: the query Gram over chunks normalized by the row count, and the
  attention-weighted value covariance normalized by the device-side weight total, against
  float64 sums (and the weights against ``oracle/calibration_oracle.key_weights``);
* eigensolver + composition: residual below 1e-6, U recovered as R Pbr^T H^T (explicit
  permutation and Sylvester matrices) reconstructs the covariance, R orthogonal, eigenvalues
  against LAPACK, and U's columns against the float64 Jacobi oracle up to sign;
* a non-finite covariance is rejected; argument errors raise before any launch.
"""

import math

import pytest
import torch

from oracle import calibration_oracle as CO

pytestmark = pytest.mark.gpu


def _ops():
    from oscar_new_amd import calibration

    return calibration


def sylvester(dim):
    h = torch.ones((1, 1), dtype=torch.float64)
    while h.shape[0] < dim:
        h = torch.cat((torch.cat((h, h), 1), torch.cat((h, -h), 1)), 0) / math.sqrt(2)
    return h


def pbr(dim):
    bits = dim.bit_length() - 1
    perm = torch.empty(dim, dtype=torch.long)
    for i in range(dim):
        perm[CO.bit_reverse(i, bits)] = dim - 1 - i
    return torch.eye(dim, dtype=torch.float64)[:, perm]


def test_streamed_covariances_against_float64_sums():
    ops = _ops()
    g = torch.Generator().manual_seed(88)
    q = torch.randn(137, 6, 256, generator=g).bfloat16()
    k = torch.randn(137, 1, 256, generator=g).bfloat16()
    v = torch.randn(137, 1, 256, generator=g).bfloat16()
    qsum = torch.zeros((256, 256), device="cuda", dtype=torch.float32)
    for chunk in q.split(32):
        ops.accumulate_gram(chunk.cuda(), qsum)
    qcov = ops.normalize(qsum, 137 * 6)
    want_q = q.double().reshape(-1, 256).T @ q.double().reshape(-1, 256) / (137 * 6)
    torch.testing.assert_close(qcov.cpu().double(), want_q, atol=2e-5, rtol=2e-5)
    vsum = torch.zeros_like(qsum)
    total = torch.zeros((), device="cuda", dtype=torch.float32)
    weights = []
    for kc, vc in zip(k.split(32), v.split(32)):
        w = ops.sst_weights(kc.cuda(), qcov, total)
        weights.append(w.cpu())
        ops.accumulate_gram(vc.cuda(), vsum, w)
    vcov = ops.normalize(vsum, total).cpu().double()
    want_w = CO.key_weights(k[:, 0], want_q)
    torch.testing.assert_close(torch.cat(weights).double(), want_w, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(float(total), float(want_w.sum()), atol=0, rtol=1e-5)
    want_v = v[:, 0].double().T @ (v[:, 0].double() * want_w[:, None]) / want_w.sum()
    torch.testing.assert_close(vcov, want_v, atol=2e-4, rtol=2e-4)


def test_gram_of_strided_fp32_rows_with_weights():
    ops = _ops()
    g = torch.Generator().manual_seed(4)
    base = torch.randn(40, 3, 320, generator=g)
    x = base[:, :, 32:288]  # strided fp32 view [40, 3, 256]
    w = torch.rand(120, generator=g)
    cov = torch.full((256, 256), 0.5, device="cuda")
    ops.accumulate_gram(x.cuda(), cov, w.cuda())
    want = 0.5 + CO.gram(x, w)
    torch.testing.assert_close(cov.cpu().double(), want, atol=1e-4, rtol=1e-5)
    small = torch.zeros((64, 64), device="cuda")
    ops.accumulate_gram(x[..., :64].contiguous().cuda(), small)
    torch.testing.assert_close(small.cpu().double(), CO.gram(x[..., :64]), atol=1e-4, rtol=1e-5)


def test_eigensolver_and_composition_reconstruct_the_covariance():
    ops = _ops()
    g = torch.Generator().manual_seed(23)
    x = torch.randn(2, 320, 256, generator=g)
    covariance = x.transpose(-1, -2) @ x / 320
    r, eigenvalues, info = ops.calibrated_rotations(covariance.cuda())
    assert info["relative_off_diagonal"] < 1e-6 and 2 <= info["sweeps"] <= 12
    r, eigenvalues = r.cpu().double(), eigenvalues.cpu().double()
    assert bool((eigenvalues[:, 1:] >= eigenvalues[:, :-1]).all())
    u = r @ pbr(256).T @ sylvester(256).T
    reconstruction = (u * eigenvalues[:, None, :]) @ u.transpose(-1, -2)
    torch.testing.assert_close(reconstruction, covariance.double(), atol=2e-4, rtol=2e-3)
    torch.testing.assert_close(r.transpose(-1, -2) @ r,
                               torch.eye(256, dtype=torch.float64).expand(2, -1, -1),
                               atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(eigenvalues, torch.linalg.eigvalsh(covariance.double()),
                               atol=2e-4, rtol=2e-3)
    # Columns with a clear eigengap against the float64 Jacobi oracle, up to sign.
    ref_u, ref_vals = CO.jacobi_eigh(covariance[0], sweeps=8)
    gaps = torch.minimum(torch.diff(ref_vals, prepend=ref_vals[:1] - 1),
                         torch.diff(ref_vals, append=ref_vals[-1:] + 1))
    keep = gaps > 2e-3 * ref_vals.abs().max()  # about 100 of 256 columns
    signs = torch.sign((u[0] * ref_u).sum(0))
    err = (u[0] * signs - ref_u).abs()[:, keep].max()
    assert keep.sum() > 80 and err < 1e-2, (int(keep.sum()), float(err))


def test_non_finite_covariance_and_bad_arguments_are_rejected():
    ops = _ops()
    bad = torch.eye(256, device="cuda").expand(2, -1, -1).contiguous()
    bad[1, 3, 5] = float("nan")
    with pytest.raises(RuntimeError, match="NaN or infinite"):
        ops.calibrated_rotations(bad)
    ident, vals, info = ops.calibrated_rotations(torch.eye(256, device="cuda")[None] * 2.0)
    assert info["relative_off_diagonal"] == 0.0
    torch.testing.assert_close(vals.cpu(), torch.full((1, 256), 2.0))
    with pytest.raises(ValueError):
        ops.calibrated_rotations(torch.eye(128, device="cuda")[None])
    with pytest.raises(ValueError):
        ops.sst_weights(torch.zeros(4, 2, 256, device="cuda"), torch.eye(256, device="cuda"),
                        torch.zeros((), device="cuda"))
    with pytest.raises(ValueError):
        ops.accumulate_gram(torch.zeros(4, 1, 256, device="cuda"), torch.zeros(128, 128,
                                                                                 device="cuda"))
