"""Rotation artefacts and the CPU calibration oracle (reference rotations.py,
calibration_kernels.py:159-327, tests/test_calibration_math.py), CPU.

Pins of ``oracle/calibration_oracle.py``: the butterfly Hadamard against the recursive
Sylvester matrix; the bit-reversed scatter against the explicit permutation-matrix product
(and a hand-worked D = 4 case); the round-robin schedule covers every pair once per sweep;
the Jacobi eigenpairs against LAPACK (torch.linalg.eigh), by reconstruction and against a
diagonal covariance's known answer; R orthogonal; the streaming weighted covariance against
the one-shot normalization of the reference test.
"""

import math

import pytest
import torch

from oracle import calibration_oracle as C
from oscar_new_amd import rotations as R


def sylvester(dim):
    h = torch.ones((1, 1), dtype=torch.float64)
    while h.shape[0] < dim:
        h = torch.cat((torch.cat((h, h), 1), torch.cat((h, -h), 1)), 0)
    return h / math.sqrt(dim)


def permutation_matrix(dim):
    bits = dim.bit_length() - 1
    perm = torch.empty(dim, dtype=torch.long)
    for i in range(dim):
        perm[int(format(i, f"0{bits}b")[::-1], 2)] = dim - 1 - i
    return torch.eye(dim, dtype=torch.float64)[:, perm]


@pytest.mark.parametrize("dim", [4, 16, 256])
def test_hadamard_butterfly_is_the_sylvester_matrix(dim):
    x = torch.randn(3, dim, dtype=torch.float64, generator=torch.Generator().manual_seed(dim))
    torch.testing.assert_close(C.hadamard_rows(x), x @ sylvester(dim), atol=1e-12, rtol=1e-12)


def test_composition_is_u_h_pbr_and_orthogonal():
    g = torch.Generator().manual_seed(14)
    x = torch.randn(48, 16, dtype=torch.float64, generator=g)
    u, _ = C.eigenpairs(x.T @ x)
    r = C.compose_rotation(u)
    torch.testing.assert_close(r, u @ sylvester(16) @ permutation_matrix(16), atol=1e-12,
                               rtol=1e-12)
    torch.testing.assert_close(r.T @ r, torch.eye(16, dtype=torch.float64), atol=1e-10,
                               rtol=1e-10)
    # D = 4 by hand: bit reversal [0, 2, 1, 3]; element i of (U H) goes to column
    # bitrev(3 - i) = [3, 1, 2, 0].
    y = C.hadamard_rows(torch.eye(4, dtype=torch.float64))
    r4 = C.compose_rotation(torch.eye(4, dtype=torch.float64))
    for i, col in enumerate([3, 1, 2, 0]):
        torch.testing.assert_close(r4[:, col], y[:, i])


def test_eigenpairs_reconstruct_and_sort_ascending():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(300, 256, dtype=torch.float64, generator=g)
    cov = x.T @ x / 300
    u, values = C.eigenpairs(cov)
    assert bool((values[1:] >= values[:-1]).all())
    torch.testing.assert_close(u @ torch.diag(values) @ u.T, cov, atol=1e-9, rtol=0)
    rotation = C.compose_rotation(u)
    torch.testing.assert_close(rotation.T @ rotation, torch.eye(256, dtype=torch.float64),
                               atol=1e-9, rtol=0)
    diag = torch.diag(torch.tensor([3.0, 1.0, 2.0, 0.5], dtype=torch.float64))
    u, vals = C.eigenpairs(diag)
    torch.testing.assert_close(vals, torch.tensor([0.5, 1.0, 2.0, 3.0], dtype=torch.float64))
    torch.testing.assert_close(u.abs(), torch.eye(4, dtype=torch.float64)[:, [3, 1, 2, 0]])


@pytest.mark.parametrize("dim", [4, 16, 256])
def test_round_robin_schedule_covers_every_pair_once_per_sweep(dim):
    seen = set()
    for r in range(dim - 1):
        p, q = C.round_pairs(dim, r)
        assert len(set(p.tolist()) | set(q.tolist())) == dim  # disjoint pairs cover 0..dim-1
        seen.update(tuple(sorted(pq)) for pq in zip(p.tolist(), q.tolist()))
    assert len(seen) == dim * (dim - 1) // 2


def test_jacobi_matches_lapack_and_reconstructs():
    g = torch.Generator().manual_seed(14)
    x = torch.randn(48, 16, dtype=torch.float64, generator=g)
    cov = x.T @ x
    u, values = C.jacobi_eigh(cov)
    torch.testing.assert_close(values, torch.linalg.eigvalsh(cov), atol=1e-9, rtol=1e-10)
    # Rotations stop once |a_pq| <= 1e-8 (|a_pp| + |a_qq|), which bounds the reconstruction.
    torch.testing.assert_close(u @ torch.diag(values) @ u.T, cov, atol=1e-5, rtol=1e-6)
    ref, _ = C.eigenpairs(cov)
    signs = torch.sign((u * ref).sum(0))
    torch.testing.assert_close(u * signs, ref, atol=1e-6, rtol=0)
    torch.testing.assert_close(C.jacobi_eigh(torch.diag(torch.tensor([3.0, 1.0, 2.0])))[1],
                               torch.tensor([1.0, 2.0, 3.0], dtype=torch.float64))


def test_gram_and_key_weights_against_direct_sums():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(5, 3, 8, dtype=torch.float64, generator=g)
    w = torch.rand(15, dtype=torch.float64, generator=g)
    direct = sum(w[i] * torch.outer(x.reshape(15, 8)[i], x.reshape(15, 8)[i]) for i in range(15))
    torch.testing.assert_close(C.gram(x, w), direct)
    qcov = -torch.eye(8, dtype=torch.float64)  # negative quadratic forms clamp to zero
    assert (C.key_weights(x[:, 0], qcov) == 0).all()


def test_streaming_weighted_covariance_matches_one_shot_normalization():
    g = torch.Generator().manual_seed(62)
    q = torch.randn(45, 6, 16, dtype=torch.float64, generator=g)
    k = torch.randn(45, 16, dtype=torch.float64, generator=g)
    v = torch.randn(45, 16, dtype=torch.float64, generator=g)
    qcov = C.query_covariance(q)
    torch.testing.assert_close(qcov, q.reshape(-1, 16).T @ q.reshape(-1, 16) / 270)
    w = C.key_weights(k, qcov)
    vw = v * (w / w.sum() * 45).sqrt()[:, None]
    official = vw.T @ vw / 45
    acc = C.WeightedCovariance(16)
    for start in range(0, 45, 7):
        acc.update(v[start : start + 7], w[start : start + 7])
    torch.testing.assert_close(acc.finalize(), official)
    with pytest.raises(RuntimeError):
        C.WeightedCovariance(16).finalize()


def test_rotation_artefacts_round_trip_and_rejections(tmp_path):
    assert R.layer_index("model.layers.17.self_attn") == 17
    with pytest.raises(ValueError):
        R.layer_index("model.embed_tokens")
    g = torch.Generator().manual_seed(5)
    good = {3: C.compose_rotation(C.eigenpairs(torch.randn(64, 256, dtype=torch.float64,
                                                           generator=g).T.cov())[0])}
    path = tmp_path / "k.pt"
    R.save_rotations(path, good)
    r = R.get_rotation(str(path), "model.layers.3.self_attn", "cpu")
    assert r.dtype == torch.bfloat16 and r.shape == (256, 256)
    torch.testing.assert_close(r.float(), good[3].float(), atol=1e-2, rtol=0)
    with pytest.raises(ValueError, match="no rotation for layer 4"):
        R.get_rotation(str(path), "model.layers.4.self_attn", "cpu")
    stacked = tmp_path / "stack.pt"
    torch.save(torch.stack([torch.eye(256), 2 * torch.eye(256)]), stacked)
    assert R.get_rotation(str(stacked), "layers.0", "cpu").shape == (256, 256)
    with pytest.raises(ValueError, match="departs from the identity"):
        R.get_rotation(str(stacked), "layers.1", "cpu")
    # The acceptance bound is 0.015 off the diagonal and 0.03 on it (the reference's).
    nearly = torch.eye(256) * (1.014 ** 0.5)
    R.check_rotation(nearly)
    with pytest.raises(ValueError):
        R.check_rotation(torch.eye(256) * (1.031 ** 0.5))
    bad = tmp_path / "bad.pt"
    torch.save({"layers": {0: torch.eye(128), 1: torch.full((256, 256), float("inf"))}}, bad)
    with pytest.raises(ValueError, match="expected 256x256"):
        R.get_rotation(str(bad), "layers.0", "cpu")
    with pytest.raises(ValueError, match="NaN or infinite"):
        R.get_rotation(str(bad), "layers.1", "cpu")
    odd = tmp_path / "odd.pt"
    torch.save([torch.eye(256)], odd)
    with pytest.raises(ValueError, match="unrecognized rotation artefact"):
        R.load_checkpoint(str(odd))
    with pytest.raises(ValueError, match="VLLM_OSCAR_K_ROTATION_PATH"):
        R.load_checkpoint("")
    assert R.layer_index("layers.2") == 2 and R.layer_index("a.layers.x.layers.5.b") == 5
