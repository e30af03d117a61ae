"""The torch float32 CPU restatement that bench.py times as its CPU baseline
(``oracle/cpu_torch.py``), checked against the numpy oracle: dequantized rows and slot
images bit-exact, rotation within one bf16 step, attention within float32 rounding."""

import numpy as np
import pytest
import torch

import oracle as O
from oracle import cpu_torch as T
from tests.test_oracle import _paged_state


def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def test_dequant_is_bit_exact_with_the_oracle():
    rng = np.random.default_rng(5)
    n = 257
    history = rng.integers(0, 256, n * 80, dtype=np.uint8)
    offs = np.arange(n) * 80 + rng.integers(0, 12, n)
    sz = np.stack([rng.uniform(1e-3, 2.0, n), rng.uniform(-3, 3, n)], 1).astype(np.float16)
    for i, o in enumerate(offs):
        history[o + 64 : o + 68] = sz[i].view(np.uint8)
    want = O.dequant_rows(history, offs)
    got = T.dequant(torch.from_numpy(history), torch.from_numpy(offs))
    assert np.array_equal(got.numpy().view(np.uint32) >> 16, want.astype(np.uint32))


@pytest.mark.parametrize("length,prefix", [(300, 299), (300, 297), (40, 36), (3, 2)])
def test_decode_step_matches_the_cached_decode_reference(length, prefix):
    geo = O.Geometry(768, sink_tokens=4, recent_tokens=16, speculative_tokens=3)
    history, window, table, ks, vs, rk, rv = _paged_state([length], [prefix], geo, seed=11)
    t = length - prefix
    q = O.f32_to_bf16(np.random.default_rng(2).standard_normal((t, 6, 256)).astype(np.float32))
    want, want_lse = O.cached_decode_reference(history, window, table[0], length, q,
                                               ks[0][prefix:], vs[0][prefix:], rk, rv, geo,
                                               scale=1 / 16)
    got, lse = T.decode_step(torch.from_numpy(history), _bf16(window), table[0], length, _bf16(q),
                             _bf16(ks[0][prefix:]), _bf16(vs[0][prefix:]), _bf16(rk), _bf16(rv),
                             geo, scale=1 / 16)
    np.testing.assert_allclose(got.numpy(), want, rtol=1e-4, atol=2e-5)
    np.testing.assert_allclose(lse.numpy(), want_lse, atol=1e-5)


def test_rotation_is_within_one_bf16_step_of_the_oracle():
    rng = np.random.default_rng(3)
    x = O.f32_to_bf16(rng.standard_normal((64, 256)).astype(np.float32))
    r = O.f32_to_bf16(np.linalg.qr(rng.standard_normal((256, 256)))[0].astype(np.float32))
    got = T.rotate(_bf16(x), _bf16(r)).float().numpy()
    want = O.bf16_to_f32(O.rotate(x, r))
    step = np.abs(want) * 2.0 ** -7 + 1e-30
    assert (np.abs(got - want) <= step).all()
    assert (got == want).mean() > 0.99


@pytest.mark.parametrize("mode", ["percentile", "factor", "search"])
def test_slot_images_are_bit_exact_with_the_oracle(mode):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((96, 2, 256)).astype(np.float32)
    x[..., rng.choice(256, 5, replace=False)] *= 10.0  # outlier channels
    x[0, 0] = 0.5  # a constant row
    k = O.f32_to_bf16(x)
    v = O.f32_to_bf16(x[::-1].copy() * 0.3)
    cfg = {"clip_mode": mode, "k_clip_ratio": 0.96, "v_clip_ratio": 0.92,
           "k_clip_factor": 0.8, "v_clip_factor": 0.9}
    want = O.packed_slots(k, v, cfg)
    got = T.quantize_pack(_bf16(k), _bf16(v), mode, 0.96, 0.92, 0.8, 0.9)
    assert np.array_equal(got.numpy(), want)
