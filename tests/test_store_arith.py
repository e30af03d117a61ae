"""CPU checks of the quantizer's arithmetic shortcuts (csrc/quant.h), each against what the
IEEE operations they replace give:

- `search_factor`: one FMA, fl(i * f32(0.4/7) + f32(0.6)), for the eight clip factors
  f32(0.6 + 0.4 i / 7) evaluated in double (the `search` mode's factors);
- `div3`: q0 = fl(x * fl(1/3)), r = fma(-q0, 3, x), fma(r, fl(1/3), q0) against the IEEE
  quotient x / 3, for every non-negative finite float (the spread (max - min) / 3 of
  tests/oracle.py:15-17 and kernels.py:104-137 is never negative).
"""

import shutil
import subprocess
from fractions import Fraction

import numpy as np
import pytest

_DIV3_C = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#ifndef STRIDE
#define STRIDE 1
#endif
int main(void) {
  const float c = 1.0f / 3.0f;
  unsigned long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
  for (long long u = 0; u < 0x7f800000ll; u += STRIDE) {
    uint32_t v = (uint32_t)u;
    float x;
    memcpy(&x, &v, 4);
    const float q0 = x * c;
    const float r = fmaf(-q0, 3.0f, x);
    const float q = fmaf(r, c, q0);
    const float e = x / 3.0f;
    if (memcmp(&q, &e, 4)) ++bad;
  }
  printf("%llu\n", bad);
  return 0;
}
"""


def _f32(x):
    return np.float32(x)


def test_search_factor_fma_matches_the_double_formula():
    step, base = _f32(0.4 / 7.0), _f32(0.6)
    for i in range(8):
        want = _f32(0.6 + 0.4 * i / 7.0)
        # One rounding of the exact i * step + base (an FMA).
        exact = Fraction(i) * Fraction(float(step)) + Fraction(float(base))
        got = _f32(float(exact))  # float(exact) is exact here: 27 significant bits at most
        assert float(exact) == exact
        assert got == want, (i, got, want)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not found")
def test_div3_sequence_is_the_ieee_quotient_for_every_nonnegative_float(tmp_path):
    src = tmp_path / "div3.c"
    src.write_text(_DIV3_C)
    exe = tmp_path / "div3"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", str(src), "-o", str(exe),
                    "-lm"], check=True, capture_output=True, timeout=120)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=300)
    assert out.stdout.strip() == "0"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not found")
def test_div3_check_catches_a_wrong_constant(tmp_path):
    # The same loop with the correction step dropped (q = q0) must report mismatches.
    src = tmp_path / "div3_bad.c"
    src.write_text(_DIV3_C.replace("fmaf(r, c, q0)", "q0 + 0.0f * r"))
    exe = tmp_path / "div3_bad"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-DSTRIDE=4097", str(src),
                    "-o", str(exe), "-lm"], check=True, capture_output=True, timeout=120)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=300)
    assert int(out.stdout.strip()) > 0


# ---------------------------------------------------------------- clip-search fast pass bound

from oracle import oscar_oracle as ora  # noqa: E402


def _fast_and_exact(x, rcp_ulps=0, margin_scale=1.0, drop_s2=False):
    """The kernel's fast pass (quant.h candidate_fast + search_best's scaling) restated in
    numpy float32, and the oracle's exact MSE, for every row of x and every search factor.
    Returns (fast [N, 8], exact [N, 8], margin [N, 8])."""
    x = np.asarray(x, np.float32)
    n = x.shape[0]
    mn = x.min(-1)
    mx = x.max(-1)
    maxabs = np.maximum(np.abs(mn), np.abs(mx)).astype(np.float32)
    fast = np.zeros((n, 8), np.float32)
    exact = np.zeros((n, 8), np.float32)
    margin = np.zeros((n, 8), np.float32)
    valid = np.zeros((n, 8), bool)
    for i, f in enumerate(ora.search_factors()):
        t = (maxabs * f).astype(np.float32)
        lo = np.minimum(np.maximum(mn, -t), t)
        hi = np.minimum(np.maximum(mx, -t), t)
        spread_raw = ((hi - lo).astype(np.float32) / np.float32(3)).astype(np.float32)
        spread = np.maximum(spread_raw, np.float32(2.0**-14))
        z = lo.astype(np.float16).astype(np.float32)
        s = spread.astype(np.float16).astype(np.float32)
        valid[:, i] = (spread_raw >= np.float32(2.0**-14)) & (
            np.abs((lo - z).astype(np.float32)) <= np.float32(0.25) * s)
        r = (np.float32(1) / s).astype(np.float32)
        for _ in range(abs(rcp_ulps)):  # v_rcp_f32 is within one ulp of the quotient
            r = np.nextafter(r, np.float32(np.inf) if rcp_ulps > 0 else np.float32(0))
        bz = (-(z * r)).astype(np.float32)
        u = ora.fma_f32(x, r[:, None], bz[:, None])
        d = (u - np.clip(np.rint(u), 0, 3)).astype(np.float32)
        lanes = d.reshape(n, 64, 4)
        acc = np.zeros((n, 64), np.float32)
        for e in range(4):
            acc = ora.fma_f32(lanes[..., e], lanes[..., e], acc)
        total = ora._tree_sum(acc)
        s2 = np.float32(1) if drop_s2 else (s * s).astype(np.float32)
        fast[:, i] = (total * s2).astype(np.float32)
        ms = (maxabs + s).astype(np.float32)
        margin[:, i] = margin_scale * (np.float32(0.00390625) * ms * ms
                                       + np.float32(3.814697265625e-06) * fast[:, i])
        # The oracle's MSE of this candidate (oracle quantize, search branch).
        xc = ora._clip(x, t[:, None])
        code, scale, zero = ora._quantize_clipped(xc)
        decoded = (code.astype(np.float32) * scale.astype(np.float32)
                   + zero.astype(np.float32)).astype(np.float32)
        err = (x - decoded).astype(np.float32)
        exact[:, i] = ora._tree_sum((err * err).astype(np.float32))
    return fast, exact, margin, valid


def _decide(fast, exact, margin, valid):
    """search_best's decision: the fast argmin when every candidate is valid and no other
    candidate's interval reaches it, else the exact pass (first minimum)."""
    rows = np.arange(len(fast))
    best = np.argmin(fast, 1)
    reach = fast[rows, best] + margin[rows, best]
    conflict = (fast - margin) <= reach[:, None]
    conflict[rows, best] = False
    use_fast = valid.all(1) & ~conflict.any(1)
    return np.where(use_fast, best, np.argmin(exact, 1)), use_fast


def _bf16(x):
    return ora.bf16_to_f32(ora.f32_to_bf16(np.asarray(x, np.float32)))


def _vectors():
    g = np.random.default_rng(77)
    out = [g.standard_normal((1500, 256))]
    o = g.standard_normal((1000, 256))
    o[:, g.choice(256, 5, replace=False)] *= 10.0  # outlier channels
    out.append(o)
    out.append(100.0 + 0.01 * g.standard_normal((300, 256)))  # large offset, small spread
    out.append(-50.0 + g.uniform(0, 1, (300, 256)))
    out.append(1e-5 * g.standard_normal((200, 256)))  # scale clamped to 2^-14
    sparse = np.zeros((200, 256))
    sparse[np.arange(200), g.integers(0, 256, 200)] = g.standard_normal(200) * 30
    out.append(sparse + 0.001 * g.standard_normal((200, 256)))
    out.append(np.full((20, 256), 3.25))  # constant rows
    out.append(g.standard_t(2, (500, 256)))  # heavy tails
    return _bf16(np.concatenate(out).astype(np.float32))


def _tiny():
    # Spreads below 3 * 2^-14: the scale is raised to 2^-14 and clipped values can take inner
    # codes (the fast pass's assumption fails; such vectors go to the exact pass).
    g = np.random.default_rng(78)
    return _bf16(np.concatenate([1e-5 * g.standard_normal((1500, 256)),
                                 3e-5 * g.standard_normal((1500, 256))]).astype(np.float32))


@pytest.mark.parametrize("rcp_ulps", [0, 1, -1])
def test_clip_search_fast_pass_is_within_half_its_margin(rcp_ulps):
    fast, exact, margin, valid = _fast_and_exact(_vectors(), rcp_ulps=rcp_ulps)
    gap = np.abs(fast.astype(np.float64) - exact.astype(np.float64))
    ok = gap <= margin.astype(np.float64) / 2
    assert np.all(ok | ~valid), float((gap / margin)[valid].max())
    assert valid[:2500].all()  # normal rows and outlier channels: the fast pass always applies


def test_clip_search_decision_is_the_exact_argmin():
    x = np.concatenate([_vectors(), _tiny()])
    fast, exact, margin, valid = _fast_and_exact(x)
    got, _ = _decide(fast, exact, margin, valid)
    assert np.array_equal(got, np.argmin(exact, 1))


def test_clip_search_checks_catch_planted_mistakes():
    # Without the validity test the tiny vectors take wrong fast decisions; without the s^2
    # scaling the bound check fails.
    fast, exact, margin, valid = _fast_and_exact(_tiny())
    got, _ = _decide(fast, exact, margin, np.ones_like(valid))
    assert not np.array_equal(got, np.argmin(exact, 1))
    fast, exact, margin, valid = _fast_and_exact(_vectors()[:500], drop_s2=True)
    gap = np.abs(fast.astype(np.float64) - exact.astype(np.float64))
    assert not np.all((gap <= margin.astype(np.float64) / 2) | ~valid)
