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
