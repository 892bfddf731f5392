"""The fused prefill router quantizes activations without a division per
value: with ry = RN(1 / s), q0 = RN(x ry), r = fma(-q0, s, x) (exact) and
q = copysign(fma(r, ry, q0), x), q equals the IEEE quotient RN(x / s)
(Markstein's theorem, plus x's sign for x = -0) unless the residual
underflows. This checks it on the CPU (C with fmaf, no contraction) for
every bf16 x with |x| <= amax against every bf16 block maximum amax of
several binades, the scale formed as the kernel forms it:
s = max(amax, 1e-4) * RN(1 / 448): the same bits for every quotient of
2^-60 or more; below that (x so small that the residual underflows) both
quotients lie under 2^-10, the e4m3 threshold of rounding to zero, with
x's sign, so the codes are the same.
"""
import shutil
import subprocess

import pytest

C_SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t u_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
int main(void) {
  const int exps[] = {-24, -14, -13, -8, -1, 0, 1, 7, 20};
  long pairs = 0, bad = 0, tiny = 0;
  for (unsigned ei = 0; ei < sizeof exps / sizeof exps[0]; ++ei)
    for (uint32_t m = 0; m < 128; ++m) {
      const float amax = f_of(((uint32_t)(exps[ei] + 127) << 23) | (m << 16));
      const float sc = fmaxf(amax, 1e-4f) * (1.0f / 448.0f);
      const float ry = 1.0f / sc;
      for (uint32_t b = 0; b < 65536; ++b) {
        const float x = f_of(b << 16);
        if (!(fabsf(x) <= amax)) continue;  /* also skips NaN */
        const float want = x / sc;
        const float q0 = x * ry;
        const float rr = fmaf(-q0, sc, x);
        const float got = copysignf(fmaf(rr, ry, q0), x);
        ++pairs;
        /* quotients of 2^-60 or more: the same bits; below (x so small
           that the residual underflows, from about 2^-78 down): both are
           under 2^-10 with x's sign, so both encode to the same signed
           e4m3 zero */
        const int big = fabsf(want) >= 0x1p-60f || x == 0.0f;
        const int same = big ? u_of(got) == u_of(want)
                             : (fabsf(got) < 0x1p-10f && signbit(got) == signbit(want));
        tiny += !big;
        if (!same) {
          if (bad < 5)
            printf("mismatch x=%a s=%a: %a vs %a\n", x, sc, got, want);
          ++bad;
        }
      }
    }
  printf("pairs %ld (quotients below 2^-60: %ld) mismatches %ld\n", pairs, tiny, bad);
  return bad != 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_quotient_equals_ieee_division(tmp_path):
    src = tmp_path / "mdiv.c"
    exe = tmp_path / "mdiv"
    src.write_text(C_SRC)
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math",
                    str(src), "-o", str(exe), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout
    assert "mismatches 0" in res.stdout
