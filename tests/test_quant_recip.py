"""The activation quantizer (df_ssm_inference.py:147-152) divides by the fp16 scale in IEEE fp32,
rounds the quotient to fp16, rounds that to the nearest even integer and clamps to [-128, 127].
The kernels (common.h quant_rcp / quant_i8) multiply by r = fp32(1 / (double)scale) instead.
Checked exhaustively here, for every finite fp16 x >= 0 and every positive finite fp16 scale
(~1.0e9 pairs): the integer q is identical, both at the clamp 127 (x >= 0) and at the clamp 128
that the mirrored negative x meets (rounding to fp16 and to integers is symmetric in the sign).
The fp16 values themselves differ for a small number of pairs, so the check is on q, as the
kernels use it. A negative control shows the check can fail: leaving out the fp16 rounding of
the quotient changes q on many pairs.
"""
import os
import shutil
import subprocess

import pytest

SRC = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static float h2f(uint16_t h) {
  uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff, bits;
  if (e == 0) return (float)m * 5.9604644775390625e-8f; /* subnormal: m * 2^-24, exact */
  bits = ((e + 112u) << 23) | (m << 13);
  float f; memcpy(&f, &bits, 4); return f;
}
/* fp32 -> fp16, round to nearest even, overflow to inf (x >= 0 here) */
static float r16(float f) {
  uint32_t ax; memcpy(&ax, &f, 4);
  if (ax >= 0x477ff000u) return INFINITY;           /* >= 65520 */
  if (ax < 0x38800000u) return rintf(f * 16777216.0f) * 5.9604644775390625e-8f; /* < 2^-14 */
  uint32_t h = (ax - (112u << 23)) >> 13, rb = ax & 0x1fffu;
  if (rb > 0x1000u || (rb == 0x1000u && (h & 1u))) h++;
  return h2f((uint16_t)h);
}
static float clampf(float t, float hi) { return t > hi ? hi : t; }
int main(int argc, char** argv) {
  const int no_r16 = argc > 1;  /* negative control */
  long bad = 0, tot = 0, f16diff = 0;
#pragma omp parallel for reduction(+:bad,tot,f16diff) schedule(dynamic, 64)
  for (int sh = 1; sh < 0x7c00; ++sh) {
    const float s = h2f((uint16_t)sh);
    const float r = (float)(1.0 / (double)s);
    for (int xh = 0; xh < 0x7c00; ++xh) {
      const float x = h2f((uint16_t)xh);
      volatile float d = x / s;
      const float ref = rintf(r16(d));
      const float y = x * r;
      const float got = no_r16 ? rintf(y) : rintf(r16(y));
      tot++;
      if (r16(d) != r16(y)) f16diff++;
      if (clampf(ref, 127.0f) != clampf(got, 127.0f) || clampf(ref, 128.0f) != clampf(got, 128.0f)) bad++;
    }
  }
  printf("%ld %ld %ld\n", tot, bad, f16diff);
  return 0;
}
"""


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    d = tmp_path_factory.mktemp("quant_recip")
    src, exe = os.path.join(d, "check.c"), os.path.join(d, "check")
    open(src, "w").write(SRC)
    subprocess.run([cc, "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", src, "-o", exe, "-lm"],
                   check=True)
    return exe


def test_fp32_reciprocal_quantizer_equals_fp32_division(checker):
    tot, bad, f16diff = map(int, subprocess.run([checker], capture_output=True, text=True, check=True).stdout.split())
    assert tot == 0x7bff * 0x7c00  # every positive finite scale x every non-negative finite x
    assert bad == 0
    assert 0 < f16diff < 10**4     # the fp16 quotients do differ now and then: q is what agrees


def test_negative_control_without_fp16_rounding_fails(checker):
    _, bad, _ = map(int, subprocess.run([checker, "nor16"], capture_output=True, text=True, check=True).stdout.split())
    assert bad > 10**5
