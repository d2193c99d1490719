"""The rotations divide by sqrt(block) with a corrected reciprocal product
instead of an IEEE division (turbopress_amd/csrc/tp_tiled_common.h:
div_by_block_root, whose special cases -- signed zeros, infinities -- are a
class test and a select, in the rotations inside the per-linear launches;
div_by_block_root_fx, which settles them with v_div_fixup_f32, in the stack
rotation).  Both restated here in C (fmaf, and the fix-up's cases as the
ISA describes them) and checked against IEEE
division for every Hadamard block 2..16384 on a strided sample of all fp32
bit patterns plus the special values: the quotients are equal wherever
|v / c| >= 2^-100; below that the residual underflows, and both quotients
(same sign, magnitude < 2^-100) round to the same fp16 signed zero, which is
what the kernel stores.  The full 2^32 sweep gives the same result, the
largest mismatching quotient being about 2^-106."""

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
/* div_by_block_root: q = v r, e = fma(-q, c, v), q1 = fma(e, r, q); q itself for q = +-0, +-inf.
   div_by_block_root_fx: the same q1, then v_div_fixup_f32(q1, c, v), which for a finite c > 0 whose
   exponent keeps its underflow clause out of reach returns: a quiet NaN for a NaN v, the signed
   infinity for v = +-inf, the signed zero for v = +-0, else |q1| with the sign of v. */
static int variant;
static float kernel_div(float v, float c, float r) {
  const float q = v * r;
  const float e = fmaf(-q, c, v);
  const float q1 = fmaf(e, r, q);
  if (variant == 0) return (q == 0.0f || isinf(q)) ? q : q1;
  if (isnan(v)) return v;
  if (isinf(v)) return copysignf(INFINITY, v);
  if (v == 0.0f) return copysignf(0.0f, v);
  return copysignf(fabsf(q1), v);
}
static int check(float v, float c, float r, unsigned long long* bad) {
  if (isnan(v)) return 0;
  const float want = v / c, got = kernel_div(v, c, r);
  if (u_of(want) == u_of(got)) return 0;
  const int both_tiny = fabsf(want) < 0x1p-100f && fabsf(got) < 0x1p-100f && signbit(want) == signbit(got);
  if (both_tiny) return 0;
  if (*bad < 5) fprintf(stderr, "c=%a v=%a want %a got %a\n", c, v, want, got);
  ++*bad;
  return 1;
}
int main(int argc, char** argv) {
  const unsigned stride = 251u;
  unsigned long long bad = 0, n = 0;
  const uint32_t special[] = {0x00000000u, 0x80000000u, 0x7f800000u, 0xff800000u, 0x00000001u, 0x80000001u,
                              0x007fffffu, 0x00800000u, 0x7f7fffffu, 0xff7fffffu, 0x3f800000u, 0xbf800000u};
  for (variant = 0; variant < 2; ++variant) {
    for (int j = 1; j <= 14; ++j) {
      const float c = sqrtf((float)(1 << j));
      const float r = 1.0f / c;
      for (uint64_t u = 0; u < (1ull << 32); u += stride) { check(f_of((uint32_t)u), c, r, &bad); ++n; }
      for (unsigned s = 0; s < sizeof(special) / sizeof(special[0]); ++s) { check(f_of(special[s]), c, r, &bad); ++n; }
    }
  }
  printf("%llu %llu\n", n, bad);
  return bad != 0;
}
"""


def test_corrected_reciprocal_division_matches_ieee(tmp_path):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = tmp_path / "div_check.c"
    src.write_text(C_SRC)
    exe = tmp_path / "div_check"
    subprocess.run([cc, "-O2", "-ffp-contract=off", "-o", str(exe), str(src), "-lm"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    n, bad = map(int, res.stdout.split())
    assert n > 14 * (1 << 32) // 251
    assert bad == 0 and res.returncode == 0, res.stderr
