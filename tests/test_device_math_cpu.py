"""Host checks of the arithmetic identities the device kernels rely on
instead of library calls (CPU only; the GPU tests check the kernels).

- Q8_0 rounding (eg2_device.hpp q8_round): roundf(v) is computed as
  truncf(v + copysignf(0.5 - 2^-25, v)); the two agree on every finite
  float (an exhaustive 2^32 sweep was run when the identity was adopted;
  this test covers every float in [-256, 256] plus random bit patterns).
- Q8_0 scale (eg2_device.hpp div127): amax / 127 as amax * RN(1/127)
  plus one FMA correction equals the IEEE quotient (exhaustive sweep when
  adopted; here every float in [0.5, 1024) and a stride over all of them,
  in C so that fmaf is the real fused operation).
- GELU (eg2_device.hpp gelu_mul): 0.5 g (1 + tanh z) evaluated as
  g / (1 + e^(-2z)); same function, and in fp32 (with correctly rounded
  exp and reciprocal standing in for the hardware's) within a few ulps of
  the exact value where the reference's fp32 form is itself accurate.
"""
import os
import shutil
import subprocess
import tempfile

import numpy as np
import pytest

F = np.float32
HALF_MINUS = np.nextafter(F(0.5), F(0))  # 0x1.fffffep-2


def fast_round(v):
    s = (v + np.copysign(HALF_MINUS, v)).astype(F)  # one fp32 add, round to nearest even
    return np.trunc(s)


def check_round(v):
    """fast_round(v) == C roundf(v) (half away from zero), computed exactly in float64."""
    v = v[np.isfinite(v)]
    w = v.astype(np.float64)
    want = np.where(w >= 0, np.floor(w + 0.5), -np.floor(-w + 0.5))
    bad = fast_round(v).astype(np.float64) != want
    assert not bad.any(), v[bad][:8]


def test_fast_roundf_on_every_float_in_the_quantizer_range():
    # Every float with 0.25 <= |v| < 256 (the quantizer sees |v * id| <=
    # 127.x; below 0.25 both sides are 0), both signs.
    lo_bits, hi_bits = 0x3E800000, 0x43800000
    for lo in range(lo_bits, hi_bits, 1 << 24):
        v = np.arange(lo, min(lo + (1 << 24), hi_bits), dtype=np.uint32).view(F)
        check_round(v)
        check_round(-v)


def test_fast_roundf_special_cases_and_random_patterns():
    specials = np.array([0.5, 1.5, 2.5, 126.5, 127.5, 0.49999997, 0.50000006, 1.4999999, 2 ** 23 - 0.5,
                         2 ** 23, 2 ** 23 + 1, 2 ** 24 + 2, 3.4e38, 1e-45, 0.0], dtype=F)
    check_round(specials)
    check_round(-specials)
    rng = np.random.default_rng(5)
    check_round(rng.integers(0, 2 ** 32, 1 << 22, dtype=np.uint64).astype(np.uint32).view(F))


def test_gelu_sigmoid_form_is_the_tanh_form():
    g = np.concatenate([np.linspace(-12, 12, 200001), np.random.default_rng(6).standard_normal(200000) * 3])
    z = 0.7978845608028654 * g * (1 + 0.044715 * g * g)
    tanh_form = 0.5 * g * (1 + np.tanh(z))
    sigmoid_form = g / (1 + np.exp(-2 * z))
    # float64's own 1 + tanh(z) cancels for negative z: compare relatively
    # where it is accurate and absolutely elsewhere.
    ok = z > -5
    assert np.allclose(sigmoid_form[ok], tanh_form[ok], rtol=1e-12, atol=0)
    assert np.abs(sigmoid_form[~ok] - tanh_form[~ok]).max() < 1e-12


def test_gelu_sigmoid_form_fp32_accuracy():
    """fp32 evaluation in the kernel's order (capped exponent, one Newton
    step modelled by a correctly rounded reciprocal, exactly 0 below
    z = -9) against the exact value: a few ulps where the result is not
    tiny, while the reference's fp32 0.5 g (1 + tanhf z) cancels."""
    g = np.concatenate([np.linspace(-12, 12, 400001), np.random.default_rng(7).standard_normal(400000) * 3]).astype(F)
    inner = (F(0.7978845608028654) * g).astype(F) * (F(1) + (F(0.044715) * g).astype(F) * g).astype(F)
    inner = inner.astype(F)
    arg = np.minimum((inner * F(-2.8853900817779268)).astype(F), F(126))
    e = np.exp2(arg.astype(np.float64)).astype(F)
    den = (F(1) + e).astype(F)
    r = (1.0 / den.astype(np.float64)).astype(F)
    r = np.where(inner < -9, F(0), r)
    got = (g * r).astype(F)
    exact = 0.5 * g.astype(np.float64) * (1 + np.tanh(inner.astype(np.float64)))
    ulp = np.spacing(np.abs(exact).astype(F)).astype(np.float64)
    err = np.abs(got - exact) / ulp
    assert err[inner >= -0.5].max() <= 3
    assert err[(inner >= -9) & (np.abs(exact) > 1e-30)].max() <= 20
    assert (got[inner < -9] == 0).all()


DIV127_C = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
static int check(uint32_t u) {
  float a; memcpy(&a, &u, 4);
  const float r = 1.0f / 127.0f;
  volatile float want = a / 127.0f;
  float q = a * r;
  float got = fmaf(fmaf(-q, 127.0f, a), r, q);
  return memcmp(&got, (const void*)&want, 4) != 0;
}
int main(int argc, char** argv) {
  uint64_t bad = 0;
  for (uint64_t u = 0x3F000000u; u < 0x44800000u; ++u) bad += check((uint32_t)u);  /* [0.5, 1024) */
  for (uint64_t u = 0; u < 0x7F800000u; u += 7) bad += check((uint32_t)u);           /* all, stride 7 */
  printf("%llu\n", (unsigned long long)bad);
  return bad != 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_div127_fma_correction_is_the_ieee_quotient():
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "div127.c"), os.path.join(d, "div127")
        open(src, "w").write(DIV127_C)
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, src, "-lm"], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
        assert out.returncode == 0 and out.stdout.strip() == "0", out.stdout
