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
- The host libm's expf and tanhf restated (eg2_libm.hpp: fdlibm's tanhf
  and expm1f, and tanhf's branch-free form, the table method of glibc's
  expf): the header, built for the
  host with g++, equals the host's libm on every 61st float bit pattern
  and every 7th in the GELU's and the softmax's working ranges (an
  exhaustive 2^32 sweep of all three functions was run when they were
  adopted; the GPU test repeats a sweep on the device).
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


LIBM_CPP = r"""
#include <cmath>
#include <cstdio>
#include <cstdint>
#include <thread>
#include <vector>
#include "eg2_libm.hpp"
using namespace eg2::libm;
static unsigned long long sweep(uint64_t lo, uint64_t hi, uint64_t stride) {
  const int T = 8;
  std::vector<unsigned long long> bad(T, 0);
  std::vector<std::thread> th;
  for (int i = 0; i < T; ++i)
    th.emplace_back([&, i] {
      for (uint64_t u = lo + stride * i; u < hi; u += stride * T) {
        const float x = ffrom((uint32_t)u);
        if (std::isnan(x)) continue;
        bad[i] += fbits(::tanhf(x)) != fbits(eg2::libm::tanhf(x));
        if (std::isfinite(x)) bad[i] += fbits(::tanhf(x)) != fbits(eg2::libm::tanhf_flat(x));
        bad[i] += fbits(::expm1f(x)) != fbits(eg2::libm::expm1f(x));
        bad[i] += fbits(::expf(x)) != fbits(eg2::libm::expf(x));
      }
    });
  for (auto& t : th) t.join();
  unsigned long long s = 0;
  for (auto b : bad) s += b;
  return s;
}
int main() {
  unsigned long long bad = sweep(0, 1ull << 32, 61);        // every 61st bit pattern
  bad += sweep(0x00000000u, 0x41200000u, 7);                 // every 7th of [0, 10]
  bad += sweep(0x80000000u, 0xC2D00000u, 7);                 // every 7th of [-104, -0]
  std::printf("%llu\n", bad);
  return bad != 0;
}
"""


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_libm_restatement_equals_host_libm():
    hdr = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "embeddinggemma2-amdkfd_amd",
                       "csrc")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "libm.cpp"), os.path.join(d, "libm")
        open(src, "w").write(LIBM_CPP)
        subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-I", hdr, "-o", exe, src, "-lm", "-pthread"],
                       check=True)
        out = subprocess.run([exe], capture_output=True, text=True, timeout=600)
        assert out.returncode == 0 and out.stdout.strip() == "0", out.stdout
