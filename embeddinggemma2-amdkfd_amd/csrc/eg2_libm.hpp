// The two libm functions on the reference CPU path, restated so that the
// device computes exactly what the host's libm returns for every input.
//
// The reference's x86-64 build calls glibc's tanhf (GELU, kernels.c:367-371)
// and expf (softmax, kernels.c:324-360). Neither is correctly rounded (the
// installed glibc 2.35 tanhf differs from the correctly rounded tanh on 2.8%
// of all floats, expf on about 1 in 10^4 arguments below zero), so a device
// evaluation of the mathematical function would differ in the last bit, and
// through the Q8_0 quantization that follows each of them a last-bit
// difference becomes a different quantum. These are the published
// algorithms glibc compiles for them:
//
//  - tanhf and expm1f: Sun's fdlibm (s_tanhf.c, s_expm1f.c; freely
//    redistributable), in plain float arithmetic, one rounding per
//    operation, no contraction;
//  - expf: the double-precision table method of the Arm Optimized Routines
//    (e_expf.c, exp2f_data.c; N = 32 table entries 2^(i/32), degree-3
//    polynomial), as glibc's x86-64 build selects it on FMA-capable CPUs:
//    the compiler contracts the argument reduction and the polynomial into
//    fused multiply-adds, which is what is written here.
//
// Both restatements were checked against the host's libm on all 2^32 float
// inputs (tanhf and expm1f: 0 differences; expf: 0 differences); the tests
// repeat a strided sweep on the CPU and compare the device's results with
// the host's.
//
// The header compiles for the host too (the CPU test builds it with g++),
// so it uses only builtins both compilers provide.
//
// Notices of the upstream works whose algorithms and constants are restated
// here:
//
// tanhf, expm1f (fdlibm, float versions):
//   Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//   Developed at SunPro, a Sun Microsystems, Inc. business.
//   Permission to use, copy, modify, and distribute this software is freely
//   granted, provided that this notice is preserved.
//   (Conversion to float by Ian Lance Taylor, Cygnus Support.)
//
// expf and its 2^(i/32) table (Arm Optimized Routines):
//   Copyright (c) 2017-2018, Arm Limited.
//   SPDX-License-Identifier: MIT
//   Permission is hereby granted, free of charge, to any person obtaining a
//   copy of this software and associated documentation files (the
//   "Software"), to deal in the Software without restriction, including
//   without limitation the rights to use, copy, modify, merge, publish,
//   distribute, sublicense, and/or sell copies of the Software, and to
//   permit persons to whom the Software is furnished to do so, subject to
//   the following conditions: The above copyright notice and this permission
//   notice shall be included in all copies or substantial portions of the
//   Software. THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND,
//   EXPRESS OR IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF
//   MERCHANTABILITY, FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN
//   NO EVENT SHALL THE AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM,
//   DAMAGES OR OTHER LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR
//   OTHERWISE, ARISING FROM, OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE
//   USE OR OTHER DEALINGS IN THE SOFTWARE.
#pragma once

#include <stdint.h>

#ifndef __HIP__
#ifndef __host__
#define __host__
#endif
#ifndef __device__
#define __device__
#endif
#endif

namespace eg2 {
namespace libm {

__host__ __device__ inline uint32_t fbits(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float ffrom(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ inline uint64_t dbits(double d) { return __builtin_bit_cast(uint64_t, d); }
__host__ __device__ inline double dfrom(uint64_t u) { return __builtin_bit_cast(double, u); }

// fdlibm expm1f: argument reduction x = k ln2 + r (ln2 split hi/lo), the
// rational correction from a 5-term polynomial in r^2/2, then
// reconstruction by exponent arithmetic. Every operation is a single
// rounded float operation in the order written.
__host__ __device__ inline float expm1f(float x) {
  const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
  const float o_threshold = 8.8721679688e+01f;
  const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
              Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
  uint32_t hx = fbits(x);
  const uint32_t xsb = hx & 0x80000000u;
  hx &= 0x7fffffffu;
  // |x| >= 27 ln2: saturates to -1 below, overflows above 88.72.
  if (hx >= 0x4195b844u) {
    if (hx >= 0x42b17218u) {
      if (hx > 0x7f800000u) return x + x;  // NaN
      if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
      if (x > o_threshold) return __builtin_inff();
    }
    if (xsb != 0) return -1.0f;
  }
  float hi, lo, c = 0.0f, t;
  int32_t k;
  if (hx > 0x3eb17218u) {  // |x| > 0.5 ln2
    if (hx < 0x3F851592u) {  // and |x| < 1.5 ln2
      if (xsb == 0) {
        hi = x - ln2_hi;
        lo = ln2_lo;
        k = 1;
      } else {
        hi = x + ln2_hi;
        lo = -ln2_lo;
        k = -1;
      }
    } else {
      k = (int32_t)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
      t = (float)k;
      hi = x - t * ln2_hi;
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x33000000u) {  // |x| < 2^-25: x itself
    return x;
  } else {
    k = 0;
  }
  const float hfx = 0.5f * x;
  const float hxs = x * hfx;
  const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  t = 3.0f - r1 * hfx;
  float e = hxs * ((r1 - t) / (6.0f - x * t));
  if (k == 0) return x - (x * e - hxs);
  e = x * (e - c) - c;
  e -= hxs;
  if (k == -1) return 0.5f * (x - e) - 0.5f;
  if (k == 1) {
    if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
    return 1.0f + 2.0f * (x - e);
  }
  float y;
  if (k <= -2 || k > 56) {  // 2^k (1 + x - e) - 1, the scaling by exponent arithmetic
    y = 1.0f - (e - x);
    y = ffrom(fbits(y) + ((uint32_t)k << 23));
    return y - 1.0f;
  }
  if (k < 23) {
    t = ffrom(0x3f800000u - (0x1000000u >> k));  // 1 - 2^-k
    y = t - (e - x);
  } else {
    t = ffrom((uint32_t)(0x7f - k) << 23);  // 2^-k
    y = x - (e + t);
    y += 1.0f;
  }
  return ffrom(fbits(y) + ((uint32_t)k << 23));
}

// fdlibm tanhf: sign-symmetric; x itself below 2^-55, 1 - 2/(e^(2|x|) + 1)
// from expm1f for |x| >= 1, -expm1f(-2|x|) / (expm1f(-2|x|) + 2) below 1,
// and +-(1 - 2^-100) = +-1 from 22 on.
__host__ __device__ inline float tanhf(float x) {
  const uint32_t jx = fbits(x), ix = jx & 0x7fffffffu;
  if (ix >= 0x7f800000u) return (int32_t)jx >= 0 ? 1.0f / x + 1.0f : 1.0f / x - 1.0f;
  float z;
  if (ix < 0x41b00000u) {  // |x| < 22
    if (ix == 0) return x;
    if (ix < 0x24000000u) return x * (1.0f + x);  // |x| < 2^-55
    if (ix >= 0x3f800000u) {
      const float t = expm1f(2.0f * __builtin_fabsf(x));
      z = 1.0f - 2.0f / (t + 2.0f);
    } else {
      const float t = expm1f(-2.0f * __builtin_fabsf(x));
      z = -t / (t + 2.0f);
    }
  } else {
    z = 1.0f - 1.0e-30f;
  }
  return (int32_t)jx >= 0 ? z : -z;
}

// The same function as tanhf, for finite x, written without branches so
// that a wave whose lanes fall in different cases runs one path. Inside
// tanhf, expm1f sees a = 2|x| >= 2 or a = -2|x| in (-2, 0], so of its
// reconstructions only these occur: k = 0, k = -1, k <= -2 ("1 - (e - r)",
// scaled, minus 1), 2 <= k <= 22 ("(1 - 2^-k) - (e - r)", scaled) and
// 23 <= k ("r - (e + 2^-k) + 1", scaled). The k <= -2 and the 2..22 cases
// share "T - (e - r)" and the scaling, T = 1 or 1 - 2^-k. For k > 56,
// where fdlibm uses the k <= -2 form, |x| > 19.6 and tanhf is 1 either
// way (2 / (t + 2) is below half an ulp of 1 once |x| > 9.02), so the 23 <=
// k form serves. The argument reduction is shared: fdlibm's k = 0 (no
// reduction, c = 0) and k = -1 (x + ln2_hi, lo = -ln2_lo) cases are its
// general formula hi = x - k ln2_hi, lo = k ln2_lo at those k (both
// products exact). Each operation is fdlibm's, in its order.
__host__ __device__ inline float tanhf_flat(float x) {
  const float ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f, invln2 = 1.4426950216e+00f;
  const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f,
              Q4 = 4.0082177293e-06f, Q5 = -2.0109921195e-07f;
  const uint32_t jx = fbits(x), ix = jx & 0x7fffffffu;
  const bool big = ix >= 0x3f800000u;  // |x| >= 1: expm1f(2|x|), else expm1f(-2|x|)
  const float ax = __builtin_fabsf(x);
  const float a = big ? 2.0f * ax : -2.0f * ax;  // expm1f's argument
  const uint32_t ha = fbits(a) & 0x7fffffffu;
  // k: 0 for |a| <= 0.5 ln2, -1 below 1.5 ln2 (a >= 2 never is), else the
  // rounded a / ln2.
  const int32_t kr = (int32_t)(invln2 * a + (big ? 0.5f : -0.5f));
  const int32_t k = ha <= 0x3eb17218u ? 0 : (ha < 0x3F851592u ? -1 : kr);
  const float t = (float)k;
  const float hi = a - t * ln2_hi, lo = t * ln2_lo;
  const float r = hi - lo;
  const float c = (hi - r) - lo;
  const float hfx = 0.5f * r;
  const float hxs = r * hfx;
  const float r1 = 1.0f + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  const float tt = 3.0f - r1 * hfx;
  const float e0 = hxs * ((r1 - tt) / (6.0f - r * tt));
  float e = r * (e0 - c) - c;
  e -= hxs;
  const uint32_t kbits = (uint32_t)k << 23;
  const float v0 = r - (r * e0 - hxs);          // k = 0
  const float vm1 = 0.5f * (r - e) - 0.5f;      // k = -1
  const int32_t kl = k < 1 ? 1 : (k > 22 ? 22 : k);
  const float T = k < 0 ? 1.0f : ffrom(0x3f800000u - (0x1000000u >> kl));
  const float w = ffrom(fbits(T - (e - r)) + kbits);
  const float vlo = k < 0 ? w - 1.0f : w;       // k <= -2, or 2 <= k <= 22
  const int32_t kh = k < 23 ? 23 : (k > 126 ? 126 : k);
  const float vhi = ffrom(fbits((r - (e + ffrom((uint32_t)(0x7f - kh) << 23))) + 1.0f) + kbits);  // k >= 23
#ifdef __HIP_DEVICE_COMPILE__
  // All four are computed for every lane (the compiler would otherwise
  // turn the selection below into branches, which a divergent wave runs
  // one after the other).
  asm volatile("" ::"v"(v0), "v"(vm1), "v"(vlo), "v"(vhi));
#endif
  float em1 = k == 0 ? v0 : (k == -1 ? vm1 : (k >= 23 ? vhi : vlo));
  em1 = ha < 0x33000000u ? a : em1;  // |a| < 2^-25: expm1f(a) = a
  // tanhf's tail: one division, 2 / (t + 2) or -t / (t + 2).
  const float q = (big ? 2.0f : -em1) / (em1 + 2.0f);
  float z = big ? 1.0f - q : q;
  z = ix >= 0x41b00000u ? 1.0f - 1.0e-30f : z;  // |x| >= 22
  z = ix < 0x24000000u ? x * (1.0f + x) : z;    // |x| < 2^-55 (and 0): tanhf keeps x's sign itself
  return ix < 0x24000000u ? z : ((int32_t)jx >= 0 ? z : -z);
}

// 2^(i/32) for i = 0..31 as double bit patterns, minus i << 47 (the
// exponent of 2^(k/32) is added back from k); each entry is the double
// nearest 2^(i/32).
struct Exp2Table {
  uint64_t t[32];
};
constexpr Exp2Table kExp2Tab = {{
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
}};

// expf by the table method: z = x * 32/ln2 = k + r (k the nearest integer,
// found by adding and subtracting 1.5 * 2^52), 2^(r/32) by a cubic in r,
// scaled by the table entry of k mod 32 with k div 32 added to its
// exponent; one final rounding to float. `tab` is the table above (the
// device passes a copy in LDS).
__host__ __device__ inline float expf_tab(float x, const uint64_t* tab) {
  const double InvLn2N = 0x1.71547652b82fep+0 * 32, Shift = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
               C2 = 0x1.62e42ff0c52d6p-1 / 32;
  const uint32_t abstop = (fbits(x) >> 20) & 0x7ffu;
  if (abstop >= (0x42b00000u >> 20)) {  // |x| >= 88 or x is not finite
    if (fbits(x) == 0xff800000u) return 0.0f;
    if (abstop >= (0x7f800000u >> 20)) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double xd = (double)x;
  double kd = __builtin_fma(InvLn2N, xd, Shift);
  const uint64_t ki = dbits(kd);
  kd -= Shift;
  const double r = __builtin_fma(InvLn2N, xd, -kd);
  const uint64_t t = tab[ki % 32] + (ki << 47);
  const double s = dfrom(t);
  const double z = __builtin_fma(C0, r, C1);
  const double r2 = r * r;
  double y = __builtin_fma(C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

__host__ __device__ inline float expf(float x) { return expf_tab(x, kExp2Tab.t); }

}  // namespace libm
}  // namespace eg2
