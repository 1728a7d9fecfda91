// bb_expf.h — binary32 exp evaluated in binary64: device code in HIP, plain C elsewhere.
//
// The reference's sigmoid/silu call Rust's f32::exp (activation.rs:5-13), which on
// x86_64-linux-gnu resolves to glibc's expf. glibc 2.35 ships the Arm optimized-routines
// algorithm (Szabolcs Nagy, 2017; "sysdeps/ieee754/flt-32/e_expf.c"): x·N/ln2 = k + r with
// N = 32, 2^(k/N) from a 32-entry table, 2^(r/N) from a cubic in r, all in double, one final
// rounding to float. On CPUs with FMA the library's ifunc picks the build compiled with FMA
// contraction; this restatement evaluates the same steps with explicit fma() where that build
// fuses. tests/test_expf_restatement.py checks it bit-for-bit against the platform expf; run
// over all 2^32 inputs on an FMA host it matched every one (the same steps without the fused
// range reduction differ on two inputs, 0x4202422f and 0xc27c65d9).
//
// The table entries are asuint64(2^(i/32)) - (i << 47), i.e. correctly rounded 2^(i/32) with
// the exponent contribution of i removed; the cubic coefficients are the published minimax
// fit for 2^(r/N) on |r| <= 1/2.
#ifndef BB_EXPF_H
#define BB_EXPF_H
#include <stdint.h>

#if defined(__HIPCC__)
#define BB_HD __device__ __forceinline__
#else
#include <math.h>
#define BB_HD static inline
#endif

#if defined(__HIPCC__)
__device__ __constant__ static const uint64_t bb_exp2f_tab_dev[32] = {
#else
static const uint64_t bb_exp2f_tab_host[32] = {
#endif
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

BB_HD uint32_t bb_f32_bits(float f) {
  union { float f; uint32_t u; } v;
  v.f = f;
  return v.u;
}
BB_HD double bb_f64_from_bits(uint64_t u) {
  union { uint64_t u; double d; } v;
  v.u = u;
  return v.d;
}
BB_HD uint64_t bb_f64_bits(double d) {
  union { double d; uint64_t u; } v;
  v.d = d;
  return v.u;
}

// tab: the 32 table entries (kernels may pass a copy of them in LDS).
BB_HD float bb_expf_tab(float x, const uint64_t* tab) {
  const double N = 32.0;
  const double InvLn2N = 0x1.71547652b82fep+0 * N;
  const double SHIFT = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / N / N / N;
  const double C1 = 0x1.ebfce50fac4f3p-3 / N / N;
  const double C2 = 0x1.62e42ff0c52d6p-1 / N;
  const uint32_t ux = bb_f32_bits(x);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= 0x42b) {                      // |x| >= 88 or not finite
    if (ux == 0xff800000u) return 0.0f;       // exp(-inf) = 0
    if (abstop >= 0x7f8) return x + x;        // +inf, nan
    if (x > 0x1.62e42ep6f) return __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
  }
  const double xd = (double)x;
  double kd = fma(InvLn2N, xd, SHIFT);
  const uint64_t ki = bb_f64_bits(kd);
  kd -= SHIFT;
  const double r = fma(InvLn2N, xd, -kd);
  uint64_t t = tab[ki % 32];
  t += ki << (52 - 5);
  const double s = bb_f64_from_bits(t);
  const double z = fma(C0, r, C1);
  const double r2 = r * r;
  double y = fma(C2, r, 1.0);
  y = fma(z, r2, y);
  y = y * s;
  return (float)y;
}

BB_HD float bb_expf(float x) {
#if defined(__HIPCC__)
  return bb_expf_tab(x, bb_exp2f_tab_dev);
#else
  return bb_expf_tab(x, bb_exp2f_tab_host);
#endif
}

#endif
