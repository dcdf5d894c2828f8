// exact_math.h - the single-precision exponential of the reference's host
// libm, bit for bit, for device and host code.
//
// The reference computes SiLU and the softmax with Rust's f32::exp
// (layer.rs:75-79, cpu.rs:410-413), which on x86-64 Linux is glibc's expf.
// glibc (2.27 and later) evaluates expf in double precision: with N = 32,
//   z = x * N/ln2,  k = round-to-nearest-even(z) (by adding 1.5*2^52),
//   r = z - k in [-1/2, 1/2],  s = 2^(k/N) = T[k mod N] with k/N added to
//   its exponent,  exp(x) = s * (C0 r^3 + C1 r^2 + C2 r + 1)
// and rounds the double result to float once.  Its x86-64 build selects an
// FMA variant on CPUs that have FMA (every MI355X host), in which every
// a*b+c of that evaluation is one fused operation.  exact_expf() below is
// that evaluation with the same constants: T[i] = 2^(i/N) correctly rounded
// to double, minus i << 47 (the k/N exponent is added back as an integer);
// C0..C2 are glibc's cubic for 2^(r/N).  A CPU test compares it with the
// host's expf for every one of the 2^32 float inputs, and a GPU test
// compares the device evaluation with the host's expf.
//
// Compile with contraction off (-ffp-contract=off): the fused operations
// are the explicit fma() calls, everything else rounds separately.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define LLMRS_HD __host__ __device__
#else
#define LLMRS_HD
#endif

namespace llmrs {

namespace expf_detail {
// 2^(i/32) rounded to double, with (i << 52) / 32 subtracted from its bits.
constexpr uint64_t kT[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};
constexpr double kInvLn2N = 0x1.71547652b82fep+5;  // 32 / ln 2
constexpr double kShift = 0x1.8p+52;
constexpr double kC0 = 0x1.c6af84b912394p-20;     // cubic of 2^(r/32), r in [-1/2, 1/2]
constexpr double kC1 = 0x1.ebfce50fac4f3p-13;
constexpr double kC2 = 0x1.62e42ff0c52d6p-6;
}  // namespace expf_detail

// `tab` holds kT (a device kernel passes a copy in LDS, so the lookup does
// not wait on a memory round trip).
LLMRS_HD inline float exact_expf(float x, const uint64_t* tab = expf_detail::kT) {
  using namespace expf_detail;
  const uint32_t ux = __builtin_bit_cast(uint32_t, x);
  const uint32_t abstop = (ux >> 20) & 0x7ff;
  if (abstop >= 0x42b) {  // |x| >= 88, or x is inf / NaN
    if (ux == 0xff800000u) return 0.0f;                       // -inf
    if (abstop >= 0x7f8) return x + x;                         // +inf, NaN
    if (x > 0x1.62e42ep6f) return __builtin_inff();            // above log(2^128)
    if (x < -0x1.9fe368p6f) return 0.0f;                       // below log(2^-150)
  }
  const double xd = (double)x;
  const double kd0 = __builtin_fma(kInvLn2N, xd, kShift);     // k + 1.5*2^52, rounded to even
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd0);
  const double kd = kd0 - kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);           // z - k
  const uint64_t t = tab[ki % 32] + (ki << 47);
  const double s = __builtin_bit_cast(double, t);
  const double p = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(p, r2, y);
  y = y * s;
  return (float)y;
}

}  // namespace llmrs
