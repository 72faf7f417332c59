// ref_expf.h — exp(x) for fp32 exactly as the reference evaluates it.
//
// The reference's softmax calls Rust's f32::exp (tensor.rs:745-754), which on
// x86-64 Linux is the C library's expf: glibc (2.27 and later) ships the
// table-driven expf of ARM's optimized-routines, and on CPUs with FMA its
// ifunc selects the build compiled with fused multiply-add.  Its published
// algorithm, restated:
//   z   = x * 32/ln2 (in double), rounded to the integer k by adding 1.5*2^52
//   r   = z - k                                   (|r| <= 1/2)
//   2^(k/32) = table[k mod 32] with k's high bits added to the exponent
//   exp(x) ~= 2^(k/32) * (c0 r^3 + c1 r^2 + c2 r + 1), rounded once to fp32
// with the FMA build's contractions: the reduction k and r are fused with the
// multiply by 32/ln2, and the polynomial is evaluated as
//   y = fma(fma(c0, r, c1), r*r, fma(c2, r, 1)) * 2^(k/32).
// The table entries are the doubles nearest 2^(i/32), each minus i << 47 (the
// exponent bits that k adds back).  This restatement is identical to the host
// C library's expf on every fp32 input (checked exhaustively by the tests).
//
// Included by the HIP kernels and, for that check, by a host-only test build.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define MH_HOST_DEVICE __host__ __device__
#else
#define MH_HOST_DEVICE
#include <cmath>
#endif

#define MH_EXP2_TABLE_32                                                                    \
  0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL, \
      0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL,                   \
      0x3fef1e9df51fdee1ULL, 0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL,                   \
      0x3feedea64c123422ULL, 0x3feece086061892dULL, 0x3feebfdad5362a27ULL,                   \
      0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,                   \
      0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL,                   \
      0x3feea589994cce13ULL, 0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL,                   \
      0x3feec49182a3f090ULL, 0x3feed503b23e255dULL, 0x3feee89f995ad3adULL,                   \
      0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,                   \
      0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL,                   \
      0x3fefd0765b6e4540ULL

namespace mh {

// `tab` holds the 32 entries of MH_EXP2_TABLE_32 (in LDS or constant memory
// on the device).
MH_HOST_DEVICE inline float ref_expf(float x, const uint64_t* tab) {
  constexpr double kInvLn2N = 0x1.71547652b82fep+0 * 32;
  constexpr double kShift = 0x1.8p+52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / 32;
  const uint32_t ux = __builtin_bit_cast(uint32_t, x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  if (abstop >= 0x42bu) {                      // |x| >= 88 or x is NaN
    if (ux == 0xff800000u) return 0.0f;        // exp(-inf)
    if (abstop >= 0x7f8u) return x + x;        // +inf, NaN
    if (x > 0x1.62e42ep6f) return __builtin_huge_valf();  // overflow
    if (x < -0x1.9fe368p6f) return 0.0f;       // underflow
  }
  const double xd = (double)x;
  double kd = __builtin_fma(kInvLn2N, xd, kShift);
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const uint64_t t = tab[ki % 32] + (ki << 47);
  const double s = __builtin_bit_cast(double, t);
  const double z = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

}  // namespace mh
