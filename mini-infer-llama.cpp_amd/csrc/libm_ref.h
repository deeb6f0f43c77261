// libm_ref.h -- the host C library's expf, restated so that device code
// returns the same float for every input.
//
// The engine's softmax (src/ops_cpu.cpp:326-331) and SiLU (src/ops_cpu.cpp:
// 134-141) call std::exp(float), i.e. the C library's expf. On the x86-64 hosts
// here that is glibc's expf, an implementation of the published
// "optimized-routines" algorithm (Arm, Szabolcs Nagy; MIT/Apache-2.0), in its
// FMA build (the build glibc selects on CPUs with FMA):
//
//   z  = x * 32/ln2 in double;  kd = fma(32/ln2, x, 2^52 + 2^51) rounds z to
//        an integer k held in the low bits of kd;  r = fma(32/ln2, x, -(kd - shift))
//   s  = 2^(k/32) = double(T[k mod 32] + (k << 47)), T[i] = bits(2^(i/32)) - (i << 47)
//   y  = (fma(fma(C0, r, C1), r * r, fma(C2, r, 1))) * s,  result float(y)
//   with C0..C2 the minimax coefficients of 2^(r/32) below.
// Special cases: NaN -> NaN, x > 0x1.62e42ep6 -> +inf, x < -0x1.9fe368p6 -> +0
// (everything else, including subnormal results, takes the main path).
//
// Pinned exhaustively: tests/test_libm_ref.py evaluates this header on the CPU
// for all 2^32 float inputs against the host's expf (bit-identical), and the
// GPU tests compare the device build against the host on a sample.
//
// The table T[i] is correctly rounded 2^(i/32) as double bits, less i << 47.
// MI_LIBM_HD is defined by the includer (__host__ __device__ in HIP sources,
// empty in host-only checkers).
#pragma once

#include <stdint.h>

#ifndef MI_LIBM_HD
#error "define MI_LIBM_HD before including libm_ref.h"
#endif

#define MI_EXPF_TABLE                                                                   \
  {0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL, \
   0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL, \
   0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL, \
   0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL, \
   0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL, \
   0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL, \
   0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL, \
   0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL}

namespace mi {

// tab: the 32 MI_EXPF_TABLE entries (any pointer type: device code passes a
// __constant__ copy, or an LDS copy when its reads must not wait on global
// memory).
template <typename Tab>
MI_LIBM_HD inline float expf_ref(float x, Tab tab) {
  const double inv_ln2_n = 0x1.71547652b82fep+0 * 32;
  const double shift = 0x1.8p+52;
  const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
  const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
  const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  if (x != x) return x + x;
  if (x > 0x1.62e42ep6f) return __builtin_inff();
  if (x < -0x1.9fe368p6f) return 0.0f;
  const double xd = (double)x;
  double kd = __builtin_fma(inv_ln2_n, xd, shift);
  const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
  kd -= shift;
  const double r = __builtin_fma(inv_ln2_n, xd, -kd);
  const uint64_t t = tab[ki % 32] + (ki << 47);
  const double s = __builtin_bit_cast(double, t);
  const double z = __builtin_fma(c0, r, c1);
  const double r2 = r * r;
  double y = __builtin_fma(c2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  return (float)y;
}

}  // namespace mi
