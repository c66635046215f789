// f64 exp that returns the same bits as the host C library's exp on x86-64 glibc >= 2.28 (the
// FMA build it selects on CPUs with FMA), on the host and on gfx950.
//
// The sampler's probabilities are exp(l - top) and exp((l - top) / T) in f64 (the reference takes
// Rust's f64::exp, which is the platform libm: crates/engine/src/sample.rs:167,187,219,262,275,282).
// Token ids can only be bit-exact if every weight has the same bits as the host's, so the GPU
// evaluates the same published method, in the same operation order:
//   exp(x) = 2^(k/N) * exp(r),  N = 128,  x = k ln2/N + r,  |r| <= ln2/2N,
//   2^(k/N) = H_i (1 + T_i) * 2^e from a 128-entry table (exp_table.h, i = k mod N),
//   exp(r) - 1 ~ r + C2 r^2 + C3 r^3 + C4 r^4 + C5 r^5,
//   result = scale + scale * (T_i + exp(r) - 1).
// Which multiply-adds are fused matters for the last bit; the pattern below was matched bitwise
// against the host exp on 4e7 arguments over [-745, 0], [-1, 1], random exponents and the subnormal
// range, and is rechecked by tests/test_gpu_sampler.py::test_gpu_exp_is_the_hosts. Everything else must compile with
// -ffp-contract=off so that no other product is fused.
#pragma once
#include <stdint.h>
#include "exp_table.h"

#if defined(__HIPCC__)
#define AS_HD __host__ __device__
#else
#define AS_HD
#endif

namespace as_exp {

#if defined(__HIP_DEVICE_COMPILE__)
__device__ static const uint64_t kTable[256] = {AS_EXP_TABLE_WORDS};
#else
static const uint64_t kTable[256] = {AS_EXP_TABLE_WORDS};
#endif

AS_HD inline uint64_t bits_of(double x) { return __builtin_bit_cast(uint64_t, x); }
AS_HD inline double double_of(uint64_t u) { return __builtin_bit_cast(double, u); }
AS_HD inline double fused(double a, double b, double c) { return __builtin_fma(a, b, c); }

// |x| >= 512 with a finite result: the scale's exponent is out of range, so it is rebuilt with an
// offset and the result rescaled; below 2^-1022 the sum is rounded once before scaling. Out of line
// on the device, so that a loop of exp_with does not evaluate it for every argument.
#if defined(__HIP_DEVICE_COMPILE__)
__attribute__((noinline))
#endif
AS_HD inline double exp_special(double tmp, uint64_t sbits, uint64_t ki) {
  if ((ki & 0x80000000ull) == 0) {
    sbits -= 1009ull << 52;
    double scale = double_of(sbits);
    return 0x1p1009 * fused(scale, tmp, scale);
  }
  sbits += 1022ull << 52;
  double scale = double_of(sbits);
  double st = scale * tmp;
  double y = scale + st;
  if (y < 1.0) {
    double lo = (scale - y) + st;
    double hi = 1.0 + y;
    lo = ((1.0 - hi) + y) + lo;
    y = (hi + lo) - 1.0;
    if (y == 0.0) y = 0.0;
  }
  return 0x1p-1022 * y;
}

// The reduction and polynomial shared by both entry points: tmp and the scale's bits.
AS_HD inline double exp_reduced(const uint64_t* tab, double x, uint64_t* sbits_out, uint64_t* ki_out) {
  const double kInvLn2N = 0x1.71547652b82fep0 * 128.0;
  const double kNegLn2HiN = -0x1.62e42fefa0000p-8;
  const double kNegLn2LoN = -0x1.cf79abc9e3b3ap-47;
  const double kShift = 0x1.8p52;
  const double kC2 = 0x1.ffffffffffdbdp-2, kC3 = 0x1.555555555543cp-3;
  const double kC4 = 0x1.55555cf172b91p-5, kC5 = 0x1.1111167a4d017p-7;
  double kd = fused(kInvLn2N, x, kShift);
  uint64_t ki = bits_of(kd);
  kd -= kShift;
  double r = fused(kd, kNegLn2LoN, fused(kd, kNegLn2HiN, x));
  uint64_t idx = 2 * (ki % 128);
  uint64_t top = ki << 45;
  double tail = double_of(tab[idx]);
  uint64_t sbits = tab[idx + 1] + top;
  double r2 = r * r;
  double a = fused(r, kC3, kC2);
  double b = fused(r, kC5, kC4);
  double tmp = fused(r2, a, tail + r);
  tmp = fused(r2 * r2, b, tmp);
  *sbits_out = sbits;
  *ki_out = ki;
  return tmp;
}

// exp_with for -512 < x < 512 only (where it takes no special case; for |x| < 2^-54 both give
// 1 + x rounded): no branch, for loops over many arguments.
AS_HD inline double exp_core(const uint64_t* tab, double x) {
  uint64_t sbits, ki;
  const double tmp = exp_reduced(tab, x, &sbits, &ki);
  const double scale = double_of(sbits);
  return fused(scale, tmp, scale);
}

// `tab` is kTable or a copy of it (a kernel stages one in LDS).
AS_HD inline double exp_with(const uint64_t* tab, double x) {
  uint32_t abstop = (uint32_t)(bits_of(x) >> 52) & 0x7ff;
  // 0x3c9 is the exponent field of 2^-54, 0x408 of 512, 0x409 of 1024.
  if (abstop - 0x3c9u >= 0x408u - 0x3c9u) {
    if (abstop - 0x3c9u >= 0x80000000u) return 1.0 + x;  // |x| < 2^-54, and 0
    if (abstop >= 0x409u) {
      if (bits_of(x) == 0xfff0000000000000ull) return 0.0;  // -inf
      if (abstop >= 0x7ffu) return 1.0 + x;                  // +inf, NaN
      return (bits_of(x) >> 63) ? 0.0 : __builtin_inf();     // underflow, overflow
    }
    abstop = 0;  // 512 <= |x| < 1024: exp_special
  }
  uint64_t sbits, ki;
  const double tmp = exp_reduced(tab, x, &sbits, &ki);
  if (abstop == 0) return exp_special(tmp, sbits, ki);
  const double scale = double_of(sbits);
  return fused(scale, tmp, scale);
}


AS_HD inline double exp(double x) { return exp_with(kTable, x); }

}  // namespace as_exp
