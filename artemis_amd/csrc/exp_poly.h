// exp(d) for d <= 0 to within kExpPolyRel relative, without a table: for sums whose error is bounded
// anyway (a table's gathers from LDS conflict across lanes, and the host-exact exp of exp_f64.h costs
// about twice the instructions). e^d = 2^t, t = d log2(e) = k + f with k = rint(t) and |f| <= 1/2
// (f = t - k exactly), 2^f by a polynomial of degree 8, 2^k by ldexp. Below d = -708 the argument is
// clamped (the result, under 2^-1021, is then e^-708 rather than e^d).
//
// The coefficients of 2^f, highest degree first: the Chebyshev interpolant of 2^f on [-1/2, 1/2] at
// degree 8 (mpmath.chebyfit at 40 digits), rounded to f64; with the rounded coefficients its relative
// error peaks at 1.064e-12, at f = -1/2 (tests/test_lp_exp_poly.py checks it from this file). Read from
// constant memory once per thread, they stay in scalar registers, which each fused multiply-add takes
// as an operand (as immediates, each step would first rebuild its coefficient in two vector moves).
#pragma once
#include <hip/hip_runtime.h>

namespace as_dev {

// The polynomial's error, the rounding of t = d * log2(e) (|t| <= 1022 times 2^-52, times ln 2:
// 1.6e-13) and of the Horner steps (about 1e-15).
constexpr double kExpPolyRel = 1.5e-12;

constexpr int kPolyLen = 9;
static __constant__ double kExp2Poly[kPolyLen] = {
    1.3255224878668817e-06, 1.5310079402249296e-05, 0.00015403455852453838, 0.0013333450568000645,
    0.009618129159402558,   0.05550410941205933,    0.2402265069581299,     0.6931471805459335,
    1.0};

struct ExpPoly {
  double c[kPolyLen];
  __device__ __forceinline__ void load() {
#pragma unroll
    for (int i = 0; i < kPolyLen; ++i) c[i] = kExp2Poly[i];
  }
  __device__ __forceinline__ double exp_neg(double d) const {
    const double t = fmax(d, -708.0) * 1.4426950408889634;
    const double k = __builtin_rint(t);
    const double f = t - k;
    double p = c[0];
#pragma unroll
    for (int i = 1; i < kPolyLen; ++i) p = __builtin_fma(p, f, c[i]);
    return __builtin_amdgcn_ldexp(p, (int32_t)k);
  }
  // exp(d) for finite d <= 0 without exp_neg's clamp at -708: below it the result is 2^f 2^k rounded
  // to a subnormal or 0, under 2^-1021 like exp(d) itself. t is bounded at -1100 first, so that k
  // converts to an int exactly (a double far outside the int range has no defined conversion); every
  // d it moves lies below -762, where exp(d) and the result are both 0.
  __device__ __forceinline__ double exp_le0(double d) const {
    const double t = fmax(d * 1.4426950408889634, -1100.0);
    const double k = __builtin_rint(t);
    const double f = t - k;
    double p = c[0];
#pragma unroll
    for (int i = 1; i < kPolyLen; ++i) p = __builtin_fma(p, f, c[i]);
    return __builtin_amdgcn_ldexp(p, (int32_t)k);
  }
};

}  // namespace as_dev
