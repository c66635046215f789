// exp(d) for d <= 0 to within kExpPolyRel relative, without a table: for sums whose error is bounded
// anyway (a table's gathers from LDS conflict across lanes, and the host-exact exp of exp_f64.h costs
// about twice the instructions). e^d = 2^t, t = d log2(e) = k + f with k = rint(t) and |f| <= 1/2
// (f = t - k exactly), 2^f by a polynomial of degree 8, 2^k by ldexp. exp_neg clamps the argument
// below d = -708 (the result, under 2^-1021, is then e^-708 rather than e^d); exp_sat and exp_fused
// need no clamp (cvt_i32_sat).
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

// k (an integral double) to an int by v_cvt_i32_f64, which clamps values past the int range to it (a
// C++ conversion of such a double is undefined). With it a far negative argument needs no clamp of its
// own: its k converts to INT_MIN and ldexp(p, INT_MIN) is 0.
__device__ __forceinline__ int32_t cvt_i32_sat(double k) {
  int32_t r;
  __asm__("v_cvt_i32_f64 %0, %1" : "=v"(r) : "v"(k));
  return r;
}

// The fused argument below: t = x log2(e) + c in one rounding, with c = -m log2(e) rounded, for
// |m| <= kFusedMax. Its distance to (x - m) log2(e) is at most (|x| + 2.45 |m| + |t|) 2^-53 (the
// rounding of log2(e), of c and of the sum); where the term is above 2^-1100, |t| <= 1100 and
// |x| <= |m| + 763, so at most 3.05e-13, which moves 2^t by at most 2.2e-13 relative (times ln 2).
constexpr double kFusedMax = 256.0;
constexpr double kFusedArgRel = 2.2e-13;
static_assert(1.07e-12 + kFusedArgRel + 1e-15 <= kExpPolyRel, "the fused argument's terms within kExpPolyRel");
constexpr double kLog2e = 1.4426950408889634;

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
  __device__ __forceinline__ double horner(double f) const {
    double p = c[0];
#pragma unroll
    for (int i = 1; i < kPolyLen; ++i) p = __builtin_fma(p, f, c[i]);
    return p;
  }
  // exp(x - m) for x <= m, both finite, |m| <= kFusedMax, given c = fused_offset(m): within
  // kExpPolyRel relative where the result is above 2^-1021, and 0 or a subnormal below.
  static __device__ __forceinline__ double fused_offset(double m) { return -m * kLog2e; }
  __device__ __forceinline__ double exp_fused(double x, double cm) const {
    const double t = __builtin_fma(x, kLog2e, cm);
    const double k = __builtin_rint(t);
    return __builtin_amdgcn_ldexp(horner(t - k), cvt_i32_sat(k));
  }
  // exp(d) for finite d <= 0: within kExpPolyRel relative where the result is above 2^-1021, and 0 or
  // a subnormal below (2^f 2^k rounded, under 2^-1021 like exp(d) itself); a far negative d needs no
  // clamp (cvt_i32_sat).
  __device__ __forceinline__ double exp_sat(double d) const {
    const double t = d * kLog2e;
    const double k = __builtin_rint(t);
    return __builtin_amdgcn_ldexp(horner(t - k), cvt_i32_sat(k));
  }
};

}  // namespace as_dev
