// cos and sin of an f32 angle, rounded once to f32, for RoPE.
//
// The oracle (and the reference's ropeRef, ops_ref.ts:76) takes
// fr(Math.cos(theta)) and fr(Math.sin(theta)) of an f32 theta: a double-
// precision value rounded to f32. Matching it bit for bit needs the double
// result to ~1e-16, which rules out f32 arithmetic. This file evaluates it in
// double with a short method instead of a general-purpose libm routine:
//
//   * Cody-Waite reduction: k = nearest integer to theta * 2/pi, and
//     r = theta - k*P1 - k*P2 with pi/2 = P1 + P2 (P1 = pi/2 rounded to double,
//     P2 = the remainder), each step one fused multiply-add. For |theta| <
//     2^22 (k < 2^22) the reduced argument is accurate to ~1e-16 absolute.
//   * Taylor series of sin and cos about 0 on |r| <= pi/4 (plus rounding
//     slack), through x^17 / 17! and x^18 / 18!; the first omitted terms are
//     below 2e-19. Horner evaluation in double.
//   * Quadrant k mod 4 selects +-sin(r) / +-cos(r).
// Larger angles (positions beyond ~4 million) use the device libm in double.
//
// __host__ __device__ so the CPU tests can compare this exact code with the
// host libm over millions of angles.
#pragma once

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

namespace flk {

__host__ __device__ __forceinline__ void sin_cos_reduced(double r, double& s, double& c) {
  const double r2 = r * r;
  // sin r = r * (1 - r^2/3! + r^4/5! - ... + r^16/17!)
  double ps = 1.0 / 355687428096000.0;          //  1/17!
  ps = fma(ps, r2, -1.0 / 1307674368000.0);     // -1/15!
  ps = fma(ps, r2, 1.0 / 6227020800.0);         //  1/13!
  ps = fma(ps, r2, -1.0 / 39916800.0);          // -1/11!
  ps = fma(ps, r2, 1.0 / 362880.0);             //  1/9!
  ps = fma(ps, r2, -1.0 / 5040.0);              // -1/7!
  ps = fma(ps, r2, 1.0 / 120.0);                //  1/5!
  ps = fma(ps, r2, -1.0 / 6.0);                 // -1/3!
  s = fma(ps * r2, r, r);
  // cos r = 1 - r^2/2! + r^4/4! - ... + r^18/18!
  double pc = 1.0 / 6402373705728000.0;         //  1/18!
  pc = fma(pc, r2, -1.0 / 20922789888000.0);    // -1/16!
  pc = fma(pc, r2, 1.0 / 87178291200.0);        //  1/14!
  pc = fma(pc, r2, -1.0 / 479001600.0);         // -1/12!
  pc = fma(pc, r2, 1.0 / 3628800.0);            //  1/10!
  pc = fma(pc, r2, -1.0 / 40320.0);             // -1/8!
  pc = fma(pc, r2, 1.0 / 720.0);                //  1/6!
  pc = fma(pc, r2, -1.0 / 24.0);                // -1/4!
  pc = fma(pc, r2, 0.5);                        // (the -1/2! term, sign below)
  c = fma(-pc, r2, 1.0);
}

// f32(cos(theta)) and f32(sin(theta)) of an f32 angle.
__host__ __device__ __forceinline__ void sincos_f32_exact(float theta, float& s_out, float& c_out) {
  const double x = (double)theta;
  if (fabs(x) < 4194304.0) {  // 2^22
    const double two_over_pi = 0.63661977236758134308;
    const double p1 = 1.5707963267948966;      // pi/2 rounded to double
    const double p2 = 6.123233995736766e-17;   // pi/2 - p1
    const double k = rint(x * two_over_pi);
    double r = fma(-k, p1, x);
    r = fma(-k, p2, r);
    double s, c;
    sin_cos_reduced(r, s, c);
    const int q = (int)((int64_t)k & 3);
    double so, co;
    if (q == 0) {
      so = s;
      co = c;
    } else if (q == 1) {
      so = c;
      co = -s;
    } else if (q == 2) {
      so = -s;
      co = -c;
    } else {
      so = -c;
      co = s;
    }
    s_out = (float)so;
    c_out = (float)co;
  } else {
    s_out = (float)sin(x);
    c_out = (float)cos(x);
  }
}

}  // namespace flk
