// refine_lane.h -- the per-lane arithmetic of the refined score intervals
// (RefineScores, step_common.h), written for host and device so that the
// CPU suite runs exactly this code on adversarial rows
// (tests/native/refine_check.cpp).
//
// The reference score sums acc_j = fl(acc_{j-1} + p_j), j = 1..n, from
// acc_0 = 0 (src/reference_kernels.cpp:13-19).  Exactly, acc_n = S - sum e_j
// with S = sum p_j and e_j = acc_{j-1} + p_j - acc_j.  Given the exact
// prefix sums T_j (in double, t below) and a bound B >= |acc_j - T_j| for
// every j, |acc_j| lies in [|T_j| - B, |T_j| + B].  When that range sits in
// one binade [2^e, 2^(e+1)) and acc_{j-1}'s binade is certainly >= e,
// acc_{j-1} is a multiple of 2^(e-23), so acc_j = acc_{j-1} + round_e(p_j)
// and e_j = p_j - round_e(p_j) is known exactly (round_e: to the nearest
// multiple of 2^(e-23)); a tie on that grid is decided by acc_{j-1}'s last
// bit, so it is known only to within half a spacing.  Any other step has
// |e_j| <= half the spacing of the largest binade acc_j can be in.
//
// A lane walks a block of consecutive steps.  Each step is branch-free:
// the binade test reads the exponent fields of the double range ends, the
// grid arithmetic is float (scaling by powers of two and rint are exact
// here).
#pragma once

#include <math.h>

#include <cstdint>

#if defined(__HIPCC__)
#define DSD_REFINE_FN __host__ __device__ __forceinline__
#else
#define DSD_REFINE_FN inline
#endif

namespace dsd_refine {

DSD_REFINE_FN uint32_t HighWord(double x) {
  return static_cast<uint32_t>(__builtin_bit_cast(uint64_t, x) >> 32);
}

DSD_REFINE_FN float FloatOfBits(uint32_t b) { return __builtin_bit_cast(float, b); }

// The biased double exponent field of |acc|'s binade when it is certain
// (|t| - B and |t| + B in one binade), else 0.  A negative lower end keeps
// its sign bit above the field, so it never matches.
DSD_REFINE_FN uint32_t CertainField(double t, double B) {
  const double a = fabs(t);
  const uint32_t lo = HighWord(a - B) >> 20;
  const uint32_t hi = HighWord(a + B) >> 20;
  return lo == hi ? lo : 0u;
}

// B for an n-step sum from its first-pass interval [lo, hi] of the scaled
// score.  That interval holds [s - err, s + err] * scale with err >=
// u sum_j |T_j| / (1 - n u) (the sequential-sum bound the score pass
// certifies), and Higham's bound gives |acc_j - T_j| <= u sum_{i<=j} |acc_i|
// <= u (sum_i |T_i| + n B) for every prefix j, so B* = u sum|T| / (1 - n u)
// bounds every step.  err is recovered as the unscaled half-width, widened
// by the scaling's rounding (at most 2u of the larger end, taken as 2^-21).
// The double prefix sums t_j the lanes form are within (n + 64) 2^-53
// sum|p| of T_j, and sum|p| <= 2 sum|T| <= 2^25 B*, which the last factor
// covers.  A non-finite interval gives B = inf: every step unknown.
DSD_REFINE_FN double FirstPassBound(float lo, float hi, float scale, int n) {
  const double l = lo, h = hi, sc = scale;
  const double half =
      (h - l) / (2.0 * sc) * (1.0 + 0x1p-40) + 0x1p-21 * fmax(fabs(l), fabs(h)) / sc;
  return half * (1.0 + (static_cast<double>(n) + 64.0) * 0x1p-28);
}

// The refined half-width around S - K for an n-step sum with bound B: the
// unknown errors' bound U (already rounded up) plus
//   * the float summation of K (at most 64 terms per lane, 6 levels of a
//     wave tree): below 70u sum|e_j| over the known steps, where |e_j| <=
//     2^-24 |acc_j| <= 2^-24 (|T_j| + B), so sum|e_j| <= B (1 + n 2^-24)
//     (sum|T_j| <= 2^24 B); 2^-16 B covers it for n < 2^20;
//   * the double rounding of S (at most n + 64 additions of terms bounded
//     by sum|p| <= 2 sum|T| <= 2^25 B) and of the parts' K sum;
//   * the rounding of S - K itself.
DSD_REFINE_FN double HalfWidth(double center, double U, double B, int n) {
  const double dn = static_cast<double>(n);
  return U + B * (0x1p-16 + (dn + 64.0) * 0x1p-27) + fabs(center) * 0x1p-52 + 0x1p-1074;
}

// Sweep 2 of one lane.  t: the exact prefix before the lane's next step;
// prev: CertainField of the accumulator before it.  K: the known errors
// (a float sum, its rounding covered in HalfWidth), U: the bound of the
// others (a float sum of non-negative terms: at most 64 per lane and 6
// levels of a wave tree, so (1 + 2^-16) covers its rounding).
struct Sweep2 {
  double t = 0.0;
  uint32_t prev = 0u;
  float K = 0.0f;
  float U = 0.0f;
};

// Field range of a usable grid: binade e = field - 1023 in [-103, 127], so
// that 2^(e-23) and 2^(23-e) are normal floats.
constexpr uint32_t kGridFieldLo = 1023u - 103u;  // 920
constexpr uint32_t kGridFieldSpan = 230u;

// One step with product p.  first: the very first step of the whole sum
// (acc_1 = fl(0 + p_1) = p_1, no error).
DSD_REFINE_FN void Sweep2Step(Sweep2& s, float p, double B, bool first) {
  s.t += static_cast<double>(p);
  const double a = fabs(s.t);
  const uint32_t elo = HighWord(a - B) >> 20;
  const uint32_t ehi = HighWord(a + B) >> 20;
  const uint32_t cert = elo == ehi ? elo : 0u;
  const bool known = (cert - kGridFieldLo <= kGridFieldSpan) && s.prev >= cert;
  s.prev = cert;
  // Grid spacing sp = 2^(e-23) (float field e - 23 + 127 = cert - 919) and
  // its inverse 2^(23-e) (field 1173 - cert); garbage when !known, unused.
  const float inv = FloatOfBits((1173u - cert) << 23);
  const float sp = FloatOfBits((cert - 919u) << 23);
  // x = p / sp exactly unless it underflows (then |x| < 1/2: c = 0, the
  // error is p itself) or |x| >= 2^24 (p is then a multiple of sp: no
  // error).  p - c*sp is representable (p's bits below sp), so the fma
  // gives it exactly.
  const float x = p * inv;
  const float c = rintf(x);
  const bool tie = fabsf(x - c) == 0.5f;
  const bool small = fabsf(x) < 0x1p24f;
  const float err = fmaf(-c, sp, p);
  const bool settled = first || (known && !tie);
  s.K = s.K + ((known && !tie && small && !first) ? err : 0.0f);
  // Half the spacing of |t| + B's binade: float field ehi - 1023 - 24 + 127,
  // clamped to 2^-126 below (an upper bound for any smaller binade) and to
  // +inf above.  For a tie (cert == ehi) it is half of sp.
  int fh = static_cast<int>(ehi) - 920;
  fh = fh < 1 ? 1 : (fh > 255 ? 255 : fh);
  const float half = FloatOfBits(static_cast<uint32_t>(fh) << 23);
  s.U = s.U + (settled ? 0.0f : half);
}

}  // namespace dsd_refine
