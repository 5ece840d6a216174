// refine_check.cpp -- the refined score intervals (csrc/refine_lane.h, the
// per-lane arithmetic of RefineScores in csrc/step_common.h) on the CPU.
//
// For each summary row the program forms the products p_j = fl(q_j * s_j),
// runs the reference's sequential sum (acc = fl(acc + p_j), the chain of
// src/reference_kernels.cpp:13-19) and the refined interval exactly as a
// workgroup forms it for `parts` waves of 64 lanes (each lane a block of
// E / (64 * parts) consecutive steps; the starts in lane order, the error
// sums in float per lane and per wave as the device forms them),
// and requires the interval to contain the chain's result.  Rows: random
// (the summaries of N(0,1) pages), a constant query, cancelling +-1e4
// terms, a half that climbs and a half that cancels it, magnitudes spread
// over 1e-22..1e16, mostly subnormal products, a zero query, dyadic values
// with many exact ties on the grid, and permuted copies.  It also reports
// how narrow the intervals are against the first-pass interval (the score
// kernel's, from which B is taken) and requires the random rows' refined
// half-width to be at least 10 times narrower on average.
//
// usage: refine_check [rows_per_family]; prints "refine_check ok" and exits
// 0, or names the first row whose interval misses and exits 1.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <string>
#include <vector>

#include "refine_lane.h"

namespace {

constexpr int kWave = 64;

struct Result {
  double center, half;   // the refined interval of the unscaled sum
  double first_pass;     // the first-pass half-width, for comparison
};

// Float rounding of a double downward / upward, and the next float below /
// above (the device's __double2float_rd / _ru, NextDown / NextUp).
float RoundDown(double x) {
  float f = static_cast<float>(x);
  if (static_cast<double>(f) > x) f = std::nextafterf(f, -INFINITY);
  return f;
}
float RoundUp(double x) {
  float f = static_cast<float>(x);
  if (static_cast<double>(f) < x) f = std::nextafterf(f, INFINITY);
  return f;
}

// The first-pass interval of the three-kernel score kernel (WriteBounds and
// WriteInterval in step_common.h): s_hat and sum|T_j| from double prefix
// sums, the sequential-sum bound, rounded outward to floats, times scale.
void FirstPass(const std::vector<float>& p, float scale, float* lo, float* hi, double* err_out) {
  const double n = static_cast<double>(p.size());
  double t = 0.0, abs_t = 0.0, abs_p = 0.0;
  for (float x : p) {
    t += x;
    abs_t += std::fabs(t);
    abs_p += std::fabs(x);
  }
  const double u = 0x1p-24;
  const double at_up = abs_t * (1.0 + 0x1p-40) + n * n * 0x1p-52 * abs_p;
  double err = u * at_up / (1.0 - n * u) + n * 0x1p-52 * abs_p + n * 0x1p-149;
  err *= 1.001;
  const float l = std::nextafterf(RoundDown(t - err), -INFINITY);
  const float h = std::nextafterf(RoundUp(t + err), INFINITY);
  *lo = l * scale;
  *hi = h * scale;
  *err_out = err;
}

// The sum of 64 lane values as WaveTotal forms it on the device: a
// Hillis-Steele scan in float (row_shr 1, 2, 4, 8 within rows of 16, then
// lane 15 into rows 1 and 3, lane 31 into rows 2 and 3), lane 63's result.
float WaveTotal(const float* v) {
  float x[kWave];
  for (int l = 0; l < kWave; ++l) x[l] = v[l];
  for (int shift = 1; shift < 16; shift <<= 1) {
    float y[kWave];
    for (int l = 0; l < kWave; ++l) y[l] = (l % 16 >= shift) ? x[l - shift] : 0.0f;
    for (int l = 0; l < kWave; ++l) x[l] = x[l] + y[l];
  }
  const float b15a = x[15], b15b = x[47];
  for (int l = 16; l < 32; ++l) x[l] = x[l] + b15a;
  for (int l = 48; l < 64; ++l) x[l] = x[l] + b15b;
  const float b31 = x[31];
  for (int l = 32; l < 64; ++l) x[l] = x[l] + b31;
  return x[63];
}

Result Refine(const std::vector<float>& q, const std::vector<float>& s, int parts, float scale) {
  const int E = static_cast<int>(q.size());
  const int lanes = kWave * parts;
  const int Lp = E / lanes;
  std::vector<float> p(E);
  for (int j = 0; j < E; ++j) p[j] = q[j] * s[j];
  float flo, fhi;
  double first_err;
  FirstPass(p, scale, &flo, &fhi, &first_err);
  const double B = dsd_refine::FirstPassBound(flo, fhi, scale, E);
  // Sweep 1: each lane's double sum; starts in lane order.
  std::vector<double> start(lanes);
  double S = 0.0;
  for (int L = 0; L < lanes; ++L) {
    double run = 0.0;
    for (int j = 0; j < Lp; ++j) run += static_cast<double>(p[L * Lp + j]);
    start[L] = S;
    S += run;
  }
  // K and U: per lane and per wave (WaveTotal) in float, the parts in
  // double, as on the device.
  double K = 0.0, U = 0.0;
  for (int w = 0; w < parts; ++w) {
    float kl[kWave], ul[kWave];
    for (int l = 0; l < kWave; ++l) {
      const int L = w * kWave + l;
      dsd_refine::Sweep2 s2;
      s2.t = start[L];
      s2.prev = dsd_refine::CertainField(start[L], B);
      for (int j = 0; j < Lp; ++j) dsd_refine::Sweep2Step(s2, p[L * Lp + j], B, L == 0 && j == 0);
      kl[l] = s2.K;
      ul[l] = s2.U;
    }
    K += static_cast<double>(WaveTotal(kl));
    U += static_cast<double>(WaveTotal(ul));
  }
  Result r;
  r.center = S - K;
  r.half = dsd_refine::HalfWidth(r.center, U * (1.0 + 0x1p-16), B, E);
  r.first_pass = first_err;
  return r;
}

float Chain(const std::vector<float>& q, const std::vector<float>& s) {
  float acc = 0.0f;
  for (size_t j = 0; j < q.size(); ++j) acc = acc + q[j] * s[j];
  return acc;
}

}  // namespace

int main(int argc, char** argv) {
  const int rows = argc > 1 ? std::atoi(argv[1]) : 40;
  const int E = 4096;
  const float scale = 1.0f / std::sqrt(128.0f);
  std::mt19937 rng(20260);
  std::normal_distribution<float> nd;
  std::uniform_real_distribution<double> ud(0.0, 1.0);
  long long checked = 0;
  double ratio_sum = 0.0;
  int ratio_count = 0;
  int failures = 0;

  auto check = [&](const char* family, int row, const std::vector<float>& q,
                   const std::vector<float>& s) {
    const double acc = Chain(q, s);
    for (int parts : {1, 2, 4, 8}) {
      const Result r = Refine(q, s, parts, scale);
      ++checked;
      const bool inside = std::isfinite(r.half) ? (r.center - r.half <= acc && acc <= r.center + r.half)
                                                : true;
      if (!inside) {
        if (failures++ < 5) {
          std::printf("refine_check MISS: %s row %d parts %d: chain %.17g, interval %.17g +- %.6g "
                      "(off by %.6g)\n",
                      family, row, parts, acc, r.center, r.half, std::fabs(acc - r.center));
        }
      }
      if (std::string(family) == "random" && r.first_pass > 0.0) {
        ratio_sum += r.half / r.first_pass;
        ++ratio_count;
      }
    }
  };

  std::vector<float> q(E), s(E);
  for (int row = 0; row < rows; ++row) {
    // random: the query N(0,1), the summary the mean of 16 N(0,1) keys
    for (auto& x : q) x = nd(rng);
    for (auto& x : s) {
      float a = 0.0f;
      for (int t = 0; t < 16; ++t) a = a + nd(rng);
      x = a * (1.0f / 16.0f);
    }
    check("random", row, q, s);
    std::vector<float> perm = s;
    std::shuffle(perm.begin(), perm.end(), rng);
    check("permuted", row, q, perm);
    // constant query
    std::vector<float> qc(E, 0.37f);
    check("constant-query", row, qc, s);
    // cancelling +-1e4 terms with small noise
    for (int j = 0; j < E; ++j) s[j] = (j % 2 ? -1e4f : 1e4f) + 1e-3f * nd(rng);
    check("cancelling", row, q, s);
    // a half that climbs, a half that cancels it
    for (int j = 0; j < E / 2; ++j) s[j] = 100.0f + nd(rng);
    for (int j = E / 2; j < E; ++j) s[j] = -s[j - E / 2] * (1.0f + 1e-6f * nd(rng));
    std::vector<float> ones(E, 1.0f);
    check("climb-cancel", row, ones, s);
    // magnitudes spread over 1e-22 .. 1e16 with random signs
    for (auto& x : s) {
      const double m = std::pow(10.0, -22.0 + 38.0 * ud(rng));
      x = static_cast<float>(ud(rng) < 0.5 ? -m : m);
    }
    check("spread", row, q, s);
    // mostly subnormal products (about 9 in 10), some normal ones
    for (int j = 0; j < E; ++j) {
      q[j] = nd(rng) * 1e-20f;
      s[j] = (ud(rng) < 0.91 ? 1e-20f : 1e-17f) * nd(rng);
    }
    check("subnormal", row, q, s);
    // zero query
    std::vector<float> qz(E, 0.0f);
    check("zero-query", row, qz, s);
    // dyadic values: many products are exact ties on the accumulator's grid
    std::uniform_int_distribution<int> di(-(1 << 20), 1 << 20);
    for (int j = 0; j < E; ++j) {
      q[j] = 1.0f;
      s[j] = std::ldexp(static_cast<float>(di(rng)), -10 + (j % 7));
    }
    check("dyadic-ties", row, q, s);
    for (auto& x : q) x = nd(rng);
  }
  if (failures != 0) {
    std::printf("refine_check FAILED: %d of %lld intervals miss the chain\n", failures, checked);
    return 1;
  }
  const double mean_ratio = ratio_count ? ratio_sum / ratio_count : 1.0;
  std::printf("refine_check: %lld intervals contain the chain; random rows: refined / first-pass "
              "half-width %.4f on average\n",
              checked, mean_ratio);
  if (mean_ratio > 0.1) {
    std::printf("refine_check FAILED: refined intervals are not narrow enough\n");
    return 1;
  }
  std::printf("refine_check ok\n");
  return 0;
}
