// step_common.h -- device helpers shared by the decode-step kernels
// (step_kernels.hip) and the fused single-launch step (fused_step.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

namespace dsdk {
namespace {

constexpr int kWave = 64;

// ---- certified score intervals ---------------------------------------------
// The reference score is acc = fl(acc + fl(q_i*s_i)) over i = 0..E-1, then
// fl(acc*scale).  A workgroup forms the same fp32 products, sums them in
// double (s_hat) and accumulates |T_i| over the exact prefix sums T_i; the
// sequential fp32 sum then lies within u*sum|T_i|/(1 - n*u) (u = 2^-24) of
// the exact sum, plus n*2^-149 for subnormal steps, plus slack for the
// double rounding of s_hat and the T_i.  WriteBounds turns that into an
// outward-rounded float interval times scale (fl(x*scale) is monotone in x).

__device__ __forceinline__ float NextDown(float x) {
  if (x == 0.0f) return -0x1p-149f;
  uint32_t b = __float_as_uint(x);
  b = (b & 0x80000000u) ? b + 1u : b - 1u;
  return __uint_as_float(b);
}

__device__ __forceinline__ float NextUp(float x) {
  if (x == 0.0f) return 0x1p-149f;
  uint32_t b = __float_as_uint(x);
  b = (b & 0x80000000u) ? b - 1u : b + 1u;
  return __uint_as_float(b);
}

__device__ __forceinline__ double WaveSum(double v) {
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// The certified interval [fl(lo*scale), fl(hi*scale)] around s_hat*scale
// for an error bound err on the unscaled sum.
__device__ __forceinline__ void WriteInterval(double s_hat, double err, float scale,
                                              float* mid_out, float* lo_out, float* hi_out,
                                              int c) {
  float lo, hi, mid;
  if (isfinite(s_hat) && isfinite(err)) {
    lo = NextDown(__double2float_rd(s_hat - err));
    hi = NextUp(__double2float_ru(s_hat + err));
    mid = __double2float_rn(s_hat);
    if (!(mid >= lo)) mid = lo;
    if (!(mid <= hi)) mid = hi;
    lo = __fmul_rn(lo, scale);
    hi = __fmul_rn(hi, scale);
    mid = __fmul_rn(mid, scale);
  } else {
    // Non-finite sums: an unbounded interval forces the exact path.
    lo = -INFINITY;
    hi = INFINITY;
    mid = 0.0f;
  }
  mid_out[c] = mid;
  lo_out[c] = lo;
  hi_out[c] = hi;
}

// Interval from exact-order prefix sums: abs_prefix = sum_i |T_i| formed in
// double, abs_p an upper bound of sum_i |p_i|.
__device__ __forceinline__ void WriteBounds(double s_hat, double abs_prefix, double abs_p,
                                            int n, float scale, float* mid_out,
                                            float* lo_out, float* hi_out, int c) {
  const double dn = static_cast<double>(n);
  const double u = 0x1p-24;
  const double at_up = abs_prefix * (1.0 + 0x1p-40) + dn * dn * 0x1p-52 * abs_p;
  double err = u * at_up / (1.0 - dn * u) + dn * 0x1p-52 * abs_p + dn * 0x1p-149;
  err *= 1.001;
  WriteInterval(s_hat, err, scale, mid_out, lo_out, hi_out, c);
}

// Interval from a float evaluation in groups of L consecutive products.
// Within a group the local prefix sums loc_j are formed in float (recursive
// summation); P_k, the computed prefix at the start of group k, and s_hat,
// the computed sum of all products, come from float additions of the group
// sums in some tree.  `depth` bounds the roundings on any product's path
// into any P_k or into s_hat, the L - 1 local ones included.  Inputs:
// tsum >= sum_k (L*|P_k| + sum_j |loc_j|) and abs_p >= sum_i |p_i|, each
// summed in float with at most 64 roundings on any path (relative error
// below 2^-17, covered by the factor 1 + 2^-16).  With g_m = m*u/(1 - m*u)
// (Higham, Accuracy and Stability, 2nd ed., Lemma 3.1 and eq. 4.4):
//   |loc_j - t_j| <= g_L * sum|p|       (t_j: exact local prefix),
//   |P_k - exact prefix at group k| <= g_depth * sum|p|,
//   |s_hat - S| <= g_depth * sum|p|     (S: exact sum),
// so the exact prefix sums satisfy, by the triangle inequality,
//   sum_i |T_i| <= tsum + n*(g_depth + g_L)*sum|p|,
// which feeds the sequential-sum bound u*sum|T_i|/(1 - n*u) (eq. 4.3) for
// the reference chain.  Float additions are exact in the subnormal range and
// the products are the reference's own, so no subnormal term is needed;
// 4*n*2^-149 is kept as slack, and 1.001 covers this function's own double
// arithmetic (here only two products and two sums; the constants are
// computed at compile time).
// The constant factors are folded at compile time:
//   err = 1.001 * (c_t*tsum + c_p*abs_p + 4*n*2^-149)
// with c_t = u(1 + 2^-16)/(1 - n*u) and
//      c_p = (1 + 2^-16)(u*n*(g_depth + g_L)/(1 - n*u) + g_depth).
template <int kN, int kL, int kDepth>
__device__ __forceinline__ void WriteBoundsFloat(float s_hat, float tsum, float abs_p,
                                                 float scale, float* mid, float* lo,
                                                 float* hi) {
  constexpr double u = 0x1p-24;
  constexpr double dn = static_cast<double>(kN);
  constexpr double gl = kL * u / (1.0 - kL * u);
  constexpr double gd = kDepth * u / (1.0 - kDepth * u);
  constexpr double c_t = 1.001 * (1.0 + 0x1p-16) * u / (1.0 - dn * u);
  constexpr double c_p = 1.001 * (1.0 + 0x1p-16) * (u * dn * (gd + gl) / (1.0 - dn * u) + gd);
  constexpr double c_0 = 1.001 * 4.0 * dn * 0x1p-149;
  const double err = c_t * static_cast<double>(tsum) + c_p * static_cast<double>(abs_p) + c_0;
  WriteInterval(static_cast<double>(s_hat), err, scale, mid, lo, hi, 0);
}

// ---- wave scans with DPP -----------------------------------------------------
// x from lane `lane - shift` in its row of 16 (row_shr), lane 15 of the row
// below (row_bcast:15, rows 1 and 3), lane 31 (row_bcast:31, rows 2 and 3),
// or the lane below across the wave (wave_shr:1); lanes with no source read 0.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ float DppMove(float x) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(x), kCtrl, kRowMask, 0xf, true));
}
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143, kWaveShr1 = 0x138;

// Inclusive prefix sum over the 64 lanes in float (Hillis-Steele): every
// input reaches every output through at most 6 additions.
__device__ __forceinline__ float WaveInclusiveScan(float x) {
  x = __fadd_rn(x, DppMove<kRowShr1>(x));
  x = __fadd_rn(x, DppMove<kRowShr2>(x));
  x = __fadd_rn(x, DppMove<kRowShr4>(x));
  x = __fadd_rn(x, DppMove<kRowShr8>(x));
  x = __fadd_rn(x, DppMove<kRowBcast15, 0xa>(x));
  x = __fadd_rn(x, DppMove<kRowBcast31, 0xc>(x));
  return x;
}

// Sum over the 64 lanes (at most 6 roundings per input), in every lane.
__device__ __forceinline__ float WaveTotal(float x) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(WaveInclusiveScan(x)), 63));
}

// Orders this wave's LDS writes before its later LDS reads of other lanes'
// data (a wave-scope release/acquire around a wave barrier).
__device__ __forceinline__ void WaveSync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---- select keys ------------------------------------------------------------
// One 64-bit key per candidate whose unsigned order is the reference's
// comparator (src/reference_kernels.cpp:94-99): high word = order-preserving
// image of the score (-0.0 folded onto +0.0, since the reference compares
// with ==), low word = ~page_id so that a smaller id wins a tie.

__device__ __forceinline__ uint64_t SelectKey(float score, int page_id) {
  uint32_t bits = __float_as_uint(score);
  if (bits == 0x80000000u) bits = 0u;
  const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return (static_cast<uint64_t>(ord) << 32) |
         static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(page_id));
}

__device__ __forceinline__ int KeyPage(uint64_t key) {
  return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFull));
}

// ---- exact rescoring --------------------------------------------------------
constexpr int kChainPages = 8;

// acc + row[0] + row[1] + ... + row[len-1], one rounding per element in
// order (the reference chain); len % 64 == 0, row 16-byte aligned.  The LDS
// reads run 32 floats ahead of the adds.
__device__ __forceinline__ float ChainAdd(const float* row, int len, float acc) {
  const float4* r4 = reinterpret_cast<const float4*>(row);
  const int n4 = len / 4;
  float4 a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = r4[i];
  for (int base = 0; base < n4; base += 16) {
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = r4[base + 8 + i];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      acc = __fadd_rn(acc, a[i].x);
      acc = __fadd_rn(acc, a[i].y);
      acc = __fadd_rn(acc, a[i].z);
      acc = __fadd_rn(acc, a[i].w);
    }
    if (base + 16 < n4) {
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = r4[base + 16 + i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      acc = __fadd_rn(acc, b[i].x);
      acc = __fadd_rn(acc, b[i].y);
      acc = __fadd_rn(acc, b[i].z);
      acc = __fadd_rn(acc, b[i].w);
    }
  }
  return acc;
}

// Exact sequential-chain scores for `nflag` candidates of request r (their
// candidate indices in flagged[]), written as select keys into keys[].  All
// threads form the fp32 products of up to kChainPages pages per tile in LDS;
// one lane per page then runs the dependent adds, so the cost is one chain's
// latency per group of pages.  An id outside [0, capacity) reads as an empty
// page.  Must be called by the whole workgroup.
constexpr int kRankTile = 1024;
constexpr int kRankTileStride = kRankTile + 4;

__device__ void RescoreExact(const int* flagged, int nflag, const float* __restrict__ q,
                             const float* __restrict__ summaries,
                             const int* __restrict__ token_counts, int capacity,
                             const int* __restrict__ cand_ids, int begin, int E, float scale,
                             float* tile, uint64_t* keys) {
  for (int g0 = 0; g0 < nflag; g0 += kChainPages) {
    const int G = nflag - g0 < kChainPages ? nflag - g0 : kChainPages;
    float acc = 0.0f;
    for (int t0 = 0; t0 < E; t0 += kRankTile) {
      const int len = E - t0 < kRankTile ? E - t0 : kRankTile;
      for (int x = threadIdx.x; x < G * len; x += blockDim.x) {
        const int f = x / len;
        const int e = x - f * len;
        const int page = cand_ids[begin + flagged[g0 + f]];
        const bool in_pool = page >= 0 && page < capacity;
        const float sv = !in_pool || token_counts[page] == 0
                             ? 0.0f
                             : summaries[static_cast<size_t>(page) * E + t0 + e];
        tile[f * kRankTileStride + e] = __fmul_rn(q[t0 + e], sv);
      }
      __syncthreads();
      if (static_cast<int>(threadIdx.x) < G) {
        const float* row = tile + threadIdx.x * kRankTileStride;
        int e = 0;
        for (; e + 4 <= len; e += 4) {
          const float4 v = *reinterpret_cast<const float4*>(row + e);
          acc = __fadd_rn(acc, v.x);
          acc = __fadd_rn(acc, v.y);
          acc = __fadd_rn(acc, v.z);
          acc = __fadd_rn(acc, v.w);
        }
        for (; e < len; ++e) acc = __fadd_rn(acc, row[e]);
      }
      __syncthreads();
    }
    if (static_cast<int>(threadIdx.x) < G) {
      const int i = flagged[g0 + threadIdx.x];
      keys[i] = SelectKey(__fmul_rn(acc, scale), cand_ids[begin + i]);
    }
    __syncthreads();
  }
}

// ---- attention helpers ------------------------------------------------------
constexpr float kLog2e = 1.4426950408889634f;

template <int DQ>
__device__ __forceinline__ void LoadDims(const float* __restrict__ p,
                                         float (&v)[DQ]) {
  if constexpr (DQ % 4 == 0) {
#pragma unroll
    for (int i = 0; i < DQ / 4; ++i) {
      const float4 x = reinterpret_cast<const float4*>(p)[i];
      v[4 * i + 0] = x.x;
      v[4 * i + 1] = x.y;
      v[4 * i + 2] = x.z;
      v[4 * i + 3] = x.w;
    }
  } else if constexpr (DQ % 2 == 0) {
#pragma unroll
    for (int i = 0; i < DQ / 2; ++i) {
      const float2 x = reinterpret_cast<const float2*>(p)[i];
      v[2 * i + 0] = x.x;
      v[2 * i + 1] = x.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < DQ; ++i) v[i] = p[i];
  }
}

__device__ __forceinline__ float Exp2(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace
}  // namespace dsdk
