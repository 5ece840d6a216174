// step_common.h -- device helpers shared by the decode-step kernels
// (step_kernels.hip) and the fused single-launch step (fused_step.hip).
#pragma once

#include <hip/hip_runtime.h>

#include "dsd_internal.h"
#include "refine_lane.h"

#include <cmath>
#include <cstdint>

namespace dsdk {
namespace {

constexpr int kWave = 64;

// Stores (epoch << 32) | code into the launch's failure word (a system-scope
// store: the word is pinned host memory the host reads after the step).
__device__ __forceinline__ void ReportFailure(const FailReport& f, int code) {
  if (f.word == nullptr) return;
  __hip_atomic_store(f.word,
                     (static_cast<unsigned long long>(f.epoch) << 32) |
                         static_cast<unsigned>(code),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The CSR bounds of request r: false (and kFailShape reported) when its
// offsets leave [0, total] or decrease, so no candidate index outside the
// launch's buffers is ever formed.
__device__ __forceinline__ bool RequestRange(const int* cand_offsets, int r, int total,
                                             const FailReport& f, int* begin, int* n) {
  const int b = cand_offsets[r];
  const int e = cand_offsets[r + 1];
  if (b < 0 || e < b || e > total) {
    ReportFailure(f, kFailShape);
    *begin = 0;
    *n = 0;
    return false;
  }
  *begin = b;
  *n = e - b;
  return true;
}

// A candidate page id usable as an index into the pool arrays.
__device__ __forceinline__ bool InPool(int page, int capacity) {
  return page >= 0 && page < capacity;
}

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

// A double from a DPP source lane (both halves moved); lanes with no source
// read +0.0, the identity of a sum.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ double DppMoveD(double x) {
  const long long b = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b), kCtrl, kRowMask, 0xf, false);
  const int hi =
      __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), kCtrl, kRowMask, 0xf, false);
  return __longlong_as_double((static_cast<long long>(hi) << 32) |
                              static_cast<long long>(static_cast<unsigned>(lo)));
}

// Inclusive prefix sum over the 64 lanes in double (at most 6 additions on
// any input's path), and the wave's total in every lane.
__device__ __forceinline__ double WaveInclusiveScanD(double x) {
  x += DppMoveD<kRowShr1>(x);
  x += DppMoveD<kRowShr2>(x);
  x += DppMoveD<kRowShr4>(x);
  x += DppMoveD<kRowShr8>(x);
  x += DppMoveD<kRowBcast15, 0xa>(x);
  x += DppMoveD<kRowBcast31, 0xc>(x);
  return x;
}

__device__ __forceinline__ double ReadLaneD(double x, int lane) {
  const long long b = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_readlane(static_cast<int>(b), lane);
  const int hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), lane);
  return __longlong_as_double((static_cast<long long>(hi) << 32) |
                              static_cast<long long>(static_cast<unsigned>(lo)));
}

__device__ __forceinline__ double WaveSum(double v) {
  return ReadLaneD(WaveInclusiveScanD(v), kWave - 1);
}

// Sum over each row of 16 lanes, the same value in all 16 (quad swaps, then
// the half-row and row mirrors: the additions of a xor butterfly, so every
// lane forms the identical sum).
constexpr int kQuadXor1 = 0xB1, kQuadXor2 = 0x4E, kRowMirror = 0x140, kRowHalfMirror = 0x141;
__device__ __forceinline__ float RowSum16(float x) {
  x = __fadd_rn(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kQuadXor1, 0xf,
                                                           0xf, false)));
  x = __fadd_rn(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kQuadXor2, 0xf,
                                                           0xf, false)));
  x = __fadd_rn(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kRowHalfMirror,
                                                           0xf, 0xf, false)));
  x = __fadd_rn(x, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), kRowMirror, 0xf,
                                                           0xf, false)));
  return x;
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
// Candidates whose order the score intervals leave open get the reference's
// chain (src/reference_kernels.cpp:13-19, :59-80): acc = fl(acc + fl(q_i*s_i))
// for i = 0 .. E-1 in order, then fl(acc * scale).  The adds of one page are
// a dependent chain (about 4.5 cycles per v_add_f32 from registers, the
// issue time of a wave64 op), so pages run side by side in the lanes of
// wave 0 while the other
// waves form the next stretch of products in a second LDS buffer: the loads
// of stretch t+1 overlap the adds of stretch t.  With M = the largest group
// the buffers hold (32 for the select kernels, 16 for the fused step, whose
// LDS stays near its score-and-select footprint), a group takes M/4, M/2 or
// M pages (the fewest that cover what remains), with stretches of 1024, 512
// or 256 products per page.  Fed from LDS, an add costs about 7 cycles (the
// read latency is not fully hidden), so a 1024-product stretch outlasts one
// memory round trip even on a busy HBM.  Measured slower: one stretch of all
// E products per page (its whole fill latency is exposed), and fills that
// batch four units per thread.
// LDS floats of the two buffers for groups of up to kMaxGroup pages
// (kMaxGroup/4 x 1028, kMaxGroup/2 x 516 or kMaxGroup x 260 per buffer).
template <int kMaxGroup>
constexpr int RescoreFloats() {
  return 2 * kMaxGroup * (256 + 4);
}

// acc + row[0] + row[1] + ... + row[len-1], one rounding per element in
// order (the reference chain); len % 64 == 0, row 16-byte aligned.  Blocks
// of 64 floats are fully unrolled, the LDS reads of the second 32-float half
// issued while the first is added; nothing is carried in registers across
// blocks, so no register copies (a rolled loop with a carried prefetch
// buffer compiles to one v_mov per element).  Larger unrolled blocks were
// no faster and, inlined into the fused step, cost it 4 us at config 2.
__device__ __forceinline__ void AddRow8(const float4 (&v)[8], float& acc) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    acc = __fadd_rn(acc, v[i].x);
    acc = __fadd_rn(acc, v[i].y);
    acc = __fadd_rn(acc, v[i].z);
    acc = __fadd_rn(acc, v[i].w);
  }
}

template <int kHalves>  // kHalves * 32 floats, kHalves even
__device__ __forceinline__ float ChainBlock(const float4* r4, float acc) {
  float4 a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = r4[i];
#pragma unroll
  for (int h = 0; h < kHalves; h += 2) {
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = r4[(h + 1) * 8 + i];
    AddRow8(a, acc);
    if (h + 2 < kHalves) {
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] = r4[(h + 2) * 8 + i];
    }
    AddRow8(b, acc);
  }
  return acc;
}

__device__ __forceinline__ float ChainAdd(const float* row, int len, float acc) {
  const float4* r4 = reinterpret_cast<const float4*>(row);
  for (int e = 0; e < len; e += 64) acc = ChainBlock<2>(r4 + e / 4, acc);
  return acc;
}

// Exact scores of `nflag` candidates: page_of(f) gives the page id of the
// f-th (an id outside [0, capacity), or a page holding no tokens, reads as
// an all-zero summary: src/paged_kv_cache.cpp:457-459), emit(f, score)
// receives its exact score.  q is the request's query (E floats, 16-byte
// aligned), E % 64 == 0, tile holds RescoreFloats<kMaxGroup>() floats of
// LDS (kMaxGroup a multiple of 4).  Must be called by the whole workgroup
// of kThreads threads; emit runs in lanes of wave 0 only.  A
// one-wave workgroup fills each stretch itself after adding the previous one
// (no overlap).
template <int kMaxGroup, int kThreads, class PageOf, class Emit>
__device__ void RescoreChains(int nflag, PageOf page_of, Emit emit, const float* __restrict__ q,
                              const float* __restrict__ summaries,
                              const int* __restrict__ token_counts, int capacity, int E,
                              float scale, float* tile) {
  static_assert(kMaxGroup % 4 == 0, "groups of kMaxGroup / 4 pages");
  constexpr int kBuf = RescoreFloats<kMaxGroup>() / 2;  // floats per buffer
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  constexpr bool one_wave = kThreads <= kWave;
  // Threads that form the stretch after the one being added.
  const int fill_first = one_wave ? 0 : kWave;
  const int fill_count = kThreads - fill_first;
  for (int g0 = 0; g0 < nflag; ) {
    const int left = nflag - g0;
    const int width = left <= kMaxGroup / 4 ? kMaxGroup / 4
                                            : (left <= kMaxGroup / 2 ? kMaxGroup / 2 : kMaxGroup);
    const int G = left < width ? left : width;
    const int C = width == kMaxGroup / 4 ? 1024 : (width == kMaxGroup / 2 ? 512 : 256);
    const int stride = C + 4;
    const int stretches = (E + C - 1) / C;
    // Products of stretch t for the group into buffer b, by threads
    // [first, first + count) of the workgroup, one float4 per unit.
    auto fill = [&](int b, int t, int first, int count) {
      const int t0 = t * C;
      const int len4 = (E - t0 < C ? E - t0 : C) / 4;
      float* buf = tile + b * kBuf;
      for (int u = static_cast<int>(threadIdx.x) - first; u < G * len4; u += count) {
        const int f = u / len4;
        const int e4 = u - f * len4;
        const int page = page_of(g0 + f);
        const bool live = page >= 0 && page < capacity && token_counts[page] != 0;
        const float4 qv = reinterpret_cast<const float4*>(q + t0)[e4];
        const float4 sv = live ? reinterpret_cast<const float4*>(
                                     summaries + static_cast<size_t>(page) * E + t0)[e4]
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        float4 p;
        p.x = __fmul_rn(qv.x, sv.x);
        p.y = __fmul_rn(qv.y, sv.y);
        p.z = __fmul_rn(qv.z, sv.z);
        p.w = __fmul_rn(qv.w, sv.w);
        reinterpret_cast<float4*>(buf + f * stride)[e4] = p;
      }
    };
    fill(0, 0, 0, kThreads);
    __syncthreads();
    float acc = 0.0f;
    for (int t = 0; t < stretches; ++t) {
      if (wave == 0) {
        const int len = E - t * C < C ? E - t * C : C;
        if (lane < G) acc = ChainAdd(tile + (t & 1) * kBuf + lane * stride, len, acc);
      }
      if ((wave != 0 || one_wave) && t + 1 < stretches) {
        fill((t + 1) & 1, t + 1, fill_first, fill_count);
      }
      __syncthreads();
    }
    if (wave == 0 && lane < G) emit(g0 + lane, __fmul_rn(acc, scale));
    __syncthreads();
    g0 += G;
  }
}

// ---- refined intervals -------------------------------------------------------
// A much narrower certified interval for one page's reference score, for the
// pages whose order the first intervals leave open: the rounding error of
// every addition whose binade is certain is accounted for exactly, the
// others by half a grid spacing (refine_lane.h states the rule; each lane
// runs its steps there).  B >= |acc_j - T_j| comes from the page's
// first-pass interval (dsd_refine::FirstPassBound).  The interval is
// S - K -+ (U + slack), K = the known errors, U = the others' bound; on
// random data it is about 30 times narrower than the first-pass interval.
//
// Whether to refine nflag flagged pages or send them straight to the exact
// chains: refine only when every page gets at least two waves in one round
// (nflag <= waves / 2).  The refinement's cost grows with the pages per
// wave, while RescoreChains runs up to a group of chains side by side at
// the cost of one; and a batch step lasts as long as its slowest
// workgroup, so a request whose refined intervals still leave a page open
// pays for both.  Measured on 32 requests of 2048 pages, top 64 (about 7
// flagged pages a request): refining every flagged set took the select
// kernel from 31 to 45 us; with this rule it stays within 1 us of never
// refining, and small flagged sets still settle without the chain.
//
// The thread counts here and below are compile-time constants, not
// blockDim.x: that reads the dispatch's group size from memory (code
// object v5), and where the compiler re-reads it mid-kernel (it did so just
// before the single-launch step's refinement) the read waits for every
// outstanding load.
template <int kThreads>
__device__ __forceinline__ bool RefineWorthwhile(int nflag) {
  return 2 * nflag <= kThreads / kWave;
}

// Refined intervals of nflag pages: page_of(f) gives the f-th page's summary
// row (nullptr: an all-zero summary), bound_of(f) its B, emit(f, mid, lo,
// hi) receives its interval (in lane 0 of the page's first wave).  q: the request's query (E floats).  E % 256 == 0; rows
// 16-byte aligned.  Called by the whole workgroup (its waves take `parts`
// waves per page, 1..8, so a few flagged pages use every wave); returns
// after a barrier, so every wave sees what emit wrote.  scratch holds 8
// doubles per wave (LDS).
//
// Wave `part` of a page takes the elements [part*E/parts, (part+1)*E/parts),
// lane l the block of Lp = E/(64*parts) consecutive ones in it, as float4
// chunks.  The products of the first kKeep chunks stay in registers between
// the sweeps (all of them when Lp <= 4*kKeep: one load round trip); later
// chunks are loaded again.  Sweep 1: the block's double sum; the blocks'
// starts come from a wave scan plus the earlier parts' totals (LDS, one
// barrier).  Sweep 2: every step through dsd_refine::Sweep2Step,
// straight-line code with no divergence between lanes; each wave's sums go
// to LDS (one barrier) and each page's first wave combines its parts.
template <int kThreads, class PageOf, class BoundOf, class Emit>
__device__ void RefineScores(int nflag, PageOf page_of, BoundOf bound_of, Emit emit,
                             const float* __restrict__ q, int E, float scale, double* scratch) {
  constexpr int kKeep = 2;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  constexpr int nwaves = kThreads / kWave;
  const int busy = nflag < nwaves ? nflag : nwaves;
  int parts = 1;
  while (parts < 8 && parts * 2 * busy <= nwaves && (E / (kWave * parts * 2)) % 4 == 0) parts *= 2;
  const int per_round = nwaves / parts;
  const int Lp = E / (kWave * parts);
  const int nch = Lp / 4;
  const int slot = wave / parts;
  const int part = wave - slot * parts;
  // LDS per wave: [0] its part's total, [3] K, [4] U; a page's first wave
  // also [6] the page's total S and [7] its B.
  double* mine = scratch + 8 * wave;
  const double* page_parts = scratch + 8 * (slot * parts);
  for (int f0 = 0; f0 < nflag; f0 += per_round) {
    const int f = f0 + slot;
    const bool active = slot < per_round && f < nflag;  // uniform per wave
    const float* s = active ? page_of(f) : nullptr;
    const size_t first = static_cast<size_t>(part) * (E / parts) + static_cast<size_t>(lane) * Lp;
    const float4* q4 = reinterpret_cast<const float4*>(q + first);
    const float4* s4 = s == nullptr ? nullptr : reinterpret_cast<const float4*>(s + first);
    auto products = [&](int c, float (&p)[4]) {
      const float4 a = q4[c];
      const float4 b = s4 != nullptr ? s4[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      p[0] = __fmul_rn(a.x, b.x);
      p[1] = __fmul_rn(a.y, b.y);
      p[2] = __fmul_rn(a.z, b.z);
      p[3] = __fmul_rn(a.w, b.w);
    };
    // Sweep 1 (the kept chunks' loads are all issued before their use).
    float keep[kKeep][4];
    double run = 0.0;
    double B = 0.0;
    if (active) {
      B = bound_of(f);
#pragma unroll
      for (int c = 0; c < kKeep; ++c) {
        if (c < nch) products(c, keep[c]);
      }
#pragma unroll
      for (int c = 0; c < kKeep; ++c) {
        if (c < nch) {
#pragma unroll
          for (int i = 0; i < 4; ++i) run += static_cast<double>(keep[c][i]);
        }
      }
#pragma unroll 1
      for (int c = kKeep; c < nch; ++c) {
        float p[4];
        products(c, p);
#pragma unroll
        for (int i = 0; i < 4; ++i) run += static_cast<double>(p[i]);
      }
    }
    const double incl = WaveInclusiveScanD(run);
    if (lane == kWave - 1) mine[0] = incl;  // this part's total
    __syncthreads();
    double before = 0.0, S = 0.0;
    for (int k = 0; k < parts; ++k) {
      const double tk = page_parts[8 * k];
      if (k < part) before += tk;
      S += tk;
    }
    // Sweep 2 from T before this lane's first step.
    dsd_refine::Sweep2 s2;
    if (active) {
      const double start = before + (incl - run);
      const bool global_first = part == 0 && lane == 0;
      s2.t = start;
      s2.prev = dsd_refine::CertainField(start, B);
#pragma unroll
      for (int c = 0; c < kKeep; ++c) {
        if (c < nch) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            dsd_refine::Sweep2Step(s2, keep[c][i], B, global_first && c == 0 && i == 0);
          }
        }
      }
#pragma unroll 1
      for (int c = kKeep; c < nch; ++c) {
        float p[4];
        products(c, p);
#pragma unroll
        for (int i = 0; i < 4; ++i) dsd_refine::Sweep2Step(s2, p[i], B, false);
      }
    }
    const float K = WaveTotal(s2.K);
    const float U = WaveTotal(s2.U);
    if (lane == 0) {
      mine[3] = static_cast<double>(K);
      mine[4] = static_cast<double>(U);
      if (part == 0) {
        mine[6] = S;
        mine[7] = B;
      }
    }
    __syncthreads();
    // Lane 0 of each page's first wave combines its parts.  Those waves'
    // slots are only rewritten after the next round's first barrier, which
    // this wave reaches after this.
    if (active && part == 0 && lane == 0) {
      double Kt = 0.0, Ut = 0.0;
      for (int k = 0; k < parts; ++k) {
        Kt += page_parts[8 * k + 3];
        Ut += page_parts[8 * k + 4];
      }
      const double center = mine[6] - Kt;
      const double half = dsd_refine::HalfWidth(center, Ut * (1.0 + 0x1p-16), mine[7], E);
      float m_, l_, h_;
      WriteInterval(center, half, scale, &m_, &l_, &h_, 0);
      emit(f, m_, l_, h_);
    }
  }
  __syncthreads();
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
