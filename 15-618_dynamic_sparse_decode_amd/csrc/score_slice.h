// score_slice.h -- the certified score pass at E = 4096 (gfx950), shared by
// the single-launch step and the stand-alone score kernel (fused_step.hip)
// and the wide step (step_kernels.hip): a workgroup of 1024 threads scores
// eight pages per pass, two waves per page, and publishes each page's
// certified interval (mid, lo, hi) as plain floats and, when asked, as
// epoch-tagged 64-bit words (below).  Reference: ScorePagesCpu,
// src/reference_kernels.cpp:59-80 (the exact score the interval contains).
#pragma once

#include "dsd_internal.h"
#include "step_common.h"

namespace dsdk {
namespace {

constexpr int kFThreads = 1024;             // one workgroup per CU
constexpr int kFWaves = kFThreads / kWave;  // 16
constexpr int kFE = 4096;
constexpr int kFPagesPerPass = 8;           // score pass = 8 pages, 2 waves each
constexpr int kFPageLanes = 2 * kWave;      // 128 lanes per page
constexpr int kFPerLane = kFE / kFPageLanes;  // 32 consecutive products per lane

// Publication without fences: a word whose high half is a launch's epoch and
// whose low half is the payload, written and read with relaxed agent-scope
// atomics; valid exactly when its tag is current.
__device__ __forceinline__ void PutTagged(unsigned long long* p, unsigned epoch,
                                          uint32_t payload) {
  __hip_atomic_store(p, (static_cast<unsigned long long>(epoch) << 32) | payload,
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long LoadWord(unsigned long long* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ bool Current(unsigned long long w, unsigned epoch) {
  return static_cast<unsigned>(w >> 32) == epoch;
}

// One score pass: certified intervals of candidates first + p, p < 8, below
// end (all of request r).  Waves 2p and 2p+1 take candidate first + p, wave
// 2p+h the elements [2048h, 2048h + 2048) as 8 rows of 64 float4: lane l of
// row j holds float4 number 512h + 64j + l, so every load instruction reads
// 1 KiB contiguously.  Each lane's float4 is a group of L = 4 consecutive
// products: the lane forms the group's local prefix sums; a DPP scan of the
// group sums along the row, plus the sums of the rows before, plus wave 2p's
// total for h = 1, gives the group's starting prefix.  All in float; the
// rounding depth on any product's path into a group's starting prefix or
// into the page sum is at most 3 local + 6 scan + 8 rows of wave 2p + 8 rows
// of wave 2p+1 + 1 = 26 (40 is used in the bound).  Called by the whole
// workgroup.
constexpr int kFRows = kFPerLane / 4;  // rows of float4 per lane and pass

// A workgroup barrier that orders LDS only.  __syncthreads() also orders
// global memory: with a global store outstanding (the previous pass's
// intervals) it waits on vmcnt(0), which on gfx950 counts loads too, and so
// would wait for the rows prefetched for the next pass.
__device__ __forceinline__ void LdsBarrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// This wave's half of page `page`'s summary (kFRows float4 per lane) and its
// token count, issued without waiting.  An id outside the pool loads page 0
// with a count of 0 (the pass reports it).
__device__ __forceinline__ void LoadPassRows(const PoolView& pool, int page,
                                             float4 (&sv)[kFRows], int& count) {
  const int lane = threadIdx.x & (kWave - 1);
  const int half = (threadIdx.x / kWave) & 1;
  count = 0;
  if (page >= 0 && page < pool.capacity) {
    count = pool.token_counts[page];
  } else {
    page = 0;
  }
  const float4* s4 =
      reinterpret_cast<const float4*>(pool.summaries + static_cast<size_t>(page) * kFE) +
      half * 512 + lane;
#pragma unroll
  for (int j = 0; j < kFRows; ++j) sv[j] = s4[j * kWave];
}

// One pass over rows already loaded (sv, count for this wave's candidate
// first + wave/2, page id `page`).  Once the products are formed, the rows
// of the next pass's candidate (page id `next`, when next_active) load into
// the same registers, so their latency overlaps this pass's reductions and
// publication.
template <class Shared>
__device__ void ScorePass(const PoolView& pool, const FusedArgs& a, int first, int end,
                          int page, float4 (&sv)[kFRows], int& count, bool next_active,
                          int next, int parity, const float4* q_lds, Shared& sh) {
  constexpr int kRows = kFRows;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int half = wave & 1;
  const int c = first + (wave >> 1);
  const bool active = c < end;  // uniform per wave
  float row_sum[kRows];   // float sums of the rows (wave-uniform)
  float excl[kRows];      // sum of the group sums of the lanes below, row j
  float loc_abs = 0.0f;   // sum of |loc| over this lane's groups
  float p_abs = 0.0f;
  if (active) {
    // An id outside the pool scores as an empty page and is reported.
    if (!InPool(page, pool.capacity) && half == 0 && lane == 0) ReportFailure(a.fail, kFailPageId);
    const float4* q4 = q_lds + half * 512 + lane;
    float4 qv[kRows];
#pragma unroll
    for (int j = 0; j < kRows; ++j) qv[j] = q4[j * kWave];
    // A page holding no tokens reads as an all-zero summary
    // (src/paged_kv_cache.cpp:457-459); the products q*0 are still formed.
    if (count == 0) {
#pragma unroll
      for (int j = 0; j < kRows; ++j) sv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      const float p0 = __fmul_rn(qv[j].x, sv[j].x);
      const float p1 = __fmul_rn(qv[j].y, sv[j].y);
      const float p2 = __fmul_rn(qv[j].z, sv[j].z);
      const float p3 = __fmul_rn(qv[j].w, sv[j].w);
      const float l2 = __fadd_rn(p0, p1);
      const float l3 = __fadd_rn(l2, p2);
      const float l4 = __fadd_rn(l3, p3);
      loc_abs = __fadd_rn(loc_abs, __fadd_rn(__fadd_rn(fabsf(p0), fabsf(l2)),
                                             __fadd_rn(fabsf(l3), fabsf(l4))));
      p_abs = __fadd_rn(p_abs, __fadd_rn(__fadd_rn(fabsf(p0), fabsf(p1)),
                                         __fadd_rn(fabsf(p2), fabsf(p3))));
      const float incl = WaveInclusiveScan(l4);
      row_sum[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(incl), kWave - 1));
      excl[j] = DppMove<kWaveShr1>(incl);  // exact: the inclusive sum of lane - 1
    }
    if (lane == 0) {
      float total = 0.0f;
#pragma unroll
      for (int j = 0; j < kRows; ++j) total = __fadd_rn(total, row_sum[j]);
      sh.wave_total[parity][wave] = total;
    }
  }
  if (next_active) LoadPassRows(pool, next, sv, count);
  LdsBarrier();
  if (active) {
    // Starting prefix of each of this lane's groups, and the bound sums.
    float base = half ? sh.wave_total[parity][wave - 1] : 0.0f;
    float tl = 0.0f;
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      const float start = __fadd_rn(base, excl[j]);
      tl = __fadd_rn(tl, 4.0f * fabsf(start));
      base = __fadd_rn(base, row_sum[j]);
    }
    const float tsum = WaveTotal(__fadd_rn(tl, loc_abs));
    const float absp = WaveTotal(p_abs);
    if (lane == 0) {
      sh.abs_prefix[parity][wave] = tsum;
      sh.abs_p[parity][wave] = absp;
    }
  }
  LdsBarrier();
  if (active && half == 0 && lane == 0) {
    const float s_hat =
        __fadd_rn(sh.wave_total[parity][wave], sh.wave_total[parity][wave + 1]);
    const float tsum =
        __fadd_rn(sh.abs_prefix[parity][wave], sh.abs_prefix[parity][wave + 1]);
    const float ap = __fadd_rn(sh.abs_p[parity][wave], sh.abs_p[parity][wave + 1]);
    float mid, lo, hi;
    WriteBoundsFloat<kFE, 4, 40>(s_hat, tsum, ap, a.scale, &mid, &lo, &hi);
    a.mid[c] = mid;
    a.lo[c] = lo;
    a.hi[c] = hi;
    if (a.rec != nullptr) {
      unsigned long long* rec = a.rec + 3 * static_cast<size_t>(c);
      PutTagged(rec + 0, a.epoch, __float_as_uint(mid));
      PutTagged(rec + 1, a.epoch, __float_as_uint(lo));
      PutTagged(rec + 2, a.epoch, __float_as_uint(hi));
    }
  }
}

// The candidates [c0, c1) of request r, eight per pass.  The query is
// staged once in LDS (in the rescoring tile, idle until the selection).
// kPipeline: the first pass's rows load alongside the query, and each later
// pass's id at the start of the pass before, its rows once that pass's
// products are formed (the stand-alone score kernel, and single-launch steps
// whose slices span several passes: 4 us off the score phase at B = 32 with
// 1024-4096-token contexts).  Otherwise each pass loads its own rows first
// (single-launch steps of one pass per slice, where the pipelined form
// measured 0.2-0.5 us slower at BASELINE config 2).
template <bool kPipeline, class Shared>
__device__ __forceinline__ void ScoreSlice(const PoolView& pool, const FusedArgs& a, int r, int c0, int c1,
                           Shared& sh) {
  if (c0 >= c1) return;
  static_assert(kFE / 4 == kFThreads, "one float4 of the query per thread");
  static_assert(sizeof(sh.tile) >= kFE * sizeof(float), "the query fits the tile");
  const int c = c0 + static_cast<int>(threadIdx.x) / (2 * kWave);
  // The query and the first ids load together.
  const float4 qv =
      reinterpret_cast<const float4*>(a.queries + static_cast<size_t>(r) * kFE)[threadIdx.x];
  int page = c < c1 ? a.cand_ids[c] : -1;
  float4 sv[kFRows];
  int count = 0;
  if (kPipeline && c < c1) LoadPassRows(pool, page, sv, count);
  float4* q_lds = reinterpret_cast<float4*>(sh.tile);
  q_lds[threadIdx.x] = qv;
  LdsBarrier();
  for (int first = c0; first < c1; first += kFPagesPerPass) {
    const int parity = ((first - c0) / kFPagesPerPass) & 1;
    if constexpr (kPipeline) {
      const int cn = c + (first - c0) + kFPagesPerPass;  // this wave's next candidate
      const bool next_active = cn < c1;
      const int next = next_active ? a.cand_ids[cn] : -1;
      ScorePass(pool, a, first, c1, page, sv, count, next_active, next, parity, q_lds, sh);
      page = next;
    } else {
      const int cp = c + (first - c0);
      if (first != c0) page = cp < c1 ? a.cand_ids[cp] : -1;
      if (cp < c1) LoadPassRows(pool, page, sv, count);
      ScorePass(pool, a, first, c1, page, sv, count, false, -1, parity, q_lds, sh);
    }
  }
}

// The stand-alone score kernel's LDS (and the wide step's score items').
struct ScoreShared {
  float wave_total[2][kFWaves];  // [pass parity]: a pass's leader reads its
  float abs_prefix[2][kFWaves];  // sums after the pass's last barrier, while
  float abs_p[2][kFWaves];       // the next pass may already write its own
  alignas(16) float tile[kFE];  // the query
};

}  // namespace
}  // namespace dsdk
