// fused_step.hip -- the whole sparse decode step in one launch (gfx950).
//
// For the hot shape (E = 4096, head_dim 128, at most 256 candidates and
// top_k <= 256 per request, certified selection) the three stages of the
// step -- page scoring (reference ScorePagesCpu, src/reference_kernels.cpp:
// 59-80), top-k (SelectTopKPagesCpu, :82-107) and gather + attention
// (GatherPagesCpu + SparseAttentionCpu, :109-194) -- run in one kernel, so the
// step pays one launch and no kernel boundary between dependent stages.
//
// Work items.  Request r owns the G = H/2 consecutive workgroups
// [r*G, r*G + G); workgroup (r, g) takes heads 2g and 2g+1.  Each does:
//   1. score: the certified intervals of its slice of the request's
//      candidates, [n*g/G, n*(g+1)/G), eight pages per pass, two waves per
//      page; publishes them and counts itself into the request's arrival
//      counter;
//   2. select: waits until the G workgroups of its request have arrived,
//      then computes the request's top-k from the intervals (the G
//      workgroups compute the same selection; g = 0 writes it out);
//   3. attend: eight waves per head over the selected pages.
// Workgroups have 1024 threads (one per CU at this kernel's register use),
// so at B*H/2 <= 256 the whole step is one dispatch wave.
//
// Every wait ends.  A workgroup waits only for the workgroups of its own
// request, which have adjacent ids.  Workgroup i goes to XCD i mod 8 and each
// XCD dispatches its share in id order.  Take the lowest-id unfinished
// workgroup u (request r): everything below u has finished, so any workgroup
// of r that an XCD has not dispatched yet is queued behind at most the other
// members of r on that XCD (ceil(G/8) in all), and an XCD that can hold that
// many workgroups dispatches it.  The members of r never wait for anything
// outside r and score before they wait, so u finishes; by induction every
// workgroup does.  The spins are bounded anyway (a timeout is reported to the
// host and gives zeros, never a hang).
//
#include "dsd_internal.h"
#include "step_common.h"

namespace dsdk {
namespace {

constexpr int kFThreads = 1024;             // one workgroup per CU
constexpr int kFWaves = kFThreads / kWave;  // 16
constexpr int kFE = 4096;
constexpr int kFD = 128;
constexpr int kFPagesPerPass = 8;           // score pass = 8 pages, 2 waves each
constexpr int kFHeadsPerItem = 2;           // workgroup = 2 heads, 8 waves each
constexpr int kFHeadWaves = kFWaves / kFHeadsPerItem;
constexpr int kFPageLanes = 2 * kWave;      // 128 lanes per page
constexpr int kFPerLane = kFE / kFPageLanes;  // 32 consecutive products per lane
constexpr int kFMaxCand = 256;
constexpr int kFMaxK = 256;
constexpr int kFLpt = 16;                 // lanes per token row (8 dims each)
constexpr int kFDq = kFD / kFLpt;         // 8
constexpr int kFTpc = kWave / kFLpt;      // 4 token rows per wave per chunk
constexpr int kFUnroll = 4;               // chunks in flight per wave
constexpr unsigned kSpinLimit = 1u << 24;  // polls of ~1 us each at most
constexpr int kCounterStride = 32;         // ints: one 128-byte line per counter
// Timing mode: per-workgroup wall clocks at start, slice scored, counter
// ready, records read, ranked, selected, end; then the hardware ids.
constexpr int kStampsPerGroup = 8;
enum Stamp { kStart, kScored, kReady, kRecords, kRanked, kSelected, kEnd, kHwId };

struct FusedShared {
  uint64_t stamp[kStampsPerGroup];  // timing mode: thread 0's clocks
  // score pass (per wave): float total (the carry into wave 2p+1) and the
  // bound sums
  float wave_total[kFWaves];
  float abs_prefix[kFWaves];
  float abs_p[kFWaves];
  int fail;
  int nflag;
  // selection (attention item)
  float mid[kFMaxCand];
  uint64_t key[kFMaxCand];
  float lo[kFMaxCand];
  float hi[kFMaxCand];
  int top[kFMaxCand];
  int flag[kFMaxCand];
  int rank[kFMaxCand];
  int cpage[kFMaxCand];  // page id and token count of candidate i
  int cntok[kFMaxCand];
  float tlo[kFMaxK];    // intervals of the top-k members, in rank order
  float thi[kFMaxK];
  float red[2][kFWaves];
  alignas(16) float tile[kChainPages * kRankTileStride];
  // attention
  int page[kFMaxK];
  int ntok[kFMaxK];
  float m[kFWaves];
  float l[kFWaves];
  alignas(16) float acc[kFWaves][kFD];
};

__device__ __forceinline__ uint64_t Now() { return static_cast<uint64_t>(wall_clock64()); }

// Timing mode only: thread 0 records the wall clock for stamp `which` in
// LDS (a global store here would make the next barrier wait for it); the
// kernel's end writes them out.
__device__ __forceinline__ void StampAt(const FusedArgs& a, FusedShared& sh, int which) {
  if (a.stamps != nullptr && threadIdx.x == 0) sh.stamp[which] = Now();
}

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

__device__ __forceinline__ void ReportFailure(const FusedArgs& a, int code) {
  __hip_atomic_store(a.fail_flag, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Arrival counter of request r for the launch with this epoch.
__device__ __forceinline__ int* ArrivalCounter(const FusedArgs& a, unsigned epoch, int r) {
  return a.arrivals + (static_cast<size_t>(epoch & 1u) * a.max_batch + r) * kCounterStride;
}

// Ranks of the n <= 256 keys in sh.key (descending; equal keys by position):
// kTpc threads per candidate count interleaved slices of the keys
// (candidate j is read by part j % kTpc: contiguous LDS words per
// instruction) and add their counts with shuffles.  Returns the rank to the
// candidate's first thread (part 0), n elsewhere.  No barrier.
constexpr int kTpc = 4;
// Every candidate below kFMaxCand has a lead thread in both rank passes.
static_assert(kFThreads / kTpc >= kFMaxCand, "PartialRanks must cover kFMaxCand");
static_assert(kFThreads / 4 >= kFMaxCand, "FloatRanks must cover kFMaxCand");

__device__ __forceinline__ int PartialRanks(const FusedShared& sh, int n, int* cand_out) {
  const int t = threadIdx.x;
  const int cand = t / kTpc;
  const int part = t - cand * kTpc;
  int partial = 0;
  if (cand < n) {
    const uint64_t key = sh.key[cand];
    int j = part;
    for (; j + 7 * kTpc < n; j += 8 * kTpc) {
      uint64_t kj[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) kj[u] = sh.key[j + u * kTpc];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        partial += (kj[u] > key || (kj[u] == key && j + u * kTpc < cand)) ? 1 : 0;
      }
    }
    for (; j < n; j += kTpc) {
      partial += (sh.key[j] > key || (sh.key[j] == key && j < cand)) ? 1 : 0;
    }
  }
#pragma unroll
  for (int o = 1; o < kTpc; o <<= 1) partial += __shfl_xor(partial, o, kWave);
  *cand_out = cand;
  return (cand < n && part == 0) ? partial : n;
}

// The common case of the same ranks from the float scores alone: tpc
// threads per candidate (as many as the workgroup allows for n: every
// candidate below n must get a lead thread) count the midpoints strictly
// above its own (two instructions per midpoint instead of a 64-bit key
// comparison).  That is the rank whenever no two candidates have equal
// midpoints; equal ones are counted into *ties (including itself), and the
// caller falls back to the key ranks when any candidate has one.
__device__ __forceinline__ int FloatRanks(const FusedShared& sh, int n, int* cand_out,
                                          int* ties) {
  const int tpc = n <= kFThreads / 16 ? 16 : (n <= kFThreads / 8 ? 8 : 4);
  const int t = threadIdx.x;
  const int cand = t / tpc;
  const int part = t - cand * tpc;
  int gt = 0, eq = 0;
  if (cand < n) {
    const float m = sh.mid[cand];
    int j = part;
    for (; j + 7 * tpc < n; j += 8 * tpc) {
      float mj[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) mj[u] = sh.mid[j + u * tpc];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        gt += mj[u] > m ? 1 : 0;
        eq += mj[u] == m ? 1 : 0;
      }
    }
    for (; j < n; j += tpc) {
      gt += sh.mid[j] > m ? 1 : 0;
      eq += sh.mid[j] == m ? 1 : 0;
    }
  }
  for (int o = 1; o < tpc; o <<= 1) {  // tpc is uniform: every lane shuffles
    gt += __shfl_xor(gt, o, kWave);
    eq += __shfl_xor(eq, o, kWave);
  }
  *cand_out = cand;
  *ties = eq;
  return (cand < n && part == 0) ? gt : n;
}

// Ranks of the keys into sh.rank (whole workgroup; ends with a barrier).
__device__ void ParallelRanks(FusedShared& sh, int n) {
  int cand;
  const int rank = PartialRanks(sh, n, &cand);
  if (rank < n) sh.rank[cand] = rank;
  __syncthreads();
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
__device__ void ScorePass(const PoolView& pool, const FusedArgs& a, int r, int first, int end,
                          FusedShared& sh) {
  constexpr int kRows = kFPerLane / 4;  // 8
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
    const int page = a.cand_ids[c];
    const float4* q4 = reinterpret_cast<const float4*>(a.queries + static_cast<size_t>(r) * kFE) +
                       half * 512 + lane;
    const float4* s4 =
        reinterpret_cast<const float4*>(pool.summaries + static_cast<size_t>(page) * kFE) +
        half * 512 + lane;
    const int count = pool.token_counts[page];
    float4 qv[kRows];
    float4 sv[kRows];
#pragma unroll
    for (int j = 0; j < kRows; ++j) {
      qv[j] = q4[j * kWave];
      sv[j] = s4[j * kWave];
    }
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
      sh.wave_total[wave] = total;
    }
  }
  __syncthreads();
  if (active) {
    // Starting prefix of each of this lane's groups, and the bound sums.
    float base = half ? sh.wave_total[wave - 1] : 0.0f;
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
      sh.abs_prefix[wave] = tsum;
      sh.abs_p[wave] = absp;
    }
  }
  __syncthreads();
  if (active && half == 0 && lane == 0) {
    const float s_hat = __fadd_rn(sh.wave_total[wave], sh.wave_total[wave + 1]);
    const float tsum = __fadd_rn(sh.abs_prefix[wave], sh.abs_prefix[wave + 1]);
    const float ap = __fadd_rn(sh.abs_p[wave], sh.abs_p[wave + 1]);
    float mid, lo, hi;
    WriteBoundsFloat(s_hat, tsum, ap, kFE, 4, 40, a.scale, &mid, &lo, &hi);
    a.mid[c] = mid;
    a.lo[c] = lo;
    a.hi[c] = hi;
    unsigned long long* rec = a.rec + 3 * static_cast<size_t>(c);
    PutTagged(rec + 0, a.epoch, __float_as_uint(mid));
    PutTagged(rec + 1, a.epoch, __float_as_uint(lo));
    PutTagged(rec + 2, a.epoch, __float_as_uint(hi));
  }
}

// The candidates [c0, c1) of request r, eight per pass; then this workgroup
// counts itself into the request's arrival counter.
__device__ void ScoreSlice(const PoolView& pool, const FusedArgs& a, int r, int c0, int c1,
                           FusedShared& sh) {
  for (int first = c0; first < c1; first += kFPagesPerPass) {
    ScorePass(pool, a, r, first, c1, sh);
  }
  __syncthreads();  // the slice's words are issued before the count
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(ArrivalCounter(a, a.epoch, r), 1, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Top-k of request r (n candidates from `begin`) from the published
// intervals into sh.page / sh.ntok, once all `groups` workgroups of the
// request have counted in; returns the count (0 on failure).
// Candidates whose order the intervals do not decide are rescored with the
// exact sequential chain (as SelectCertifiedRankKernel).  The workgroup with
// `writer` set also writes the selection out for the caller.
__device__ int SelectForRequest(const PoolView& pool, const FusedArgs& a, int r, int begin,
                                int n, int groups, bool writer, FusedShared& sh) {
  int kk = a.top_k <= 0 ? 0 : (a.top_k < n ? a.top_k : n);
  if (n > kFMaxCand) {
    // The caller's max_candidates understated the CSR: select nothing (the
    // outputs are zeros) and report it to the host.
    if (writer && threadIdx.x == 0) ReportFailure(a, 2);
    kk = 0;
  }
  const int i = threadIdx.x;
  const bool mine = kk > 0 && i < n;
  // Ids and token counts do not depend on the scores: fetch them first.
  int my_page = 0, my_ntok = 0;
  if (mine) {
    my_page = a.cand_ids[begin + i];
    my_ntok = pool.token_counts[my_page];
  }
  if (i == 0) {
    sh.fail = 0;
    sh.nflag = 0;
    if (kk > 0) {
      // One poller per workgroup: wait until every workgroup of the request
      // has published its slice (a hint; the tags below decide).
      int* counter = ArrivalCounter(a, a.epoch, r);
      unsigned spins = 0;
      while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < groups) {
        __builtin_amdgcn_s_sleep(2);
        if (++spins >= kSpinLimit) {
          sh.fail = 1;
          break;
        }
      }
    }
  }
  __syncthreads();
  StampAt(a, sh, kReady);
  if (mine && !sh.fail) {
    unsigned long long* rec = a.rec + 3 * static_cast<size_t>(begin + i);
    // First an ordinary (L2-cached) read, shared by the workgroups of this
    // request on the XCD; a word whose tag is not current (not yet visible,
    // or a stale cached line) is then polled coherently.
    unsigned long long w0 = rec[0], w1 = rec[1], w2 = rec[2];
    unsigned spins = 0;
    while (!(Current(w0, a.epoch) && Current(w1, a.epoch) && Current(w2, a.epoch))) {
      __builtin_amdgcn_s_sleep(1);
      if (++spins >= kSpinLimit) {
        sh.fail = 1;
        break;
      }
      w0 = LoadWord(rec + 0);
      w1 = LoadWord(rec + 1);
      w2 = LoadWord(rec + 2);
    }
    sh.mid[i] = __uint_as_float(static_cast<uint32_t>(w0));
    sh.key[i] = SelectKey(sh.mid[i], my_page);
    sh.lo[i] = __uint_as_float(static_cast<uint32_t>(w1));
    sh.hi[i] = __uint_as_float(static_cast<uint32_t>(w2));
    sh.cpage[i] = my_page;
    sh.cntok[i] = my_ntok;
  }
  __syncthreads();
  StampAt(a, sh, kRecords);
  if (sh.fail) {
    if (threadIdx.x == 0) ReportFailure(a, 1);
    kk = 0;
  }
  if (kk > 0) {
    // Ranks, with everything the flag test needs published in the same
    // pass: rank per candidate, the members' intervals in rank order, the
    // members' pages (speculatively: rewritten if rescoring reorders), and
    // per-wave min(lo of members) / max(hi of outsiders).  Midpoints decide
    // the ranks unless two are equal; then the (score, page id) keys do.
    int cand, ties;
    int lead_rank = FloatRanks(sh, n, &cand, &ties);
    if (__syncthreads_or(lead_rank < n && ties > 1)) {
      lead_rank = PartialRanks(sh, n, &cand);
    }
    StampAt(a, sh, kRanked);
    float my_min = INFINITY, my_max = -INFINITY;
    if (lead_rank < n) {
      sh.rank[cand] = lead_rank;
      if (lead_rank < kk) {
        sh.tlo[lead_rank] = sh.lo[cand];
        sh.thi[lead_rank] = sh.hi[cand];
        sh.page[lead_rank] = sh.cpage[cand];
        sh.ntok[lead_rank] = sh.cntok[cand];
        my_min = sh.lo[cand];
      } else {
        my_max = sh.hi[cand];
      }
    }
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
      my_min = fminf(my_min, __shfl_xor(my_min, o, kWave));
      my_max = fmaxf(my_max, __shfl_xor(my_max, o, kWave));
    }
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
      sh.red[0][wave] = my_min;
      sh.red[1][wave] = my_max;
    }
    __syncthreads();
    bool flag = false;
    if (i < n) {
      float min_t_lo = INFINITY, max_o_hi = -INFINITY;
#pragma unroll
      for (int w = 0; w < kFWaves; ++w) {
        min_t_lo = fminf(min_t_lo, sh.red[0][w]);
        max_o_hi = fmaxf(max_o_hi, sh.red[1][w]);
      }
      const int rank = sh.rank[i];
      const float l = sh.lo[i];
      const float h = sh.hi[i];
      if (rank >= kk) {
        flag = h >= min_t_lo;
      } else {
        // Overlap with any other member, or with the best outsider.  The
        // members are in midpoint order, so a member ranked above overlaps
        // iff its lo <= this hi, one ranked below iff its hi >= this lo.
        float above_lo = INFINITY, below_hi = -INFINITY;
#pragma unroll 4
        for (int j = 0; j < kk; ++j) {
          const float tl = sh.tlo[j];
          const float th = sh.thi[j];
          above_lo = j < rank ? fminf(above_lo, tl) : above_lo;
          below_hi = j > rank ? fmaxf(below_hi, th) : below_hi;
        }
        flag = l <= max_o_hi || above_lo <= h || below_hi >= l;
      }
    }
    if (__syncthreads_or(flag ? 1 : 0)) {
      // Some order is not decided by the intervals: rescore those pages
      // with the exact chain, rank again and rewrite the members.
      if (flag) sh.flag[atomicAdd(&sh.nflag, 1)] = i;
      __syncthreads();
      const int nflag = sh.nflag;
      if (writer && threadIdx.x == 0 && a.exact_pages != nullptr) {
        atomicAdd(a.exact_pages, nflag);
      }
      RescoreExact(sh.flag, nflag, a.queries + static_cast<size_t>(r) * kFE, pool.summaries,
                   pool.token_counts, a.cand_ids, begin, kFE, a.scale, sh.tile, sh.key);
      ParallelRanks(sh, n);
      if (i < n && sh.rank[i] < kk) {
        sh.page[sh.rank[i]] = sh.cpage[i];
        sh.ntok[sh.rank[i]] = sh.cntok[i];
      }
      __syncthreads();
    }
    // Every member slot holds a candidate's page id; one outside the pool
    // would be a selection bug: drop it (no K/V access) and report it.
    if (i < kk && (sh.page[i] < 0 || sh.page[i] >= pool.capacity)) {
      sh.ntok[i] = 0;
      ReportFailure(a, 3);
    }
    __syncthreads();
    if (writer && i < kk) a.selected[static_cast<size_t>(r) * a.sel_stride + i] = sh.page[i];
  }
  if (writer && threadIdx.x == 0) a.counts[r] = kk;
  return kk;
}

// Attention of workgroup (r, g), heads h0 = 2g and h0+1: select, then per
// head softmax(q_h K^T * scale) V over the selected pages' valid tokens;
// waves 0-7 take head h0 and waves 8-15 head h0+1, each as
// AttentionFastKernel<128, 16, 8, 4>.
__device__ void AttentionItem(const PoolView& pool, const FusedArgs& a, int r, int begin, int n,
                              int group, int groups, FusedShared& sh) {
  const int h0 = group * kFHeadsPerItem;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int hw = wave % kFHeadWaves;   // wave within its head
  const int h = h0 + wave / kFHeadWaves;
  const int g = lane / kFLpt;
  const int j = lane % kFLpt;
  const int head_off = h * kFD + j * kFDq;
  float q[kFDq];
  float acc[kFDq];
  {
    const float qscale = a.scale * kLog2e;
    LoadDims<kFDq>(a.queries + static_cast<size_t>(r) * kFE + head_off, q);
#pragma unroll
    for (int i = 0; i < kFDq; ++i) {
      q[i] *= qscale;
      acc[i] = 0.0f;
    }
  }
  const int kk = SelectForRequest(pool, a, r, begin, n, groups, group == 0, sh);
  StampAt(a, sh, kSelected);
  if (kk == 0) {
    // Nothing selected: zeros (src/cuda/sparse_batched_attention.cu:621-627).
    if (threadIdx.x < kFHeadsPerItem * kFD) {
      a.outputs[static_cast<size_t>(r) * kFE + static_cast<size_t>(h0) * kFD + threadIdx.x] =
          0.0f;
    }
    return;
  }

  const int E = kFE;
  const int ps = pool.page_size;
  const int total = kk * ps;
  float m = -INFINITY;
  float l = 0.0f;
  for (int base = hw * kFTpc * kFUnroll; base < total;
       base += kFHeadWaves * kFTpc * kFUnroll) {
    float kv[kFUnroll][kFDq];
    float vv[kFUnroll][kFDq];
    bool valid[kFUnroll];
#pragma unroll
    for (int u = 0; u < kFUnroll; ++u) {
      const int f = base + u * kFTpc + g;
      valid[u] = false;
      if (f < total) {
        const int slot = f / ps;
        const int t = f - slot * ps;
        valid[u] = t < sh.ntok[slot];
        if (valid[u]) {
          const size_t off = static_cast<size_t>(sh.page[slot]) * pool.page_elems +
                             static_cast<size_t>(t) * E + head_off;
          LoadDims<kFDq>(pool.keys + off, kv[u]);
          LoadDims<kFDq>(pool.values + off, vv[u]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kFUnroll; ++u) {
      float dot = 0.0f;
      if (valid[u]) {
#pragma unroll
        for (int i = 0; i < kFDq; ++i) dot = fmaf(q[i], kv[u][i], dot);
      }
#pragma unroll
      for (int o = 1; o < kFLpt; o <<= 1) dot += __shfl_xor(dot, o, kWave);
      if (valid[u]) {
        const float m_new = fmaxf(m, dot);
        const float alpha = Exp2(m - m_new);
        const float beta = Exp2(dot - m_new);
        l = fmaf(l, alpha, beta);
#pragma unroll
        for (int i = 0; i < kFDq; ++i) acc[i] = fmaf(acc[i], alpha, beta * vv[u][i]);
        m = m_new;
      }
    }
  }
  // Merge the 4 token-slot streams of this wave, then the 8 waves of each
  // head in LDS.
  float wm = m;
#pragma unroll
  for (int o = kFLpt; o < kWave; o <<= 1) wm = fmaxf(wm, __shfl_xor(wm, o, kWave));
  const float sc = (m == -INFINITY) ? 0.0f : Exp2(m - wm);
  float wl = l * sc;
#pragma unroll
  for (int i = 0; i < kFDq; ++i) acc[i] *= sc;
#pragma unroll
  for (int o = kFLpt; o < kWave; o <<= 1) {
    wl += __shfl_xor(wl, o, kWave);
#pragma unroll
    for (int i = 0; i < kFDq; ++i) acc[i] += __shfl_xor(acc[i], o, kWave);
  }
  if (g == 0) {
    if (j == 0) {
      sh.m[wave] = wm;
      sh.l[wave] = wl;
    }
#pragma unroll
    for (int i = 0; i < kFDq; ++i) sh.acc[wave][j * kFDq + i] = acc[i];
  }
  __syncthreads();
  if (threadIdx.x < kFHeadsPerItem * kFD) {
    const int hh = threadIdx.x / kFD;  // which of the two heads
    const int d = threadIdx.x - hh * kFD;
    const int w0 = hh * kFHeadWaves;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kFHeadWaves; ++w) mx = fmaxf(mx, sh.m[w0 + w]);
    float lt = 0.0f;
    float at = 0.0f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kFHeadWaves; ++w) {
        const float sw = (sh.m[w0 + w] == -INFINITY) ? 0.0f : Exp2(sh.m[w0 + w] - mx);
        lt = fmaf(sh.l[w0 + w], sw, lt);
        at = fmaf(sh.acc[w0 + w][d], sw, at);
      }
    }
    // No valid token at all: zeros, as the reference.
    a.outputs[static_cast<size_t>(r) * kFE + static_cast<size_t>(h0 + hh) * kFD + d] =
        lt == 0.0f ? 0.0f : at / lt;
  }
}

__global__ __launch_bounds__(kFThreads) void FusedStepKernel(PoolView pool, FusedArgs a) {
  __shared__ FusedShared sh;
  if (a.stamps != nullptr && threadIdx.x == 0) {
    for (int i = 0; i < kStampsPerGroup; ++i) sh.stamp[i] = 0;
  }
  StampAt(a, sh, kStart);
  const int groups = pool.num_heads / kFHeadsPerItem;
  const int r = blockIdx.x / groups;
  const int g = blockIdx.x - r * groups;
  if (blockIdx.x == 0 && static_cast<int>(threadIdx.x) < a.max_batch) {
    // Clear the arrival counters the next launch uses.
    __hip_atomic_store(ArrivalCounter(a, a.epoch + 1, threadIdx.x), 0, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
  const int begin = a.cand_offsets[r];
  const int n = a.cand_offsets[r + 1] - begin;
  // A request beyond kFMaxCand selects nothing (reported by the selection):
  // its slices are not scored.
  if (n <= kFMaxCand) {
    ScoreSlice(pool, a, r, begin + (g * n) / groups, begin + ((g + 1) * n) / groups, sh);
  }
  StampAt(a, sh, kScored);
  AttentionItem(pool, a, r, begin, n, g, groups, sh);
  StampAt(a, sh, kEnd);
  if (a.stamps != nullptr && threadIdx.x == 0) {
    // HW_ID (wave slot, SIMD, CU, shader array, shader engine) and XCC_ID.
    const uint64_t hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
    const uint64_t xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);
    sh.stamp[kHwId] = (xcc << 32) | hw;
    for (int i = 0; i < kStampsPerGroup; ++i) {
      a.stamps[kStampsPerGroup * static_cast<size_t>(blockIdx.x) + i] = sh.stamp[i];
    }
  }
}

}  // namespace

bool FusedStepSupported(const PoolView& pool, int max_candidates, int top_k) {
  return pool.elements == kFE && pool.head_dim == kFD && pool.page_size > 0 &&
         pool.num_heads % kFHeadsPerItem == 0 && max_candidates <= kFMaxCand &&
         top_k <= kFMaxK;
}

int FusedStepGrid(const PoolView& pool, int batch) {
  return batch * (pool.num_heads / kFHeadsPerItem);
}

int FusedStepStampsPerGroup() { return kStampsPerGroup; }

void LaunchFusedStep(const PoolView& pool, const FusedArgs& args, hipStream_t stream) {
  if (args.batch <= 0) return;
  const int grid = FusedStepGrid(pool, args.batch);
  hipLaunchKernelGGL(FusedStepKernel, dim3(grid), dim3(kFThreads), 0, stream, pool, args);
  DSD_HIP_CHECK(hipGetLastError());
}

}  // namespace dsdk
