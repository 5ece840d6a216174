// step_kernels.hip -- the three kernels of one sparse decode step (gfx950):
//   1. exact-order page scoring   (reference ScorePagesCpu, src/reference_kernels.cpp:59-80)
//   2. per-request top-k select   (reference SelectTopKPagesCpu, :82-107)
//   3. fused gather + attention   (reference GatherPagesCpu + SparseAttentionCpu, :109-194)
// Dense attention (reference DenseAttentionCpu, :196-203) reuses kernel 3
// with every candidate page as the list.
#include <cmath>
#include <cstdio>
#include <cstdlib>

#include "dsd_internal.h"
#include "score_slice.h"
#include "step_common.h"

namespace dsdk {
namespace {

// ---------------------------------------------------------------------------
// 1. Exact-order scoring.
//
// The reference scores a page as acc = 0; acc = fl(acc + fl(q[i]*s[i])) for
// i = 0..E-1, then fl(acc*scale).  That chain must be reproduced in order to
// keep page selection bit-exact, so one lane owns one candidate page and
// walks its summary row sequentially with separately rounded multiply and
// add (__fmul_rn / __fadd_rn; never contracted to FMA).  A wave covers 64
// candidates of one request, so the query operand is wave-uniform and is
// fetched through the scalar cache.
// ---------------------------------------------------------------------------
template <bool kVec4>
__global__ __launch_bounds__(kWave) void ScoreExactKernel(
    const float* __restrict__ queries, const float* __restrict__ summaries,
    const int* __restrict__ token_counts, int capacity, const int* __restrict__ cand_offsets,
    const int* __restrict__ cand_ids, int total, int E, float scale,
    float* __restrict__ scores, FailReport fail) {
  const int r = blockIdx.y;
  int begin, n;
  if (!RequestRange(cand_offsets, r, total, fail, &begin, &n)) return;
  const int end = begin + n;
  const int first = begin + blockIdx.x * kWave;
  if (first >= end) return;
  const int c = first + static_cast<int>(threadIdx.x);
  const bool active = c < end;
  int page = active ? cand_ids[c] : cand_ids[first];
  // A page holding no tokens reads as an all-zero summary
  // (src/paged_kv_cache.cpp:457-459); the products q*0 are still formed.  An
  // id outside the pool scores as such a page and is reported.
  bool zero = !active;
  if (!InPool(page, capacity)) {
    if (active) ReportFailure(fail, kFailPageId);
    page = 0;
    zero = true;
  }
  zero = zero || token_counts[page] == 0;
  const float* __restrict__ q = queries + static_cast<size_t>(r) * E;
  const float* __restrict__ s = summaries + static_cast<size_t>(page) * E;

  float acc = 0.0f;
  if constexpr (kVec4) {
#pragma unroll 8
    for (int i = 0; i < E; i += 4) {
      const float4 qv = *reinterpret_cast<const float4*>(q + i);
      float4 sv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (!zero) sv = *reinterpret_cast<const float4*>(s + i);
      acc = __fadd_rn(acc, __fmul_rn(qv.x, sv.x));
      acc = __fadd_rn(acc, __fmul_rn(qv.y, sv.y));
      acc = __fadd_rn(acc, __fmul_rn(qv.z, sv.z));
      acc = __fadd_rn(acc, __fmul_rn(qv.w, sv.w));
    }
  } else {
    for (int i = 0; i < E; ++i) {
      const float sv = zero ? 0.0f : s[i];
      acc = __fadd_rn(acc, __fmul_rn(q[i], sv));
    }
  }
  if (active) scores[c] = __fmul_rn(acc, scale);
}

// ---------------------------------------------------------------------------
// 1b. Certified scoring (the fast path).
//
// The sequential chain above is latency-bound (4096 dependent adds per page).
// Instead, each page gets one wave that forms the same fp32 products
// p_i = fl(q_i*s_i), sums them in double, and bounds how far the reference's
// sequential fp32 sum can be from that sum:
//   acc_i = fl(acc_{i-1} + p_i)  =>  |acc_n - S| <= u * sum_i |T_i| / (1 - n u)
// with S = sum p_i, T_i the exact prefix sums and u = 2^-24 (plus 2^-150 per
// step for subnormal results).  Each lane owns a contiguous block of BL
// products: pass 1 sums the block, a wave exclusive scan gives the block's
// starting prefix, pass 2 accumulates |T_i|.  Double rounding of the scan is
// covered by generous slack terms.  The page's score interval
// [fl(lo*scale), fl(hi*scale)] (lo/hi rounded outward to float) provably
// contains the reference score, because fl(x*scale) is monotone in x.
// At E = 4096 the fused step's float score passes (ScorePagesKernel in
// fused_step.hip) take this role; the kernel below serves the other E.
// ---------------------------------------------------------------------------
constexpr int kBoundWaves = 4;

// Any E that is a multiple of 64: runtime block length, products re-formed
// from the (cache-resident) operands in pass 2.
__global__ __launch_bounds__(kBoundWaves * kWave) void ScoreBoundGenericKernel(
    const float* __restrict__ queries, const float* __restrict__ summaries,
    const int* __restrict__ token_counts, int capacity, const int* __restrict__ cand_offsets,
    const int* __restrict__ cand_ids, int total, int E, float scale, float* __restrict__ mid_out,
    float* __restrict__ lo_out, float* __restrict__ hi_out, FailReport fail) {
  const int BL = E / kWave;
  const int r = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  int begin, n;
  if (!RequestRange(cand_offsets, r, total, fail, &begin, &n)) return;
  const int c = begin + blockIdx.x * kBoundWaves + wave;
  if (c >= begin + n) return;
  int page = cand_ids[c];
  bool zero = false;
  if (!InPool(page, capacity)) {  // scores as an empty page, reported
    if (lane == 0) ReportFailure(fail, kFailPageId);
    page = 0;
    zero = true;
  }
  zero = zero || token_counts[page] == 0;
  const float* __restrict__ q = queries + static_cast<size_t>(r) * E + lane * BL;
  const float* __restrict__ s = summaries + static_cast<size_t>(page) * E + lane * BL;
  double block = 0.0, abs_p = 0.0;
  for (int i = 0; i < BL; ++i) {
    const float pi = __fmul_rn(q[i], zero ? 0.0f : s[i]);
    block += static_cast<double>(pi);
    abs_p += fabs(static_cast<double>(pi));
  }
  double incl = block;
  for (int o = 1; o < kWave; o <<= 1) {
    const double t = __shfl_up(incl, o, kWave);
    if (lane >= o) incl += t;
  }
  double prefix = __shfl_up(incl, 1, kWave);
  if (lane == 0) prefix = 0.0;
  double abs_prefix = 0.0;
  for (int i = 0; i < BL; ++i) {
    prefix += static_cast<double>(__fmul_rn(q[i], zero ? 0.0f : s[i]));
    abs_prefix += fabs(prefix);
  }
  const double s_hat = __shfl(incl, kWave - 1, kWave);
  abs_prefix = WaveSum(abs_prefix);
  abs_p = WaveSum(abs_p);
  if (lane == 0) WriteBounds(s_hat, abs_prefix, abs_p, E, scale, mid_out, lo_out, hi_out, c);
}

// ---------------------------------------------------------------------------
// 2. Top-k select.
//
// Each candidate becomes one 64-bit key whose unsigned order is the
// reference's comparator: high word = order-preserving image of the score
// (-0.0 folded onto +0.0, since the reference compares with ==), low word =
// ~page_id so that a smaller id wins a tie.  One workgroup bitonic-sorts a
// request's keys descending in LDS and emits the first min(k, n) ids.
// ---------------------------------------------------------------------------
constexpr int kSelectMaxKeys = 8192;  // 64 KiB of LDS

__global__ __launch_bounds__(256) void SelectTopKKernel(
    const float* __restrict__ scores, const int* __restrict__ cand_offsets,
    const int* __restrict__ cand_ids, int total, int max_candidates, int top_k,
    int* __restrict__ selected, int* __restrict__ counts, FailReport fail) {
  extern __shared__ uint64_t keys[];
  const int r = blockIdx.x;
  int begin, n;
  RequestRange(cand_offsets, r, total, fail, &begin, &n);
  if (n > max_candidates) {
    // The launch (LDS, score grid) was sized for max_candidates.
    if (threadIdx.x == 0) ReportFailure(fail, kFailShape);
    n = 0;
  }
  const int kk = top_k <= 0 ? 0 : (top_k < n ? top_k : n);
  if (kk == 0) {
    if (threadIdx.x == 0) counts[r] = 0;
    return;
  }
  int m = 1;
  int log_m = 0;
  while (m < n) {
    m <<= 1;
    ++log_m;
  }
  for (int i = threadIdx.x; i < m; i += blockDim.x) {
    keys[i] = i < n ? SelectKey(scores[begin + i], cand_ids[begin + i]) : 0ull;
  }
  __syncthreads();
  const int half = m >> 1;
  for (int log_size = 1; log_size <= log_m; ++log_size) {
    const int size = 1 << log_size;
    for (int log_stride = log_size - 1; log_stride >= 0; --log_stride) {
      const int stride = 1 << log_stride;
      for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const int lo = ((i >> log_stride) << (log_stride + 1)) | (i & (stride - 1));
        const int hi = lo + stride;
        const bool descending = (lo & size) == 0;
        const uint64_t a = keys[lo];
        const uint64_t b = keys[hi];
        if ((a < b) == descending) {
          keys[lo] = b;
          keys[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  int* out = selected + static_cast<size_t>(r) * top_k;
  for (int i = threadIdx.x; i < kk; i += blockDim.x) out[i] = KeyPage(keys[i]);
  if (threadIdx.x == 0) counts[r] = kk;
}

// ---------------------------------------------------------------------------
// 2b. Certified top-k select.
//
// Candidates are sorted by (interval midpoint desc, id asc).  With T the
// first k, a candidate needs its exact score only if its interval overlaps
// another relevant one: an outsider whose hi reaches min(lo over T), or a
// member of T whose interval meets an outsider's or another member's.  Every
// other comparison is already decided by disjoint intervals, so replacing the
// flagged candidates' keys by their exact scores and sorting again yields the
// reference order exactly.  Exact scores come from the reference's sequential
// chain (RescoreChains: the lanes of wave 0 run the dependent adds of up to
// 32 pages while the other waves form the next stretch of products).
// ---------------------------------------------------------------------------
constexpr int kCertMaxKeys = 2048;   // next-pow2 candidates per request
constexpr int kSelRescoreGroup = 32;  // exact chains per rescore group (lanes of wave 0)
constexpr int kSelThreads = 1024;    // one compare-exchange per thread per stage at 2048 keys

// Radix select of the kk-th largest 64-bit key among keys[0, n): 8 bits a
// round from the top, stopping as soon as the boundary bucket holds exactly
// the members still needed.  On return *shift is the last round's shift,
// *prefix the kept bucket's key bits above it, *need how many keys of that
// bucket are members and *all whether they all are (need == bucket size).
// Keys above the bucket (key >> shift > prefix) are members.  Whole
// workgroup; hist is 256 ints of LDS.
__device__ void RadixSelectKth(const uint64_t* keys, int n, int kk, int* hist,
                               unsigned long long* s_prefix, int* s_need, int* s_all,
                               int* shift_out, uint64_t* prefix_out, int* need_out,
                               bool* all_out) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  uint64_t prefix = 0;
  int need = kk;
  int shift = 56;
  bool all = false;
  for (int round = 0; round < 8; ++round) {
    shift = 56 - 8 * round;
    for (int b = threadIdx.x; b < 256; b += kSelThreads) hist[b] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += kSelThreads) {
      const uint64_t key = keys[i];
      if (round == 0 || (key >> (shift + 8)) == prefix) {
        atomicAdd(&hist[static_cast<int>((key >> shift) & 255u)], 1);
      }
    }
    __syncthreads();
    if (wave == 0) {
      // Lane l holds bins 4l .. 4l+3; suffix sums from the top bin down find
      // the bucket b with sum(bins > b) < need <= sum(bins >= b).
      const int b0 = 4 * lane;
      const int c3 = hist[b0 + 3], c2 = hist[b0 + 2], c1 = hist[b0 + 1], c0 = hist[b0];
      int suffix = c0 + c1 + c2 + c3;  // becomes the sum over lanes >= l
      for (int o = 1; o < kWave; o <<= 1) {
        const int other = __shfl_down(suffix, o, kWave);
        if (lane + o < kWave) suffix += other;
      }
      int above = __shfl_down(suffix, 1, kWave);  // sum over lanes > l
      if (lane == kWave - 1) above = 0;
      if (suffix >= need && above < need) {
        int b = b0 + 3;
        int count = c3;
        if (above + c3 < need) { above += c3; b = b0 + 2; count = c2;
          if (above + c2 < need) { above += c2; b = b0 + 1; count = c1;
            if (above + c1 < need) { above += c1; b = b0; count = c0; } } }
        *s_prefix = (static_cast<unsigned long long>(prefix) << 8) | static_cast<unsigned>(b);
        *s_need = need - above;
        *s_all = count == need - above;
      }
    }
    __syncthreads();
    prefix = *s_prefix;
    need = *s_need;
    all = *s_all != 0;
    __syncthreads();  // the next round rewrites hist and the shared words
    if (all) break;
  }
  *shift_out = shift;
  *prefix_out = prefix;
  *need_out = need;
  *all_out = all;
}

// (key, idx) pairs [0, count) into out_keys / out_idx in descending key
// order, by counting: rank(i) = #{j : key_j > key_i} + #{j < i : key_j ==
// key_i} (a permutation even with equal keys).  Cheaper than a bitonic sort
// for the few dozen members (no stage chain); O(count^2) work in all.  Whole
// workgroup; the outputs are complete after the closing barrier.
__device__ void RankSortDesc(const uint64_t* keys, const int* idx, int count,
                             uint64_t* out_keys, int* out_idx) {
  for (int i = threadIdx.x; i < count; i += kSelThreads) {
    const uint64_t key = keys[i];
    int rank = 0;
    int j = 0;
    for (; j + 8 <= count; j += 8) {
      uint64_t kj[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) kj[u] = keys[j + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) rank += (kj[u] > key) | ((kj[u] == key) & (j + u < i));
    }
    for (; j < count; ++j) {
      const uint64_t kj = keys[j];
      rank += (kj > key) | ((kj == key) & (j < i));
    }
    out_keys[rank] = key;
    out_idx[rank] = idx[i];
  }
  __syncthreads();
}

// The LDS of one request's certified select (kSelThreads threads).
struct CertShared {
  uint64_t keys[kCertMaxKeys];   // by candidate
  float s_lo[kCertMaxKeys];
  float s_hi[kCertMaxKeys];
  uint8_t member[kCertMaxKeys];  // by candidate
  uint64_t skeys[kCertMaxKeys];  // the members, then the final set, sorted
  int sidx[kCertMaxKeys];
  int flagged[kCertMaxKeys];
  int hist[256];
  alignas(16) float tile[RescoreFloats<kSelRescoreGroup>()];
  float s_red[2][kSelThreads / kWave];
  unsigned long long s_prefix;
  int s_need, s_all, s_count, s_tie, s_nflag, s_bad;
};

// Request r's certified top-k (up to kCertMaxKeys candidates, the whole
// workgroup of kSelThreads threads).  load(c, &mid, &lo, &hi) gives candidate
// c's first-pass interval (c indexes the batch's CSR); with kPolled it may
// report that an interval never became readable (false), and the request
// then selects nothing (kFailWait).  emit(i, page) writes member i of the
// selection (rank order), emit_count(kk) the count; emit_count runs once, in
// thread 0, after the emits.
template <bool kPolled, class Load, class Emit, class EmitCount>
__device__ __forceinline__ void SelectCertifiedRequest(
    CertShared& sh, int r, Load load, Emit emit, EmitCount emit_count,
    const float* __restrict__ queries, const float* __restrict__ summaries,
    const int* __restrict__ token_counts, int capacity, const int* __restrict__ cand_offsets,
    const int* __restrict__ cand_ids, int total, int max_candidates, int E, float scale,
    int top_k, int* __restrict__ exact_pages, FailReport fail) {
  uint64_t* keys = sh.keys;
  float* s_lo = sh.s_lo;
  float* s_hi = sh.s_hi;
  uint8_t* member = sh.member;
  uint64_t* skeys = sh.skeys;
  int* sidx = sh.sidx;
  int* flagged = sh.flagged;
  int* hist = sh.hist;
  float* tile = sh.tile;
  float (&s_red)[2][kSelThreads / kWave] = sh.s_red;
  unsigned long long& s_prefix = sh.s_prefix;
  int& s_need = sh.s_need;
  int& s_all = sh.s_all;
  int& s_count = sh.s_count;
  int& s_tie = sh.s_tie;
  int& s_nflag = sh.s_nflag;
  int begin, n;
  RequestRange(cand_offsets, r, total, fail, &begin, &n);
  if (n > max_candidates || n > kCertMaxKeys) {
    // Only max_candidates were scored (and this kernel holds kCertMaxKeys):
    // select nothing and report it.
    if (threadIdx.x == 0) ReportFailure(fail, kFailShape);
    n = 0;
  }
  const int kk = top_k <= 0 ? 0 : (top_k < n ? top_k : n);
  if (kk == 0) {
    if (threadIdx.x == 0) emit_count(0);
    return;
  }
  const int* cand = cand_ids + begin;
  if constexpr (kPolled) {
    if (threadIdx.x == 0) sh.s_bad = 0;
    __syncthreads();
  }
  for (int i = threadIdx.x; i < n; i += kSelThreads) {
    float m, l, h;
    if (!load(begin + i, &m, &l, &h)) sh.s_bad = 1;
    keys[i] = SelectKey(m, cand[i]);
    s_lo[i] = l;
    s_hi[i] = h;
  }
  if (threadIdx.x == 0) {
    s_count = 0;
    s_tie = 0;
    s_nflag = 0;
  }
  __syncthreads();
  if constexpr (kPolled) {
    if (sh.s_bad != 0) {
      if (threadIdx.x == 0) {
        ReportFailure(fail, kFailWait);
        emit_count(0);
      }
      return;
    }
  }

  const int wave = threadIdx.x / kWave;
  constexpr int nwaves = kSelThreads / kWave;
  uint64_t* tkeys = reinterpret_cast<uint64_t*>(tile);
  int* tidx = reinterpret_cast<int*>(tile + 2 * kCertMaxKeys);
  // Pass 0 certifies with the score kernel's intervals; the candidates it
  // flags get refined intervals (RefineScores, several waves per page; E a
  // multiple of 256) and pass 1 selects and certifies again.  What pass 1
  // leaves open gets the exact chain (step 3).
  for (int pass = 0; pass < 2; ++pass) {
    // 1. The members: the kk largest keys (equal keys are the same page listed
    //    twice, so which of them counts is immaterial).
    int shift;
    uint64_t prefix;
    int need;
    bool all;
    RadixSelectKth(keys, n, kk, hist, &s_prefix, &s_need, &s_all, &shift, &prefix, &need, &all);
    // The members, unordered, into the rescoring tile (idle until step 3),
    // then in key order into skeys / sidx.
    for (int i = threadIdx.x; i < n; i += kSelThreads) {
      const uint64_t top = keys[i] >> shift;
      bool in = top > prefix;
      if (top == prefix) in = all || atomicAdd(&s_tie, 1) < need;
      member[i] = in ? 1 : 0;
      if (in) {
        const int pos = atomicAdd(&s_count, 1);
        tkeys[pos] = keys[i];
        tidx[pos] = i;
      }
    }
    __syncthreads();
    RankSortDesc(tkeys, tidx, kk, skeys, sidx);

    // 2. Certification.  Member intervals in rank order go to the rescoring
    //    tile (idle until step 3): mlo = tile[0, kk), mhi = tile[kk, 2kk).
    float* mlo = tile;
    float* mhi = tile + kCertMaxKeys;
    float my_min = INFINITY, my_max = -INFINITY;
    for (int t = threadIdx.x; t < kk; t += kSelThreads) {
      const int c = sidx[t];
      mlo[t] = s_lo[c];
      mhi[t] = s_hi[c];
      my_min = fminf(my_min, s_lo[c]);
    }
    for (int i = threadIdx.x; i < n; i += kSelThreads) {
      if (!member[i]) my_max = fmaxf(my_max, s_hi[i]);
    }
    for (int o = 1; o < kWave; o <<= 1) {
      my_min = fminf(my_min, __shfl_xor(my_min, o, kWave));
      my_max = fmaxf(my_max, __shfl_xor(my_max, o, kWave));
    }
    if ((threadIdx.x & (kWave - 1)) == 0) {
      s_red[0][wave] = my_min;
      s_red[1][wave] = my_max;
    }
    __syncthreads();
    float min_t_lo = INFINITY, max_o_hi = -INFINITY;
    for (int w = 0; w < nwaves; ++w) {
      min_t_lo = fminf(min_t_lo, s_red[0][w]);
      max_o_hi = fmaxf(max_o_hi, s_red[1][w]);
    }
    // An outsider is flagged when its hi reaches the members' smallest lo; a
    // member when its lo reaches the outsiders' largest hi or its interval
    // meets another member's.
    for (int i = threadIdx.x; i < n; i += kSelThreads) {
      if (!member[i] && s_hi[i] >= min_t_lo) flagged[atomicAdd(&s_nflag, 1)] = i;
    }
    for (int t = threadIdx.x; t < kk; t += kSelThreads) {
      const float l = mlo[t];
      const float h = mhi[t];
      bool flag = l <= max_o_hi;
      // Eight independent reads per round (an early exit would serialise them).
      for (int u0 = 0; u0 < kk && !flag; u0 += 8) {
  #pragma unroll
        for (int v = 0; v < 8; ++v) {
          const int u = u0 + v;
          const bool in = u < kk;
          const float lu = in ? mlo[u] : INFINITY;
          const float hu = in ? mhi[u] : -INFINITY;
          flag |= (u != t) & (l <= hu) & (lu <= h);
        }
      }
      if (flag) flagged[atomicAdd(&s_nflag, 1)] = sidx[t];
    }
    __syncthreads();
    if (s_nflag == 0 || pass == 1 || E % 256 != 0 || !RefineWorthwhile<kSelThreads>(s_nflag)) break;
    RefineScores<kSelThreads>(
        s_nflag,
        [&](int f) -> const float* {
          const int pg = cand[flagged[f]];
          const bool live = pg >= 0 && pg < capacity && token_counts[pg] != 0;
          return live ? summaries + static_cast<size_t>(pg) * E : nullptr;
        },
        [&](int f) {
          const int c = flagged[f];
          return dsd_refine::FirstPassBound(s_lo[c], s_hi[c], scale, E);
        },
        [&](int f, float m, float l, float h) {
          const int c = flagged[f];
          // LDS only: the global intervals stay the score kernel's
          // first-pass ones, which a later select over the same buffers
          // (a stage replay) needs for FirstPassBound's precondition.
          keys[c] = SelectKey(m, cand[c]);
          s_lo[c] = l;
          s_hi[c] = h;
        },
        queries + static_cast<size_t>(r) * E, E, scale, reinterpret_cast<double*>(tile));
    if (threadIdx.x == 0) {
      s_count = 0;
      s_tie = 0;
      s_nflag = 0;
    }
    __syncthreads();
  }
  const int nflag = s_nflag;
  if (nflag > 0) {
    // 3. Exact chains for the flagged candidates, then the final order over
    //    the members and the flagged outsiders: every other outsider's hi
    //    is below every member's lo, so it cannot enter the top kk.
    if (threadIdx.x == 0 && exact_pages != nullptr) atomicAdd(exact_pages, nflag);
    RescoreChains<kSelRescoreGroup, kSelThreads>(
        nflag, [&](int f) { return cand[flagged[f]]; },
        [&](int f, float score) {
          const int c = flagged[f];
          keys[c] = SelectKey(score, cand[c]);
        },
        queries + static_cast<size_t>(r) * E, summaries, token_counts, capacity, E, scale, tile);
    if (threadIdx.x == 0) s_count = kk;
    __syncthreads();
    for (int t = threadIdx.x; t < kk; t += kSelThreads) skeys[t] = keys[sidx[t]];
    for (int f = threadIdx.x; f < nflag; f += kSelThreads) {
      const int c = flagged[f];
      if (!member[c]) {
        const int pos = atomicAdd(&s_count, 1);
        skeys[pos] = keys[c];
        sidx[pos] = c;
      }
    }
    __syncthreads();
    RankSortDesc(skeys, sidx, s_count, tkeys, tidx);
  }
  const uint64_t* final_keys = nflag > 0 ? tkeys : skeys;
  for (int i = threadIdx.x; i < kk; i += kSelThreads) emit(i, KeyPage(final_keys[i]));
  if constexpr (kPolled) __syncthreads();  // every member out before the count
  if (threadIdx.x == 0) emit_count(kk);
}

__global__ __launch_bounds__(kSelThreads) void SelectCertifiedKernel(
    const float* __restrict__ mid, const float* __restrict__ lo,
    const float* __restrict__ hi, const float* __restrict__ queries,
    const float* __restrict__ summaries, const int* __restrict__ token_counts, int capacity,
    const int* __restrict__ cand_offsets, const int* __restrict__ cand_ids, int total,
    int max_candidates, int E, float scale, int top_k, int* __restrict__ selected,
    int* __restrict__ counts, int* __restrict__ exact_pages, FailReport fail) {
  __shared__ CertShared sh;
  const int r = blockIdx.x;
  int* out = selected + static_cast<size_t>(r) * top_k;
  SelectCertifiedRequest<false>(
      sh, r,
      [&](int c, float* m, float* l, float* h) {
        *m = mid[c];
        *l = lo[c];
        *h = hi[c];
        return true;
      },
      [&](int i, int page) { out[i] = page; }, [&](int kk) { counts[r] = kk; }, queries,
      summaries, token_counts, capacity, cand_offsets, cand_ids, total, max_candidates, E,
      scale, top_k, exact_pages, fail);
}

// Certified select for up to 256 candidates per request: thread i owns
// candidate i and finds its rank by counting larger keys (broadcast LDS reads,
// no barrier chain), ties broken by position so ranks are distinct.
constexpr int kRankMax = 256;

__global__ __launch_bounds__(kRankMax) void SelectCertifiedRankKernel(
    const float* __restrict__ mid, const float* __restrict__ lo,
    const float* __restrict__ hi, const float* __restrict__ queries,
    const float* __restrict__ summaries, const int* __restrict__ token_counts, int capacity,
    const int* __restrict__ cand_offsets, const int* __restrict__ cand_ids, int total,
    int max_candidates, int E, float scale, int top_k, int* __restrict__ selected,
    int* __restrict__ counts, int* __restrict__ exact_pages, FailReport fail) {
  __shared__ uint64_t s_key[kRankMax];
  __shared__ float s_lo[kRankMax];
  __shared__ float s_hi[kRankMax];
  __shared__ int s_top[kRankMax];
  __shared__ int s_flag[kRankMax];
  __shared__ float s_red[2][kRankMax / kWave];
  __shared__ int s_nflag;
  __shared__ __align__(16) float tile[RescoreFloats<kSelRescoreGroup>()];
  const int r = blockIdx.x;
  int begin, n;
  RequestRange(cand_offsets, r, total, fail, &begin, &n);
  if (n > max_candidates || n > kRankMax) {
    // Only max_candidates were scored (and this kernel holds kRankMax):
    // select nothing and report it.
    if (threadIdx.x == 0) ReportFailure(fail, kFailShape);
    n = 0;
  }
  const int kk = top_k <= 0 ? 0 : (top_k < n ? top_k : n);
  if (kk == 0) {
    if (threadIdx.x == 0) counts[r] = 0;
    return;
  }
  const int i = threadIdx.x;
  const bool active = i < n;
  if (active) {
    s_key[i] = SelectKey(mid[begin + i], cand_ids[begin + i]);
    s_lo[i] = lo[begin + i];
    s_hi[i] = hi[begin + i];
  }
  if (i == 0) s_nflag = 0;
  __syncthreads();
  // Keys are read 8 at a time (independent broadcast LDS reads in flight).
  auto rank_of = [&](int me) {
    const uint64_t key = s_key[me];
    int rank = 0;
    int j = 0;
    for (; j + 8 <= n; j += 8) {
      uint64_t kj[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) kj[u] = s_key[j + u];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        rank += (kj[u] > key || (kj[u] == key && j + u < me)) ? 1 : 0;
      }
    }
    for (; j < n; ++j) {
      const uint64_t kj = s_key[j];
      rank += (kj > key || (kj == key && j < me)) ? 1 : 0;
    }
    return rank;
  };
  const int wave = threadIdx.x / kWave;
  constexpr int nwaves = kRankMax / kWave;
  const int* cand = cand_ids + begin;
  int rank = n;
  int nflag = 0;
  // Pass 0 certifies with the score kernel's intervals; pages it leaves
  // open get refined intervals (RefineScores, several waves per page; E a
  // multiple of 256) and pass 1 certifies again.  What pass 1 leaves open
  // gets the exact chain.
  for (int pass = 0; pass < 2; ++pass) {
    rank = active ? rank_of(i) : n;
    if (active && rank < kk) s_top[rank] = i;
    float my_min = (active && rank < kk) ? s_lo[i] : INFINITY;
    float my_max = (active && rank >= kk) ? s_hi[i] : -INFINITY;
    for (int o = 1; o < kWave; o <<= 1) {
      my_min = fminf(my_min, __shfl_xor(my_min, o, kWave));
      my_max = fmaxf(my_max, __shfl_xor(my_max, o, kWave));
    }
    if ((threadIdx.x & (kWave - 1)) == 0) {
      s_red[0][wave] = my_min;
      s_red[1][wave] = my_max;
    }
    __syncthreads();
    float min_t_lo = INFINITY, max_o_hi = -INFINITY;
    for (int w = 0; w < nwaves; ++w) {
      min_t_lo = fminf(min_t_lo, s_red[0][w]);
      max_o_hi = fmaxf(max_o_hi, s_red[1][w]);
    }
    if (active) {
      const float l = s_lo[i];
      const float h = s_hi[i];
      bool flag;
      if (rank >= kk) {
        flag = h >= min_t_lo;
      } else {
        flag = l <= max_o_hi;
        for (int j = 0; j < kk && !flag; ++j) {
          if (j == rank) continue;
          const int c2 = s_top[j];
          flag = l <= s_hi[c2] && s_lo[c2] <= h;
        }
      }
      if (flag) s_flag[atomicAdd(&s_nflag, 1)] = i;
    }
    __syncthreads();
    nflag = s_nflag;
    if (nflag == 0 || pass == 1 || E % 256 != 0 || !RefineWorthwhile<kRankMax>(nflag)) break;
    RefineScores<kRankMax>(
        nflag,
        [&](int f) -> const float* {
          const int pg = cand[s_flag[f]];
          const bool live = pg >= 0 && pg < capacity && token_counts[pg] != 0;
          return live ? summaries + static_cast<size_t>(pg) * E : nullptr;
        },
        [&](int f) {
          const int c = s_flag[f];
          return dsd_refine::FirstPassBound(s_lo[c], s_hi[c], scale, E);
        },
        [&](int f, float m, float l, float h) {
          const int c = s_flag[f];
          // LDS only (see SelectCertifiedKernel).
          s_key[c] = SelectKey(m, cand[c]);
          s_lo[c] = l;
          s_hi[c] = h;
        },
        queries + static_cast<size_t>(r) * E, E, scale, reinterpret_cast<double*>(tile));
    if (i == 0) s_nflag = 0;
    __syncthreads();
  }
  if (nflag > 0) {
    if (threadIdx.x == 0 && exact_pages != nullptr) atomicAdd(exact_pages, nflag);
    RescoreChains<kSelRescoreGroup, kRankMax>(
        nflag, [&](int f) { return cand[s_flag[f]]; },
        [&](int f, float score) {
          const int c = s_flag[f];
          s_key[c] = SelectKey(score, cand[c]);
        },
        queries + static_cast<size_t>(r) * E, summaries, token_counts, capacity, E, scale, tile);
    rank = active ? rank_of(i) : n;
  }
  if (active && rank < kk) selected[static_cast<size_t>(r) * top_k + rank] = cand_ids[begin + i];
  if (threadIdx.x == 0) counts[r] = kk;
}

// ---------------------------------------------------------------------------
// 3. Fused gather + softmax attention (flash-decoding inside a workgroup).
//
// Workgroup = (head h, request r); its waves stride over 16-token chunks of
// the request's page list.  Lane (g, j) = (lane/4, lane%4) owns token slot g
// of the chunk and the j-th quarter of the head's dims, so a 4-lane group
// reads one 4*DQ-float K row and one V row (contiguous, vectorised).  Each
// lane keeps its own online-softmax stream (m, l, acc[DQ]) over the tokens
// it sees: the only per-token cross-lane traffic is the 2-step dot-product
// reduction within the group.  Streams are merged once at the end: across
// the 16 token slots with xor shuffles, across waves through LDS.  Logits
// live in the log2 domain (q pre-scaled by scale*log2 e) so each exponential
// is one v_exp_f32.
// ---------------------------------------------------------------------------
constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kChunk = 16;
// DQ > 0: head_dim == 4*DQ, lane j covers dims [j*DQ, (j+1)*DQ).
// DQ == 0: generic head_dim <= 256, lane j covers dims j, j+4, j+8, ...
template <int DQ>
__global__ __launch_bounds__(kAttnThreads) void AttentionKernel(
    PoolView pool, AttentionArgs args) {
  constexpr int kRegs = DQ > 0 ? DQ : 64;
  const int h = blockIdx.x;
  const int r = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int g = lane >> 2;
  const int j = lane & 3;
  const int D = pool.head_dim;
  const int E = pool.elements;
  const int ps = pool.page_size;

  int start, count;
  if (args.list_stride > 0) {
    start = r * args.list_stride;
    count = args.list_counts[r];
  } else {
    start = args.list_offsets[r];
    count = args.list_offsets[r + 1] - start;
  }

  const int nd = DQ > 0 ? DQ : (D - j + 3) / 4;
  const int dim0 = DQ > 0 ? j * DQ : j;
  const int dstep = DQ > 0 ? 1 : 4;
  const int head_off = h * D + dim0;

  float q[kRegs];
  float acc[kRegs];
  {
    const float qscale = args.scale * kLog2e;
    const float* qp = args.queries + static_cast<size_t>(r) * E + head_off;
    if constexpr (DQ > 0) {
      LoadDims<DQ>(qp, q);
    } else {
#pragma unroll
      for (int i = 0; i < kRegs; ++i) q[i] = i < nd ? qp[i * dstep] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kRegs; ++i) {
      q[i] *= qscale;
      acc[i] = 0.0f;
    }
  }

  float m = -INFINITY;
  float l = 0.0f;
  const int total = count * ps;
  for (int base = wave * kChunk; base < total; base += kAttnWaves * kChunk) {
    const int f = base + g;
    bool valid = false;
    float kv[kRegs];
    float vv[kRegs];
    if (f < total) {
      const int slot = f / ps;
      const int t = f - slot * ps;
      const int page = args.list_ids[start + slot];
      valid = InPool(page, pool.capacity) && t < pool.token_counts[page];
      if (valid) {
        const size_t off = static_cast<size_t>(page) * pool.page_elems +
                           static_cast<size_t>(t) * E + head_off;
        if constexpr (DQ > 0) {
          LoadDims<DQ>(pool.keys + off, kv);
          LoadDims<DQ>(pool.values + off, vv);
        } else {
#pragma unroll
          for (int i = 0; i < kRegs; ++i) {
            kv[i] = i < nd ? pool.keys[off + i * dstep] : 0.0f;
            vv[i] = i < nd ? pool.values[off + i * dstep] : 0.0f;
          }
        }
      }
    }
    float dot = 0.0f;
    if (valid) {
#pragma unroll
      for (int i = 0; i < kRegs; ++i) dot = fmaf(q[i], kv[i], dot);
    }
    dot += __shfl_xor(dot, 1, kWave);
    dot += __shfl_xor(dot, 2, kWave);
    if (valid) {
      const float m_new = fmaxf(m, dot);
      const float alpha = Exp2(m - m_new);
      const float beta = Exp2(dot - m_new);
      l = fmaf(l, alpha, beta);
#pragma unroll
      for (int i = 0; i < kRegs; ++i) acc[i] = fmaf(acc[i], alpha, beta * vv[i]);
      m = m_new;
    }
  }

  // Merge the 16 token-slot streams of this wave (lanes differing in g).
  float wm = m;
#pragma unroll
  for (int o = 4; o < kWave; o <<= 1) wm = fmaxf(wm, __shfl_xor(wm, o, kWave));
  const float sc = (m == -INFINITY) ? 0.0f : Exp2(m - wm);
  float wl = l * sc;
#pragma unroll
  for (int i = 0; i < kRegs; ++i) acc[i] *= sc;
#pragma unroll
  for (int o = 4; o < kWave; o <<= 1) {
    wl += __shfl_xor(wl, o, kWave);
#pragma unroll
    for (int i = 0; i < kRegs; ++i) acc[i] += __shfl_xor(acc[i], o, kWave);
  }

  // Merge the waves through LDS: s_acc[wave][D], s_m/s_l[wave].
  extern __shared__ float smem[];
  float* s_m = smem;
  float* s_l = smem + kAttnWaves;
  float* s_acc = smem + 2 * kAttnWaves;
  if (g == 0) {
    if (j == 0) {
      s_m[wave] = wm;
      s_l[wave] = wl;
    }
#pragma unroll
    for (int i = 0; i < kRegs; ++i) {
      if (i < nd) s_acc[wave * D + dim0 + i * dstep] = acc[i];
    }
  }
  __syncthreads();
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) mx = fmaxf(mx, s_m[w]);
  float* out = args.outputs + static_cast<size_t>(r) * E + static_cast<size_t>(h) * D;
  for (int d = threadIdx.x; d < D; d += kAttnThreads) {
    float lt = 0.0f;
    float at = 0.0f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) {
        const float s = (s_m[w] == -INFINITY) ? 0.0f : Exp2(s_m[w] - mx);
        lt = fmaf(s_l[w], s, lt);
        at = fmaf(s_acc[w * D + d], s, at);
      }
    }
    // No valid token at all: the reference returns zeros
    // (src/cuda/sparse_batched_attention.cu:364-369; CPU :159-161).
    out[d] = lt == 0.0f ? 0.0f : at / lt;
  }
}

// Fixed-D variant for the hot shape (D = 128) with the lane split, the
// waves per workgroup and the chunks in flight per wave as parameters:
// LPT lanes per token (each owns D/LPT contiguous dims), 64/LPT tokens per
// chunk, UNROLL chunks whose K and V rows are all requested before any is
// consumed (bytes in flight per wave = UNROLL * 64/LPT * 2 * D * 4).
template <int WAVES, int D>
struct AttnFastShared {
  float m[WAVES];
  float l[WAVES];
  alignas(16) float acc[WAVES][D];
};

// Head h of request r over the `count` pages of `list` (global or LDS), by
// WAVES waves whose thread index within the head is tid; ends with a
// workgroup barrier (every thread of the workgroup must call it).
template <int D, int LPT, int WAVES, int UNROLL, class List>
__device__ __forceinline__ void AttentionFastHead(const PoolView& pool, const AttentionArgs& args,
                                                  int h, int r, int tid, List list, int count,
                                                  AttnFastShared<WAVES, D>& sh) {
  constexpr int DQ = D / LPT;
  constexpr int TPC = kWave / LPT;
  static_assert(DQ % 4 == 0, "float4 rows");
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int g = lane / LPT;
  const int j = lane % LPT;
  const int E = pool.elements;
  const int ps = pool.page_size;
  const int head_off = h * D + j * DQ;
  float q[DQ];
  float acc[DQ];
  {
    const float qscale = args.scale * kLog2e;
    LoadDims<DQ>(args.queries + static_cast<size_t>(r) * E + head_off, q);
#pragma unroll
    for (int i = 0; i < DQ; ++i) {
      q[i] *= qscale;
      acc[i] = 0.0f;
    }
  }
  float m = -INFINITY;
  float l = 0.0f;
  const int total = count * ps;
  for (int base = wave * TPC * UNROLL; base < total; base += WAVES * TPC * UNROLL) {
    float kv[UNROLL][DQ];
    float vv[UNROLL][DQ];
    bool valid[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int f = base + u * TPC + g;
      valid[u] = false;
      if (f < total) {
        const int slot = f / ps;
        const int t = f - slot * ps;
        const int page = list[slot];
        valid[u] = InPool(page, pool.capacity) && t < pool.token_counts[page];
        if (valid[u]) {
          const size_t off = static_cast<size_t>(page) * pool.page_elems +
                             static_cast<size_t>(t) * E + head_off;
          LoadDims<DQ>(pool.keys + off, kv[u]);
          LoadDims<DQ>(pool.values + off, vv[u]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      float dot = 0.0f;
      if (valid[u]) {
#pragma unroll
        for (int i = 0; i < DQ; ++i) dot = fmaf(q[i], kv[u][i], dot);
      }
#pragma unroll
      for (int o = 1; o < LPT; o <<= 1) dot += __shfl_xor(dot, o, kWave);
      if (valid[u]) {
        const float m_new = fmaxf(m, dot);
        const float alpha = Exp2(m - m_new);
        const float beta = Exp2(dot - m_new);
        l = fmaf(l, alpha, beta);
#pragma unroll
        for (int i = 0; i < DQ; ++i) acc[i] = fmaf(acc[i], alpha, beta * vv[u][i]);
        m = m_new;
      }
    }
  }
  // merge the TPC token-slot streams of this wave
  float wm = m;
#pragma unroll
  for (int o = LPT; o < kWave; o <<= 1) wm = fmaxf(wm, __shfl_xor(wm, o, kWave));
  const float sc = (m == -INFINITY) ? 0.0f : Exp2(m - wm);
  float wl = l * sc;
#pragma unroll
  for (int i = 0; i < DQ; ++i) acc[i] *= sc;
#pragma unroll
  for (int o = LPT; o < kWave; o <<= 1) {
    wl += __shfl_xor(wl, o, kWave);
#pragma unroll
    for (int i = 0; i < DQ; ++i) acc[i] += __shfl_xor(acc[i], o, kWave);
  }
  float* s_m = sh.m;
  float* s_l = sh.l;
  float (&s_acc)[WAVES][D] = sh.acc;
  if (g == 0) {
    if (j == 0) {
      s_m[wave] = wm;
      s_l[wave] = wl;
    }
#pragma unroll
    for (int i = 0; i < DQ; ++i) s_acc[wave][j * DQ + i] = acc[i];
  }
  __syncthreads();
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) mx = fmaxf(mx, s_m[w]);
  float* out = args.outputs + static_cast<size_t>(r) * E + static_cast<size_t>(h) * D;
  for (int d = tid; d < D; d += WAVES * kWave) {
    float lt = 0.0f;
    float at = 0.0f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < WAVES; ++w) {
        const float sw = (s_m[w] == -INFINITY) ? 0.0f : Exp2(s_m[w] - mx);
        lt = fmaf(s_l[w], sw, lt);
        at = fmaf(s_acc[w][d], sw, at);
      }
    }
    out[d] = lt == 0.0f ? 0.0f : at / lt;
  }
}

template <int D, int LPT, int WAVES, int UNROLL>
__global__ __launch_bounds__(WAVES * kWave) void AttentionFastKernel(
    PoolView pool, AttentionArgs args) {
  __shared__ AttnFastShared<WAVES, D> sh;
  const int r = blockIdx.y;
  int start, count;
  if (args.list_stride > 0) {
    start = r * args.list_stride;
    count = args.list_counts[r];
  } else {
    start = args.list_offsets[r];
    count = args.list_offsets[r + 1] - start;
  }
  AttentionFastHead<D, LPT, WAVES, UNROLL>(pool, args, blockIdx.x, r, threadIdx.x,
                                           args.list_ids + start, count, sh);
}


// ---------------------------------------------------------------------------
// 4. The wide step: the three-kernel step (E = 4096, head_dim 128, up to
// kCertMaxKeys candidates per request) in one launch.
//
// Items: score slices (request r, slice x: candidates [P*x, P*x + P), G
// slices per request) and attention items (request r, head h).  The
// workgroup that scores a request's last slice (an arrival counter per
// request) runs that request's certified select.  Every score slice comes
// before every attention item (WideItemOf with lag = batch): an attention
// item dispatched in the first round would hold its CU from the launch on
// while it waits for its select (at 32 requests of 2048 pages the step
// spanned 379 us with all slices first, 427-489 us with 4 to 16 requests'
// slices between a request's slices and its attention).  HBM streams K/V
// for the requests selected first while the others still score and select:
// the stages of different requests overlap instead of running one after
// another with HBM idle between them (reference: the score -> top-k ->
// attention sequence of src/cuda/sparse_batched_attention.cu:665-762 and
// its k > 16 path, :703-731).
//
// Tickets.  A workgroup takes the next item from a counter as it starts,
// and the grid holds half as many spare workgroups again, which find the
// items gone and leave.  Workgroup i goes to XCD i mod
// 8 and each XCD runs its own share of the grid: with items tied to
// workgroup ids, the XCDs whose CUs ran the selects (each holds its CU for
// about 47 us) finished up to 25 us after the others; with tickets an XCD
// that frees up early takes more items (config 3: 381 against 395 us per
// step; spares of 1 and 2 per item measured 383 and 388 us).
//
// Intervals, selected ids and counts cross workgroups as epoch-tagged
// words (score_slice.h): no fences.
//
// Every wait ends.  A score slice never waits; the select that follows a
// request's last slice waits only for interval words that the request's
// slices wrote before they arrived.  An attention item waits for its
// request's select, that is for score slices with lower tickets, which
// workgroups already running took: they finish without waiting, the last
// of them runs the select, and the select ends.  (Without tickets, the
// lowest-id attention item that waits has, on every XCD, only score slices
// and attention items that do not wait forever ahead of it in dispatch
// order, and the same follows.)  The polls are bounded anyway (kFailWait,
// zero outputs, never a hang).  The ticket and arrival counters come in two
// sets that launches use in turn; workgroup 0 of each launch zeroes the set
// the next launch will use (the previous launch used it and has finished),
// so no workgroup waits at the end to reset anything and a spare leaves
// after one load.
//
// A persistent form (one workgroup per CU taking items from a counter)
// spilled 188 bytes per lane: values the compiler hoisted out of the item
// loop stay live across all three item kinds.
// ---------------------------------------------------------------------------
constexpr int kWideStamps = 5;  // per item in timing mode

// An attention item is one head of one request, all kFWaves waves on it,
// with the lane split of the three-kernel step's attention for the same
// batches (kWideAttnLpt, kWideAttnUnroll; LaunchAttention with
// wide_partition): both step forms give bit-identical outputs.  Two heads
// per item (8 waves each) measured 10 us slower at 32 requests of 2048
// pages: the attention of the requests selected last ends later.
constexpr int kWideAttnLpt = 16;
constexpr int kWideAttnUnroll = 4;

struct WideShared {
  union {
    ScoreShared score;
    CertShared cert;
    AttnFastShared<kFWaves, 128> attn;
  };
  int page[kCertMaxKeys];  // an attention item's selected pages
  int item;
  int last;
  int count;
  unsigned long long stamp[3];  // timing mode: start, select start and end
};

// A tagged word once it carries `tag` (spin_limit polls, sleeping between),
// or false.
__device__ __forceinline__ bool AwaitTagged(unsigned long long* p, unsigned tag,
                                            unsigned spin_limit, unsigned long long* out) {
  unsigned long long w = LoadWord(p);
  for (unsigned i = 0; static_cast<unsigned>(w >> 32) != tag; ++i) {
    if (i >= spin_limit) return false;
    __builtin_amdgcn_s_sleep(1);
    w = LoadWord(p);
  }
  *out = w;
  return true;
}

// Item i's kind (0 score slice, 1 attention), request and slice or head:
// request r's G slices, then (for r >= lag) request r - lag's Q heads,
// request by request; after the last request the remaining lag requests'
// heads.  (lag = batch: all slices, then all heads; DSD_WIDE_LAG.)
__device__ __forceinline__ int WideItemOf(int i, int batch, int G, int Q, int lag, int* r,
                                          int* sub) {
  const int head = lag * G;
  if (i < head) {
    *r = i / G;
    *sub = i - *r * G;
    return 0;
  }
  const int block = G + Q;
  const int j = (i - head) / block;
  if (j < batch - lag) {
    const int off = i - head - j * block;
    if (off < G) {
      *r = lag + j;
      *sub = off;
      return 0;
    }
    *r = j;
    *sub = off - G;
    return 1;
  }
  const int t = i - head - (batch - lag) * block;
  *r = batch - lag + t / Q;
  *sub = t - (t / Q) * Q;
  return 1;
}

// Item `item` of the step (WideItemOf), by the whole workgroup.
__device__ __forceinline__ void WideStepItem(const PoolView& pool, const WideArgs& w, int item,
                                             WideShared& sh) {
  const FusedArgs& a = w.a;
  const int stride = a.sel_stride;
  int item_r, item_sub;
  const int kind =
      WideItemOf(item, a.batch, w.groups, pool.num_heads, w.lag, &item_r, &item_sub);
  // Timing mode: thread 0's clocks (start, select start and end, end) and
  // the item kind, written out at the end.
  // (kept in LDS: a register would stay live across the whole item)
  if (a.stamps != nullptr && threadIdx.x == 0) {
    sh.stamp[0] = wall_clock64();
    sh.stamp[1] = 0;
    sh.stamp[2] = 0;
  }
  if (kind == 0) {
    const int r = item_r;
    const int x = item_sub;
    int begin, n;
    if (RequestRange(a.cand_offsets, r, a.total, x == 0 ? a.fail : FailReport{}, &begin, &n)) {
      const int c0 = x * w.pages_per_group;
      if (c0 < n) {
        const int c1 = n - c0 < w.pages_per_group ? n : c0 + w.pages_per_group;
        ScoreSlice<true>(pool, a, r, begin + c0, begin + c1, sh.score);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      const unsigned prev = __hip_atomic_fetch_add(w.counters + 1 + r, 1u, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
      sh.last = prev == static_cast<unsigned>(w.groups - 1) ? 1 : 0;
    }
    __syncthreads();
    if (sh.last != 0) {
      if (a.stamps != nullptr && threadIdx.x == 0) sh.stamp[1] = wall_clock64();
      unsigned long long* sel = w.sel_rec + static_cast<size_t>(r) * stride;
      int* out = a.selected + static_cast<size_t>(r) * stride;
      SelectCertifiedRequest<true>(
          sh.cert, r,
          [&](int c, float* m, float* l, float* h) {
            unsigned long long* p = a.rec + 3 * static_cast<size_t>(c);
            unsigned long long w0 = 0, w1 = 0, w2 = 0;
            const bool ok = AwaitTagged(p, a.wait_tag, a.spin_limit, &w0) &&
                            AwaitTagged(p + 1, a.wait_tag, a.spin_limit, &w1) &&
                            AwaitTagged(p + 2, a.wait_tag, a.spin_limit, &w2);
            *m = __uint_as_float(static_cast<uint32_t>(w0));
            *l = __uint_as_float(static_cast<uint32_t>(w1));
            *h = __uint_as_float(static_cast<uint32_t>(w2));
            return ok;
          },
          [&](int i, int page) {
            out[i] = page;
            PutTagged(sel + i, a.epoch, static_cast<uint32_t>(page));
          },
          [&](int kk) {
            a.counts[r] = kk;
            PutTagged(w.cnt_rec + r, a.epoch, static_cast<uint32_t>(kk));
          },
          a.queries, pool.summaries, pool.token_counts, pool.capacity, a.cand_offsets,
          a.cand_ids, a.total, a.max_candidates, pool.elements, a.scale, a.top_k,
          a.exact_pages, a.fail);
      if (a.stamps != nullptr && threadIdx.x == 0) sh.stamp[2] = wall_clock64();
    }
  } else {
    const int r = item_r;
    const int head = item_sub;
    unsigned long long* sel = w.sel_rec + static_cast<size_t>(r) * stride;
    // Each thread reads its id word along with thread 0's read of the count:
    // when the select finished before this item started (most items), the
    // ids arrive in the same round trip; a word not yet current is polled
    // below.
    const unsigned long long early =
        static_cast<int>(threadIdx.x) < stride ? LoadWord(sel + threadIdx.x) : 0ull;
    if (threadIdx.x == 0) {
      unsigned long long word = 0;
      int count = 0;
      if (AwaitTagged(w.cnt_rec + r, a.wait_tag, a.spin_limit, &word)) {
        count = static_cast<int>(static_cast<uint32_t>(word));
      } else {
        ReportFailure(a.fail, kFailWait);
      }
      sh.count = count < stride ? count : stride;
    }
    __syncthreads();
    const int count = sh.count;
    for (int i = threadIdx.x; i < count; i += kFThreads) {
      unsigned long long word = i == static_cast<int>(threadIdx.x) ? early : 0ull;
      int page = -1;  // never attended (InPool fails)
      if (static_cast<unsigned>(word >> 32) == a.wait_tag ||
          AwaitTagged(sel + i, a.wait_tag, a.spin_limit, &word)) {
        page = static_cast<int>(static_cast<uint32_t>(word));
      } else {
        ReportFailure(a.fail, kFailWait);
      }
      sh.page[i] = page;
    }
    __syncthreads();
    AttentionArgs args;
    args.queries = a.queries;
    args.scale = a.scale;
    args.outputs = a.outputs;
    AttentionFastHead<128, kWideAttnLpt, kFWaves, kWideAttnUnroll>(
        pool, args, head, r, threadIdx.x, sh.page, count, sh.attn);
  }
  if (a.stamps != nullptr && threadIdx.x == 0) {
    unsigned long long* st = a.stamps + static_cast<size_t>(kWideStamps) * item;
    st[0] = sh.stamp[0];
    st[1] = static_cast<unsigned long long>(kind) | (static_cast<unsigned long long>(item_r) << 8) |
            (static_cast<unsigned long long>(blockIdx.x) << 32);
    st[2] = sh.stamp[1];
    st[3] = sh.stamp[2];
    st[4] = wall_clock64();
  }
}

// One thread advances a captured wide step's epoch (as EpochBumpKernel:
// within [2^30, 2^31)) and its launch count (the parity picks the counter
// set).
__global__ void WideBumpKernel(unsigned* epoch, unsigned* seq) {
  if (threadIdx.x == 0) {
    *epoch = ((*epoch + 1u) & 0x3FFFFFFFu) | 0x40000000u;
    *seq = *seq + 1u;
  }
}

__global__ __launch_bounds__(kFThreads) void WideStepKernel(PoolView pool, WideArgs w) {
  __shared__ WideShared sh;
  if (w.a.epoch_src != nullptr) {
    // Replayed from a captured graph: the epoch and the counter set that
    // the bump kernel just before this launch advanced.
    w.a.epoch = *w.a.epoch_src;
    w.a.wait_tag = w.a.epoch | w.a.wait_mask;
    w.a.fail.epoch = w.a.epoch;
    const unsigned n = *w.seq_src;
    w.counters = w.capture_counters + (n & 1u) * static_cast<size_t>(w.counter_words);
    w.next_counters = w.capture_counters + ((n + 1u) & 1u) * static_cast<size_t>(w.counter_words);
  }
  if (blockIdx.x == 0) {
    // Zero the other counter set for the next launch (the launch before
    // this one used it and has finished).
    for (int t = static_cast<int>(threadIdx.x); t < w.counter_words; t += kFThreads) {
      __hip_atomic_store(w.next_counters + t, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  int item = static_cast<int>(blockIdx.x);
  if (w.tickets) {
    if (threadIdx.x == 0) {
      // A spare workgroup that starts after every item was taken sees so
      // with a load and leaves without touching the counter.
      unsigned t = static_cast<unsigned>(w.items);
      if (__hip_atomic_load(w.counters, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
          static_cast<unsigned>(w.items)) {
        t = __hip_atomic_fetch_add(w.counters, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      sh.item = t < static_cast<unsigned>(w.items) ? static_cast<int>(t) : w.items;
    }
    __syncthreads();
    item = sh.item;
  }
  if (item < w.items) WideStepItem(pool, w, item, sh);
}

using AttnKernelFn = void (*)(PoolView, AttentionArgs);

struct AttnVariant {
  int lpt, waves, unroll;
  AttnKernelFn fn;
};

#define DSD_ATTN_VARIANT(L, W, U) \
  AttnVariant{L, W, U, AttentionFastKernel<128, L, W, U>}
const AttnVariant kAttnVariants[] = {
    DSD_ATTN_VARIANT(4, 4, 1),  DSD_ATTN_VARIANT(4, 4, 2),  DSD_ATTN_VARIANT(4, 8, 1),
    DSD_ATTN_VARIANT(8, 4, 1),  DSD_ATTN_VARIANT(8, 4, 2),  DSD_ATTN_VARIANT(8, 4, 4),
    DSD_ATTN_VARIANT(8, 8, 1),  DSD_ATTN_VARIANT(8, 8, 2),  DSD_ATTN_VARIANT(16, 4, 2),
    DSD_ATTN_VARIANT(16, 4, 4), DSD_ATTN_VARIANT(16, 8, 2), DSD_ATTN_VARIANT(16, 8, 4),
    DSD_ATTN_VARIANT(16, 16, 4),
};
#undef DSD_ATTN_VARIANT

// The D = 128 variant in use: DSD_ATTN_VARIANT="LPTxWAVESxUNROLL" selects
// one of kAttnVariants (a tuning knob); otherwise the measured default.
const AttnVariant& SelectAttnVariant() {
  int lpt = 16, waves = 8, unroll = 4;
  if (const char* env = std::getenv("DSD_ATTN_VARIANT")) {
    int a = 0, b = 0, c = 0;
    if (std::sscanf(env, "%dx%dx%d", &a, &b, &c) == 3) {
      lpt = a;
      waves = b;
      unroll = c;
    }
  }
  for (const auto& v : kAttnVariants) {
    if (v.lpt == lpt && v.waves == waves && v.unroll == unroll) return v;
  }
  throw std::invalid_argument("unknown DSD_ATTN_VARIANT");
}

template <int DQ>
void LaunchAttentionT(const PoolView& pool, const AttentionArgs& args,
                      hipStream_t stream) {
  const size_t lds = sizeof(float) * (2 * kAttnWaves + kAttnWaves * pool.head_dim);
  hipLaunchKernelGGL(AttentionKernel<DQ>, dim3(pool.num_heads, args.batch),
                     dim3(kAttnThreads), lds, stream, pool, args);
}

}  // namespace

void LaunchScoreExact(const PoolView& pool, const float* d_queries,
                      const int* d_cand_offsets, const int* d_cand_ids,
                      int batch, int total_candidates, int max_candidates, float scale,
                      float* d_scores, FailReport fail, hipStream_t stream) {
  if (batch <= 0 || max_candidates <= 0) return;
  const dim3 grid((max_candidates + kWave - 1) / kWave, batch);
  if (pool.elements % 4 == 0) {
    hipLaunchKernelGGL(ScoreExactKernel<true>, grid, dim3(kWave), 0, stream,
                       d_queries, pool.summaries, pool.token_counts, pool.capacity,
                       d_cand_offsets, d_cand_ids, total_candidates, pool.elements, scale,
                       d_scores, fail);
  } else {
    hipLaunchKernelGGL(ScoreExactKernel<false>, grid, dim3(kWave), 0, stream,
                       d_queries, pool.summaries, pool.token_counts, pool.capacity,
                       d_cand_offsets, d_cand_ids, total_candidates, pool.elements, scale,
                       d_scores, fail);
  }
  DSD_HIP_CHECK(hipGetLastError());
}

bool CertifiedScoringSupported(int elements, int max_candidates) {
  int m = 1;
  while (m < max_candidates) m <<= 1;
  return elements % kWave == 0 && elements >= kWave && m <= kCertMaxKeys;
}

void LaunchScoreBounds(const PoolView& pool, const float* d_queries,
                       const int* d_cand_offsets, const int* d_cand_ids, int batch,
                       int total_candidates, int max_candidates, float scale, float* d_mid,
                       float* d_lo, float* d_hi, FailReport fail, hipStream_t stream) {
  if (batch <= 0 || max_candidates <= 0) return;
  const dim3 grid((max_candidates + kBoundWaves - 1) / kBoundWaves, batch);
  const dim3 block(kBoundWaves * kWave);
  if (pool.elements == 4096) {
    // The fused step's float score passes, 8..128 pages per workgroup.
    LaunchScorePages(pool, d_queries, d_cand_offsets, d_cand_ids, batch, total_candidates,
                     max_candidates, scale, d_mid, d_lo, d_hi, fail, stream);
    return;
  } else {
    hipLaunchKernelGGL(ScoreBoundGenericKernel, grid, block, 0, stream, d_queries,
                       pool.summaries, pool.token_counts, pool.capacity, d_cand_offsets,
                       d_cand_ids, total_candidates, pool.elements, scale, d_mid, d_lo, d_hi,
                       fail);
  }
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchSelectCertified(const PoolView& pool, const float* d_mid, const float* d_lo,
                           const float* d_hi,
                           const float* d_queries,
                           const int* d_cand_offsets, const int* d_cand_ids, int batch,
                           int total_candidates, int max_candidates, float scale, int top_k,
                           int* d_selected, int* d_counts, int* d_exact_pages, FailReport fail,
                           hipStream_t stream) {
  if (batch <= 0) return;
  if (max_candidates <= kRankMax) {
    // Always four waves: three of them form products while wave 0 runs the
    // exact chains.
    hipLaunchKernelGGL(SelectCertifiedRankKernel, dim3(batch), dim3(kRankMax), 0, stream,
                       d_mid, d_lo, d_hi, d_queries, pool.summaries, pool.token_counts,
                       pool.capacity, d_cand_offsets, d_cand_ids, total_candidates,
                       max_candidates, pool.elements, scale, top_k, d_selected, d_counts,
                       d_exact_pages, fail);
    DSD_HIP_CHECK(hipGetLastError());
    return;
  }
  int m = 1;
  while (m < max_candidates) m <<= 1;
  if (m > kCertMaxKeys) {
    throw std::invalid_argument("certified select supports up to " +
                                std::to_string(kCertMaxKeys) + " candidates per request");
  }
  if (pool.elements % kWave != 0) {
    throw std::invalid_argument("certified select needs E % 64 == 0");
  }
  hipLaunchKernelGGL(SelectCertifiedKernel, dim3(batch), dim3(kSelThreads), 0, stream, d_mid,
                     d_lo, d_hi, d_queries, pool.summaries, pool.token_counts, pool.capacity,
                     d_cand_offsets, d_cand_ids, total_candidates, max_candidates,
                     pool.elements, scale, top_k, d_selected, d_counts, d_exact_pages, fail);
  DSD_HIP_CHECK(hipGetLastError());
}

int SelectMaxCandidates() { return kSelectMaxKeys; }

bool WideStepSupported(const PoolView& pool, int max_candidates, int top_k) {
  return pool.elements == kFE && pool.head_dim == 128 &&
         pool.page_size > 0 && max_candidates > 0 && max_candidates <= kCertMaxKeys &&
         top_k <= kCertMaxKeys;
}

int WideStepMaxCandidates() { return kCertMaxKeys; }

int WideStepStampsPerGroup() { return kWideStamps; }

int WideStepItems(const PoolView& pool, int batch, int groups) {
  return batch * groups + batch * pool.num_heads;
}

int WideStepGrid(int items, bool tickets) { return tickets ? items + items / 2 : items; }

void LaunchWideStep(const PoolView& pool, const WideArgs& w, hipStream_t stream) {
  if (w.a.batch <= 0) return;
  if (!WideStepSupported(pool, w.a.max_candidates, w.a.top_k)) {
    throw std::invalid_argument("the wide step needs E = 4096, head_dim 128 and at most 2048 "
                                "candidates per request");
  }
  if (w.pages_per_group <= 0 || w.pages_per_group % kFPagesPerPass != 0 ||
      static_cast<long long>(w.groups) * w.pages_per_group < w.a.max_candidates) {
    throw std::invalid_argument("wide step slices do not cover max_candidates");
  }
  if (w.a.rec == nullptr || w.sel_rec == nullptr || w.cnt_rec == nullptr ||
      w.counters == nullptr || w.next_counters == nullptr || w.counter_words < w.a.batch + 1 ||
      w.a.sel_stride < (w.a.top_k > 0 ? w.a.top_k : 1)) {
    throw std::invalid_argument("wide step scratch missing");
  }
  if (w.a.epoch_src != nullptr) {
    if (w.seq_src == nullptr || w.capture_counters == nullptr) {
      throw std::invalid_argument("a captured wide step needs its device launch count");
    }
    hipLaunchKernelGGL(WideBumpKernel, dim3(1), dim3(kWave), 0, stream,
                       const_cast<unsigned*>(w.a.epoch_src), w.seq_src);
    DSD_HIP_CHECK(hipGetLastError());
  }
  if (w.items != WideStepItems(pool, w.a.batch, w.groups)) {
    throw std::invalid_argument("wide step item count does not match its slices");
  }
  const int grid = WideStepGrid(w.items, w.tickets);
  hipLaunchKernelGGL(WideStepKernel, dim3(grid), dim3(kFThreads), 0, stream, pool, w);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchSelectTopK(const float* d_scores, const int* d_cand_offsets,
                      const int* d_cand_ids, int batch, int total_candidates,
                      int max_candidates, int top_k, int* d_selected, int* d_counts,
                      FailReport fail, hipStream_t stream) {
  if (batch <= 0) return;
  int m = 1;
  while (m < max_candidates) m <<= 1;
  if (m > kSelectMaxKeys) {
    throw std::invalid_argument(
        "candidate pages per request exceed the top-k select limit of " +
        std::to_string(kSelectMaxKeys));
  }
  int threads = m / 2;
  if (threads < kWave) threads = kWave;
  if (threads > 256) threads = 256;
  hipLaunchKernelGGL(SelectTopKKernel, dim3(batch), dim3(threads),
                     sizeof(uint64_t) * static_cast<size_t>(m), stream, d_scores,
                     d_cand_offsets, d_cand_ids, total_candidates, max_candidates, top_k,
                     d_selected, d_counts, fail);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchAttention(const PoolView& pool, const AttentionArgs& args,
                     hipStream_t stream) {
  if (args.batch <= 0 || pool.num_heads <= 0) return;
  const int D = pool.head_dim;
  if (D <= 0 || D > 256) {
    throw std::invalid_argument("head_dim must be in (0, 256]");
  }
  if (D == 128 && args.wide_partition && pool.elements == kFE) {
    // the wide step's partition of a head (kFWaves waves)
    hipLaunchKernelGGL((AttentionFastKernel<128, kWideAttnLpt, kFWaves, kWideAttnUnroll>),
                       dim3(pool.num_heads, args.batch), dim3(kFThreads), 0, stream, pool, args);
    DSD_HIP_CHECK(hipGetLastError());
    return;
  }
  if (D == 128) {
    const AttnVariant& v = SelectAttnVariant();
    hipLaunchKernelGGL(v.fn, dim3(pool.num_heads, args.batch), dim3(v.waves * kWave), 0,
                       stream, pool, args);
    DSD_HIP_CHECK(hipGetLastError());
    return;
  }
  switch (D % 4 == 0 ? D / 4 : 0) {
    case 1: LaunchAttentionT<1>(pool, args, stream); break;
    case 2: LaunchAttentionT<2>(pool, args, stream); break;
    case 4: LaunchAttentionT<4>(pool, args, stream); break;
    case 8: LaunchAttentionT<8>(pool, args, stream); break;
    case 16: LaunchAttentionT<16>(pool, args, stream); break;
    case 20: LaunchAttentionT<20>(pool, args, stream); break;
    case 32: LaunchAttentionT<32>(pool, args, stream); break;
    case 64: LaunchAttentionT<64>(pool, args, stream); break;
    default: LaunchAttentionT<0>(pool, args, stream); break;
  }
  DSD_HIP_CHECK(hipGetLastError());
}

void PreloadStepKernels() {
  PreloadKernel(WideStepKernel);
  PreloadKernel(WideBumpKernel);
  PreloadKernel(AttentionFastKernel<128, kWideAttnLpt, kFWaves, kWideAttnUnroll>);
  PreloadKernel(SelectAttnVariant().fn);
  PreloadKernel(SelectCertifiedKernel);
  PreloadKernel(SelectCertifiedRankKernel);
  PreloadKernel(ScoreBoundGenericKernel);
}

}  // namespace dsdk
