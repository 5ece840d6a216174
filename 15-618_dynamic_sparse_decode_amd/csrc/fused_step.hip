// fused_step.hip -- the whole sparse decode step in one launch (gfx950).
//
// For the hot shape (E = 4096, head_dim 128, at most 256 candidates and
// top_k <= 256 per request, certified selection) the three stages of the
// step -- page scoring (reference ScorePagesCpu, src/reference_kernels.cpp:
// 59-80), top-k (SelectTopKPagesCpu, :82-107) and gather + attention
// (GatherPagesCpu + SparseAttentionCpu, :109-194) -- run in one kernel, so the
// step pays one launch and no kernel boundary between dependent stages.
//
// Work items.  Request r owns the G = H/hpw consecutive workgroups
// [r*G, r*G + G); workgroup (r, g) takes heads hpw*g .. hpw*g + hpw - 1,
// where hpw (1, 2, 4 or 8 heads per workgroup) is the fewest that keeps the
// grid within one dispatch wave (B*H/hpw <= CUs) when that is possible.
// Each does:
//   1. score: the certified intervals of its slice of the request's
//      candidates, [n*g/G, n*(g+1)/G), eight pages per pass, two waves per
//      page, published as tagged words (below); when some slice spans
//      several passes the launch uses FusedStepKernel<true>, whose passes
//      load the next pass's rows while they reduce;
//   2. select: waits until every interval of its request is published,
//      then computes the request's top-k from them (the G workgroups
//      compute the same selection; g = 0 writes it out);
//   3. attend: 16/hpw waves per head over the selected pages.
// Workgroups have 1024 threads (one per CU at this kernel's register use),
// so the whole step is one dispatch wave whenever B*H/8 <= the CU count.
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
// Publication without fences.  Each interval crosses workgroups as three
// 64-bit words (mid, lo, hi) whose high half is this launch's epoch (a
// per-context counter, never 0) and whose low half is the float: written
// with relaxed agent-scope atomic stores, read with relaxed agent-scope
// atomic loads until the epoch matches.  A word is valid exactly when its
// tag is current, so no ordering between words is needed and there is no
// release/acquire (each would write back or invalidate the XCD's L2).  Wave
// 0 of each workgroup polls its request's words directly (a cached read
// first, then coherent re-reads of the words whose tag is not yet current,
// with a short sleep between rounds) and shares them through LDS.
#include "dsd_internal.h"
#include "step_common.h"
#include "score_slice.h"

namespace dsdk {
namespace {

constexpr int kFD = 128;
constexpr int kFMaxHeadsPerGroup = 8;       // workgroup = 1, 2, 4 or 8 heads (16/hpw waves each)
constexpr int kFMaxCand = 256;
constexpr int kFMaxK = 256;
constexpr int kFLpt = 16;                 // lanes per token row (8 dims each)
constexpr int kFDq = kFD / kFLpt;         // 8
constexpr int kFTpc = kWave / kFLpt;      // 4 token rows per wave per chunk
constexpr int kFUnroll = 4;               // chunks in flight per wave
constexpr int kFSlots = kFMaxCand / kWave;  // candidates (or ranks) per lane: l + 64m
constexpr int kFRescoreGroup = 16;            // exact chains per rescore group
static_assert(kFMaxK <= kFMaxCand, "rank slots cover the candidate slots");
// Timing mode: per-workgroup wall clocks at start, slice scored, counter
// ready, records read, ranked, selected, end, refinement begun and ended
// (0 when none ran); then the hardware ids.
constexpr int kStampsPerGroup = 10;
enum Stamp { kStart, kScored, kReady, kRecords, kRanked, kSelected, kEnd, kRefine, kRefined, kHwId };

struct FusedShared {
  uint64_t stamp[kStampsPerGroup];  // timing mode: thread 0's clocks
  // score pass (per wave): float total (the carry into wave 2p+1) and the
  // bound sums
  float wave_total[2][kFWaves];  // [pass parity]: a pass's leader reads its
  float abs_prefix[2][kFWaves];  // sums after the pass's last barrier, while
  float abs_p[2][kFWaves];       // the next pass may already write its own
  int fail;
  int nflag;
  int certified;  // FastSelect's verdict, for every wave
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
  alignas(16) float tile[RescoreFloats<kFRescoreGroup>()];  // exact rescore; the staged query before
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

// Ranks of the n <= 256 keys in sh.key (descending; equal keys by position):
// kTpc threads per candidate count interleaved slices of the keys
// (candidate j is read by part j % kTpc: contiguous LDS words per
// instruction) and add their counts with shuffles.  Returns the rank to the
// candidate's first thread (part 0), n elsewhere.  No barrier.
constexpr int kTpc = 4;
// Every candidate below kFMaxCand has a lead thread.
static_assert(kFThreads / kTpc >= kFMaxCand, "PartialRanks must cover kFMaxCand");

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

// Ranks of the keys into sh.rank (whole workgroup; ends with a barrier).
__device__ void ParallelRanks(FusedShared& sh, int n) {
  int cand;
  const int rank = PartialRanks(sh, n, &cand);
  if (rank < n) sh.rank[cand] = rank;
  __syncthreads();
}

// ---- selection helpers: wave scans with identities (lanes with no source
// keep the identity) -----------------------------------------------------------
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ float DppOr(float x, float identity) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(identity), __float_as_int(x),
                                                    kCtrl, kRowMask, 0xf, false));
}
constexpr int kRowShl1 = 0x101, kRowShl2 = 0x102, kRowShl4 = 0x104, kRowShl8 = 0x108;
constexpr int kWaveShl1 = 0x130;

__device__ __forceinline__ float ReadLane(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

// Inclusive minimum over lanes 0..l.
__device__ __forceinline__ float WaveMinPrefix(float x) {
  x = fminf(x, DppOr<kRowShr1>(x, INFINITY));
  x = fminf(x, DppOr<kRowShr2>(x, INFINITY));
  x = fminf(x, DppOr<kRowShr4>(x, INFINITY));
  x = fminf(x, DppOr<kRowShr8>(x, INFINITY));
  x = fminf(x, DppOr<kRowBcast15, 0xa>(x, INFINITY));
  x = fminf(x, DppOr<kRowBcast31, 0xc>(x, INFINITY));
  return x;
}

// Inclusive maximum over lanes l..63: within each row of 16 by row shifts
// toward lane 0, then the rows above through their first lanes.
__device__ __forceinline__ float WaveMaxSuffix(float x) {
  x = fmaxf(x, DppOr<kRowShl1>(x, -INFINITY));
  x = fmaxf(x, DppOr<kRowShl2>(x, -INFINITY));
  x = fmaxf(x, DppOr<kRowShl4>(x, -INFINITY));
  x = fmaxf(x, DppOr<kRowShl8>(x, -INFINITY));
  const float r3 = ReadLane(x, 48);
  const float r2 = fmaxf(ReadLane(x, 32), r3);
  const float r1 = fmaxf(ReadLane(x, 16), r2);
  const int row = (threadIdx.x & (kWave - 1)) >> 4;
  const float above = row == 0 ? r1 : (row == 1 ? r2 : (row == 2 ? r3 : -INFINITY));
  return fmaxf(x, above);
}

__device__ __forceinline__ float WaveMax(float x) { return ReadLane(WaveMaxSuffix(x), 0); }

__device__ __forceinline__ int Popc(uint64_t m) { return __popcll(m); }

// Steps 2 and 3 of SelectForRequest for CS candidate slots and RS rank slots
// (compile-time counts, so the slot loops are straight-line code).  Reads the
// intervals from LDS, ranks, certifies; when some order is undecided, wave 0
// also lists the flagged candidates and all keys for the exact path.
// Returns whether anything is flagged (the same in every wave).
template <int CS, int RS>
__device__ bool RankAndCertify(const FusedArgs& a, int n, int kk, const int (&page)[kFSlots],
                               const int (&ntok)[kFSlots], FusedShared& sh) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  float mid[CS], lo[CS], hi[CS];
#pragma unroll
  for (int m = 0; m < CS; ++m) {
    const int i = lane + kWave * m;  // < kFMaxCand: the LDS reads stay in bounds
    const bool in = i < n;
    const float x = sh.mid[i], l = sh.lo[i], h = sh.hi[i];
    // Midpoints are finite; -inf marks the empty slots.
    mid[m] = in ? x : -INFINITY;
    lo[m] = in ? l : INFINITY;
    hi[m] = in ? h : -INFINITY;
  }
  // 2. ranks: wave w ranks candidate i = 64m + l for l = w + 16q and keeps
  // the rank in lane l (a uniform loop: ballots need every lane).
  int my_rank[CS];
#pragma unroll
  for (int m = 0; m < CS; ++m) {
    my_rank[m] = n;
#pragma unroll
    for (int q = 0; q < kWave / kFWaves; ++q) {
      const int l = wave + kFWaves * q;
      const int i = kWave * m + l;
      const float s_mid = ReadLane(mid[m], l);
      int above = 0, equal = 0;
#pragma unroll
      for (int m2 = 0; m2 < CS; ++m2) {
        above += Popc(__ballot(mid[m2] > s_mid));
        equal += Popc(__ballot(mid[m2] == s_mid));
      }
      if (equal > 1) {
        // Equal midpoints (rare): order them by (page id, position).
        const int s_page = __builtin_amdgcn_readlane(page[m], l);
#pragma unroll
        for (int m2 = 0; m2 < CS; ++m2) {
          const int j = kWave * m2 + lane;
          const bool tie_before = (mid[m2] == s_mid) &
                                  ((page[m2] < s_page) | ((page[m2] == s_page) & (j < i)));
          above += Popc(__ballot(tie_before));
        }
      }
      my_rank[m] = (lane == l && i < n) ? above : my_rank[m];
    }
  }
#pragma unroll
  for (int m = 0; m < CS; ++m) {
    const int i = lane + kWave * m;
    if ((lane & (kFWaves - 1)) == wave && i < n) {
      const int rank = my_rank[m];
      sh.rank[i] = rank;
      if (rank < kk) {
        sh.page[rank] = page[m];
        sh.ntok[rank] = ntok[m];
        sh.tlo[rank] = lo[m];
        sh.thi[rank] = hi[m];
        sh.top[rank] = i;
      }
    }
  }
  __syncthreads();
  StampAt(a, sh, kRanked);
  // 3. certification (every wave, same result)
  float max_o_hi = -INFINITY;
  bool outsider[CS];
#pragma unroll
  for (int m = 0; m < CS; ++m) {
    const int i = lane + kWave * m;
    const int rank = sh.rank[i];
    outsider[m] = (i < n) & (rank >= kk);
    max_o_hi = fmaxf(max_o_hi, outsider[m] ? hi[m] : -INFINITY);
  }
  max_o_hi = WaveMax(max_o_hi);
  // The members in rank order: rank t = lane + 64m.
  float tlo[RS], thi[RS], pmin[RS], smax[RS];
#pragma unroll
  for (int m = 0; m < RS; ++m) {
    const int t = lane + kWave * m;
    const float l = sh.tlo[t], h = sh.thi[t];
    tlo[m] = t < kk ? l : INFINITY;
    thi[m] = t < kk ? h : -INFINITY;
  }
  float carry = INFINITY;  // min lo over the ranks of the slots before
#pragma unroll
  for (int m = 0; m < RS; ++m) {
    const float incl = fminf(WaveMinPrefix(tlo[m]), carry);
    pmin[m] = DppOr<kWaveShr1>(incl, carry);  // every rank below t
    carry = ReadLane(incl, kWave - 1);
  }
  const float min_t_lo = carry;
  carry = -INFINITY;  // max hi over the ranks of the slots after
#pragma unroll
  for (int m = RS - 1; m >= 0; --m) {
    const float incl = fmaxf(WaveMaxSuffix(thi[m]), carry);
    smax[m] = DppOr<kWaveShl1>(incl, carry);  // every rank above t
    carry = ReadLane(incl, 0);
  }
  uint64_t oflag[CS], mflag[CS];
  bool any = false;
#pragma unroll
  for (int m = 0; m < CS; ++m) {
    oflag[m] = __ballot(outsider[m] & (hi[m] >= min_t_lo));
    mflag[m] = 0;
    if (m < RS) {
      const int t = lane + kWave * m;
      mflag[m] = __ballot((t < kk) & ((tlo[m] <= max_o_hi) | (pmin[m] <= thi[m]) |
                                      (smax[m] >= tlo[m])));
    }
    any = any || oflag[m] != 0 || mflag[m] != 0;
  }
  if (any && wave == 0) {
    const uint64_t below = (1ull << lane) - 1ull;
    int base = 0;
#pragma unroll
    for (int m = 0; m < CS; ++m) {
      const int i = lane + kWave * m;
      if ((oflag[m] >> lane) & 1ull) sh.flag[base + Popc(oflag[m] & below)] = i;
      base += Popc(oflag[m]);
      if ((mflag[m] >> lane) & 1ull) sh.flag[base + Popc(mflag[m] & below)] = sh.top[i];
      base += Popc(mflag[m]);
      if (i < n) {
        sh.key[i] = SelectKey(mid[m], page[m]);
        sh.cpage[i] = page[m];
        sh.cntok[i] = ntok[m];
      }
    }
    if (lane == 0) sh.nflag = base;
  }
  return any;
}

// ---- selection for small k (kk <= kFFastK): one wave, kk rounds ----------
// The ballot ranks of RankAndCertify rank all n candidates with every wave;
// for a few members it is shorter for one wave to take the best remaining
// candidate kk times.  Same order (midpoint descending, then page id
// ascending, then position) and the same certification, so the result is
// the one RankAndCertify would give.
constexpr int kFFastK = 32;

__device__ __forceinline__ uint32_t OrderBits(float x) {
  return static_cast<uint32_t>(SelectKey(x, 0) >> 32);
}

// x from a DPP source lane; lanes with no source (or outside kRowMask) read
// 0, the identity of an unsigned maximum.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ uint32_t DppU32(uint32_t x) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(x), kCtrl, kRowMask, 0xf, false));
}

// Maximum over the wave, in every lane.
__device__ __forceinline__ uint32_t WaveMaxU32(uint32_t x) {
  x = max(x, DppU32<kRowShr1>(x));
  x = max(x, DppU32<kRowShr2>(x));
  x = max(x, DppU32<kRowShr4>(x));
  x = max(x, DppU32<kRowShr8>(x));
  x = max(x, DppU32<kRowBcast15, 0xa>(x));
  x = max(x, DppU32<kRowBcast31, 0xc>(x));
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(x), kWave - 1));
}

// Wave 0 only.  Candidate i = lane + 64m (m < CS, i < n) has interval
// (mid, lo, hi)[m], the same values as sh.mid / sh.lo / sh.hi[i]; its page id
// and token count are in sh.cpage / sh.cntok.  Takes the best remaining
// candidate kk times: a round is a wave maximum of the midpoints' order bits,
// one ballot per slot and the winner's index kept in lane t, so it stays
// short and runs warm after the first (a first run of one-shot code pays for
// every instruction-cache line it touches, which dominates a round).  The
// members' intervals are then read once from LDS, lane t holding member t,
// for the certification.  Writes the members in rank order to sh.top
// (candidate index), sh.page and sh.ntok.  Returns 1 when the intervals
// certify the selection; 0 when they do not, after listing the flagged
// candidates in sh.flag / sh.nflag (an outsider whose hi reaches the
// members' smallest lo; a member whose lo reaches an outsider's hi or whose
// interval overlaps another member's) and writing every candidate's key to
// sh.key; -1 when a round's maximum is not unique (equal midpoints: the
// ballot ranks then order them).  Nothing else is written before a -1.
template <int CS>
__device__ int FastSelect(int n, int kk, const float (&mid)[kFSlots], const float (&hi)[kFSlots],
                          FusedShared& sh, bool dry) {
  const int lane = threadIdx.x & (kWave - 1);
  uint32_t kh[CS];  // order bits of the midpoint; 0: empty or taken
#pragma unroll
  for (int m = 0; m < CS; ++m) kh[m] = lane + kWave * m < n ? OrderBits(mid[m]) : 0u;
  int m_top = 0;     // lane t: candidate index of member t
  bool dup = false;  // some round's maximum was not unique
#pragma nounroll
  for (int t = 0; t < kk; ++t) {
    uint32_t x = kh[0];
#pragma unroll
    for (int m = 1; m < CS; ++m) x = max(x, kh[m]);
    const uint32_t best = WaveMaxU32(x);
    int count = 0;
    int winner = -1;
#pragma unroll
    for (int m = 0; m < CS; ++m) {
      const uint64_t b = __ballot(kh[m] == best);
      count += __popcll(b);
      winner = (winner < 0 && b != 0) ? kWave * m + __ffsll(static_cast<long long>(b)) - 1
                                      : winner;
    }
    dup = dup || count != 1;
    m_top = lane == t ? winner : m_top;
#pragma unroll
    for (int m = 0; m < CS; ++m) kh[m] = lane + kWave * m == winner ? 0u : kh[m];
  }
  if (dup) return -1;
  float m_lo = INFINITY, m_hi = -INFINITY;
  if (lane < kk) {
    if (dry) {
      // The warm-up: the members' intervals are the made-up midpoints.
      m_lo = m_hi = -static_cast<float>(m_top);
    } else {
      sh.top[lane] = m_top;
      sh.page[lane] = sh.cpage[m_top];
      sh.ntok[lane] = sh.cntok[m_top];
      m_lo = sh.lo[m_top];
      m_hi = sh.hi[m_top];
    }
  }
  float oh = -INFINITY;  // the outsiders' largest hi
#pragma unroll
  for (int m = 0; m < CS; ++m) oh = fmaxf(oh, kh[m] != 0u ? hi[m] : -INFINITY);
  const float max_o_hi = WaveMax(oh);
  const float min_lo = ReadLane(WaveMinPrefix(m_lo), kWave - 1);
  // Members in order: each one's lo above the next one's hi (lo <= hi, so
  // adjacent pairs decide every pair).
  const float next_hi = DppOr<kWaveShl1>(m_hi, -INFINITY);
  const bool ordered = __ballot(lane + 1 < kk && !(m_lo > next_hi)) == 0;
  if (ordered && max_o_hi < min_lo) return 1;
  if (dry) return 0;
  // Flags, as RankAndCertify's (members are lanes 0..kk-1 here).
  const float pmin = DppOr<kWaveShr1>(WaveMinPrefix(m_lo), INFINITY);   // members above
  const float smax = DppOr<kWaveShl1>(WaveMaxSuffix(m_hi), -INFINITY);  // members below
  const uint64_t mflag =
      __ballot(lane < kk && (m_lo <= max_o_hi || pmin <= m_hi || smax >= m_lo));
  const uint64_t below = (1ull << lane) - 1ull;
  int base = 0;
#pragma unroll
  for (int m = 0; m < CS; ++m) {
    const int i = lane + kWave * m;
    const uint64_t of = __ballot(kh[m] != 0u && hi[m] >= min_lo);
    if ((of >> lane) & 1ull) sh.flag[base + __popcll(of & below)] = i;
    base += __popcll(of);
    if (i < n) sh.key[i] = SelectKey(mid[m], sh.cpage[i]);
  }
  if ((mflag >> lane) & 1ull) sh.flag[base + __popcll(mflag & below)] = m_top;
  base += __popcll(mflag);
  if (lane == 0) sh.nflag = base;
  return 0;
}

__device__ __forceinline__ int FastSelectSlots(int n, int kk, const float (&mid)[kFSlots],
                                               const float (&hi)[kFSlots], FusedShared& sh,
                                               bool dry) {
  switch ((n + kWave - 1) / kWave) {
    case 1: return FastSelect<1>(n, kk, mid, hi, sh, dry);
    case 2: return FastSelect<2>(n, kk, mid, hi, sh, dry);
    case 3: return FastSelect<3>(n, kk, mid, hi, sh, dry);
    default: return FastSelect<4>(n, kk, mid, hi, sh, dry);
  }
}

// Top-k of request r (n candidates from `begin`) from the published
// intervals into sh.page / sh.ntok (rank order); returns the count (0 on
// failure).  The order is that of the (score desc, page id asc) key of the
// reference comparator; equal keys (a page listed twice) by position.
//   1. Every lane holds candidates l + 64m (id, token count); wave 0 polls
//      the interval words and shares them in LDS; one barrier.
//   2. Ranks by ballots: rank(i) = #{j : mid_j > mid_i} + #{j : mid_j ==
//      mid_i and (page_j, j) < (page_i, i)}.  Wave w ranks the candidates
//      whose lane is w mod 16 and writes the members' rank slots; one
//      barrier.
//   3. Certification, computed identically by every wave (no barrier): an
//      outsider is flagged when its hi reaches the members' smallest lo; a
//      member when its lo reaches the outsiders' largest hi, or when it
//      overlaps a member ranked above (prefix minimum of lo) or below
//      (suffix maximum of hi).  The members are in midpoint order, so these
//      cover every overlapping pair.
//   4. Only if some pair is flagged: those pages are rescored with the exact
//      sequential chain (as SelectCertifiedRankKernel) and ranked again.
// Workgroup `group` of the request's `groups` (group 0 also writes the
// selection out).
__device__ __forceinline__ int SelectForRequest(const PoolView& pool, const FusedArgs& a, int r, int begin,
                                int n, int group, int groups, FusedShared& sh) {
  const bool writer = group == 0;
  int kk = a.top_k <= 0 ? 0 : (a.top_k < n ? a.top_k : n);
  if (n > a.max_candidates || n > kFMaxCand) {
    // The caller's max_candidates understated the CSR: select nothing (the
    // outputs are zeros) and report it to the host.
    if (writer && threadIdx.x == 0) ReportFailure(a.fail, kFailShape);
    kk = 0;
  }
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  // Ids and token counts do not depend on the scores: every wave loads them
  // for all candidates first.  An id outside the pool keeps no tokens (the
  // score pass reported it).
  int page[kFSlots], ntok[kFSlots];
#pragma unroll
  for (int m = 0; m < kFSlots; ++m) {
    const int i = lane + kWave * m;
    page[m] = 0x7fffffff;
    ntok[m] = 0;
    if (kk > 0 && i < n) {
      page[m] = a.cand_ids[begin + i];
      if (page[m] >= 0 && page[m] < pool.capacity) ntok[m] = pool.token_counts[page[m]];
    }
  }
  if (threadIdx.x == 0) sh.fail = 0;
  if (wave == 0 && kk > 0) {
    // With FastSelect, two runs of one loop body (the same code, so not
    // inlined twice): run 0 selects one member from made-up distinct
    // intervals while the other slices finish, which brings FastSelect's
    // code into the instruction cache; it is a dry run (no LDS reads or
    // writes of candidate state, its verdict unused).  Run 1 waits for the
    // published intervals and selects.
    const bool fast = kk <= kFFastK;
    bool timed_out = false;
#pragma nounroll
    for (int run = fast ? 0 : 1; run < 2; ++run) {
      float mid[kFSlots], lo[kFSlots], hi[kFSlots];
      if (run == 1) {
        // First an ordinary (L2-cached) read; words whose tag is not current
        // (not yet visible, or a stale cached line) are then polled
        // coherently.
        unsigned long long w[kFSlots][3];
        bool ok = true;
#pragma unroll
        for (int m = 0; m < kFSlots; ++m) {
          const int i = lane + kWave * m;
          w[m][0] = w[m][1] = w[m][2] = static_cast<unsigned long long>(a.wait_tag) << 32;
          if (i < n) {
            const unsigned long long* rec = a.rec + 3 * static_cast<size_t>(begin + i);
            w[m][0] = rec[0];
            w[m][1] = rec[1];
            w[m][2] = rec[2];
            ok = ok && Current(w[m][0], a.wait_tag) && Current(w[m][1], a.wait_tag) &&
                 Current(w[m][2], a.wait_tag);
          }
        }
        unsigned spins = 0;
        while (__ballot(!ok) != 0) {
          if (++spins >= a.spin_limit) {
            if (lane == 0) sh.fail = 1;
            timed_out = true;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          ok = true;
#pragma unroll
          for (int m = 0; m < kFSlots; ++m) {
            const int i = lane + kWave * m;
            if (i < n) {
              unsigned long long* rec = a.rec + 3 * static_cast<size_t>(begin + i);
#pragma unroll
              for (int x = 0; x < 3; ++x) {
                if (!Current(w[m][x], a.wait_tag)) w[m][x] = LoadWord(rec + x);
              }
              ok = ok && Current(w[m][0], a.wait_tag) && Current(w[m][1], a.wait_tag) &&
                   Current(w[m][2], a.wait_tag);
            }
          }
        }
#pragma unroll
        for (int m = 0; m < kFSlots; ++m) {
          const int i = lane + kWave * m;
          mid[m] = __uint_as_float(static_cast<uint32_t>(w[m][0]));
          lo[m] = __uint_as_float(static_cast<uint32_t>(w[m][1]));
          hi[m] = __uint_as_float(static_cast<uint32_t>(w[m][2]));
          if (i < n) {
            sh.mid[i] = mid[m];
            sh.lo[i] = lo[m];
            sh.hi[i] = hi[m];
            sh.cpage[i] = page[m];
            sh.cntok[i] = ntok[m];
          }
        }
        StampAt(a, sh, kReady);
      } else {
#pragma unroll
        for (int m = 0; m < kFSlots; ++m) {
          mid[m] = lo[m] = hi[m] = -static_cast<float>(lane + kWave * m);
        }
      }
      if (fast && !timed_out) {
        const int verdict = FastSelectSlots(n, run == 1 ? kk : 1, mid, hi, sh, run == 0);
        if (run == 1 && lane == 0) sh.certified = verdict;
      }
    }
    if (fast) StampAt(a, sh, kRanked);
  }
  __syncthreads();
  StampAt(a, sh, kRecords);
  if (sh.fail) {
    if (threadIdx.x == 0) ReportFailure(a.fail, kFailWait);
    kk = 0;
  }
  if (kk > 0) {
    // The common case, FastSelect's intervals certified the selection
    // (sh.certified > 0, wave 0 wrote it before the barrier): nothing to
    // rank, refine or rescore.  It skips the block below, whose loop the
    // compiler prepares with a few hundred instructions of hoisted masks:
    // about 1 us, run cold, of every step that took them.
    const bool settled = kk <= kFFastK && sh.certified > 0;
    if (!settled) {
      // 2-3 with the slot counts fixed at compile time (straight-line code).
      const int cs = (n + kWave - 1) / kWave;    // candidate slots, 1..4
      const int rs = (kk + kWave - 1) / kWave;   // rank slots, 1..cs
      bool any = false;
      bool ballot = kk > kFFastK;  // the ballot ranks (every wave) or FastSelect
      for (int pass = 0; pass < 2; ++pass) {
        if (!ballot) {
          if (pass == 1) {
            // Select again from the refined intervals.
            if (wave == 0) {
              float mid[kFSlots], hi[kFSlots];
  #pragma unroll
              for (int m = 0; m < kFSlots; ++m) {
                const int i = lane + kWave * m;  // < kFMaxCand: in bounds
                mid[m] = sh.mid[i];
                hi[m] = sh.hi[i];
              }
              const int verdict = FastSelectSlots(n, kk, mid, hi, sh, false);
              if (lane == 0) sh.certified = verdict;
            }
            __syncthreads();
          }
          const int verdict = sh.certified;
          ballot = verdict < 0;  // equal midpoints: rank with ballots instead
          any = verdict == 0;
        }
        if (ballot) switch (cs * 8 + rs) {
          case 1 * 8 + 1: any = RankAndCertify<1, 1>(a, n, kk, page, ntok, sh); break;
          case 2 * 8 + 1: any = RankAndCertify<2, 1>(a, n, kk, page, ntok, sh); break;
          case 2 * 8 + 2: any = RankAndCertify<2, 2>(a, n, kk, page, ntok, sh); break;
          case 3 * 8 + 1: any = RankAndCertify<3, 1>(a, n, kk, page, ntok, sh); break;
          case 3 * 8 + 2: any = RankAndCertify<3, 2>(a, n, kk, page, ntok, sh); break;
          case 3 * 8 + 3: any = RankAndCertify<3, 3>(a, n, kk, page, ntok, sh); break;
          case 4 * 8 + 1: any = RankAndCertify<4, 1>(a, n, kk, page, ntok, sh); break;
          case 4 * 8 + 2: any = RankAndCertify<4, 2>(a, n, kk, page, ntok, sh); break;
          case 4 * 8 + 3: any = RankAndCertify<4, 3>(a, n, kk, page, ntok, sh); break;
          default: any = RankAndCertify<4, 4>(a, n, kk, page, ntok, sh); break;
        }
        if (!any || pass == 1) break;
        // 4a. Some order is not decided by the intervals: the flagged pages
        // get refined intervals (RefineScores, the whole workgroup, several
        // waves per page), and the ranks and certification run again; more
        // flagged pages than that pays for go straight to the exact chains
        // (sh.nflag read after the barrier: wave 0 wrote it).
        __syncthreads();
        const int nflag = sh.nflag;
        if (!RefineWorthwhile<kFThreads>(nflag)) break;
        StampAt(a, sh, kRefine);
        // The request's workgroups share the work: flagged page f is refined
        // by workgroup f mod groups, which publishes its interval as tagged
        // words (a.refined, slot f of the request); the others read it.  Every
        // workgroup of the request holds the same intervals and so forms the
        // same flag list (ballots over the same values), and each page's
        // interval is computed once: all of them certify from identical
        // intervals.  (The refinement is VALU-bound: at 8 flagged pages one
        // workgroup took 11 us for all of them.)
        const bool share = a.refined != nullptr && groups > 1 && nflag <= kFRefineSlots;
        const int stride = share ? groups : 1;
        const int first = share ? group : 0;
        const int nmine = first < nflag ? (nflag - first + stride - 1) / stride : 0;
        unsigned long long* xr =
            share ? a.refined + static_cast<size_t>(r) * (3 * kFRefineSlots) : nullptr;
        RefineScores<kFThreads>(
            nmine,
            [&](int f) -> const float* {
              const int i = sh.flag[first + f * stride];
              const int pg = sh.cpage[i];
              const bool live = pg >= 0 && pg < pool.capacity && sh.cntok[i] != 0;
              return live ? pool.summaries + static_cast<size_t>(pg) * kFE : nullptr;
            },
            [&](int f) {
              const int i = sh.flag[first + f * stride];
              return dsd_refine::FirstPassBound(sh.lo[i], sh.hi[i], a.scale, kFE);
            },
            [&](int f, float m, float l, float h) {
              // In LDS (the score passes of the request's other workgroups
              // wrote the global intervals, with no ordering against this
              // one), and for the other workgroups in the request's slot.
              const int ff = first + f * stride;
              const int i = sh.flag[ff];
              sh.mid[i] = m;
              sh.lo[i] = l;
              sh.hi[i] = h;
              if (xr != nullptr) {
                PutTagged(xr + 3 * ff + 0, a.epoch, __float_as_uint(m));
                PutTagged(xr + 3 * ff + 1, a.epoch, __float_as_uint(l));
                PutTagged(xr + 3 * ff + 2, a.epoch, __float_as_uint(h));
              }
            },
            a.queries + static_cast<size_t>(r) * kFE, kFE, a.scale,
            reinterpret_cast<double*>(sh.tile));
        if (share) {
          // The other workgroups' pages.  A wait that gives up keeps that
          // page's first-pass interval (still sound: the certification then
          // flags it again and the exact chain decides) and is reported.
          const int f = static_cast<int>(threadIdx.x);
          if (f < nflag && f % groups != group) {
            unsigned long long w[3];
            bool ok = true;
            for (int x = 0; x < 3; ++x) {
              unsigned spins = 0;
              w[x] = LoadWord(xr + 3 * f + x);
              while (ok && !Current(w[x], a.wait_tag)) {
                if (++spins >= a.spin_limit) {
                  ok = false;
                  break;
                }
                __builtin_amdgcn_s_sleep(1);
                w[x] = LoadWord(xr + 3 * f + x);
              }
            }
            const int i = sh.flag[f];
            if (ok) {
              sh.mid[i] = __uint_as_float(static_cast<uint32_t>(w[0]));
              sh.lo[i] = __uint_as_float(static_cast<uint32_t>(w[1]));
              sh.hi[i] = __uint_as_float(static_cast<uint32_t>(w[2]));
            } else {
              ReportFailure(a.fail, kFailWait);
            }
          }
          __syncthreads();
        }
        StampAt(a, sh, kRefined);
      }
      if (any) {
        // 4b. What the refined intervals leave open: rescore those pages with
        // the exact chain, rank again and rewrite the members.
        __syncthreads();
        const int nflag = sh.nflag;
        if (writer && threadIdx.x == 0 && a.exact_pages != nullptr) {
          atomicAdd(a.exact_pages, nflag);
        }
        RescoreChains<kFRescoreGroup, kFThreads>(
            nflag, [&](int f) { return sh.cpage[sh.flag[f]]; },
            [&](int f, float score) {
              const int i = sh.flag[f];
              sh.key[i] = SelectKey(score, sh.cpage[i]);
            },
            a.queries + static_cast<size_t>(r) * kFE, pool.summaries, pool.token_counts,
            pool.capacity, kFE, a.scale, sh.tile);
        ParallelRanks(sh, n);
        const int i = threadIdx.x;
        if (i < n && sh.rank[i] < kk) {
          sh.top[sh.rank[i]] = i;
          sh.page[sh.rank[i]] = sh.cpage[i];
          sh.ntok[sh.rank[i]] = sh.cntok[i];
        }
        __syncthreads();
      }
    }
    if (writer && static_cast<int>(threadIdx.x) < kk) {
      // Every rank below kk holds the page of one of the request's
      // candidates (sh.top its index, sh.cpage its id); a slot that does not
      // is reported and written as -1 (the attention never loads through
      // it: sh.page starts at -1 and sh.ntok at 0 in every launch).
      const int t = threadIdx.x;
      const int i = sh.top[t];
      const int pg = sh.page[t];
      const bool ok = i >= 0 && i < n && sh.cpage[i] == pg;
      if (!ok) ReportFailure(a.fail, kFailSelect);
      a.selected[static_cast<size_t>(r) * a.sel_stride + t] = ok ? pg : -1;
    }
  }
  if (writer && threadIdx.x == 0) a.counts[r] = kk;
  return kk;
}

// Attention of workgroup (r, g), heads h0 = 2g and h0+1: select, then per
// head softmax(q_h K^T * scale) V over the selected pages' valid tokens;
// waves 0-7 take head h0 and waves 8-15 head h0+1, each as
// AttentionFastKernel<128, 16, 8, 4>.
__device__ __forceinline__ void AttentionItem(const PoolView& pool, const FusedArgs& a, int r, int begin, int n,
                              int group, FusedShared& sh) {
  const int hpw = a.heads_per_group;
  const int wph = kFWaves / hpw;       // waves per head
  const int h0 = group * hpw;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int hw = wave % wph;   // wave within its head
  const int h = h0 + wave / wph;
  const int g = lane / kFLpt;
  const int j = lane % kFLpt;
  const int head_off = h * kFD + j * kFDq;
  const int kk =
      SelectForRequest(pool, a, r, begin, n, group, pool.num_heads / a.heads_per_group, sh);
  StampAt(a, sh, kSelected);
  // The query row loads with the first K/V rows (it is not held through the
  // selection, whose registers it would take).
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
  if (kk == 0) {
    // Nothing selected: zeros (src/cuda/sparse_batched_attention.cu:621-627).
    if (static_cast<int>(threadIdx.x) < hpw * kFD) {
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
       base += wph * kFTpc * kFUnroll) {
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
      static_assert(kFLpt == 16, "one token row per DPP row");
      dot = RowSum16(dot);  // the token's 16 lanes: one row
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
  // Merge the 4 token-slot streams of this wave, then the waves of each
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
  if (static_cast<int>(threadIdx.x) < hpw * kFD) {
    const int hh = threadIdx.x / kFD;  // which of the workgroup's heads
    const int d = threadIdx.x - hh * kFD;
    const int w0 = hh * wph;
    float mx = -INFINITY;
    for (int w = 0; w < wph; ++w) mx = fmaxf(mx, sh.m[w0 + w]);
    float lt = 0.0f;
    float at = 0.0f;
    if (mx != -INFINITY) {
      for (int w = 0; w < wph; ++w) {
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

// kMultiPass: some workgroup's slice spans several score passes; those
// slices pipeline their passes (each pass's rows load while the previous
// pass reduces).  Single-pass launches keep the plain form, which measured
// faster there.
template <bool kMultiPass>
__global__ __launch_bounds__(kFThreads) void FusedStepKernel(PoolView pool, FusedArgs a) {
  __shared__ FusedShared sh;
  if (a.epoch_src != nullptr) {
    // Replayed from a captured graph: the epoch the bump kernel just set.
    a.epoch = *a.epoch_src;
    a.wait_tag = a.epoch | a.wait_mask;
    a.fail.epoch = a.epoch;
  }
  if (a.stamps != nullptr && threadIdx.x == 0) {
    for (int i = 0; i < kStampsPerGroup; ++i) sh.stamp[i] = 0;
  }
  if (threadIdx.x < kFMaxK) {
    // No member slot keeps a previous workgroup's LDS: an unwritten slot
    // reads as no page with no tokens.  Slots below 64 are set by wave 0,
    // which alone writes them before the selection's first barrier; the
    // others are written only after that barrier.
    sh.top[threadIdx.x] = -1;
    sh.page[threadIdx.x] = -1;
    sh.ntok[threadIdx.x] = 0;
  }
  StampAt(a, sh, kStart);
  const int groups = pool.num_heads / a.heads_per_group;
  const int r = blockIdx.x / groups;
  const int g = blockIdx.x - r * groups;
  // A request whose offsets leave [0, total] is skipped (n = 0: nothing
  // scored or selected, zero outputs) and reported.
  int begin, n;
  RequestRange(a.cand_offsets, r, a.total, g == 0 ? a.fail : FailReport{}, &begin, &n);
  // A request beyond the caller's max_candidates (or kFMaxCand) selects
  // nothing (reported by the selection): its slices are not scored.
  if (n <= a.max_candidates && n <= kFMaxCand) {
    ScoreSlice<kMultiPass>(pool, a, r, begin + (g * n) / groups,
                           begin + ((g + 1) * n) / groups, sh);
  }
  StampAt(a, sh, kScored);
  AttentionItem(pool, a, r, begin, n, g, sh);
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

// ---- stand-alone score kernel (the three-kernel step at E = 4096) ----------
// Workgroup (x, r) scores candidates [P*x, P*x + P) of request r, P =
// pages_per_group (a multiple of 8), with the score passes above: the query
// staged once per workgroup, eight pages per pass.  Intervals go to
// mid/lo/hi[c] only.

__global__ __launch_bounds__(kFThreads) void ScorePagesKernel(PoolView pool, FusedArgs a,
                                                              int pages_per_group) {
  __shared__ ScoreShared sh;
  const int r = blockIdx.y;
  int begin, n;
  if (!RequestRange(a.cand_offsets, r, a.total, blockIdx.x == 0 ? a.fail : FailReport{}, &begin,
                    &n)) {
    return;
  }
  const int c0 = static_cast<int>(blockIdx.x) * pages_per_group;
  if (c0 >= n) return;
  const int c1 = n - c0 < pages_per_group ? n : c0 + pages_per_group;
  ScoreSlice<true>(pool, a, r, begin + c0, begin + c1, sh);
}

}  // namespace

void LaunchScorePages(const PoolView& pool, const float* d_queries, const int* d_cand_offsets,
                      const int* d_cand_ids, int batch, int total_candidates,
                      int max_candidates, float scale, float* d_mid, float* d_lo, float* d_hi,
                      FailReport fail, hipStream_t stream) {
  if (batch <= 0 || max_candidates <= 0 || total_candidates <= 0) return;
  if (pool.elements != kFE) throw std::invalid_argument("ScorePages needs E = 4096");
  const int per = ScorePagesPerGroup(total_candidates);
  FusedArgs a;
  a.queries = d_queries;
  a.cand_offsets = d_cand_offsets;
  a.cand_ids = d_cand_ids;
  a.batch = batch;
  a.total = total_candidates;
  a.scale = scale;
  a.mid = d_mid;
  a.lo = d_lo;
  a.hi = d_hi;
  a.fail = fail;
  const dim3 grid((max_candidates + per - 1) / per, batch);
  hipLaunchKernelGGL(ScorePagesKernel, grid, dim3(kFThreads), 0, stream, pool, a, per);
  DSD_HIP_CHECK(hipGetLastError());
}

int ScorePagesPerGroup(int total_candidates) {
  // About two workgroups per CU in all, 8..128 pages each (config 3,
  // 65,536 candidates: 128 pages per workgroup scored in 184.7 us, against
  // 187.5 at 64, 191.4 at 256 and 188.6 at 32).
  int per = (total_candidates + 511) / 512;
  per = ((per + kFPagesPerPass - 1) / kFPagesPerPass) * kFPagesPerPass;
  if (per < kFPagesPerPass) per = kFPagesPerPass;
  if (per > 128) per = 128;
  return per;
}

bool FusedStepMultiPass(const PoolView& pool, int max_candidates, int heads_per_group) {
  // Slices of a request split its candidates evenly over its workgroups.
  const int groups = pool.num_heads / heads_per_group;
  return (max_candidates + groups - 1) / groups > kFPagesPerPass;
}

bool FusedStepSupported(const PoolView& pool, int max_candidates, int top_k) {
  return pool.elements == kFE && pool.head_dim == kFD && pool.page_size > 0 &&
         pool.num_heads % 2 == 0 && max_candidates <= kFMaxCand && top_k <= kFMaxK;
}

int FusedStepHeadsPerGroup(const PoolView& pool, int batch, int compute_units) {
  // The fewest heads per workgroup (most waves per head) that keeps the
  // grid within one dispatch wave; 8 when none does.
  for (int hpw = 1; hpw < kFMaxHeadsPerGroup; hpw *= 2) {
    if (pool.num_heads % (2 * hpw) != 0) return hpw;
    if (static_cast<int64_t>(batch) * (pool.num_heads / hpw) <= compute_units) return hpw;
  }
  return kFMaxHeadsPerGroup;
}

int FusedStepGrid(const PoolView& pool, int batch, int heads_per_group) {
  return batch * (pool.num_heads / heads_per_group);
}

int FusedStepStampsPerGroup() { return kStampsPerGroup; }

// One thread advances the device epoch counter of captured steps, within
// [2^30, 2^31) (host epochs stay below 2^30, so the two never meet).
__global__ void EpochBumpKernel(unsigned* epoch) {
  if (threadIdx.x == 0) *epoch = ((*epoch + 1u) & 0x3FFFFFFFu) | 0x40000000u;
}

void LaunchEpochBump(unsigned* epoch, hipStream_t stream) {
  hipLaunchKernelGGL(EpochBumpKernel, dim3(1), dim3(kWave), 0, stream, epoch);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchFusedStep(const PoolView& pool, const FusedArgs& args, hipStream_t stream) {
  if (args.batch <= 0) return;
  const int hpw = args.heads_per_group;
  if (hpw != 1 && hpw != 2 && hpw != 4 && hpw != 8) {
    throw std::invalid_argument("heads per group must be 1, 2, 4 or 8");
  }
  if (pool.num_heads % hpw != 0) throw std::invalid_argument("heads per group must divide num_heads");
  const int grid = FusedStepGrid(pool, args.batch, hpw);
  if (args.epoch_src != nullptr) {
    hipLaunchKernelGGL(EpochBumpKernel, dim3(1), dim3(kWave), 0, stream,
                       const_cast<unsigned*>(args.epoch_src));
    DSD_HIP_CHECK(hipGetLastError());
  }
  if (FusedStepMultiPass(pool, args.max_candidates, hpw)) {
    hipLaunchKernelGGL(FusedStepKernel<true>, dim3(grid), dim3(kFThreads), 0, stream, pool, args);
  } else {
    hipLaunchKernelGGL(FusedStepKernel<false>, dim3(grid), dim3(kFThreads), 0, stream, pool, args);
  }
  DSD_HIP_CHECK(hipGetLastError());
}

void PreloadFusedKernels() {
  PreloadKernel(FusedStepKernel<true>);
  PreloadKernel(FusedStepKernel<false>);
  PreloadKernel(ScorePagesKernel);
  PreloadKernel(EpochBumpKernel);
}

}  // namespace dsdk
