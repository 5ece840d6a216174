// dsd_internal.h -- kernel launch interface shared by the HIP translation
// units of libdsd_hip.so.  Not part of the public ABI (include/dsd_hip.h).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace dsdk {

// Raw view of a device page pool (see the layout in include/dsd_hip.h).
struct PoolView {
  float* keys = nullptr;        // [capacity][page_size][E]
  float* values = nullptr;      // [capacity][page_size][E]
  float* summaries = nullptr;   // [capacity][E]
  int* token_counts = nullptr;  // [capacity]
  uint8_t* live = nullptr;      // [capacity]
  int num_heads = 0;
  int head_dim = 0;
  int page_size = 0;
  int elements = 0;   // E = num_heads * head_dim
  int capacity = 0;
  int64_t page_elems = 0;  // page_size * E
};

// A HIP runtime failure; the C ABI maps it to DSD_ERR_HIP.
struct HipError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

inline void CheckHip(hipError_t status, const char* expr) {
  if (status != hipSuccess) {
    throw HipError(std::string(expr) + " failed: " + hipGetErrorString(status));
  }
}

#define DSD_HIP_CHECK(expr) ::dsdk::CheckHip((expr), #expr)

// Loads a kernel's code on the current device now: the runtime otherwise
// loads it at its first launch, about a millisecond for the step kernels,
// which would land in the first step a caller runs (and times).
template <typename K>
void PreloadKernel(K kernel) {
  hipFuncAttributes attr{};
  DSD_HIP_CHECK(hipFuncGetAttributes(&attr, reinterpret_cast<const void*>(kernel)));
}
// The hot kernels of each translation unit (sparse contexts and tables
// call these at creation).
void PreloadStepKernels();
void PreloadFusedKernels();
void PreloadPoolKernels();
void PreloadTableKernels();

// Where a step's kernels report an input they cannot use: they store
// (epoch << 32) | code into *word, a host-visible pinned word, so the host
// can tell which launch failed.  Codes: 1 a cross-workgroup wait of the
// single-launch step gave up, 2 a request's candidate list does not fit what
// the launch was told (max_candidates, total_candidates, or a malformed CSR),
// 3 a candidate page id outside the pool.  The request is then skipped
// (nothing selected, zero outputs); every kernel still exits normally.
struct FailReport {
  unsigned long long* word = nullptr;  // null: failures are not reported
  unsigned epoch = 0;
};
// kFailSelect: a selection kernel was about to emit an id that is not the
// page of one of the request's candidates (an internal invariant; the slot
// is written as -1 and never attended).
enum FailCode { kFailWait = 1, kFailShape = 2, kFailPageId = 3, kFailSelect = 4 };

// ---- pool kernels (pool_kernels.hip) --------------------------------------

// For each of n pages: token count and live flag, then the summary row --
// copied from rows[n][E] when rows != nullptr, else computed from the page's
// keys with the host rule (sum in token order, times fl(1/count)).
void LaunchFinishPageUpload(const PoolView& pool, const int* d_page_ids,
                            const int* d_token_counts, const float* d_rows,
                            int n, hipStream_t stream);

// Token append.  Tokens are grouped in segments of one page each (host
// sorted by (page, offset)): seg_start[nseg+1] indexes order[], order[q] is
// the token index into the staged rows keys/values[n][E] and the per-token
// arrays.  Writes K/V rows, then the summary (rows copy or running mean in
// offset order), token count and live flag.
void LaunchAppendTokens(const PoolView& pool, const int* d_seg_start,
                        const int* d_order, const int* d_page_ids,
                        const int* d_offsets, const int* d_counts,
                        const float* d_keys, const float* d_values,
                        const float* d_rows, int num_segments,
                        hipStream_t stream);

// Synthetic GPU-resident admission (integer-hash payloads).
void LaunchPrefillSynthetic(const PoolView& pool, const int* d_page_ids,
                            const int* d_token_counts, int n, int request_id,
                            hipStream_t stream);
// meta: device-readable (pinned, coherent) ints, seg_start[num_segments + 1]
// then five arrays of n in page / offset order: page ids, token offsets, page
// token counts, request ids, decode steps.
void LaunchAppendSynthetic(const PoolView& pool, const int* meta, int n, int num_segments,
                           hipStream_t stream);

// Clears token count, live flag and summary row of n pages.
void LaunchMarkFree(const PoolView& pool, const int* d_page_ids, int n,
                    hipStream_t stream);

// ---- request -> page table (page_table.hip) ---------------------------------

// A pool's request -> page table and free-page stack in device memory.
struct TableView {
  int* pages = nullptr;       // [max_slots][max_pages]: slot s's pages in logical order
  int* npages = nullptr;      // [max_slots]
  int* free_stack = nullptr;  // [pool capacity]: free page ids, top at free_top - 1
  int* free_top = nullptr;    // [1]
  int max_slots = 0;
  int max_pages = 0;
};

// A host-visible progress word: once the kernels of a launch have read their
// host-side arguments, the launch's last kernel stores `seq` into *word
// (pinned, coherent; a release at system scope).  The host polls the word
// instead of recording an event, whose barrier idles the stream for
// microseconds.  word == nullptr: no mark.
struct ProgressMark {
  unsigned long long* word = nullptr;
  unsigned long long seq = 0;
};
__device__ inline void StoreProgress(const ProgressMark& m) {
  if (m.word != nullptr) {
    __hip_atomic_store(m.word, m.seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

// Stack = [0 .. capacity-1], every slot empty.
void LaunchTableReset(const TableView& t, int capacity, hipStream_t stream);
// Slot `slot` (empty) takes the n pages on top of the stack, ascending.
void LaunchTableReserve(const TableView& t, int slot, int n, hipStream_t stream);
// d_keys / d_values: tokens x E rows (device) into the pages of `slot`.
void LaunchTableScatter(const PoolView& pool, const TableView& t, int slot, int tokens,
                        const float* d_keys, const float* d_values, hipStream_t stream);
// One token for each of n slots: page allocation, then the plan of the m
// uploaded tokens (layout in page_table.hip) for LaunchAppendSynthetic
// (meta = d_plan) or LaunchAppendTokens (d_order and the plan's arrays).
// args (device-readable, e.g. pinned): slots[n], flags[n], request ids[n],
// decode steps[n].  `mark` is stored once args has been read.
void LaunchTablePlanAppend(const PoolView& pool, const TableView& t, const int* args, int n,
                           int m, int* d_plan, int* d_order, hipStream_t stream,
                           ProgressMark mark = {});
// n <= 1024 slots (device-readable) back to the stack; `clear` also clears
// their pages' counts, live flags and summaries.  `mark` is stored once
// slots has been read.
void LaunchTableRelease(const PoolView& pool, const TableView& t, const int* slots, int n,
                        int released_pages, bool clear, hipStream_t stream,
                        ProgressMark mark = {});

// Up to four segments of 4-byte words, each 16-byte aligned at both ends of
// the copy: src in pinned host memory the device reads directly, dst in
// device memory.  Optionally also a row gather: nrows rows of row_words
// words (a multiple of 4), row r from rows[r] (a device-visible table of
// device-visible, 16-byte aligned pointers) to rows_dst + r * row_words.
// Optionally also the candidate lists of a batch from a page table: request
// b's list is table.pages[slots[b]] (slots device-readable), written as the
// CSR csr_offsets[table_batch + 1] / csr_ids.
struct StageSegments {
  const uint32_t* src[4] = {};
  uint32_t* dst[4] = {};
  int words[4] = {};
  int count = 0;
  const float* const* rows = nullptr;
  float* rows_dst = nullptr;
  int nrows = 0;
  int row_words = 0;
  TableView table;
  const int* table_slots = nullptr;
  int table_batch = 0;
  int* csr_offsets = nullptr;
  int* csr_ids = nullptr;
  // When non-null: the device clock (wall_clock64) as workgroup 0 starts,
  // stored here (pinned) -- an asynchronous step's start stamp.
  unsigned long long* start_stamp = nullptr;
};
void LaunchStageIn(const StageSegments& s, hipStream_t stream);
// An asynchronous step's completion mark, after every earlier kernel on the
// stream: words[1] = the device clock, then words[0] = ticket (a release at
// system scope; words pinned and coherent).
void LaunchStepMark(unsigned long long* words, unsigned long long ticket, hipStream_t stream);

// ---- decode-step kernels (step_kernels.hip) --------------------------------

// Exact-order page scores: scores[c] = fl(sum_seq q*s) * scale, bit-equal to
// the reference's sequential CPU loop.
void LaunchScoreExact(const PoolView& pool, const float* d_queries,
                      const int* d_cand_offsets, const int* d_cand_ids,
                      int batch, int total_candidates, int max_candidates, float scale,
                      float* d_scores, FailReport fail, hipStream_t stream);

// Certified scoring: per candidate an interval [lo, hi] that provably holds
// the reference's sequential-fp32 score, and its midpoint.  Needs E % 64 == 0
// and at most 2048 candidates per request (next power of two).
bool CertifiedScoringSupported(int elements, int max_candidates);
void LaunchScoreBounds(const PoolView& pool, const float* d_queries,
                       const int* d_cand_offsets, const int* d_cand_ids, int batch,
                       int total_candidates, int max_candidates, float scale, float* d_mid,
                       float* d_lo, float* d_hi, FailReport fail, hipStream_t stream);

// Top-k from certified intervals; candidates whose order is not decided by
// disjoint intervals get refined intervals (kept in LDS: mid/lo/hi stay the
// score kernel's first-pass intervals, so the select can run again on the
// same buffers) and, where those still leave it open, the exact sequential
// chain.  Adds the
// number of rescored pages to *d_exact_pages when non-null.  A request whose
// candidate list is longer than max_candidates (the score kernels covered
// only that many) or whose offsets leave [0, total_candidates] selects
// nothing and is reported (kFailShape).
void LaunchSelectCertified(const PoolView& pool, const float* d_mid, const float* d_lo,
                           const float* d_hi,
                           const float* d_queries,
                           const int* d_cand_offsets, const int* d_cand_ids, int batch,
                           int total_candidates, int max_candidates, float scale, int top_k,
                           int* d_selected, int* d_counts, int* d_exact_pages, FailReport fail,
                           hipStream_t stream);

// Largest next-pow2 candidate count the LDS select handles.
int SelectMaxCandidates();

// Per-request top-k by (score desc, id asc): selected[r*top_k + j],
// counts[r] = min(top_k, n_r).
void LaunchSelectTopK(const float* d_scores, const int* d_cand_offsets,
                      const int* d_cand_ids, int batch, int total_candidates,
                      int max_candidates, int top_k, int* d_selected, int* d_counts,
                      FailReport fail, hipStream_t stream);

// Fused gather + softmax attention over page lists.  Request r attends over
// list_ids[start_r .. start_r + count_r): with list_stride > 0, start_r =
// r*list_stride and count_r = list_counts[r]; otherwise CSR list_offsets.
// A list id outside the pool holds no tokens (never read).
struct AttentionArgs {
  const float* queries = nullptr;  // [batch][E]
  const int* list_ids = nullptr;
  const int* list_offsets = nullptr;
  const int* list_counts = nullptr;
  int list_stride = 0;
  int batch = 0;
  float scale = 0.0f;
  float* outputs = nullptr;  // [batch][E]
  // D = 128, E = 4096: split each head as the wide step's attention items
  // do (bit-identical outputs), for the batches that step takes.
  bool wide_partition = false;
};
void LaunchAttention(const PoolView& pool, const AttentionArgs& args,
                     hipStream_t stream);

// ---- the fused single-launch step (fused_step.hip) --------------------------

// Arguments of the one-launch decode step.  Intervals cross workgroups as
// epoch-tagged 64-bit words in context-owned device memory (zero at
// creation): rec[total][3] = (mid, lo, hi) of each candidate.  epoch is
// non-zero and differs between consecutive launches on the context.
struct FusedArgs {
  const float* queries = nullptr;     // [batch][E]
  const int* cand_offsets = nullptr;  // [batch + 1]
  const int* cand_ids = nullptr;      // [total]
  int batch = 0;
  int total = 0;
  int top_k = 0;
  int sel_stride = 1;                 // row stride of selected
  int heads_per_group = 2;            // heads per workgroup: 1, 2, 4 or 8
  int max_candidates = 0;             // the largest request's candidate count
  float scale = 0.0f;
  float* mid = nullptr;               // [total] certified intervals (caller copy)
  float* lo = nullptr;
  float* hi = nullptr;
  int* selected = nullptr;            // [batch][sel_stride] (caller copy)
  int* counts = nullptr;              // [batch]
  float* outputs = nullptr;           // [batch][E]
  unsigned long long* rec = nullptr;
  // [batch][kFRefineSlots][3] tagged refined intervals that a request's
  // workgroups exchange (each refines a share of the flagged pages); null:
  // every workgroup refines all of them.
  unsigned long long* refined = nullptr;
  unsigned epoch = 0;
  int* exact_pages = nullptr;         // may be null
  FailReport fail;                    // kFailWait / kFailShape / kFailPageId / kFailSelect
  unsigned spin_limit = 0;            // polls of a cross-workgroup wait before it gives up
  unsigned wait_tag = 0;              // the tag the waits look for: epoch | wait_mask
  unsigned wait_mask = 0;             // 0, or a bit no epoch has (a test hook: every
                                      // wait gives up)
  // Non-null for launches captured into a graph: the device counter that
  // LaunchFusedStep advances in a one-thread kernel just before the step;
  // the step reads its epoch there (so every replay tags afresh) instead of
  // `epoch`.  Host epochs lie in [1, 2^30), device epochs in [2^30, 2^31).
  const unsigned* epoch_src = nullptr;
  unsigned long long* stamps = nullptr;  // null, or [grid][FusedStepStampsPerGroup()]:
                                         // clocks at start, slice scored, counter
                                         // ready, records read, ranked, selected,
                                         // end; then the hardware ids
};

// Flagged pages a request refines at most (RefineWorthwhile with 1024
// threads) and so the refined-interval slots per request.
constexpr int kFRefineSlots = 8;

// E = 4096, head_dim = 128, max_candidates <= 256, top_k <= 256.
bool FusedStepSupported(const PoolView& pool, int max_candidates, int top_k);
// Heads per workgroup for a batch: the fewest (1, 2, 4, 8) that keep the grid
// within `compute_units` workgroups, else 8.
int FusedStepHeadsPerGroup(const PoolView& pool, int batch, int compute_units);
// Workgroups of one launch: num_heads / heads_per_group per request.
int FusedStepGrid(const PoolView& pool, int batch, int heads_per_group);
int FusedStepStampsPerGroup();
// Whether a launch takes FusedStepKernel<true> (a slice spans several score
// passes of 8 pages, so each pass's rows load while the previous one reduces).
bool FusedStepMultiPass(const PoolView& pool, int max_candidates, int heads_per_group);
// Pages per workgroup of the stand-alone score kernel (E = 4096).
int ScorePagesPerGroup(int total_candidates);
void LaunchFusedStep(const PoolView& pool, const FusedArgs& args, hipStream_t stream);

// The wide step (step_kernels.hip): the certified three-kernel step for
// E = 4096, head_dim 128 and up to WideStepMaxCandidates() candidates per
// request in one launch: score slices (groups per request), then one
// attention item per (request, head), taken by workgroups in start order;
// the last slice of a request to finish selects it.  a: as for
// LaunchFusedStep (rec: the interval words, 3 per candidate; sel_stride =
// top_k).  sel_rec: [batch][sel_stride] tagged selected ids; cnt_rec:
// [batch] tagged counts; counters: this launch's set, [0] item tickets,
// [1 .. 1 + batch) arrivals, zero at the launch; next_counters: the other
// set (counter_words words), which workgroup 0 zeroes for the next launch.
// Launches alternate between the two sets.  A launch captured into a graph
// (a.epoch_src set) takes its epoch there and its set from the parity of
// *seq_src, one of the two sets at capture_counters; LaunchWideStep then
// first advances both counters in a one-thread kernel.
struct WideArgs {
  FusedArgs a;
  unsigned long long* sel_rec = nullptr;
  unsigned long long* cnt_rec = nullptr;
  unsigned* counters = nullptr;
  unsigned* next_counters = nullptr;
  unsigned* seq_src = nullptr;           // captured launches: the device launch count
  unsigned* capture_counters = nullptr;  // captured launches: their two sets
  int counter_words = 0;    // words per set, at least batch + 1
  int pages_per_group = 0;  // candidates per score item (a multiple of 8)
  int groups = 0;           // score items per request
  int lag = 0;              // a request's attention items follow the score
                            // items of the request `lag` places later
  int items = 0;            // WideStepItems
  bool tickets = true;      // items in the order workgroups start (a
                            // counter in counters[0]), not by workgroup id
};
bool WideStepSupported(const PoolView& pool, int max_candidates, int top_k);
int WideStepMaxCandidates();
// Score slices plus attention items.
int WideStepItems(const PoolView& pool, int batch, int groups);
// Workgroups launched: with tickets, half as many again as items (spares let
// an XCD whose CUs free up early take items another XCD would have run).
int WideStepGrid(int items, bool tickets);
// Timing mode (FusedArgs::stamps): per item the clocks at start, select
// start and end (0 when it selected nothing), end, and in slot 1 the item
// kind (bits 0-7: 0 score slice, 1 attention item), request (bits 8-31) and
// the workgroup that ran it (bits 32+).
int WideStepStampsPerGroup();
void LaunchWideStep(const PoolView& pool, const WideArgs& w, hipStream_t stream);
// One thread advances a captured step's device epoch counter (see FusedArgs).
void LaunchEpochBump(unsigned* epoch, hipStream_t stream);

// Certified intervals for E = 4096 with the fused step's score passes
// (float, query staged in LDS, 8..64 pages per 1024-thread workgroup).
void LaunchScorePages(const PoolView& pool, const float* d_queries, const int* d_cand_offsets,
                      const int* d_cand_ids, int batch, int total_candidates,
                      int max_candidates, float scale, float* d_mid, float* d_lo, float* d_hi,
                      FailReport fail, hipStream_t stream);

}  // namespace dsdk
