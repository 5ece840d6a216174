/*
 * dsd_hip.h -- C ABI of the MI355X (gfx950) batched page-level sparse decode
 * library, libdsd_hip.so.
 *
 * This is the drop-in boundary.  Every entry point is plain C: opaque
 * handles, raw pointers and sizes, an int status.  The reference's C++ API
 * (PagePool / PagedKvCache / DevicePagePool / SparseCudaContext::RunBatch /
 * DenseCudaContext, the headers under include/dsd/) is implemented in host C++ on top
 * of these calls only; each entry below names the reference interface it
 * replaces (/root/reference/<file>:<line>).
 *
 * Status codes map 1:1 onto the reference's exception types; the message of
 * the last failure on the calling thread is returned by dsd_last_error().
 *
 * Device memory layout (HBM), owned by a pool handle:
 *   keys, values   float[capacity][page_size][E]   token-major, E = H*D
 *   summaries      float[capacity][E]              per-page key mean
 *   token_counts   int32[capacity]
 *   live           uint8[capacity]
 * Element (page p, token t, head h, dim d) is at p*page_size*E + t*E + h*D + d
 * (reference src/page_pool.cpp:58-59, src/cuda/sparse_batched_attention.cu:330).
 *
 * Threading: a handle is not thread-safe.  Pool calls are synchronous with
 * respect to the host (the reference's pool copies are blocking cudaMemcpy,
 * src/device_page_pool.cpp:1138-1166).  Sparse/dense host-buffer calls return
 * after their outputs are in host memory; *_device calls are asynchronous on
 * the given stream.
 */
#ifndef DSD_HIP_H_
#define DSD_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status ------------------------------------------------------------ */
enum {
  DSD_OK = 0,
  DSD_ERR_INVALID_ARGUMENT = 1, /* reference: std::invalid_argument */
  DSD_ERR_OUT_OF_RANGE = 2,     /* reference: std::out_of_range */
  DSD_ERR_RUNTIME = 3,          /* reference: std::runtime_error */
  DSD_ERR_HIP = 4               /* HIP runtime failure (reference: DSD_CUDA_CHECK,
                                   include/dsd/cuda_utils.h:43-53) */
};

/* Message of the last failure on this thread ("" if none). */
const char* dsd_last_error(void);

/* 1 when a gfx950-class device is visible, else 0.
 * Replaces SparseAttentionCudaAvailable / DenseAttentionCudaAvailable
 * (include/dsd/cuda_sparse_attention.h:17, cuda_dense_attention.h:16). */
int dsd_gpu_available(void);

/* Wait for all work on the current device. */
int dsd_device_synchronize(void);

/* ---- device page pool -------------------------------------------------- */
/* Replaces dsd::DevicePagePool (include/dsd/device_page_pool.h:17-140). */
typedef struct dsd_pool dsd_pool;

typedef struct dsd_transfer_stats {
  uint64_t h2d_bytes;
  uint64_t d2h_bytes;
  uint64_t h2d_calls;
  uint64_t d2h_calls;
  uint64_t h2d_large_calls; /* >= 1 MiB, as src/device_page_pool.cpp:13 */
  uint64_t d2h_large_calls;
} dsd_transfer_stats; /* include/dsd/types.h:50-57 */

/* DevicePagePool(config, capacity_pages) (device_page_pool.h:19). */
int dsd_pool_create(int num_heads, int head_dim, int page_size,
                    int capacity_pages, dsd_pool** out_pool);
int dsd_pool_destroy(dsd_pool* pool);

/* Reset(): all pages free, counts/live/summaries zero (device_page_pool.h:21). */
int dsd_pool_reset(dsd_pool* pool);

/* Upload n whole pages from host memory.  Page i gets id page_ids[i] and
 * token_counts[i] in (0, page_size] tokens whose K/V rows are the
 * token_counts[i]*E contiguous floats starting at element src_offsets[i] of
 * keys / values.  summaries: NULL => the device computes each page summary
 * with the host rule (sum in token order, then times fl(1/count));
 * otherwise [n][E] rows copied verbatim.
 * Covers UploadPage (device_page_pool.h:23-27), UploadPagesFromCache
 * (:31-33, with src_offsets = id*page_size*E into the cache pools and the
 * cache's summary rows) and UploadPromptDirect (:37-42, src_offsets = first
 * prompt token of each page * E). */
int dsd_pool_upload_pages(dsd_pool* pool, int n, const int* page_ids,
                          const int* token_counts, const int64_t* src_offsets,
                          const float* keys, const float* values,
                          const float* summaries);

/* Upload n single tokens: token i's K/V rows ([n][E] in keys/values) go to
 * (page_ids[i], token_offsets[i]); the page's token count becomes
 * page_token_counts[i].  summaries: NULL => the device applies the
 * running-mean update s = (s*old + k)/(old+1) in offset order (requires
 * each page's first offset to equal its current device count); otherwise
 * [n][E] rows copied.  Replaces UploadTokensFromCache / UploadTokensDirect
 * (device_page_pool.h:55-63). */
int dsd_pool_upload_tokens(dsd_pool* pool, int n, const int* page_ids,
                           const int* token_offsets,
                           const int* page_token_counts, const float* keys,
                           const float* values, const float* summaries);

/* MarkPagesFree (device_page_pool.h:71-72): counts, live flags and summary
 * rows of the listed pages are cleared on the device. */
int dsd_pool_mark_free(dsd_pool* pool, int n, const int* page_ids);

/* DownloadPage (device_page_pool.h:74-77): copies token_count*E floats of
 * K and V; *token_count receives the count.  Free page => DSD_ERR_RUNTIME. */
int dsd_pool_download_page(const dsd_pool* pool, int page_id, float* keys,
                           float* values, int* token_count);

/* DownloadMetadata (device_page_pool.h:79-81): capacity entries each. */
int dsd_pool_download_meta(const dsd_pool* pool, int* token_counts,
                           uint8_t* live);

/* Device summary rows of n pages into out[n][E] (parity checks). */
int dsd_pool_download_summaries(const dsd_pool* pool, int n,
                                const int* page_ids, float* out);

/* Device addresses of the pool arrays (key_base_device, value_base_device,
 * page_summary_base_device, page_token_counts_device, page_live_mask_device,
 * page_k_offsets_device, page_v_offsets_device, device_page_pool.h:92-100).
 * k_offsets[p] = v_offsets[p] = p * page_size * E. */
typedef struct dsd_pool_arrays {
  float* keys;
  float* values;
  float* summaries;
  int* token_counts;
  uint8_t* live;
  uint64_t* k_offsets;
  uint64_t* v_offsets;
} dsd_pool_arrays;
int dsd_pool_device_arrays(const dsd_pool* pool, dsd_pool_arrays* out);

/* PrefillPromptSynthetic (device_page_pool.h:44-48): K/V of n prompt pages of
 * request_id generated on the device from the reference's integer hash
 * (src/device_page_pool.cpp:102-120; page i of the call is prompt page i),
 * summaries by the host rule. */
int dsd_pool_prefill_synthetic(dsd_pool* pool, int n, const int* page_ids,
                               const int* token_counts, int request_id);

/* AppendTokensSynthetic (device_page_pool.h:65-69): token i's K/V generated
 * from (request_ids[i], decode_steps[i]) (src/device_page_pool.cpp:122-138),
 * written at (page_ids[i], token_offsets[i]), running-mean summary.  Returns
 * once the work is enqueued: every later call on the pool, and every step on
 * a context using the pool, is ordered after it. */
int dsd_pool_append_synthetic(dsd_pool* pool, int n, const int* page_ids,
                              const int* token_offsets,
                              const int* page_token_counts,
                              const int* request_ids, const int* decode_steps);

/* transfer_stats / ResetTransferStats (device_page_pool.h:85-86). */
int dsd_pool_transfer_stats(const dsd_pool* pool, dsd_transfer_stats* out);
int dsd_pool_reset_transfer_stats(dsd_pool* pool);

int dsd_pool_capacity(const dsd_pool* pool);

/* ---- sparse decode step ------------------------------------------------ */
/* Replaces dsd::SparseCudaContext (include/dsd/cuda_sparse_attention.h:50-137). */
typedef struct dsd_sparse_ctx dsd_sparse_ctx;

enum {
  DSD_OUTPUT_NONE = 0,    /* SparseBatchOutputMode::kNoOutputs   (:19-23) */
  DSD_OUTPUT_OUTPUTS = 1, /* SparseBatchOutputMode::kOutputsOnly */
  DSD_OUTPUT_DEBUG = 2    /* SparseBatchOutputMode::kDebugTensors */
};
enum {
  DSD_TIMING_NONE = 0,  /* SparseBatchTimingMode::kNone (:25-28) */
  DSD_TIMING_EVENTS = 1 /* SparseBatchTimingMode::kKernelEvents */
};

/* Per-call timings, ms (StageTimings + RuntimeOverheadTimings,
 * include/dsd/types.h:40-48,65-71). */
typedef struct dsd_step_timings {
  double score_ms;
  double topk_ms;
  double attention_ms;
  double kernel_ms;
  double h2d_ms;
  double d2h_ms;
  double launch_ms;
  double sync_ms;
} dsd_step_timings;

/* SparseCudaContext(cache, config, max_batch_size, max_total_candidates,
 * max_total_selected_pages) (cuda_sparse_attention.h:52-57).  The context
 * reads pages from `pool`, which must outlive it.  top_k >= 0. */
int dsd_sparse_create(dsd_pool* pool, int top_k, int max_batch,
                      int max_total_candidates, int max_total_selected,
                      dsd_sparse_ctx** out_ctx);
int dsd_sparse_destroy(dsd_sparse_ctx* ctx);

/* RunBatch (cuda_sparse_attention.h:60-68) over host buffers.
 *   queries      [batch][E]
 *   cand_offsets [batch+1]   CSR offsets into cand_ids (cand_offsets[0] == 0)
 *   cand_ids     [cand_offsets[batch]] candidate page ids per request
 * Outputs (host; may be NULL when not requested by output_mode):
 *   outputs          [batch][E]
 *   scores           [total candidates]             (DSD_OUTPUT_DEBUG)
 *   selected         [sum min(k, n_r)] compact       (DSD_OUTPUT_DEBUG, or
 *   selected_counts  [batch]                          DSD_OUTPUT_OUTPUTS when
 *                                                     both are non-NULL)
 * Selected ids equal the reference sparse_cpu selection bit-exactly.
 * timings may be NULL. */
int dsd_sparse_run_batch(dsd_sparse_ctx* ctx, int batch, const float* queries,
                         const int* cand_offsets, const int* cand_ids,
                         int output_mode, int timing_mode, float* outputs,
                         float* scores, int* selected, int* selected_counts,
                         dsd_step_timings* timings);

/* The context's pinned host staging, for callers that assemble a step in
 * place (no copy of the inputs): queries [max_batch][E], cand_offsets
 * [max_batch + 1], cand_ids [max_total_candidates], and outputs
 * [max_batch][E] where dsd_sparse_run_staged leaves a step's outputs.  Any
 * pointer argument may be NULL.  The buffers live as long as the context.
 * No reference counterpart: the reference's RunBatch packs into its own
 * host vectors (src/cuda/sparse_batched_attention.cu:24-96, :807-828). */
int dsd_sparse_staging(dsd_sparse_ctx* ctx, float** queries, int** cand_offsets,
                       int** cand_ids, float** outputs);

/* dsd_sparse_run_batch on inputs already written to the staging: the same
 * checks, output modes DSD_OUTPUT_NONE / DSD_OUTPUT_OUTPUTS (outputs stay in
 * the staging), ids into selected / selected_counts when both are non-NULL,
 * and the same timings. */
int dsd_sparse_run_staged(dsd_sparse_ctx* ctx, int batch, int output_mode,
                          int timing_mode, int* selected, int* selected_counts,
                          dsd_step_timings* timings);

/* dsd_sparse_run_staged with request r's query read from query_rows[r]
 * (E floats) instead of the staging's queries; the candidate lists come
 * from the staging as before.  Every row must be 16-byte aligned and lie
 * inside a dsd_host_alloc or dsd_device_alloc block, or be the staging's
 * own row r; anything
 * else fails with DSD_ERR_INVALID_ARGUMENT before any work.  The rows are
 * read by the device directly (no host copy), and the call returns after
 * the step, so they may change once it has returned.
 * No reference counterpart: lets a serving loop that keeps its queries in
 * pinned memory skip the per-step packing copy (the reference packs into
 * host vectors, src/cuda/sparse_batched_attention.cu:24-96). */
int dsd_sparse_run_staged_rows(dsd_sparse_ctx* ctx, int batch,
                               const float* const* query_rows, int output_mode,
                               int timing_mode, int* selected, int* selected_counts,
                               dsd_step_timings* timings);

/* Pinned host memory the device reads directly (coherent, so rows written
 * by the host between steps are seen by the next step).  dsd_host_free
 * takes only pointers from dsd_host_alloc (NULL is a no-op).  No reference
 * counterpart: the memory behind dsd_sparse_run_staged_rows. */
int dsd_host_alloc(size_t bytes, void** out);
int dsd_host_free(void* p);

/* Device memory whose rows the steps above accept as query rows, as they
 * accept dsd_host_alloc rows: for queries that already live in HBM, as a
 * model's own outputs do, so the step's stage-in reads them from HBM
 * instead of across PCIe.  dsd_device_upload copies bytes of host memory
 * (any kind) into such a block, synchronously; dsd_device_free takes only
 * pointers from dsd_device_alloc (NULL is a no-op) and waits for the
 * device first.  No reference counterpart: the reference's queries are host
 * vectors copied in every step (src/cuda/sparse_batched_attention.cu:
 * 24-96,600-640). */
int dsd_device_alloc(size_t bytes, void** out);
int dsd_device_upload(void* dst, const void* src, size_t bytes);
int dsd_device_free(void* p);

/* ---- synthetic inputs --------------------------------------------------- */
/* BuildSyntheticBatch's draw order (src/synthetic_data.cpp:23-68): one
 * std::mt19937(seed); the batch's context lengths first
 * (uniform_int_distribution<int>(min, max)) into context_tokens[batch]; then
 * for each request, page by page, its keys, then its values, then the
 * request's query.  DSD_SYNTHETIC_UNIFORM draws U(-1, 1) as the reference
 * does (its values bit for bit); DSD_SYNTHETIC_NORMAL draws
 * std::normal_distribution<float>(0, 1) on the same engine in the same
 * order (the benchmark's N(0, 1) inputs).  The batch's page g (requests in
 * order, pages in logical order) is pool page capacity_pages - 1 - g, as the
 * reference's LIFO page pool hands them out; key_pool / value_pool are
 * [capacity_pages][page_size][E], queries [batch][E], rows past a page's
 * tokens zero.  With key_pool, value_pool and queries all NULL only the
 * lengths are drawn. */
enum { DSD_SYNTHETIC_UNIFORM = 0, DSD_SYNTHETIC_NORMAL = 1 };
int dsd_synthetic_batch(int num_heads, int head_dim, int page_size, int batch,
                        int min_context_tokens, int max_context_tokens, int seed,
                        int distribution, int capacity_pages, int* context_tokens,
                        float* key_pool, float* value_pool, float* queries);

/* Device-resident step: every pointer is device memory and the call only
 * enqueues work on `stream` (a hipStream_t; NULL = the context's stream).
 * total_candidates and max_candidates (largest n_r) must describe the CSR.
 * selected ([batch][top_k], unused slots untouched), selected_counts,
 * scores may be NULL (context scratch is used).
 * The inputs are checked on the device, not the host: a request whose
 * offsets leave [0, total_candidates] or whose list is longer than
 * max_candidates selects nothing, and a candidate id outside the pool scores
 * as an empty page; either way the step's kernels finish normally, the
 * request's outputs are zeros, and dsd_sparse_device_status reports it.
 * Steps on one context share its scratch: a step on a stream other than the
 * previous step's first waits for the previous stream's work, so that
 * stream must still be valid then (it is used for an event record).
 * Graph capture: on a stream that is capturing, the call records the step
 * into the graph.  A captured single-launch step (fused or wide) takes its
 * epoch (the tag of the words its workgroups exchange) from a device
 * counter that a one-thread kernel, captured with it, advances on every
 * replay, so each replay reads its own inputs; the wide step's item
 * counters alternate between two sets by a device count the same kernel
 * advances.  The caller orders the graph's replays
 * against the context's other steps (no event wait is captured), and a
 * pool append must have completed (dsd_pool_* synchronised) before the
 * capture, or the call fails with DSD_ERR_INVALID_ARGUMENT. */
int dsd_sparse_run_batch_device(dsd_sparse_ctx* ctx, int batch,
                                int total_candidates, int max_candidates,
                                const float* d_queries,
                                const int* d_cand_offsets,
                                const int* d_cand_ids, float* d_outputs,
                                float* d_scores, int* d_selected,
                                int* d_selected_counts, void* stream);

/* The launch form of the context's last step (for tests and benchmarks
 * that must know which kernels ran).  No reference counterpart. */
typedef struct dsd_launch_info {
  int fused;                 /* 1: the single-launch step, 0: otherwise */
  int certified;             /* 1: certified scoring, 0: exact chains */
  int multi_pass;            /* fused: slices span several 8-page passes */
  int heads_per_group;       /* fused: heads per 1024-thread workgroup */
  int grid;                  /* fused, wide: workgroups launched (wide:
                                items plus spares); three-kernel at
                                E = 4096: score workgroups */
  int score_pages_per_group; /* wide, three-kernel at E = 4096: pages per
                                score workgroup */
  int wide;                  /* 1: the wide single launch (257 to 2048
                                candidates per request: score slices, the
                                select and the attention overlap in one
                                kernel; DSD_WIDE_STEP=0 at context creation
                                gives three kernels) */
} dsd_launch_info;
int dsd_sparse_last_launch(const dsd_sparse_ctx* ctx, dsd_launch_info* out);

/* Per-workgroup wall-clock stamps of the context's last timed single-launch
 * step (a host-buffer step in DSD_TIMING_EVENTS mode): *grid workgroups of
 * *per_group stamps each -- start, slice scored, intervals ready, intervals
 * read, ranked, selected, end, refinement begun and ended (0 when none ran),
 * then the hardware ids (HW_ID, XCC_ID << 32) -- at *khz ticks per
 * millisecond.  For the wide launch (dsd_launch_info.wide) *grid counts
 * items (score slices, then attention items) and each item's stamps are
 * start; kind (bits 0-7: 0 score slice, 1 attention), request (bits 8-31)
 * and the workgroup that ran it (bits 32+); select start and end (0 when
 * the item selected nothing); end.  out == NULL queries the sizes only.
 * For profiling; no reference counterpart. */
int dsd_sparse_step_stamps(const dsd_sparse_ctx* ctx, int* grid, int* per_group, double* khz,
                           uint64_t* out, size_t capacity);

/* Synchronizes the device, then reports (as its status, with the message in
 * dsd_last_error) the last input failure any step of the context recorded
 * and not yet reported -- e.g. from dsd_sparse_run_batch_device, which
 * cannot report it itself -- and clears it: DSD_ERR_INVALID_ARGUMENT for a
 * candidate list that does not fit the step's sizes, DSD_ERR_OUT_OF_RANGE
 * for a page id outside the pool, DSD_ERR_RUNTIME for a timed-out wait or
 * for a selection slot that did not hold one of the request's candidates
 * (an internal invariant the step checks before it writes each id: such a
 * slot is written as -1 and never attended).
 * Host-buffer steps report their own failures when they return.  No
 * reference counterpart (the reference's RunBatch checks on the host,
 * src/cuda/sparse_batched_attention.cu:600-608). */
int dsd_sparse_device_status(dsd_sparse_ctx* ctx);

/* The single-launch step's cross-workgroup waits poll at most spin_limit
 * times (default 2^17, about 0.1-0.3 s) before they give up: the step then
 * selects nothing for the request, its outputs are zeros and the failure is
 * reported (DSD_ERR_RUNTIME).  never_ready != 0 makes every wait look for a
 * tag no workgroup writes, so every wait gives up: a test hook for that
 * path, which never reaches a GPU hang.  No reference counterpart. */
int dsd_sparse_set_wait_limit(dsd_sparse_ctx* ctx, unsigned spin_limit, int never_ready);

/* dsd_sparse_run_batch_device without a context and without any
 * allocation: for callers that cannot allocate device memory during a step
 * -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  No counterpart in the reference (whose RunBatch
 * allocates nothing per step only because its context preallocated,
 * src/cuda/sparse_batched_attention.cu:444-528).
 * The step's scratch (publication words, score intervals, and ids / counts
 * when d_selected / d_selected_counts are NULL) lives in a static device
 * array of 2.7 MiB that each GPU holds until the process ends; the call
 * makes no hipMalloc / hipFree and no allocating library call.  Limits:
 * batch <= 1024, total_candidates <= 65536 and, when d_selected is NULL,
 * batch * max(1, top_k) <= 65536; larger calls fail with
 * DSD_ERR_INVALID_ARGUMENT before any work.  Every call on one GPU shares
 * the array, so calls that overlap on one GPU (on different streams, or
 * from several threads) race: order them.  Ids and counts left in the
 * array are overwritten by the next call.
 * Arguments as dsd_sparse_run_batch_device, plus the pool and top_k of the
 * context it replaces; selection is certified (bit-exact with sparse_cpu).
 * d_fail (may be NULL): memory the device writes (epoch << 32) | code to
 * when a request is skipped (1 timed-out wait, 2 sizes, 3 page id outside
 * the pool, 4 selection slot not a candidate: as dsd_sparse_device_status);
 * the caller clears it before the call and reads it after.
 * Under graph capture the step's epoch is a device counter kept in the same
 * static array, as for dsd_sparse_run_batch_device. */
int dsd_sparse_run_batch_device_static(dsd_pool* pool, int top_k, int batch,
                                       int total_candidates, int max_candidates,
                                       const float* d_queries, const int* d_cand_offsets,
                                       const int* d_cand_ids, float* d_outputs, float* d_scores,
                                       int* d_selected, int* d_selected_counts,
                                       unsigned long long* d_fail, void* stream);

/* Re-enqueue one stage of the last dsd_sparse_run_batch_device call on the
 * same buffers (stage 0 = score, 1 = select, 2 = attention, each as its own
 * kernel; 3 = the single-launch fused step, when the last call used it).
 * For per-kernel timing of the hot loop. */
int dsd_sparse_replay_stage(dsd_sparse_ctx* ctx, int stage, void* stream);

/* The stream the context's host-buffer steps run on (hipStream_t): the
 * pool's stream, so steps and pool work are ordered by the stream. */
void* dsd_sparse_stream(dsd_sparse_ctx* ctx);

/* Scoring mode (no counterpart in the reference, whose GPU scores are a
 * tree-reduced approximation, src/cuda/sparse_batched_attention.cu:133-151):
 *   DSD_SCORE_CERTIFIED (default) -- every page gets a rigorous interval
 *     around its sequential-fp32 score from an HBM-bound parallel kernel;
 *     only pages whose order the intervals leave open are rescored with the
 *     sequential chain.  Selection equals sparse_cpu bit for bit.
 *   DSD_SCORE_EXACT -- every page is scored with the sequential chain.
 * DSD_OUTPUT_DEBUG always uses exact scores (they are returned). */
enum { DSD_SCORE_CERTIFIED = 0, DSD_SCORE_EXACT = 1 };
int dsd_sparse_set_score_mode(dsd_sparse_ctx* ctx, int mode);

/* The first n certified score intervals of the last step (midpoint, lower
 * and upper bound per candidate, in CSR order).  For verification. */
int dsd_sparse_score_bounds(dsd_sparse_ctx* ctx, int n, float* mid, float* lo,
                            float* hi);

/* Pages rescored with the exact chain by certified selects so far (*out);
 * reset != 0 zeroes the counter.  Synchronizes the device. */
int dsd_sparse_exact_rescored_pages(dsd_sparse_ctx* ctx, int reset, int* out);

/* ---- request -> page table in HBM --------------------------------------- */
/* The reference keeps the request -> page table (PagedKvCache::
 * request_to_pages_, include/dsd/paged_kv_cache.h:120) and the free-page
 * list (PagePool, src/page_pool.cpp:36-44) on the host and packs every
 * step's candidate lists there (PackSparseBatchInto,
 * src/cuda/sparse_batched_attention.cu:24-96).  dsd_table keeps both in
 * device memory beside a pool: max_slots request slots of at most max_pages
 * page ids each, and a stack of free page ids with the PagePool order
 * (initially [0 .. capacity-1], the first page handed out capacity-1).  The
 * calls below enqueue kernels on the pool's stream and return; the host
 * keeps only counts (pages per slot, tokens in each tail page, free pages),
 * so it can check every call before enqueueing it and never reads page ids
 * back unless asked (dsd_table_download).  A table owns the pages it hands
 * out: use it, not dsd_pool_upload_* / mark_free, for those pages.  Only one
 * table per pool. */
typedef struct dsd_table dsd_table;

int dsd_table_create(dsd_pool* pool, int max_slots, int max_pages,
                     dsd_table** out);
int dsd_table_destroy(dsd_table* table);
/* Every slot empty, every page free (as at creation). */
int dsd_table_reset(dsd_table* table);
/* Pages of a slot; free pages (host mirror, no device access). */
int dsd_table_slot_pages(const dsd_table* table, int slot, int* count);
int dsd_table_free_pages(const dsd_table* table, int* count);
/* The slot's page ids in list order, and the free stack bottom to top
 * (synchronous downloads, for tests and observers). */
int dsd_table_download(dsd_table* table, int slot, int* page_ids, int capacity,
                       int* count);
int dsd_table_free_stack(dsd_table* table, int* page_ids, int capacity,
                         int* count);

/* Prompt admission into an empty slot: ceil(tokens / page_size) pages off
 * the stack, kept ascending (PagedKvCache::ReservePagesForRequest,
 * src/paged_kv_cache.cpp:114-160), then the prompt's rows
 * (keys / values: tokens x E host floats, token t to page t / page_size)
 * and each page's summary by the host cache's rule.  Replaces
 * ReservePagesForRequest + DevicePagePool::UploadPromptDirect
 * (src/device_page_pool.cpp:491-624).  The caller's buffers may be reused
 * on return. */
int dsd_table_admit_prompt(dsd_table* table, int slot, int tokens,
                           const float* keys, const float* values);
/* The same with the synthetic integer-hash prompt of request_id generated
 * on the device (DevicePagePool::PrefillPromptSynthetic,
 * src/device_page_pool.cpp:626-679). */
int dsd_table_admit_synthetic(dsd_table* table, int slot, int tokens,
                              int request_id);
/* Prompt upload ahead of admission, so that it overlaps the decode steps
 * (the reference admits synchronously, src/continuous_batching.cpp:208-239).
 * dsd_table_staging_init makes `buffers` device staging buffers of up to
 * max_tokens tokens and a copy stream.  dsd_table_stage_prompt uploads a
 * prompt (tokens x E host rows, pageable) into staging buffer `buffer` on
 * that stream and returns once the host rows have been copied out (the DMA
 * may still run).  dsd_table_admit_staged is dsd_table_admit_prompt from a
 * staged buffer: the pool's stream waits for that buffer's upload, then
 * pages are reserved, filled from it (device to device) and summarised.
 * dsd_table_stage_prompt waits for the previous admission from the same
 * buffer to have read it.  It may run on another host thread than the other
 * calls; the caller orders each buffer's staging after the admission
 * call that consumed its previous contents. */
int dsd_table_staging_init(dsd_table* table, int buffers, int max_tokens);
int dsd_table_stage_prompt(dsd_table* table, int buffer, int tokens,
                           const float* keys, const float* values);
int dsd_table_admit_staged(dsd_table* table, int slot, int buffer, int tokens);
/* One decode token for each of n distinct slots, in batch order
 * (PagedKvCache::AppendTokenMetadataOnly, src/paged_kv_cache.cpp:312-351,
 * then DevicePagePool::UploadTokensDirect / AppendTokensSynthetic,
 * src/device_page_pool.cpp:700-983): a slot whose tail page is full, that
 * has no page, or with fresh_page[i] != 0 takes the next page off the stack
 * (batch order).  Tokens with upload[i] != 0 get their payload: rows of
 * keys / values (m x E host floats, the uploaded tokens in batch order), or
 * with keys == values == NULL the device hash of (request_ids[i],
 * decode_steps[i]); the page summary follows the running mean.  A token
 * without upload only takes its page (the reference uploads every token but
 * a request's last).  fresh_page may be NULL. */
int dsd_table_append(dsd_table* table, int n, const int* slots,
                     const unsigned char* fresh_page, const unsigned char* upload,
                     const float* keys, const float* values,
                     const int* request_ids, const int* decode_steps);
/* The pages of n distinct slots back on the stack, in list order, slots in
 * order (PagedKvCache::ReleaseRequest, src/paged_kv_cache.cpp:354-373);
 * clear != 0 also clears their token counts, live flags and summaries
 * (DevicePagePool::MarkPagesFree, src/device_page_pool.cpp:989-1043). */
int dsd_table_release(dsd_table* table, int n, const int* slots, int clear);

/* The sparse step (dsd_sparse_run_batch) with request r's candidate list
 * the page list of table slot slots[r]: the CSR is built on the device from
 * the table, so only the queries and the slot ids cross PCIe.  Queries:
 * `queries` ([batch][E] host floats, or the staging's own rows) or
 * query_rows (as dsd_sparse_run_staged_rows).  Output modes NONE / OUTPUTS;
 * outputs NULL leaves them in the staging (dsd_sparse_staging).  Replaces
 * SparseCudaContext::RunBatch's packing
 * (src/cuda/sparse_batched_attention.cu:24-96,554-838). */
int dsd_sparse_run_table(dsd_sparse_ctx* ctx, dsd_table* table, int batch,
                         const int* slots, const float* queries,
                         const float* const* query_rows, int output_mode,
                         int timing_mode, float* outputs, int* selected,
                         int* selected_counts, dsd_step_timings* timings);
/* The CSR of the last step (cand_offsets[batch + 1], cand_ids) as the step
 * read it; synchronous.  For observers of table steps. */
int dsd_sparse_last_csr(dsd_sparse_ctx* ctx, int batch, int* cand_offsets,
                        int* cand_ids, int capacity);
/* The selected ids of the last step on the context's stream, packed per
 * request as dsd_sparse_run_batch returns them (selected[sum of counts],
 * selected_counts[batch]); synchronous.  For observers of table steps. */
int dsd_sparse_last_selection(dsd_sparse_ctx* ctx, int batch, int* selected,
                              int* selected_counts);

/* ---- asynchronous table steps ------------------------------------------ */
/* The serving loop's step without a host wait: the reference's loop calls
 * SparseCudaContext::RunBatch and waits for every step
 * (src/continuous_batching.cpp:497-696,
 * src/cuda/sparse_batched_attention.cu:554-838); here the host enqueues a
 * step, the step's append and release (dsd_table_append / _release, on the
 * same stream), and goes on to the next step while the device runs them.
 *
 * dsd_sparse_run_table_async is dsd_sparse_run_table that returns once the
 * step is enqueued, with *ticket its sequence number (0: batch was 0,
 * nothing enqueued).  Its slot ids and a `queries` block are copied at the
 * call; query_rows (dsd_host_alloc memory) are read by the device when the
 * step runs, so the caller keeps them unchanged until the step has
 * completed (dsd_sparse_async_wait).  Outputs stay in the staging
 * (dsd_sparse_staging), where later steps overwrite them; no ids are
 * returned (dsd_sparse_last_selection after a wait).  At most 4 steps are in
 * flight: a call first waits for the step enqueued 4 calls before it.
 * host_timings (may be NULL) gets the host side: h2d_ms staging, launch_ms
 * enqueue, sync_ms the wait for a free ring slot.
 *
 * dsd_sparse_async_wait blocks until every step up to `ticket` has completed;
 * dsd_sparse_async_collect until every enqueued step has, then hands over up
 * to `capacity` of the oldest records (*count of them; call again for the
 * rest).  A failure a step reported (the codes of dsd_sparse_device_status)
 * is returned by the call that waits for that step; its record is dropped.
 * A record's times are device event times from a base recorded before the
 * first step of its timeline (a timeline starts when nothing is in flight
 * and every record has been collected). */
typedef struct dsd_async_step {
  long long ticket;
  int batch;
  int fused;
  double start_ms;     /* the step's first command (the stage-in) */
  double done_ms;      /* its last command */
  double score_ms;     /* DSD_TIMING_EVENTS only, as dsd_step_timings */
  double topk_ms;
  double attention_ms;
  double kernel_ms;    /* the wide launch: its whole time (no stage split) */
  int wide;            /* 1: the wide single launch ran the step */
} dsd_async_step;
int dsd_sparse_run_table_async(dsd_sparse_ctx* ctx, dsd_table* table, int batch,
                               const int* slots, const float* queries,
                               const float* const* query_rows, int output_mode,
                               int timing_mode, long long* ticket,
                               dsd_step_timings* host_timings);
int dsd_sparse_async_wait(dsd_sparse_ctx* ctx, long long ticket);
int dsd_sparse_async_collect(dsd_sparse_ctx* ctx, dsd_async_step* steps, int capacity,
                             int* count);

/* ---- dense decode step ------------------------------------------------- */
/* DenseCudaContext::RunBatch (include/dsd/cuda_dense_attention.h:18-44):
 * attention over every candidate page, host buffers as above.
 * kernel_ms may be NULL. */
int dsd_dense_run_batch(dsd_pool* pool, int batch, const float* queries,
                        const int* cand_offsets, const int* cand_ids,
                        float* outputs, double* kernel_ms);

/* Device-resident dense step on `stream` (NULL = default stream). */
int dsd_dense_run_batch_device(dsd_pool* pool, int batch,
                               const float* d_queries,
                               const int* d_cand_offsets,
                               const int* d_cand_ids, float* d_outputs,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSD_HIP_H_ */
