// sparse_context.cpp -- SparseCudaContext on the libdsd_hip.so C ABI.
// Behaviour of reference src/cuda/sparse_batched_attention.cu:444-966:
// constructor checks and upload of the cache's live pages, RunBatch packing
// (PackSparseBatchInto, :24-96) and capacity checks, the three output modes,
// kernel-event and host-overhead timings, Sync* pass-throughs, and the
// one-shot helpers SparseDecodeCuda / SparseAttentionCuda.
#include "dsd/cuda_sparse_attention.h"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <stdexcept>

#include "dsd_hip.h"
#include "status.h"

namespace dsd {

using detail::ThrowOnError;

namespace {

using Clock = std::chrono::steady_clock;

double MsSince(Clock::time_point t0) {
  return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

void Pack(const std::vector<const RequestState*>& requests, const ModelConfig& config,
          PackedSparseBatch* packed) {
  if (config.head_dim <= 0 || config.head_dim > 128) {
    throw std::invalid_argument("sparse decode supports head_dim in (0, 128]");
  }
  const int E = config.num_heads * config.head_dim;
  packed->queries.clear();
  packed->request_candidate_offsets.assign(1, 0);
  packed->candidate_page_ids.clear();
  packed->selected_offsets.assign(1, 0);
  packed->selected_counts.clear();
  packed->num_requests = static_cast<int>(requests.size());
  packed->num_heads = config.num_heads;
  packed->head_dim = config.head_dim;
  packed->elements_per_token = E;
  packed->max_candidates_per_request = 0;
  for (const RequestState* r : requests) {
    if (r == nullptr) throw std::invalid_argument("request pointer must be non-null");
    if (static_cast<int>(r->query.size()) != E) {
      throw std::invalid_argument("query length does not match model config");
    }
    packed->queries.insert(packed->queries.end(), r->query.begin(), r->query.end());
    packed->candidate_page_ids.insert(packed->candidate_page_ids.end(),
                                      r->candidate_page_ids.begin(),
                                      r->candidate_page_ids.end());
    const int n = static_cast<int>(r->candidate_page_ids.size());
    packed->request_candidate_offsets.push_back(
        static_cast<int>(packed->candidate_page_ids.size()));
    packed->max_candidates_per_request = std::max(packed->max_candidates_per_request, n);
    const int sel = std::max(0, std::min(config.top_k_pages, n));
    packed->selected_counts.push_back(sel);
    packed->selected_offsets.push_back(packed->selected_offsets.back() + sel);
  }
  packed->total_candidates = static_cast<int>(packed->candidate_page_ids.size());
  packed->total_selected_pages = packed->selected_offsets.back();
}

}  // namespace

bool SparseAttentionCudaAvailable() { return dsd_gpu_available() != 0; }

SparseCudaContext::SparseCudaContext(const PagedKvCache& cache, const ModelConfig& config,
                                     int max_batch_size, int max_total_candidates,
                                     int max_total_selected_pages)
    : cache_(&cache),
      config_(config),
      elements_per_token_(config.num_heads * config.head_dim),
      max_batch_size_(max_batch_size),
      max_total_candidates_(max_total_candidates),
      max_total_selected_pages_(max_total_selected_pages),
      device_page_pool_(config, cache.CapacityPages()) {
  if (!SparseAttentionCudaAvailable()) {
    throw std::runtime_error("sparse decode requires a visible gfx950 (MI355X) GPU");
  }
  if (config.head_dim <= 0 || config.head_dim > 128) {
    throw std::invalid_argument("sparse decode supports head_dim in (0, 128]");
  }
  if (max_batch_size < 0 || max_total_candidates < 0 || max_total_selected_pages < 0) {
    throw std::invalid_argument("sparse context capacities must be non-negative");
  }
  device_page_pool_.UploadActivePagesFromCache(cache);
  ThrowOnError(dsd_sparse_create(device_page_pool_.handle(), std::max(0, config.top_k_pages),
                                 max_batch_size, max_total_candidates,
                                 max_total_selected_pages, &ctx_));
}

SparseCudaContext::~SparseCudaContext() {
  if (ctx_ != nullptr) dsd_sparse_destroy(ctx_);
}

SparseBatchCudaResult SparseCudaContext::RunBatch(const std::vector<RequestState>& requests,
                                                  SparseBatchOutputMode output_mode) {
  SparseRunBatchOptions options;
  options.output_mode = output_mode;
  options.timing_mode = SparseBatchTimingMode::kKernelEvents;
  return RunBatch(requests, options);
}

SparseBatchCudaResult SparseCudaContext::RunBatch(const std::vector<RequestState>& requests,
                                                  SparseRunBatchOptions options) {
  request_ptr_scratch_.clear();
  for (const auto& r : requests) request_ptr_scratch_.push_back(&r);
  return RunBatch(request_ptr_scratch_, options);
}

SparseBatchCudaResult SparseCudaContext::RunBatch(
    const std::vector<const RequestState*>& requests, SparseRunBatchOptions options) {
  SparseBatchCudaResult result;
  if (requests.empty()) return result;
  const bool timing = options.timing_mode == SparseBatchTimingMode::kKernelEvents;
  const bool debug = options.output_mode == SparseBatchOutputMode::kDebugTensors;
  const bool outputs = options.output_mode != SparseBatchOutputMode::kNoOutputs;

  if (!debug) return RunBatchStaged(requests, timing, outputs);
  const auto t0 = Clock::now();
  Pack(requests, config_, &packed_scratch_);
  const double layout_ms = MsSince(t0);
  const auto& p = packed_scratch_;
  if (p.num_requests > max_batch_size_) {
    throw std::invalid_argument("request batch exceeds sparse context capacity");
  }
  if (p.total_candidates > max_total_candidates_) {
    throw std::invalid_argument("candidate page count exceeds sparse context capacity");
  }
  if (p.total_selected_pages > max_total_selected_pages_) {
    throw std::invalid_argument("selected page count exceeds sparse context capacity");
  }

  const std::size_t out_elems = static_cast<std::size_t>(p.num_requests) * elements_per_token_;
  host_outputs_.resize(outputs ? out_elems : 0);
  host_scores_.resize(debug ? std::max(1, p.total_candidates) : 0);
  host_selected_.resize(debug ? std::max(1, p.total_selected_pages) : 0);
  host_counts_.resize(debug ? p.num_requests : 0);
  const int mode = options.output_mode == SparseBatchOutputMode::kNoOutputs ? DSD_OUTPUT_NONE
                   : debug ? DSD_OUTPUT_DEBUG
                           : DSD_OUTPUT_OUTPUTS;
  dsd_step_timings t{};
  ThrowOnError(dsd_sparse_run_batch(
      ctx_, p.num_requests, p.queries.data(), p.request_candidate_offsets.data(),
      p.candidate_page_ids.data(), mode, timing ? DSD_TIMING_EVENTS : DSD_TIMING_NONE,
      outputs ? host_outputs_.data() : nullptr, debug ? host_scores_.data() : nullptr,
      debug ? host_selected_.data() : nullptr, debug ? host_counts_.data() : nullptr, &t));

  if (timing) {
    result.aggregate_timings.page_scoring_ms = t.score_ms;
    result.aggregate_timings.topk_ms = t.topk_ms;
    result.aggregate_timings.attention_ms = t.attention_ms;
    result.aggregate_timings.gather_ms = 0.0;  // fused into attention
    result.aggregate_timings.total_ms = t.score_ms + t.topk_ms + t.attention_ms;
    result.kernel_ms = result.aggregate_timings.total_ms;
    result.runtime_overheads.time_prepare_sparse_layout_ms = layout_ms;
    result.runtime_overheads.time_memcpy_h2d_ms = t.h2d_ms;
    result.runtime_overheads.time_memcpy_d2h_ms = t.d2h_ms;
    result.runtime_overheads.time_kernel_launch_ms = t.launch_ms;
    result.runtime_overheads.time_sync_ms = t.sync_ms;
  }
  if (!outputs) return result;

  result.per_request.reserve(requests.size());
  int selected_at = 0;
  for (int r = 0; r < p.num_requests; ++r) {
    SparseDecodeResult one;
    one.request_id = requests[static_cast<std::size_t>(r)]->request_id;
    if (debug) {
      const int b = p.request_candidate_offsets[r];
      const int e = p.request_candidate_offsets[r + 1];
      one.scores.reserve(static_cast<std::size_t>(e - b));
      for (int c = b; c < e; ++c) {
        one.scores.push_back(PageScore{p.candidate_page_ids[c], host_scores_[c]});
      }
      const int cnt = host_counts_[r];
      one.selected_page_ids.assign(host_selected_.begin() + selected_at,
                                   host_selected_.begin() + selected_at + cnt);
      selected_at += cnt;
    }
    const auto begin = host_outputs_.begin() + static_cast<std::ptrdiff_t>(r) * elements_per_token_;
    one.output.output.assign(begin, begin + elements_per_token_);
    result.per_request.push_back(std::move(one));
  }
  return result;
}

// The outputs / no-outputs modes: PackSparseBatchInto's checks, then the
// queries and the CSR go straight into the context's pinned staging and the
// outputs are read from it (one copy each way).
SparseBatchCudaResult SparseCudaContext::RunBatchStaged(
    const std::vector<const RequestState*>& requests, bool timing, bool outputs) {
  SparseBatchCudaResult result;
  const auto t0 = Clock::now();
  if (config_.head_dim <= 0 || config_.head_dim > 128) {
    throw std::invalid_argument("sparse decode supports head_dim in (0, 128]");
  }
  const int B = static_cast<int>(requests.size());
  const int E = elements_per_token_;
  int total = 0;
  int total_selected = 0;
  for (const RequestState* r : requests) {
    if (r == nullptr) throw std::invalid_argument("request pointer must be non-null");
    if (static_cast<int>(r->query.size()) != E) {
      throw std::invalid_argument("query length does not match model config");
    }
    const int n = static_cast<int>(r->candidate_page_ids.size());
    total += n;
    total_selected += std::max(0, std::min(config_.top_k_pages, n));
  }
  if (B > max_batch_size_) {
    throw std::invalid_argument("request batch exceeds sparse context capacity");
  }
  if (total > max_total_candidates_) {
    throw std::invalid_argument("candidate page count exceeds sparse context capacity");
  }
  if (total_selected > max_total_selected_pages_) {
    throw std::invalid_argument("selected page count exceeds sparse context capacity");
  }
  float* queries = nullptr;
  int* offsets = nullptr;
  int* ids = nullptr;
  float* out = nullptr;
  ThrowOnError(dsd_sparse_staging(ctx_, &queries, &offsets, &ids, &out));
  offsets[0] = 0;
  int at = 0;
  for (int b = 0; b < B; ++b) {
    const RequestState& r = *requests[static_cast<std::size_t>(b)];
    std::memcpy(queries + static_cast<std::size_t>(b) * E, r.query.data(), sizeof(float) * E);
    const int n = static_cast<int>(r.candidate_page_ids.size());
    if (n > 0) std::memcpy(ids + at, r.candidate_page_ids.data(), sizeof(int) * n);
    at += n;
    offsets[b + 1] = at;
  }
  const double layout_ms = MsSince(t0);
  dsd_step_timings t{};
  ThrowOnError(dsd_sparse_run_staged(ctx_, B, outputs ? DSD_OUTPUT_OUTPUTS : DSD_OUTPUT_NONE,
                                     timing ? DSD_TIMING_EVENTS : DSD_TIMING_NONE, nullptr,
                                     nullptr, &t));
  if (timing) {
    result.aggregate_timings.page_scoring_ms = t.score_ms;
    result.aggregate_timings.topk_ms = t.topk_ms;
    result.aggregate_timings.attention_ms = t.attention_ms;
    result.aggregate_timings.gather_ms = 0.0;  // fused into attention
    result.aggregate_timings.total_ms = t.score_ms + t.topk_ms + t.attention_ms;
    result.kernel_ms = result.aggregate_timings.total_ms;
    result.runtime_overheads.time_prepare_sparse_layout_ms = layout_ms;
    result.runtime_overheads.time_memcpy_h2d_ms = t.h2d_ms;
    result.runtime_overheads.time_memcpy_d2h_ms = t.d2h_ms;
    result.runtime_overheads.time_kernel_launch_ms = t.launch_ms;
    result.runtime_overheads.time_sync_ms = t.sync_ms;
  }
  if (!outputs) return result;
  result.per_request.reserve(requests.size());
  for (int b = 0; b < B; ++b) {
    SparseDecodeResult one;
    one.request_id = requests[static_cast<std::size_t>(b)]->request_id;
    const float* o = out + static_cast<std::size_t>(b) * E;
    one.output.output.assign(o, o + E);
    result.per_request.push_back(std::move(one));
  }
  return result;
}

void SparseCudaContext::SyncPageFromCache(const PagedKvCache& cache, PageId page_id) {
  SyncPagesFromCache(cache, std::vector<PageId>{page_id});
}

void SparseCudaContext::SyncPagesFromCache(const PagedKvCache& cache,
                                           const std::vector<PageId>& page_ids) {
  cache_ = &cache;
  device_page_pool_.UploadPagesFromCache(cache, page_ids);
}

void SparseCudaContext::SyncPromptDirect(const PagedKvCache& cache,
                                         const std::vector<PageId>& page_ids,
                                         const std::vector<int>& token_counts,
                                         const float* prompt_keys,
                                         const float* prompt_values) {
  cache_ = &cache;
  device_page_pool_.UploadPromptDirect(cache, page_ids, token_counts, prompt_keys,
                                       prompt_values);
}

void SparseCudaContext::PrefillPromptSynthetic(const PagedKvCache& cache,
                                               const std::vector<PageId>& page_ids,
                                               const std::vector<int>& token_counts,
                                               int request_id) {
  cache_ = &cache;
  device_page_pool_.PrefillPromptSynthetic(cache, page_ids, token_counts, request_id);
}

void SparseCudaContext::SyncAppendedToken(const PagedKvCache& cache,
                                          const AppendTokenResult& result) {
  SyncAppendedTokens(cache, std::vector<AppendTokenResult>{result});
}

void SparseCudaContext::SyncAppendedTokens(const PagedKvCache& cache,
                                           const std::vector<AppendTokenResult>& results) {
  cache_ = &cache;
  device_page_pool_.UploadTokensFromCache(cache, results);
}

void SparseCudaContext::SyncAppendedTokensDirect(const PagedKvCache& cache,
                                                 const std::vector<AppendTokenResult>& results,
                                                 const std::vector<float>& token_keys,
                                                 const std::vector<float>& token_values) {
  cache_ = &cache;
  device_page_pool_.UploadTokensDirect(cache, results, token_keys, token_values);
}

void SparseCudaContext::AppendSyntheticTokens(const PagedKvCache& cache,
                                              const std::vector<AppendTokenResult>& results,
                                              const std::vector<int>& request_ids,
                                              const std::vector<int>& decode_steps) {
  cache_ = &cache;
  device_page_pool_.AppendTokensSynthetic(cache, results, request_ids, decode_steps);
}

void SparseCudaContext::SyncFreedPages(const std::vector<PageId>& page_ids) {
  device_page_pool_.MarkPagesFree(page_ids);
}

void SparseCudaContext::ResetDeviceTransferStats() { device_page_pool_.ResetTransferStats(); }

DeviceTransferStats SparseCudaContext::DeviceTransfers() const {
  return device_page_pool_.transfer_stats();
}

SparseDecodeResult SparseDecodeCuda(const PagedKvCache& cache, const RequestState& request,
                                    const ModelConfig& config) {
  const int n = static_cast<int>(request.candidate_page_ids.size());
  SparseCudaContext context(cache, config, 1, n, std::max(0, std::min(config.top_k_pages, n)));
  auto batch = context.RunBatch(std::vector<RequestState>{request},
                                SparseBatchOutputMode::kDebugTensors);
  SparseDecodeResult result;
  if (!batch.per_request.empty()) result = std::move(batch.per_request.front());
  result.request_id = request.request_id;
  result.timings = batch.aggregate_timings;
  result.runtime_overheads = batch.runtime_overheads;
  return result;
}

AttentionResult SparseAttentionCuda(const PagedKvCache& cache, const std::vector<float>& query,
                                    const std::vector<PageId>& selected_page_ids,
                                    const ModelConfig& config, double* gather_ms,
                                    double* attention_ms,
                                    RuntimeOverheadTimings* runtime_overheads) {
  RequestState request;
  request.request_id = 0;
  request.query = query;
  request.candidate_page_ids = selected_page_ids;
  request.context_tokens = static_cast<int>(selected_page_ids.size()) * config.page_size;
  ModelConfig local = config;
  local.top_k_pages = static_cast<int>(selected_page_ids.size());
  const auto result = SparseDecodeCuda(cache, request, local);
  if (gather_ms != nullptr) *gather_ms = result.timings.gather_ms;
  if (attention_ms != nullptr) *attention_ms = result.timings.attention_ms;
  if (runtime_overheads != nullptr) *runtime_overheads = result.runtime_overheads;
  return result.output;
}

}  // namespace dsd
