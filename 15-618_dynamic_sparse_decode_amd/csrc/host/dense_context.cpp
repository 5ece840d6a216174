// dense_context.cpp -- DenseCudaContext on the C ABI (behaviour of reference
// src/cuda/kernels.cu:175-330: availability and head_dim checks, upload of
// the cache's live pages, attention over every candidate page per request).
#include "dsd/cuda_dense_attention.h"

#include <chrono>
#include <stdexcept>

#include "dsd_hip.h"
#include "status.h"

namespace dsd {

using detail::ThrowOnError;

bool DenseAttentionCudaAvailable() { return dsd_gpu_available() != 0; }

DenseCudaContext::DenseCudaContext(const PagedKvCache& cache, const ModelConfig& config)
    : cache_(&cache),
      config_(config),
      elements_per_token_(config.num_heads * config.head_dim),
      device_page_pool_(config, cache.CapacityPages()) {
  if (!DenseAttentionCudaAvailable()) {
    throw std::runtime_error("no visible gfx950 (MI355X) GPU");
  }
  if (config.head_dim <= 0 || config.head_dim > 256) {
    throw std::invalid_argument("head_dim must be in (0, 256]");
  }
  device_page_pool_.UploadActivePagesFromCache(cache);
}

DenseBatchResult DenseCudaContext::RunBatch(const std::vector<RequestState>& requests) {
  DenseBatchResult result;
  result.outputs.resize(requests.size());
  if (requests.empty()) return result;
  const auto t0 = std::chrono::steady_clock::now();
  std::vector<float> queries;
  std::vector<int> offsets{0};
  std::vector<int> ids;
  queries.reserve(requests.size() * static_cast<std::size_t>(elements_per_token_));
  for (const auto& r : requests) {
    if (static_cast<int>(r.query.size()) != elements_per_token_) {
      throw std::invalid_argument("request query length does not match model config");
    }
    queries.insert(queries.end(), r.query.begin(), r.query.end());
    ids.insert(ids.end(), r.candidate_page_ids.begin(), r.candidate_page_ids.end());
    offsets.push_back(static_cast<int>(ids.size()));
  }
  std::vector<float> out(queries.size());
  double kernel_ms = 0.0;
  ThrowOnError(dsd_dense_run_batch(device_page_pool_.handle(), static_cast<int>(requests.size()),
                                   queries.data(), offsets.data(), ids.data(), out.data(),
                                   &kernel_ms));
  result.kernel_ms = kernel_ms;
  const double total_ms =
      std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  result.runtime_overheads.time_sync_ms = total_ms > kernel_ms ? total_ms - kernel_ms : 0.0;
  for (std::size_t r = 0; r < requests.size(); ++r) {
    const auto begin = out.begin() + static_cast<std::ptrdiff_t>(r) * elements_per_token_;
    result.outputs[r].output.assign(begin, begin + elements_per_token_);
  }
  return result;
}

void DenseCudaContext::SyncPageFromCache(const PagedKvCache& cache, PageId page_id) {
  SyncPagesFromCache(cache, std::vector<PageId>{page_id});
}

void DenseCudaContext::SyncPagesFromCache(const PagedKvCache& cache,
                                          const std::vector<PageId>& page_ids) {
  cache_ = &cache;
  device_page_pool_.UploadPagesFromCache(cache, page_ids);
}

void DenseCudaContext::SyncAppendedToken(const PagedKvCache& cache,
                                         const AppendTokenResult& result) {
  SyncAppendedTokens(cache, std::vector<AppendTokenResult>{result});
}

void DenseCudaContext::SyncAppendedTokens(const PagedKvCache& cache,
                                          const std::vector<AppendTokenResult>& results) {
  cache_ = &cache;
  device_page_pool_.UploadTokensFromCache(cache, results);
}

void DenseCudaContext::SyncFreedPages(const std::vector<PageId>& page_ids) {
  device_page_pool_.MarkPagesFree(page_ids);
}

DenseBatchResult DenseAttentionCudaBatch(const PagedKvCache& cache,
                                         const std::vector<RequestState>& requests,
                                         const ModelConfig& config) {
  DenseCudaContext context(cache, config);
  return context.RunBatch(requests);
}

}  // namespace dsd
