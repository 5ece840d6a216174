// cuda_dense_attention.h -- attention over every candidate page (reference
// include/dsd/cuda_dense_attention.h:14-49); same names, gfx950 implementation.
#pragma once

#include <vector>

#include "dsd/config.h"
#include "dsd/device_page_pool.h"
#include "dsd/paged_kv_cache.h"
#include "dsd/types.h"

namespace dsd {

bool DenseAttentionCudaAvailable();

class DenseCudaContext {
 public:
  DenseCudaContext(const PagedKvCache& cache, const ModelConfig& config);

  DenseBatchResult RunBatch(const std::vector<RequestState>& requests);

  void SyncPageFromCache(const PagedKvCache& cache, PageId page_id);
  void SyncPagesFromCache(const PagedKvCache& cache, const std::vector<PageId>& page_ids);
  void SyncAppendedToken(const PagedKvCache& cache, const AppendTokenResult& result);
  void SyncAppendedTokens(const PagedKvCache& cache,
                          const std::vector<AppendTokenResult>& results);
  void SyncFreedPages(const std::vector<PageId>& page_ids);

 private:
  const PagedKvCache* cache_ = nullptr;
  ModelConfig config_{};
  int elements_per_token_ = 0;
  DevicePagePool device_page_pool_;
};

DenseBatchResult DenseAttentionCudaBatch(const PagedKvCache& cache,
                                         const std::vector<RequestState>& requests,
                                         const ModelConfig& config);

}  // namespace dsd
