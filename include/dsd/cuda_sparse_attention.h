// cuda_sparse_attention.h -- the batched sparse decode step (reference
// include/dsd/cuda_sparse_attention.h:15-151).  The header keeps the
// reference's file name and type names so callers written against it compile
// unchanged; the implementation is libdsd_hip.so on gfx950 (no CUDA).
//
// Selection is bit-exact with the reference CPU path (SelectTopKPagesCpu):
// page scores are certified intervals around the reference's sequential fp32
// dot product, with exact rescoring of the pages whose order is undecided.
#pragma once

#include <cstdint>
#include <vector>

#include "dsd/config.h"
#include "dsd/device_page_pool.h"
#include "dsd/paged_kv_cache.h"
#include "dsd/types.h"

struct dsd_sparse_ctx;

namespace dsd {

// True when a gfx950 (MI355X) device is visible.
bool SparseAttentionCudaAvailable();

enum class SparseBatchOutputMode {
  kNoOutputs,
  kOutputsOnly,
  kDebugTensors,
};

enum class SparseBatchTimingMode {
  kNone,
  kKernelEvents,
};

struct SparseRunBatchOptions {
  SparseBatchOutputMode output_mode = SparseBatchOutputMode::kOutputsOnly;
  SparseBatchTimingMode timing_mode = SparseBatchTimingMode::kKernelEvents;
};

struct PackedSparseBatch {
  std::vector<float> queries;
  std::vector<int> request_candidate_offsets;
  std::vector<int> candidate_page_ids;
  std::vector<int> selected_offsets;
  std::vector<int> selected_counts;
  int num_requests = 0;
  int total_candidates = 0;
  int total_selected_pages = 0;
  int num_heads = 0;
  int head_dim = 0;
  int elements_per_token = 0;
  int max_candidates_per_request = 0;
};

class SparseCudaContext {
 public:
  SparseCudaContext(const PagedKvCache& cache, const ModelConfig& config, int max_batch_size,
                    int max_total_candidates, int max_total_selected_pages);
  ~SparseCudaContext();
  SparseCudaContext(const SparseCudaContext&) = delete;
  SparseCudaContext& operator=(const SparseCudaContext&) = delete;

  SparseBatchCudaResult RunBatch(
      const std::vector<RequestState>& requests,
      SparseBatchOutputMode output_mode = SparseBatchOutputMode::kOutputsOnly);
  SparseBatchCudaResult RunBatch(const std::vector<RequestState>& requests,
                                 SparseRunBatchOptions options);
  SparseBatchCudaResult RunBatch(const std::vector<const RequestState*>& requests,
                                 SparseRunBatchOptions options);

  void SyncPageFromCache(const PagedKvCache& cache, PageId page_id);
  void SyncPagesFromCache(const PagedKvCache& cache, const std::vector<PageId>& page_ids);
  void SyncPromptDirect(const PagedKvCache& cache, const std::vector<PageId>& page_ids,
                        const std::vector<int>& token_counts, const float* prompt_keys,
                        const float* prompt_values);
  void PrefillPromptSynthetic(const PagedKvCache& cache, const std::vector<PageId>& page_ids,
                              const std::vector<int>& token_counts, int request_id);
  void SyncAppendedToken(const PagedKvCache& cache, const AppendTokenResult& result);
  void SyncAppendedTokens(const PagedKvCache& cache,
                          const std::vector<AppendTokenResult>& results);
  void SyncAppendedTokensDirect(const PagedKvCache& cache,
                                const std::vector<AppendTokenResult>& results,
                                const std::vector<float>& token_keys,
                                const std::vector<float>& token_values);
  void AppendSyntheticTokens(const PagedKvCache& cache,
                             const std::vector<AppendTokenResult>& results,
                             const std::vector<int>& request_ids,
                             const std::vector<int>& decode_steps);
  void SyncFreedPages(const std::vector<PageId>& page_ids);
  void ResetDeviceTransferStats();
  DeviceTransferStats DeviceTransfers() const;

  // The C-ABI step handle (device-resident entry points, dsd_hip.h).
  ::dsd_sparse_ctx* handle() const { return ctx_; }
  // The C-ABI pool the context steps over (for a dsd_table beside it).  No
  // reference counterpart.
  ::dsd_pool* pool_handle() const { return device_page_pool_.handle(); }

 private:
  SparseBatchCudaResult RunBatchStaged(const std::vector<const RequestState*>& requests,
                                       bool timing, bool outputs);

  const PagedKvCache* cache_ = nullptr;
  ModelConfig config_{};
  int elements_per_token_ = 0;
  int max_batch_size_ = 0;
  int max_total_candidates_ = 0;
  int max_total_selected_pages_ = 0;
  PackedSparseBatch packed_scratch_;
  std::vector<const RequestState*> request_ptr_scratch_;
  DevicePagePool device_page_pool_;
  ::dsd_sparse_ctx* ctx_ = nullptr;
  std::vector<float> host_outputs_;
  std::vector<float> host_scores_;
  std::vector<int> host_selected_;
  std::vector<int> host_counts_;
};

SparseDecodeResult SparseDecodeCuda(const PagedKvCache& cache, const RequestState& request,
                                    const ModelConfig& config);

AttentionResult SparseAttentionCuda(const PagedKvCache& cache, const std::vector<float>& query,
                                    const std::vector<PageId>& selected_page_ids,
                                    const ModelConfig& config, double* gather_ms = nullptr,
                                    double* attention_ms = nullptr,
                                    RuntimeOverheadTimings* runtime_overheads = nullptr);

}  // namespace dsd
