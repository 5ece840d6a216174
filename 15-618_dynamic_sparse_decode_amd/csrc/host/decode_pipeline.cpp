// decode_pipeline.cpp -- the GPU methods of DecodePipeline and request
// metadata (reference src/decode_pipeline.cpp:11,54-87 and
// src/reference_kernels.cpp:44-57).  The CPU methods (sparse_cpu / dense_cpu)
// are the checker and are defined in oracle/liboracle_cpu.so.
#include "dsd/decode_pipeline.h"

#include <utility>

namespace dsd {

DecodePipeline::DecodePipeline(ModelConfig config) : config_(config) {}

AttentionResult DecodePipeline::RunDenseStepCuda(const PagedKvCache& cache,
                                                 const RequestState& request) const {
  auto batch = DenseAttentionCudaBatch(cache, std::vector<RequestState>{request}, config_);
  if (batch.outputs.empty()) return {};
  return batch.outputs.front();
}

SparseDecodeResult DecodePipeline::RunNaiveSparseStepCuda(const PagedKvCache& cache,
                                                          const RequestState& request) const {
  return SparseDecodeCuda(cache, request, config_);
}

DenseBatchResult DecodePipeline::RunDenseBatchCuda(
    const PagedKvCache& cache, const std::vector<RequestState>& requests) const {
  return DenseAttentionCudaBatch(cache, requests, config_);
}

DenseBatchResult DecodePipeline::RunDenseBatchCuda(
    DenseCudaContext& context, const std::vector<RequestState>& requests) const {
  return context.RunBatch(requests);
}

SparseBatchCudaResult DecodePipeline::RunNaiveSparseBatchCuda(
    SparseCudaContext& context, const std::vector<RequestState>& requests) const {
  return context.RunBatch(requests, SparseBatchOutputMode::kDebugTensors);
}

RequestState MakeRequestState(int request_id, std::vector<float> query,
                              const PagedKvCache& cache, int context_tokens) {
  RequestState r;
  r.request_id = request_id;
  r.query = std::move(query);
  r.context_tokens = context_tokens;
  const auto& pages = cache.GetRequestPages(request_id);
  r.candidate_page_ids.assign(pages.begin(), pages.end());
  return r;
}

}  // namespace dsd
