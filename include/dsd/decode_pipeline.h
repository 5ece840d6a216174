// decode_pipeline.h -- per-request and batched decode steps (reference
// include/dsd/decode_pipeline.h:14-54).  The *Cuda methods run on the GPU
// (libdsd.so); RunNaiveSparseStep / RunNaiveSparseBatch / RunDenseStep are the
// reference's CPU rows (sparse_cpu / dense_cpu), provided by the checker
// library oracle/liboracle_cpu.so.
#pragma once

#include <vector>

#include "dsd/config.h"
#include "dsd/cuda_dense_attention.h"
#include "dsd/cuda_sparse_attention.h"
#include "dsd/paged_kv_cache.h"
#include "dsd/reference_kernels.h"
#include "dsd/types.h"

namespace dsd {

class DecodePipeline {
 public:
  explicit DecodePipeline(ModelConfig config);

  SparseDecodeResult RunNaiveSparseStep(const PagedKvCache& cache,
                                        const RequestState& request) const;
  AttentionResult RunDenseStep(const PagedKvCache& cache, const RequestState& request) const;
  AttentionResult RunDenseStepCuda(const PagedKvCache& cache,
                                   const RequestState& request) const;
  SparseDecodeResult RunNaiveSparseStepCuda(const PagedKvCache& cache,
                                            const RequestState& request) const;
  DenseBatchResult RunDenseBatchCuda(const PagedKvCache& cache,
                                     const std::vector<RequestState>& requests) const;
  DenseBatchResult RunDenseBatchCuda(DenseCudaContext& context,
                                     const std::vector<RequestState>& requests) const;
  SparseBatchCudaResult RunNaiveSparseBatchCuda(
      SparseCudaContext& context, const std::vector<RequestState>& requests) const;
  BatchDecodeResult RunNaiveSparseBatch(const PagedKvCache& cache,
                                        const std::vector<RequestState>& requests) const;

  const ModelConfig& config() const { return config_; }

 private:
  ModelConfig config_;
};

}  // namespace dsd
