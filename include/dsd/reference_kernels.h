// reference_kernels.h -- the CPU reference path (reference
// include/dsd/reference_kernels.h:11-43).
//
// MakeRequestState is part of libdsd.so (request metadata).  The CPU kernels
// (ScorePagesCpu .. DenseAttentionCpu, MaxAbsDiff) are the parity checker:
// they live in oracle/liboracle_cpu.so, which callers that want the
// reference's sparse_cpu / dense_cpu rows (tests, the bench drivers) link
// next to libdsd.so.  The product never calls them.
#pragma once

#include <vector>

#include "dsd/config.h"
#include "dsd/paged_kv_cache.h"
#include "dsd/types.h"

namespace dsd {

RequestState MakeRequestState(int request_id, std::vector<float> query,
                              const PagedKvCache& cache, int context_tokens);

std::vector<PageScore> ScorePagesCpu(const PagedKvCache& cache, const RequestState& request,
                                     const ModelConfig& config);

std::vector<PageId> SelectTopKPagesCpu(std::vector<PageScore> scores, int top_k);

GatheredPages GatherPagesCpu(const PagedKvCache& cache, const std::vector<PageId>& page_ids,
                             const ModelConfig& config);

AttentionResult SparseAttentionCpu(const std::vector<float>& query,
                                   const GatheredPages& gathered, const ModelConfig& config);

AttentionResult DenseAttentionCpu(const PagedKvCache& cache, const RequestState& request,
                                  const ModelConfig& config);

float MaxAbsDiff(const std::vector<float>& lhs, const std::vector<float>& rhs);

}  // namespace dsd
