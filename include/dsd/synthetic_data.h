// synthetic_data.h -- seeded synthetic batches (reference
// include/dsd/synthetic_data.h:11-24): context lengths, then per request and
// page the keys and values, then the query, all from one std::mt19937 stream
// with U(-1,1) values, into a cache whose capacity is exactly the pages used.
#pragma once

#include <vector>

#include "dsd/config.h"
#include "dsd/paged_kv_cache.h"
#include "dsd/types.h"

namespace dsd {

struct SyntheticBatch {
  explicit SyntheticBatch(const ModelConfig& config, int capacity_pages = 1024)
      : cache(config, capacity_pages) {}

  PagedKvCache cache;
  std::vector<RequestState> requests;
};

SyntheticBatch BuildSyntheticBatch(const ModelConfig& config, int batch_size,
                                   int min_context_tokens, int max_context_tokens, int seed);

}  // namespace dsd
