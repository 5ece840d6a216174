// synthetic_data.cpp -- BuildSyntheticBatch (reference
// src/synthetic_data.cpp:12-68).  The draw order defines the workload, so it
// is kept: one std::mt19937(seed); all context lengths first
// (uniform_int_distribution); then per request and page the keys, then the
// values (uniform_real_distribution(-1, 1), one distribution object per
// vector); then the request's query.
#include "dsd/synthetic_data.h"

#include <algorithm>
#include <random>

#include "dsd/reference_kernels.h"

namespace dsd {

namespace {
std::vector<float> Uniform(int count, std::mt19937& rng) {
  std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
  std::vector<float> v(static_cast<std::size_t>(count));
  for (float& x : v) x = dist(rng);
  return v;
}
}  // namespace

SyntheticBatch BuildSyntheticBatch(const ModelConfig& config, int batch_size,
                                   int min_context_tokens, int max_context_tokens, int seed) {
  std::mt19937 rng(static_cast<std::mt19937::result_type>(seed));
  std::uniform_int_distribution<int> length(min_context_tokens, max_context_tokens);
  std::vector<int> lengths(static_cast<std::size_t>(std::max(batch_size, 0)));
  int pages = 0;
  for (int& n : lengths) {
    n = length(rng);
    pages += (n + config.page_size - 1) / config.page_size;
  }
  SyntheticBatch batch(config, pages);
  const int E = config.num_heads * config.head_dim;
  for (int r = 0; r < batch_size; ++r) {
    const int n = lengths[static_cast<std::size_t>(r)];
    const int page_count = (n + config.page_size - 1) / config.page_size;
    for (int p = 0; p < page_count; ++p) {
      const int tokens = std::min(config.page_size, n - p * config.page_size);
      const auto keys = Uniform(tokens * E, rng);
      const auto values = Uniform(tokens * E, rng);
      batch.cache.AppendPage(r, keys, values, tokens);
    }
    batch.requests.push_back(MakeRequestState(r, Uniform(E, rng), batch.cache, n));
  }
  return batch;
}

}  // namespace dsd
