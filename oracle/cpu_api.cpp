// cpu_api.cpp -- TEST INFRASTRUCTURE ONLY: the reference's CPU rows
// (sparse_cpu / dense_cpu) behind the reference's own C++ names, built on the
// C oracle (dsd_oracle.c) and linked against libdsd.so for PagedKvCache.
// Output: oracle/liboracle_cpu.so.  Tests and the C++ test drivers link it to
// check the GPU path; the product libraries never load it.
//
// Each function follows the reference file:line named in its comment and
// adds no arithmetic of its own: every float operation is one of the C
// oracle's (compiled -ffp-contract=off, no -march), so the results are the
// reference's bit for bit (pinned in tests/test_oracle.py).
#include <cstddef>
#include <limits>
#include <stdexcept>
#include <vector>

#include "dsd/decode_pipeline.h"
#include "dsd/profiler.h"
#include "dsd/reference_kernels.h"
#include "dsd_oracle.h"

namespace dsd {

// src/reference_kernels.cpp:59-80 (stored summary; zero for an empty page,
// src/paged_kv_cache.cpp:454-461).
std::vector<PageScore> ScorePagesCpu(const PagedKvCache& cache, const RequestState& request,
                                     const ModelConfig& config) {
  const int E = config.num_heads * config.head_dim;
  if (static_cast<int>(request.query.size()) != E) {
    throw std::invalid_argument("query length does not match model config");
  }
  const float scale = oracle_scale(config.head_dim);
  std::vector<PageScore> scores;
  scores.reserve(request.candidate_page_ids.size());
  for (PageId id : request.candidate_page_ids) {
    const auto summary = cache.BuildPageSummary(id);
    const float dot = oracle_dot(request.query.data(), summary.data(), E);
    scores.push_back(PageScore{id, dot * scale});
  }
  return scores;
}

// src/reference_kernels.cpp:82-107.
std::vector<PageId> SelectTopKPagesCpu(std::vector<PageScore> scores, int top_k) {
  if (top_k <= 0 || scores.empty()) return {};
  std::vector<float> s(scores.size());
  std::vector<int> ids(scores.size());
  for (std::size_t i = 0; i < scores.size(); ++i) {
    s[i] = scores[i].score;
    ids[i] = scores[i].page_id;
  }
  std::vector<int> out(static_cast<std::size_t>(top_k < static_cast<int>(s.size())
                                                    ? top_k
                                                    : static_cast<int>(s.size())));
  const int n = oracle_select_topk(s.data(), ids.data(), static_cast<int>(s.size()), top_k,
                                   out.data());
  out.resize(static_cast<std::size_t>(n));
  return out;
}

// src/reference_kernels.cpp:109-147.
GatheredPages GatherPagesCpu(const PagedKvCache& cache, const std::vector<PageId>& page_ids,
                             const ModelConfig& config) {
  GatheredPages g;
  g.page_ids = page_ids;
  const int E = config.num_heads * config.head_dim;
  int running = 0;
  for (PageId id : page_ids) {
    const auto& page = cache.GetPage(id);
    g.token_offsets.push_back(running);
    g.token_counts.push_back(page.token_count);
    running += page.token_count;
    const auto k = cache.CopyPageKeys(id);
    const auto v = cache.CopyPageValues(id);
    g.keys.insert(g.keys.end(), k.begin(), k.end());
    g.values.insert(g.values.end(), v.begin(), v.end());
  }
  const std::size_t expected = static_cast<std::size_t>(running) * E;
  if (g.keys.size() != expected || g.values.size() != expected) {
    throw std::runtime_error("gather stage produced an inconsistent layout");
  }
  return g;
}

// src/reference_kernels.cpp:149-194: the gathered tokens, in order, are
// attended as one-token pages so the oracle's pool-indexed loop visits them
// in the same sequence.
AttentionResult SparseAttentionCpu(const std::vector<float>& query,
                                   const GatheredPages& gathered, const ModelConfig& config) {
  const int E = config.num_heads * config.head_dim;
  if (static_cast<int>(query.size()) != E) {
    throw std::invalid_argument("query length does not match model config");
  }
  const int tokens = static_cast<int>(gathered.keys.size()) / E;
  AttentionResult r;
  r.output.assign(static_cast<std::size_t>(E), 0.0f);
  if (tokens == 0) return r;
  std::vector<int> ones(static_cast<std::size_t>(tokens), 1);
  std::vector<int> ids(static_cast<std::size_t>(tokens));
  for (int t = 0; t < tokens; ++t) ids[static_cast<std::size_t>(t)] = t;
  oracle_attention(query.data(), gathered.keys.data(), gathered.values.data(), ones.data(),
                   ids.data(), tokens, config.num_heads, config.head_dim, 1, r.output.data());
  return r;
}

// src/reference_kernels.cpp:196-203.
AttentionResult DenseAttentionCpu(const PagedKvCache& cache, const RequestState& request,
                                  const ModelConfig& config) {
  return SparseAttentionCpu(request.query, GatherPagesCpu(cache, request.candidate_page_ids,
                                                          config),
                            config);
}

// src/reference_kernels.cpp:205-217.
float MaxAbsDiff(const std::vector<float>& lhs, const std::vector<float>& rhs) {
  if (lhs.size() != rhs.size()) return std::numeric_limits<float>::infinity();
  return oracle_max_abs_diff(lhs.data(), static_cast<int64_t>(lhs.size()), rhs.data(),
                             static_cast<int64_t>(rhs.size()));
}

// src/decode_pipeline.cpp:13-46.
SparseDecodeResult DecodePipeline::RunNaiveSparseStep(const PagedKvCache& cache,
                                                      const RequestState& request) const {
  SparseDecodeResult result;
  result.request_id = request.request_id;
  GatheredPages gathered;
  {
    ScopedStageTimer total(&result.timings.total_ms);
    {
      ScopedStageTimer t(&result.timings.page_scoring_ms);
      result.scores = ScorePagesCpu(cache, request, config_);
    }
    {
      ScopedStageTimer t(&result.timings.topk_ms);
      result.selected_page_ids = SelectTopKPagesCpu(result.scores, config_.top_k_pages);
    }
    {
      ScopedStageTimer t(&result.timings.gather_ms);
      gathered = GatherPagesCpu(cache, result.selected_page_ids, config_);
    }
    {
      ScopedStageTimer t(&result.timings.attention_ms);
      result.output = SparseAttentionCpu(request.query, gathered, config_);
    }
  }
  return result;
}

// src/decode_pipeline.cpp:48-52.
AttentionResult DecodePipeline::RunDenseStep(const PagedKvCache& cache,
                                             const RequestState& request) const {
  return DenseAttentionCpu(cache, request, config_);
}

// src/decode_pipeline.cpp:89-107.
BatchDecodeResult DecodePipeline::RunNaiveSparseBatch(
    const PagedKvCache& cache, const std::vector<RequestState>& requests) const {
  BatchDecodeResult batch;
  batch.per_request.reserve(requests.size());
  for (const auto& request : requests) {
    auto r = RunNaiveSparseStep(cache, request);
    batch.aggregate_timings.page_scoring_ms += r.timings.page_scoring_ms;
    batch.aggregate_timings.topk_ms += r.timings.topk_ms;
    batch.aggregate_timings.gather_ms += r.timings.gather_ms;
    batch.aggregate_timings.attention_ms += r.timings.attention_ms;
    batch.aggregate_timings.total_ms += r.timings.total_ms;
    batch.per_request.push_back(std::move(r));
  }
  return batch;
}

}  // namespace dsd
