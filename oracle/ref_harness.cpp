// ref_harness.cpp -- extern "C" probe around the reference's own CPU units.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles this file together with
// the reference's CPU translation units, in place under /root/reference, into
// oracle/_ref/libdsd_ref.so.  Tests use it to pin the C oracle (and the
// product's synthetic-data generator) against the reference's own code:
// BuildSyntheticBatch (src/synthetic_data.cpp:23-68), the sparse_cpu step
// (src/decode_pipeline.cpp:13-46), dense_cpu (src/reference_kernels.cpp:196)
// BuildSyntheticContinuousWorkload (src/continuous_batching.cpp:336-381)
// and the decode-token running mean (PagedKvCache::AppendToken /
// AppendTokenMetadataOnly, src/paged_kv_cache.cpp:182-306).
#include <algorithm>
#include <cstring>
#include <vector>

#include "dsd/config.h"
#include "dsd/continuous_batching.h"
#include "dsd/decode_pipeline.h"
#include "dsd/paged_kv_cache.h"
#include "dsd/reference_kernels.h"
#include "dsd/synthetic_data.h"

namespace {

struct RefBatch {
  dsd::ModelConfig config;
  dsd::SyntheticBatch batch;
  RefBatch(const dsd::ModelConfig& c, dsd::SyntheticBatch&& b)
      : config(c), batch(std::move(b)) {}
};

dsd::ModelConfig MakeConfig(int heads, int head_dim, int page_size, int top_k) {
  dsd::ModelConfig c;
  c.num_heads = heads;
  c.head_dim = head_dim;
  c.page_size = page_size;
  c.top_k_pages = top_k;
  return c;
}

}  // namespace

extern "C" {

void* ref_batch_build(int heads, int head_dim, int page_size, int top_k,
                      int batch, int min_ctx, int max_ctx, int seed) {
  const auto config = MakeConfig(heads, head_dim, page_size, top_k);
  auto built = dsd::BuildSyntheticBatch(config, batch, min_ctx, max_ctx, seed);
  return new RefBatch(config, std::move(built));
}

void ref_batch_free(void* handle) { delete static_cast<RefBatch*>(handle); }

// capacity pages and total candidate count.
void ref_batch_info(void* handle, int* capacity, int* total_candidates) {
  const auto* h = static_cast<RefBatch*>(handle);
  *capacity = h->batch.cache.CapacityPages();
  int total = 0;
  for (const auto& r : h->batch.requests) {
    total += static_cast<int>(r.candidate_page_ids.size());
  }
  *total_candidates = total;
}

void ref_batch_get(void* handle, int* ctx_tokens, int* cand_offsets,
                   int* cand_ids, int* token_counts, float* key_pool,
                   float* value_pool, float* summaries, float* queries) {
  const auto* h = static_cast<RefBatch*>(handle);
  const auto& cache = h->batch.cache;
  const int ept = h->config.num_heads * h->config.head_dim;
  int offset = 0;
  cand_offsets[0] = 0;
  for (std::size_t r = 0; r < h->batch.requests.size(); ++r) {
    const auto& req = h->batch.requests[r];
    ctx_tokens[r] = req.context_tokens;
    for (int id : req.candidate_page_ids) cand_ids[offset++] = id;
    cand_offsets[r + 1] = offset;
    std::memcpy(queries + r * static_cast<std::size_t>(ept), req.query.data(),
                sizeof(float) * static_cast<std::size_t>(ept));
  }
  for (const auto& page : cache.Pages()) {
    token_counts[page.id] = page.token_count;
  }
  std::memcpy(key_pool, cache.KeyPool().data(),
              sizeof(float) * cache.KeyPool().size());
  std::memcpy(value_pool, cache.ValuePool().data(),
              sizeof(float) * cache.ValuePool().size());
  std::memcpy(summaries, cache.PageSummaryPool().data(),
              sizeof(float) * cache.PageSummaryPool().size());
}

// sparse_cpu through the reference DecodePipeline.  selected is [B][top_k].
void ref_batch_sparse_cpu(void* handle, float* scores, int* selected,
                          int* counts, float* outputs) {
  const auto* h = static_cast<RefBatch*>(handle);
  dsd::DecodePipeline pipeline(h->config);
  const int ept = h->config.num_heads * h->config.head_dim;
  int offset = 0;
  for (std::size_t r = 0; r < h->batch.requests.size(); ++r) {
    const auto res = pipeline.RunNaiveSparseStep(h->batch.cache, h->batch.requests[r]);
    for (const auto& s : res.scores) scores[offset++] = s.score;
    counts[r] = static_cast<int>(res.selected_page_ids.size());
    for (std::size_t j = 0; j < res.selected_page_ids.size(); ++j) {
      selected[r * static_cast<std::size_t>(h->config.top_k_pages) + j] =
          res.selected_page_ids[j];
    }
    std::memcpy(outputs + r * static_cast<std::size_t>(ept),
                res.output.output.data(), sizeof(float) * static_cast<std::size_t>(ept));
  }
}

void ref_batch_dense_cpu(void* handle, float* outputs) {
  const auto* h = static_cast<RefBatch*>(handle);
  dsd::DecodePipeline pipeline(h->config);
  const int ept = h->config.num_heads * h->config.head_dim;
  for (std::size_t r = 0; r < h->batch.requests.size(); ++r) {
    const auto out = pipeline.RunDenseStep(h->batch.cache, h->batch.requests[r]);
    std::memcpy(outputs + r * static_cast<std::size_t>(ept), out.output.data(),
                sizeof(float) * static_cast<std::size_t>(ept));
  }
}

// Decode-token appends through the reference's own PagedKvCache
// (src/paged_kv_cache.cpp:182-242 AppendToken, :244-306
// AppendTokenMetadataOnly): `tokens` rows of keys (and values) appended to
// request 0 in order, a fresh page forced where force_new[t] != 0; the
// cache's summary row of every page the request holds is copied out in list
// order (n_pages rows of heads * head_dim floats, at most max_pages), with
// each page's token count.  metadata_only selects AppendTokenMetadataOnly
// (values unused).  Returns the page count.
int ref_append_tokens(int heads, int head_dim, int page_size, int capacity, int tokens,
                      const float* keys, const float* values, const unsigned char* force_new,
                      int metadata_only, int max_pages, float* summaries, int* token_counts) {
  const auto config = MakeConfig(heads, head_dim, page_size, 8);
  dsd::PagedKvCache cache(config, capacity, metadata_only == 0);
  const std::size_t ept = static_cast<std::size_t>(heads) * head_dim;
  std::vector<int> pages;
  for (int t = 0; t < tokens; ++t) {
    const bool fresh = force_new != nullptr && force_new[t] != 0;
    const auto res = metadata_only != 0
                         ? cache.AppendTokenMetadataOnly(0, keys + t * ept, fresh)
                         : cache.AppendToken(0, keys + t * ept, values + t * ept, fresh);
    if (res.allocated_new_page) pages.push_back(res.page_id);
  }
  const int n = static_cast<int>(pages.size());
  for (int j = 0; j < n && j < max_pages; ++j) {
    const float* s = cache.PageSummaryPool().data() + static_cast<std::size_t>(pages[j]) * ept;
    std::memcpy(summaries + j * ept, s, sizeof(float) * ept);
    token_counts[j] = cache.Pages()[static_cast<std::size_t>(pages[j])].token_count;
  }
  return n;
}

// Continuous workload (src/continuous_batching.cpp:336-381).  Returns the
// request count; meta is [n][4] = request_id, arrival, prompt_tokens,
// decode_steps; the sums are per-request float sums of prompt keys, prompt
// values and the initial query (a compact fingerprint of the payloads).
int ref_workload(int heads, int head_dim, int page_size, int top_k,
                 int num_requests, int window, int min_prompt, int max_prompt,
                 int min_decode, int max_decode, int seed, int* meta,
                 double* sums) {
  const auto config = MakeConfig(heads, head_dim, page_size, top_k);
  const auto specs = dsd::BuildSyntheticContinuousWorkload(
      config, num_requests, window, min_prompt, max_prompt, min_decode,
      max_decode, seed);
  for (std::size_t i = 0; i < specs.size(); ++i) {
    const auto& s = specs[i];
    meta[4 * i + 0] = s.request_id;
    meta[4 * i + 1] = s.arrival_step;
    meta[4 * i + 2] = s.prompt_tokens;
    meta[4 * i + 3] = s.decode_steps;
    double a = 0.0, b = 0.0, c = 0.0;
    for (float x : s.prompt_keys) a += x;
    for (float x : s.prompt_values) b += x;
    for (float x : s.initial_query) c += x;
    sums[3 * i + 0] = a;
    sums[3 * i + 1] = b;
    sums[3 * i + 2] = c;
  }
  return static_cast<int>(specs.size());
}

}  // extern "C"
