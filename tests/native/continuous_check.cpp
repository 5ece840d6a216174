// continuous_check.cpp -- the continuous-batching serving loop
// (RunContinuousSparseDecode, reference src/continuous_batching.cpp:392-741)
// checked step by step against the CPU oracle.
//
// The loop runs as a caller runs it (this build's libdsd.so, on the GPU).  A
// step observer (include/dsd/step_observer.h) hands every `every`-th step's
// requests, page lists, queries, selected ids and outputs to this program.
// For each request of such a step it rebuilds, independently of the loop,
// what that request's pages hold at that step:
//   * prompt pages: the workload's prompt K/V (BuildSyntheticContinuousWorkload,
//     whose values the CPU suite pins against the reference's own build),
//     summaries by the host rule (oracle_page_summary);
//   * decode pages: with GPU-side admission the first decode token opens a
//     new page (:614-624); token i < decode_step has K/V =
//     DeterministicTokenVector(E, id, i, 1 / 2) (oracle_token_vector, pinned
//     against the reference) and the page summary is the running mean
//     (oracle_append_summary, src/paged_kv_cache.cpp:299-306);
//   * the query: the initial query at decode step 0, else
//     DeterministicTokenVector(E, id, decode_step, 0).
// With DSD_PAYLOAD_DIST=normal (the N(0, 1) payload mode) the prompts and
// decode tokens are the N(0, 1) generator's (oracle_prompt_normal /
// oracle_token_vector_normal restate it; the prompts are checked against
// that restatement on the CPU).
// Then the oracle's sparse_cpu rows (score, top-k with the reference's
// tie-break on the real page ids, gather + attention) give the expected
// selection, which must equal the device's id for id, and the expected
// output, within 1e-4 of the device's.
//
//   continuous_check num_requests max_active window min_prompt max_prompt
//                    min_decode max_decode seed heads head_dim page_size top_k
//                    every [precompute]
// Prints one line per checked step and a summary; exit status 0 when every
// checked request matches.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <string>
#include <vector>

#include "dsd/continuous_batching.h"
#include "dsd/step_observer.h"
#include "dsd_oracle.h"

namespace {

struct Args {
  int num_requests, max_active, window, min_prompt, max_prompt, min_decode, max_decode, seed;
  int heads, head_dim, page_size, top_k, every, precompute;
};

// The decode payload generator of the mode the loop runs in: the reference's
// U(-1, 1), or N(0, 1) when DSD_PAYLOAD_DIST=normal (oracle restatements).
void token_vector(int count, int request_id, int decode_step, int stream, float* out) {
  const char* e = std::getenv("DSD_PAYLOAD_DIST");
  if (e != nullptr && std::string(e) == "normal") {
    oracle_token_vector_normal(count, request_id, decode_step, stream, out);
  } else {
    oracle_token_vector(count, request_id, decode_step, stream, out);
  }
}

int Check(const Args& a, const std::vector<dsd::ContinuousRequestSpec>& specs,
          const dsd::ObservedDecodeStep& s, double* worst, long* requests) {
  const int E = a.heads * a.head_dim;
  const int ps = a.page_size;
  const float scale = oracle_scale(a.head_dim);
  std::map<int, const dsd::ContinuousRequestSpec*> by_id;
  for (const auto& sp : specs) by_id[sp.request_id] = &sp;
  const int B = static_cast<int>(s.request_ids.size());
  int failures = 0;
  int sel_at = 0;
  double step_worst = 0.0;
  for (int b = 0; b < B; ++b) {
    const auto& sp = *by_id.at(s.request_ids[b]);
    const int rid = sp.request_id;
    const int d = s.decode_steps[b];
    const int n = s.cand_offsets[b + 1] - s.cand_offsets[b];
    const int* pages = s.cand_ids.data() + s.cand_offsets[b];
    const int prompt_pages = (sp.prompt_tokens + ps - 1) / ps;
    const int decode_pages = (d + ps - 1) / ps;
    const int kk = std::min(a.top_k, n);
    const int got_k = s.selected_counts[b];
    const int* got_sel = s.selected.data() + sel_at;
    sel_at += got_k;
    if (n != prompt_pages + decode_pages) {
      std::printf("FAIL step %d request %d: %d pages, expected %d + %d\n", s.step, rid, n,
                  prompt_pages, decode_pages);
      ++failures;
      continue;
    }
    std::vector<float> keys(static_cast<size_t>(n) * ps * E, 0.0f);
    std::vector<float> values(keys.size(), 0.0f);
    std::vector<float> summ(static_cast<size_t>(n) * E, 0.0f);
    std::vector<int> counts(n, 0);
    for (int j = 0; j < prompt_pages; ++j) {
      const int t0 = j * ps;
      const int c = std::min(ps, sp.prompt_tokens - t0);
      counts[j] = c;
      std::copy(sp.prompt_keys.begin() + static_cast<size_t>(t0) * E,
                sp.prompt_keys.begin() + static_cast<size_t>(t0 + c) * E,
                keys.begin() + static_cast<size_t>(j) * ps * E);
      std::copy(sp.prompt_values.begin() + static_cast<size_t>(t0) * E,
                sp.prompt_values.begin() + static_cast<size_t>(t0 + c) * E,
                values.begin() + static_cast<size_t>(j) * ps * E);
      oracle_page_summary(keys.data() + static_cast<size_t>(j) * ps * E, c, E,
                          summ.data() + static_cast<size_t>(j) * E);
    }
    for (int i = 0; i < d; ++i) {
      const int j = prompt_pages + i / ps;
      const int off = i % ps;
      float* k = keys.data() + (static_cast<size_t>(j) * ps + off) * E;
      float* v = values.data() + (static_cast<size_t>(j) * ps + off) * E;
      token_vector(E, rid, i, 1, k);
      token_vector(E, rid, i, 2, v);
      oracle_append_summary(summ.data() + static_cast<size_t>(j) * E, k, off, E);
      counts[j] = off + 1;
    }
    std::vector<float> q(E);
    if (d == 0) {
      q = sp.initial_query;
    } else {
      token_vector(E, rid, d, 0, q.data());
    }
    const float* got_q = s.queries.data() + static_cast<size_t>(b) * E;
    if (!std::equal(q.begin(), q.end(), got_q)) {
      std::printf("FAIL step %d request %d: the loop's query differs from the oracle's\n",
                  s.step, rid);
      ++failures;
      continue;
    }
    std::vector<int> pos(n);
    for (int j = 0; j < n; ++j) pos[j] = j;
    std::vector<float> scores(n);
    oracle_score_pages(q.data(), summ.data(), counts.data(), pos.data(), n, E, scale,
                       scores.data());
    std::vector<int> sel(std::max(1, kk));
    const int m = oracle_select_topk(scores.data(), pages, n, a.top_k, sel.data());
    bool same = m == got_k;
    for (int j = 0; same && j < m; ++j) same = sel[j] == got_sel[j];
    if (!same) {
      std::printf("FAIL step %d request %d: selection differs (%d vs %d ids)\n", s.step, rid,
                  got_k, m);
      ++failures;
      continue;
    }
    std::vector<int> sel_pos(std::max(1, m));
    for (int j = 0; j < m; ++j) {
      sel_pos[j] = static_cast<int>(std::find(pages, pages + n, sel[j]) - pages);
    }
    std::vector<float> out(E);
    oracle_attention(q.data(), keys.data(), values.data(), counts.data(), sel_pos.data(), m,
                     a.heads, a.head_dim, ps, out.data());
    const float diff = oracle_max_abs_diff(out.data(), E,
                                           s.outputs.data() + static_cast<size_t>(b) * E, E);
    step_worst = std::max(step_worst, static_cast<double>(diff));
    if (!(diff <= 1e-4f)) {
      std::printf("FAIL step %d request %d: output max abs diff %.3g\n", s.step, rid, diff);
      ++failures;
    }
    ++*requests;
  }
  *worst = std::max(*worst, step_worst);
  std::printf("step %d: %d requests, max abs diff %.3g, %d failures\n", s.step, B, step_worst,
              failures);
  std::fflush(stdout);
  return failures;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 14) {
    std::fprintf(stderr,
                 "usage: %s requests max_active window min_prompt max_prompt min_decode "
                 "max_decode seed heads head_dim page_size top_k every [precompute]\n",
                 argv[0]);
    return 2;
  }
  Args a{};
  int* fields[] = {&a.num_requests, &a.max_active, &a.window,   &a.min_prompt, &a.max_prompt,
                   &a.min_decode,   &a.max_decode, &a.seed,     &a.heads,      &a.head_dim,
                   &a.page_size,    &a.top_k,      &a.every};
  for (int i = 0; i < 13; ++i) *fields[i] = std::atoi(argv[i + 1]);
  a.precompute = argc > 14 ? std::atoi(argv[14]) : 0;
  if (!dsd::SparseAttentionCudaAvailable()) {
    std::printf("continuous check skipped: no visible gfx950 GPU\n");
    return 3;
  }
  dsd::ModelConfig config;
  config.num_heads = a.heads;
  config.head_dim = a.head_dim;
  config.page_size = a.page_size;
  config.top_k_pages = a.top_k;
  const auto specs = dsd::BuildSyntheticContinuousWorkload(
      config, a.num_requests, a.window, a.min_prompt, a.max_prompt, a.min_decode, a.max_decode,
      a.seed);
  std::vector<dsd::ObservedDecodeStep> seen;
  dsd::SetContinuousStepObserver([&](const dsd::ObservedDecodeStep& s) { seen.push_back(s); },
                                 a.every);
  dsd::ContinuousDecodeOptions options;
  options.max_active_requests = a.max_active;
  options.prompt_admission_mode = dsd::ContinuousPromptAdmissionMode::kDirectGpuUpload;
  options.lazy_release = false;
  options.precompute_decode_payloads = a.precompute != 0;
  const auto stats = dsd::RunContinuousSparseDecode(config, specs, options);
  dsd::SetContinuousStepObserver(nullptr, 0);
  std::printf("loop: %d tokens, %.1f tokens/s, avg active %.2f, %zu steps observed\n",
              stats.total_generated_tokens, stats.tokens_per_second,
              stats.avg_active_batch_size, seen.size());
  std::fflush(stdout);
  int failures = 0;
  long requests = 0;
  double worst = 0.0;
  for (const auto& s : seen) failures += Check(a, specs, s, &worst, &requests);
  std::printf("continuous check: %zu steps, %ld request-steps, max abs diff %.3g, %d failures\n",
              seen.size(), requests, worst, failures);
  return failures == 0 && !seen.empty() ? 0 : 1;
}
