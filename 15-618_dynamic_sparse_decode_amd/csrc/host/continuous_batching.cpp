// continuous_batching.cpp -- the continuous-batching serving loop (behaviour
// of reference src/continuous_batching.cpp:24-1039): workload generation,
// the three prompt admission modes, per-step RunBatch over the active set,
// decode-token append (host payloads, or device-generated in the synthetic
// mode), page release, and the step statistics.  Every device-side update
// goes through SparseCudaContext / DenseCudaContext (libdsd_hip.so).
#include "dsd/continuous_batching.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <condition_variable>
#include <deque>
#include <memory>
#include <mutex>
#include <thread>
#include <numeric>
#include <random>
#include <stdexcept>
#include <string>
#include <unordered_set>
#include <utility>

#include "dsd/cuda_dense_attention.h"
#include "dsd/paged_kv_cache.h"
#include "dsd/reference_kernels.h"
#include "dsd/step_observer.h"
#include "dsd_hip.h"
#include "host_workers.h"
#include "status.h"

namespace dsd {

namespace {

using Clock = std::chrono::steady_clock;

ContinuousStepObserver g_observer;
int g_observe_every = 0;

double Ms(Clock::time_point a, Clock::time_point b) {
  return std::chrono::duration<double, std::milli>(b - a).count();
}

int Ept(const ModelConfig& c) { return c.num_heads * c.head_dim; }

int PagesFor(const ModelConfig& c, int tokens) {
  return tokens <= 0 ? 0 : (tokens + c.page_size - 1) / c.page_size;
}

std::vector<float> Uniform(int count, std::mt19937& rng) {
  std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
  std::vector<float> v(static_cast<std::size_t>(count));
  for (float& x : v) x = dist(rng);
  return v;
}

// Seed of the per-(request, step, stream) decode payload generator
// (reference src/continuous_batching.cpp:44-59); streams 0 = next query,
// 1 = key, 2 = value.
std::uint32_t StepSeed(int request_id, int decode_step, int stream) {
  std::uint32_t x = 0x9e3779b9u;
  x ^= static_cast<std::uint32_t>(request_id) + 0x85ebca6bu + (x << 6) + (x >> 2);
  x ^= static_cast<std::uint32_t>(decode_step) + 0xc2b2ae35u + (x << 6) + (x >> 2);
  x ^= static_cast<std::uint32_t>(stream) + 0x27d4eb2fu + (x << 6) + (x >> 2);
  return x;
}

// The payload distribution of the synthetic serving workload: the
// reference's U(-1, 1) (src/continuous_batching.cpp:35-42), or N(0, 1) when
// the environment sets DSD_PAYLOAD_DIST=normal (BASELINE config 5 states
// N(0, 1) decode K/V; the reference has no such mode).  Read once.
bool NormalPayloads() {
  static const bool normal = [] {
    const char* e = std::getenv("DSD_PAYLOAD_DIST");
    return e != nullptr && std::strcmp(e, "normal") == 0;
  }();
  return normal;
}

// N(0, 1) floats by the Box-Muller transform (Box and Muller, Ann. Math.
// Statist. 29(2), 1958) on consecutive pairs of 32-bit draws a, b:
// u1 = (a + 1/2) 2^-32 in (0, 1), u2 = b 2^-32, r = sqrt(-2 ln u1),
// z0 = fl(r cos(2 pi u2)), z1 = fl(r sin(2 pi u2)), in double with libm; an
// odd count ends with a pair's z0.
std::vector<float> Normal(int count, std::mt19937& rng) {
  std::vector<float> v(static_cast<std::size_t>(count));
  for (int i = 0; i < count; i += 2) {
    const double u1 = (static_cast<double>(rng()) + 0.5) * 0x1p-32;
    const double u2 = static_cast<double>(rng()) * 0x1p-32;
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double t = 6.283185307179586476925 * u2;
    v[static_cast<std::size_t>(i)] = static_cast<float>(r * std::cos(t));
    if (i + 1 < count) v[static_cast<std::size_t>(i) + 1] = static_cast<float>(r * std::sin(t));
  }
  return v;
}

std::vector<float> TokenVector(int count, int request_id, int decode_step, int stream) {
  std::mt19937 rng(StepSeed(request_id, decode_step, stream));
  return NormalPayloads() ? Normal(count, rng) : Uniform(count, rng);
}

int CapacityFor(const ModelConfig& c, const std::vector<ContinuousRequestSpec>& specs) {
  int pages = 0;
  for (const auto& s : specs) pages += PagesFor(c, s.prompt_tokens) + PagesFor(c, s.decode_steps);
  return std::max(pages, 1);
}

int MaxPagesPerRequest(const ModelConfig& c, const std::vector<ContinuousRequestSpec>& specs) {
  int m = 0;
  for (const auto& s : specs) {
    m = std::max(m, PagesFor(c, s.prompt_tokens) + PagesFor(c, s.decode_steps));
  }
  return std::max(m, 1);
}

void Add(StageTimings* d, const StageTimings& s) {
  d->page_scoring_ms += s.page_scoring_ms;
  d->topk_ms += s.topk_ms;
  d->gather_ms += s.gather_ms;
  d->attention_ms += s.attention_ms;
  d->total_ms += s.total_ms;
}

void Add(RuntimeOverheadTimings* d, const RuntimeOverheadTimings& s) {
  d->time_malloc_ms += s.time_malloc_ms;
  d->time_memcpy_h2d_ms += s.time_memcpy_h2d_ms;
  d->time_memcpy_d2h_ms += s.time_memcpy_d2h_ms;
  d->time_free_ms += s.time_free_ms;
  d->time_kernel_launch_ms += s.time_kernel_launch_ms;
  d->time_sync_ms += s.time_sync_ms;
  d->time_prepare_sparse_layout_ms += s.time_prepare_sparse_layout_ms;
}

void Add(DeviceTransferStats* d, const DeviceTransferStats& s) {
  d->h2d_bytes += s.h2d_bytes;
  d->d2h_bytes += s.d2h_bytes;
  d->h2d_calls += s.h2d_calls;
  d->d2h_calls += s.d2h_calls;
  d->h2d_large_calls += s.h2d_large_calls;
  d->d2h_large_calls += s.d2h_large_calls;
}

void Scale(StageTimings* t, double f) {
  t->page_scoring_ms *= f;
  t->topk_ms *= f;
  t->gather_ms *= f;
  t->attention_ms *= f;
  t->total_ms *= f;
}

void Scale(RuntimeOverheadTimings* t, double f) {
  t->time_malloc_ms *= f;
  t->time_memcpy_h2d_ms *= f;
  t->time_memcpy_d2h_ms *= f;
  t->time_free_ms *= f;
  t->time_kernel_launch_ms *= f;
  t->time_sync_ms *= f;
  t->time_prepare_sparse_layout_ms *= f;
}

double Percentile(std::vector<double> v, double q) {
  if (v.empty()) return 0.0;
  std::sort(v.begin(), v.end());
  const double pos = q * static_cast<double>(v.size() - 1);
  const auto lo = static_cast<std::size_t>(std::floor(pos));
  const auto hi = static_cast<std::size_t>(std::ceil(pos));
  if (lo == hi) return v[lo];
  const double f = pos - static_cast<double>(lo);
  return v[lo] * (1.0 - f) + v[hi] * f;
}

void Validate(const ModelConfig& c, const std::vector<ContinuousRequestSpec>& specs) {
  const int E = Ept(c);
  std::unordered_set<int> ids;
  for (const auto& s : specs) {
    if (s.request_id < 0) throw std::invalid_argument("request_id must be non-negative");
    if (s.arrival_step < 0 || s.prompt_tokens < 0 || s.decode_steps < 0) {
      throw std::invalid_argument("continuous request counts must be non-negative");
    }
    const std::size_t n = static_cast<std::size_t>(s.prompt_tokens) * E;
    if (s.prompt_keys.size() != n || s.prompt_values.size() != n) {
      throw std::invalid_argument("prompt payload size does not match prompt_tokens");
    }
    if (static_cast<int>(s.initial_query.size()) != E) {
      throw std::invalid_argument("initial query size does not match model config");
    }
  }
  for (const auto& s : specs) {
    if (!ids.insert(s.request_id).second) {
      throw std::invalid_argument("continuous workload request_id values must be unique");
    }
  }
}

std::vector<int> PromptPageCounts(const ModelConfig& c, const ContinuousRequestSpec& s) {
  std::vector<int> counts;
  for (int t = 0; t < s.prompt_tokens; t += c.page_size) {
    counts.push_back(std::min(c.page_size, s.prompt_tokens - t));
  }
  return counts;
}

// kCpuCache admission: pages appended to the host cache.  A tail page that
// will receive decode tokens keeps a summary (reference :167-193).
std::vector<PageId> AdmitToCache(const ModelConfig& c, const ContinuousRequestSpec& s,
                                 PagedKvCache* cache) {
  const int E = Ept(c);
  std::vector<PageId> ids;
  for (int t = 0; t < s.prompt_tokens; t += c.page_size) {
    const int n = std::min(c.page_size, s.prompt_tokens - t);
    const bool tail = t + n == s.prompt_tokens;
    const bool summary = tail && n < c.page_size && s.decode_steps > 0;
    const std::size_t at = static_cast<std::size_t>(t) * E;
    ids.push_back(cache->AppendPage(s.request_id, s.prompt_keys.data() + at,
                                    s.prompt_values.data() + at, n, summary));
  }
  return ids;
}

std::vector<PageId> AdmitPrompt(const ModelConfig& c, const ContinuousRequestSpec& s,
                                ContinuousPromptAdmissionMode mode, PagedKvCache* cache,
                                SparseCudaContext* ctx) {
  if (mode == ContinuousPromptAdmissionMode::kCpuCache) {
    auto ids = AdmitToCache(c, s, cache);
    ctx->SyncPagesFromCache(*cache, ids);
    return ids;
  }
  const auto counts = PromptPageCounts(c, s);
  auto ids = cache->ReservePagesForRequest(s.request_id, counts);
  if (mode == ContinuousPromptAdmissionMode::kDirectGpuUpload) {
    ctx->SyncPromptDirect(*cache, ids, counts, s.prompt_keys.data(), s.prompt_values.data());
    return ids;
  }
  if (mode == ContinuousPromptAdmissionMode::kSyntheticGpuPrefill) {
    ctx->PrefillPromptSynthetic(*cache, ids, counts, s.request_id);
    return ids;
  }
  throw std::invalid_argument("unknown prompt admission mode");
}

// Pinned host memory from dsd_host_alloc: the device reads rows in it
// directly, so a step can take its queries in place.
class PinnedFloats {
 public:
  PinnedFloats() = default;
  explicit PinnedFloats(std::size_t count) {
    if (count == 0) return;
    void* p = nullptr;
    detail::ThrowOnError(dsd_host_alloc(sizeof(float) * count, &p));
    ptr_ = static_cast<float*>(p);
  }
  PinnedFloats(PinnedFloats&& o) noexcept : ptr_(o.ptr_) { o.ptr_ = nullptr; }
  PinnedFloats& operator=(PinnedFloats&& o) noexcept {
    std::swap(ptr_, o.ptr_);
    return *this;
  }
  PinnedFloats(const PinnedFloats&) = delete;
  PinnedFloats& operator=(const PinnedFloats&) = delete;
  ~PinnedFloats() {
    if (ptr_ != nullptr) (void)dsd_host_free(ptr_);
  }
  float* data() const { return ptr_; }

 private:
  float* ptr_ = nullptr;
};

// A dsd_device_alloc block of floats (HBM rows the steps read in place).
class DeviceFloats {
 public:
  DeviceFloats() = default;
  DeviceFloats(const float* host, std::size_t count) {
    if (count == 0) return;
    void* p = nullptr;
    detail::ThrowOnError(dsd_device_alloc(sizeof(float) * count, &p));
    ptr_ = static_cast<float*>(p);
    detail::ThrowOnError(dsd_device_upload(ptr_, host, sizeof(float) * count));
  }
  DeviceFloats(DeviceFloats&& o) noexcept : ptr_(o.ptr_) { o.ptr_ = nullptr; }
  DeviceFloats& operator=(DeviceFloats&& o) noexcept {
    std::swap(ptr_, o.ptr_);
    return *this;
  }
  DeviceFloats(const DeviceFloats&) = delete;
  DeviceFloats& operator=(const DeviceFloats&) = delete;
  ~DeviceFloats() {
    if (ptr_ != nullptr) (void)dsd_device_free(ptr_);
  }
  const float* data() const { return ptr_; }

 private:
  float* ptr_ = nullptr;
};

// DSD_QUERY_STORE=host keeps the pipelined loop's precomputed queries in
// pinned host memory only, read across PCIe by every step's stage-in.  By
// default the store is also uploaded to HBM with the payloads, where a
// model's own queries would be, and the steps read it there.
bool DeviceQueryStore() {
  static const bool on = [] {
    const char* e = std::getenv("DSD_QUERY_STORE");
    return e == nullptr || std::strcmp(e, "host") != 0;
  }();
  return on;
}

// The precomputed payloads (src/continuous_batching.cpp:272-300, :444-454): every
// request's next-step queries in one pinned block, request i's rows from
// query_row0[i] on (and, for the pipelined loop, a copy in HBM), and the
// appended keys / values per request.
struct DecodePayloads {
  PinnedFloats queries;
  DeviceFloats device_queries;
  std::size_t query_rows = 0;
  std::vector<std::size_t> query_row0;
  std::vector<std::vector<float>> keys, values;
  std::size_t RowOf(std::size_t spec, int step, int E) const {
    return (query_row0[spec] + static_cast<std::size_t>(step)) * static_cast<std::size_t>(E);
  }
  const float* NextQuery(std::size_t spec, int step, int E) const {
    return queries.data() + RowOf(spec, step, E);
  }
  // The HBM copy's row, or nullptr without one.
  const float* NextQueryDevice(std::size_t spec, int step, int E) const {
    return device_queries.data() == nullptr ? nullptr
                                            : device_queries.data() + RowOf(spec, step, E);
  }
};

// Every vector has its own seed, so the host threads form the requests'
// payloads in any order with the reference's values.
DecodePayloads BuildPayloads(const ModelConfig& c,
                             const std::vector<ContinuousRequestSpec>& specs, bool kv) {
  const int E = Ept(c);
  DecodePayloads p;
  p.query_row0.resize(specs.size());
  std::size_t rows = 0;
  for (std::size_t i = 0; i < specs.size(); ++i) {
    p.query_row0[i] = rows;
    rows += static_cast<std::size_t>(std::max(0, specs[i].decode_steps));
  }
  p.queries = PinnedFloats(rows * static_cast<std::size_t>(E));
  p.query_rows = rows;
  if (kv) {
    p.keys.resize(specs.size());
    p.values.resize(specs.size());
  }
  const std::size_t row_bytes = sizeof(float) * static_cast<std::size_t>(E);
  dsd_host::Workers::Get().ParallelFor(static_cast<int>(specs.size()), [&](int i) {
    const auto& s = specs[static_cast<std::size_t>(i)];
    const std::size_t steps = static_cast<std::size_t>(std::max(0, s.decode_steps));
    if (kv) {
      p.keys[static_cast<std::size_t>(i)].resize(steps * static_cast<std::size_t>(E));
      p.values[static_cast<std::size_t>(i)].resize(steps * static_cast<std::size_t>(E));
    }
    for (int step = 0; step < s.decode_steps; ++step) {
      const auto q = TokenVector(E, s.request_id, step + 1, 0);
      std::memcpy(const_cast<float*>(p.NextQuery(static_cast<std::size_t>(i), step, E)),
                  q.data(), row_bytes);
      if (kv) {
        const std::size_t at = static_cast<std::size_t>(step) * static_cast<std::size_t>(E);
        const auto k = TokenVector(E, s.request_id, step, 1);
        const auto v = TokenVector(E, s.request_id, step, 2);
        std::memcpy(p.keys[static_cast<std::size_t>(i)].data() + at, k.data(), row_bytes);
        std::memcpy(p.values[static_cast<std::size_t>(i)].data() + at, v.data(), row_bytes);
      }
    }
  });
  return p;
}

const float* Row(const std::vector<float>& v, int step, int E) {
  return v.data() + static_cast<std::size_t>(step) * static_cast<std::size_t>(E);
}

// An active request of the sparse loop: the reference's state plus where
// its next query lives: a row of the pinned payload store, which the step
// reads in place, or its own buffer, which the step copies into the
// context's pinned staging.
struct LiveRequest {
  ActiveDecodeRequest a;
  const float* query = nullptr;  // payload-store row when !own
  std::vector<float> query_buf;  // the query when own
  bool own = true;
  // The same query in HBM (the pipelined loop's device query store), read
  // by the step instead of `query`; nullptr when there is none.
  const float* device_query = nullptr;
  const float* Query() const { return own ? query_buf.data() : query; }
};

// DSD_VERIFY_STAGED=1 (a self-check for tests; the loop's step outputs are
// not otherwise observable): each staged step is run again through
// SparseCudaContext::RunBatch, whose packing copies every query and page
// list, and the two steps' outputs must agree bit for bit.
bool VerifyStagedSteps() {
  static const bool on = [] {
    const char* e = std::getenv("DSD_VERIFY_STAGED");
    return e != nullptr && std::strcmp(e, "0") != 0;
  }();
  return on;
}

long long g_verified_steps = 0;  // staged steps checked in this process

void VerifyStagedStep(SparseCudaContext& ctx, const PagedKvCache& cache,
                      const std::vector<LiveRequest>& active, int E) {
  using detail::ThrowOnError;
  float* staged_out = nullptr;
  ThrowOnError(dsd_sparse_staging(ctx.handle(), nullptr, nullptr, nullptr, &staged_out));
  const std::size_t B = active.size();
  const std::vector<float> staged(staged_out, staged_out + B * static_cast<std::size_t>(E));
  std::vector<RequestState> states(B);
  std::vector<const RequestState*> ptrs;
  for (std::size_t b = 0; b < B; ++b) {
    const LiveRequest& l = active[b];
    states[b].request_id = l.a.state.request_id;
    states[b].query.assign(l.Query(), l.Query() + E);
    states[b].candidate_page_ids = cache.GetRequestPages(l.a.state.request_id);
    states[b].context_tokens = l.a.state.context_tokens;
    ptrs.push_back(&states[b]);
  }
  SparseRunBatchOptions o;
  o.output_mode = SparseBatchOutputMode::kOutputsOnly;
  o.timing_mode = SparseBatchTimingMode::kNone;
  const auto check = ctx.RunBatch(ptrs, o);
  for (std::size_t b = 0; b < B; ++b) {
    const auto& out = check.per_request[b].output.output;
    if (out.size() != static_cast<std::size_t>(E) ||
        std::memcmp(out.data(), staged.data() + b * static_cast<std::size_t>(E),
                    sizeof(float) * static_cast<std::size_t>(E)) != 0) {
      throw std::runtime_error("staged step differs from RunBatch for request " +
                               std::to_string(states[b].request_id));
    }
  }
  ++g_verified_steps;
}

// One RunBatch of the loop in the outputs / no-outputs modes, on the C ABI:
// PackSparseBatchInto's checks and layout written into the pinned staging
// (candidate lists from the cache; queries that live in the pinned payload
// store are read in place, the others copied into the staging), the step,
// and the same timings RunBatch reports.  Outputs stay in the staging.
SparseBatchCudaResult StagedStep(SparseCudaContext& ctx, const PagedKvCache& cache,
                                 const std::vector<LiveRequest>& active, int E, int top_k,
                                 int max_batch, int max_candidates, int max_selected,
                                 const SparseRunBatchOptions& run,
                                 std::vector<const float*>* rows,
                                 ObservedDecodeStep* observe) {
  using detail::ThrowOnError;
  SparseBatchCudaResult result;
  const auto t0 = Clock::now();
  const int B = static_cast<int>(active.size());
  int total = 0;
  int total_selected = 0;
  for (const auto& l : active) {
    const int n = static_cast<int>(cache.GetRequestPages(l.a.state.request_id).size());
    total += n;
    total_selected += std::max(0, std::min(top_k, n));
  }
  if (B > max_batch) throw std::invalid_argument("request batch exceeds sparse context capacity");
  if (total > max_candidates) {
    throw std::invalid_argument("candidate page count exceeds sparse context capacity");
  }
  if (total_selected > max_selected) {
    throw std::invalid_argument("selected page count exceeds sparse context capacity");
  }
  float* queries = nullptr;
  int* offsets = nullptr;
  int* ids = nullptr;
  ThrowOnError(dsd_sparse_staging(ctx.handle(), &queries, &offsets, &ids, nullptr));
  offsets[0] = 0;
  int at = 0;
  bool in_place = false;
  rows->resize(static_cast<std::size_t>(B));
  for (int b = 0; b < B; ++b) {
    const LiveRequest& l = active[static_cast<std::size_t>(b)];
    float* row = queries + static_cast<std::size_t>(b) * E;
    if (l.own) {
      std::memcpy(row, l.query_buf.data(), sizeof(float) * E);
      (*rows)[static_cast<std::size_t>(b)] = row;
    } else {
      (*rows)[static_cast<std::size_t>(b)] = l.query;
      in_place = true;
    }
    const auto& pages = cache.GetRequestPages(l.a.state.request_id);
    const int n = static_cast<int>(pages.size());
    if (n > 0) std::memcpy(ids + at, pages.data(), sizeof(int) * n);
    at += n;
    offsets[b + 1] = at;
  }
  const double layout_ms = Ms(t0, Clock::now());
  const bool timing = run.timing_mode == SparseBatchTimingMode::kKernelEvents;
  const bool outputs = run.output_mode != SparseBatchOutputMode::kNoOutputs || observe;
  dsd_step_timings t{};
  const int out_mode = outputs ? DSD_OUTPUT_OUTPUTS : DSD_OUTPUT_NONE;
  const int time_mode = timing ? DSD_TIMING_EVENTS : DSD_TIMING_NONE;
  int* sel = nullptr;
  int* sel_counts = nullptr;
  if (observe != nullptr) {
    // The inputs as staged, before the step runs.
    observe->cand_offsets.assign(offsets, offsets + B + 1);
    observe->cand_ids.assign(ids, ids + at);
    observe->queries.resize(static_cast<std::size_t>(B) * E);
    for (int b = 0; b < B; ++b) {
      std::memcpy(observe->queries.data() + static_cast<std::size_t>(b) * E,
                  (*rows)[static_cast<std::size_t>(b)], sizeof(float) * E);
    }
    observe->selected.assign(static_cast<std::size_t>(std::max(1, total_selected)), 0);
    observe->selected_counts.assign(static_cast<std::size_t>(B), 0);
    sel = observe->selected.data();
    sel_counts = observe->selected_counts.data();
  }
  if (in_place) {
    ThrowOnError(dsd_sparse_run_staged_rows(ctx.handle(), B, rows->data(), out_mode, time_mode,
                                            sel, sel_counts, &t));
  } else {
    ThrowOnError(dsd_sparse_run_staged(ctx.handle(), B, out_mode, time_mode, sel, sel_counts,
                                       &t));
  }
  if (observe != nullptr) {
    float* staged_out = nullptr;
    ThrowOnError(dsd_sparse_staging(ctx.handle(), nullptr, nullptr, nullptr, &staged_out));
    observe->outputs.assign(staged_out, staged_out + static_cast<std::size_t>(B) * E);
    observe->selected.resize(static_cast<std::size_t>(total_selected));
  }
  if (VerifyStagedSteps()) VerifyStagedStep(ctx, cache, active, E);
  if (timing) {
    result.aggregate_timings.page_scoring_ms = t.score_ms;
    result.aggregate_timings.topk_ms = t.topk_ms;
    result.aggregate_timings.attention_ms = t.attention_ms;
    result.aggregate_timings.gather_ms = 0.0;  // fused into attention
    result.aggregate_timings.total_ms = t.score_ms + t.topk_ms + t.attention_ms;
    result.kernel_ms = result.aggregate_timings.total_ms;
    result.runtime_overheads.time_prepare_sparse_layout_ms = layout_ms;
    result.runtime_overheads.time_memcpy_h2d_ms = t.h2d_ms;
    result.runtime_overheads.time_memcpy_d2h_ms = t.d2h_ms;
    result.runtime_overheads.time_kernel_launch_ms = t.launch_ms;
    result.runtime_overheads.time_sync_ms = t.sync_ms;
  }
  return result;
}

// The loop's request -> page table in device memory (dsd_table beside the
// context's pool) and the slots of the admitted requests.  In the
// GPU-resident admission modes the loop keeps no page lists on the host:
// admission, append and release are table kernels, and each step's
// candidate lists are packed on the device from slot ids.  DSD_DEVICE_TABLE=0
// keeps the host lists (the reference's PagedKvCache) and stages each step's
// candidate lists from them instead.
bool DeviceTableEnabled() {
  static const bool on = [] {
    const char* e = std::getenv("DSD_DEVICE_TABLE");
    return e == nullptr || std::strcmp(e, "0") != 0;
  }();
  return on;
}

bool PrefetchEnabled() {
  static const bool on = [] {
    const char* e = std::getenv("DSD_PREFETCH");
    return e == nullptr || std::strcmp(e, "0") != 0;
  }();
  return on;
}
constexpr int kPrefetchDepth = 8;

class LoopTable {
 public:
  LoopTable(::dsd_pool* pool, int slots, int max_pages) {
    detail::ThrowOnError(dsd_table_create(pool, slots, max_pages, &t_));
    for (int s = slots - 1; s >= 0; --s) free_.push_back(s);
  }
  ~LoopTable() {
    if (t_ != nullptr) (void)dsd_table_destroy(t_);
  }
  LoopTable(const LoopTable&) = delete;
  LoopTable& operator=(const LoopTable&) = delete;
  ::dsd_table* get() const { return t_; }
  int Take(int request) {
    if (free_.empty()) throw std::runtime_error("device page table has no free slot");
    const int slot = free_.back();
    free_.pop_back();
    slot_of_[request] = slot;
    return slot;
  }
  int SlotOf(int request) const { return slot_of_.at(request); }
  // Releases the slots of `requests` (in order) in one call.
  void Release(const std::vector<int>& requests, bool clear) {
    if (requests.empty()) return;
    std::vector<int> slots;
    slots.reserve(requests.size());
    for (int id : requests) slots.push_back(slot_of_.at(id));
    detail::ThrowOnError(
        dsd_table_release(t_, static_cast<int>(slots.size()), slots.data(), clear ? 1 : 0));
    for (std::size_t i = 0; i < requests.size(); ++i) {
      slot_of_.erase(requests[i]);
      free_.push_back(slots[i]);
    }
  }

 private:
  ::dsd_table* t_ = nullptr;
  std::vector<int> free_;
  std::unordered_map<int, int> slot_of_;
};

// Prompt uploads ahead of admission (direct GPU upload through the table):
// a host thread of its own uploads the prompts in admission order (the
// workload's order) into `depth` device staging buffers in turn, on the
// table's copy stream, so the PCIe transfers run while the loop steps;
// admission then only waits for its prompt's upload on the device and
// fills its pages from the staging buffer.  The pages are still reserved at
// admission, in the reference's order.
class PromptPrefetcher {
 public:
  PromptPrefetcher(::dsd_table* table, const std::vector<ContinuousRequestSpec>& specs,
                   int depth)
      : table_(table), specs_(specs), depth_(depth) {
    int max_tokens = 1;
    for (const auto& s : specs) max_tokens = std::max(max_tokens, s.prompt_tokens);
    detail::ThrowOnError(dsd_table_staging_init(table, depth, max_tokens));
    thread_ = std::thread([this] { Run(); });
  }
  ~PromptPrefetcher() {
    {
      std::lock_guard<std::mutex> lock(mu_);
      stop_ = true;
    }
    cv_.notify_all();
    thread_.join();
  }
  PromptPrefetcher(const PromptPrefetcher&) = delete;
  PromptPrefetcher& operator=(const PromptPrefetcher&) = delete;
  // The staging buffer holding request i's prompt once its upload is
  // enqueued (call in increasing i, then Admitted(i)).
  int Await(std::size_t i) {
    std::unique_lock<std::mutex> lock(mu_);
    cv_.wait(lock, [&] { return staged_ > i || !error_.empty(); });
    if (!error_.empty()) throw std::runtime_error("prompt upload failed: " + error_);
    return static_cast<int>(i % static_cast<std::size_t>(depth_));
  }
  void Admitted(std::size_t i) {
    {
      std::lock_guard<std::mutex> lock(mu_);
      admitted_ = i + 1;
    }
    cv_.notify_all();
  }

 private:
  void Run() {
    const std::size_t depth = static_cast<std::size_t>(depth_);
    for (std::size_t i = 0; i < specs_.size(); ++i) {
      {
        // The buffer's previous prompt (request i - depth) is admitted.
        std::unique_lock<std::mutex> lock(mu_);
        cv_.wait(lock, [&] { return stop_ || i < depth || admitted_ >= i - depth + 1; });
        if (stop_) return;
      }
      const auto& s = specs_[i];
      if (dsd_table_stage_prompt(table_, static_cast<int>(i % depth), s.prompt_tokens,
                                 s.prompt_keys.data(), s.prompt_values.data()) != 0) {
        std::lock_guard<std::mutex> lock(mu_);
        error_ = dsd_last_error();
        cv_.notify_all();
        return;
      }
      {
        std::lock_guard<std::mutex> lock(mu_);
        staged_ = i + 1;
      }
      cv_.notify_all();
    }
  }

  ::dsd_table* table_;
  const std::vector<ContinuousRequestSpec>& specs_;
  int depth_;
  std::mutex mu_;
  std::condition_variable cv_;
  std::size_t staged_ = 0, admitted_ = 0;
  bool stop_ = false;
  std::string error_;
  std::thread thread_;
};

// DSD_PIPELINE=0 keeps the table loop's synchronous step (the reference's
// RunBatch shape: the host waits for every step).  By default the loop
// enqueues each step, its append and its release on the pool's stream
// without waiting (dsd_sparse_run_table_async) and forms the next step while
// the device runs them; the steps' device times are collected at the end.
bool PipelineEnabled() {
  static const bool on = [] {
    const char* e = std::getenv("DSD_PIPELINE");
    return e == nullptr || std::strcmp(e, "0") != 0;
  }();
  return on;
}

// The pinned payload rows of the pipelined loop, one slab per step in a ring
// of kSlabs.  The device reads a step's query rows when the step runs and
// its appended K/V rows when the append's copy runs, so the host writes
// step j's slab only after step j - kSlabs (for K/V, the step after it,
// which follows its append on the stream) has completed.  A query slab
// holds the queries generated after the previous step in rows
// [0, max_active) (row = the request's place in that step's batch) and the
// initial queries of the requests admitted for step j in rows
// [max_active, 2 max_active); a K/V slab holds the step's uploaded tokens in
// batch order.
class PayloadSlabs {
 public:
  static constexpr int kSlabs = 6;
  PayloadSlabs(int max_active, int E, bool kv) : max_(max_active), E_(E) {
    const std::size_t rows = static_cast<std::size_t>(max_active) * static_cast<std::size_t>(E);
    for (int i = 0; i < kSlabs; ++i) {
      q_.emplace_back(2 * rows);
      if (kv) {
        k_.emplace_back(rows);
        v_.emplace_back(rows);
      }
    }
  }
  float* Query(long long step, int row) const {
    return q_[Index(step)].data() + static_cast<std::size_t>(row) * static_cast<std::size_t>(E_);
  }
  float* Admitted(long long step, int n) const { return Query(step, max_ + n); }
  float* Keys(long long step) const { return k_[Index(step)].data(); }
  float* Values(long long step) const { return v_[Index(step)].data(); }

 private:
  static std::size_t Index(long long step) { return static_cast<std::size_t>(step % kSlabs); }
  int max_, E_;
  std::vector<PinnedFloats> q_, k_, v_;
};

// The pipelined loop's step tickets (index = the loop's step number) and
// the waits that guard the payload slabs.
class StepTickets {
 public:
  explicit StepTickets(::dsd_sparse_ctx* ctx) : ctx_(ctx) {}
  // On scope exit (also by an exception) every enqueued step has finished
  // before the slabs it reads are freed.
  ~StepTickets() {
    if (!tickets_.empty()) (void)dsd_device_synchronize();
  }
  StepTickets(const StepTickets&) = delete;
  StepTickets& operator=(const StepTickets&) = delete;
  void Push(long long ticket) { tickets_.push_back(ticket); }
  // Blocks until loop step `step` (if it ran) has completed.
  void WaitFor(long long step) const {
    if (step < 0 || step >= static_cast<long long>(tickets_.size())) return;
    detail::ThrowOnError(dsd_sparse_async_wait(ctx_, tickets_[static_cast<std::size_t>(step)]));
  }

 private:
  ::dsd_sparse_ctx* ctx_;
  std::vector<long long> tickets_;
};

// Prompt admission into the table (GPU-resident modes); with `mirror`, the
// host cache reserves the same pages (for verification).
void AdmitToTable(const ModelConfig& c, const ContinuousRequestSpec& s, std::size_t index,
                  ContinuousPromptAdmissionMode mode, LoopTable* table, PagedKvCache* mirror,
                  PromptPrefetcher* prefetch) {
  const int slot = table->Take(s.request_id);
  if (mirror != nullptr) mirror->ReservePagesForRequest(s.request_id, PromptPageCounts(c, s));
  if (prefetch != nullptr) {
    const int buffer = prefetch->Await(index);
    detail::ThrowOnError(
        dsd_table_admit_staged(table->get(), slot, buffer, s.prompt_tokens));
    prefetch->Admitted(index);
  } else if (mode == ContinuousPromptAdmissionMode::kDirectGpuUpload) {
    detail::ThrowOnError(dsd_table_admit_prompt(table->get(), slot, s.prompt_tokens,
                                                s.prompt_keys.data(), s.prompt_values.data()));
  } else {
    detail::ThrowOnError(
        dsd_table_admit_synthetic(table->get(), slot, s.prompt_tokens, s.request_id));
  }
}

// The observed step's page lists and outputs, once it has completed (its
// queries and selection are filled by the caller).
void ObserveTableStep(SparseCudaContext& ctx, const LoopTable& table,
                      const std::vector<int>& slots, int E, ObservedDecodeStep* observe) {
  using detail::ThrowOnError;
  const int B = static_cast<int>(slots.size());
  int total = 0;
  for (int slot : slots) {
    int n = 0;
    ThrowOnError(dsd_table_slot_pages(table.get(), slot, &n));
    total += n;
  }
  observe->cand_offsets.assign(static_cast<std::size_t>(B) + 1, 0);
  observe->cand_ids.assign(static_cast<std::size_t>(std::max(1, total)), 0);
  ThrowOnError(dsd_sparse_last_csr(ctx.handle(), B, observe->cand_offsets.data(),
                                   observe->cand_ids.data(), std::max(1, total)));
  observe->cand_ids.resize(static_cast<std::size_t>(total));
  int selected_total = 0;
  for (int b = 0; b < B; ++b) selected_total += observe->selected_counts[static_cast<std::size_t>(b)];
  observe->selected.resize(static_cast<std::size_t>(selected_total));
  float* staged_out = nullptr;
  ThrowOnError(dsd_sparse_staging(ctx.handle(), nullptr, nullptr, nullptr, &staged_out));
  observe->outputs.assign(staged_out, staged_out + static_cast<std::size_t>(B) * E);
}

// One step of the table loop: the queries as StagedStep takes them (rows
// in the pinned payload store read in place, the others copied into the
// staging), candidate lists from the table.  Outputs stay in the staging.
SparseBatchCudaResult TableStep(SparseCudaContext& ctx, const LoopTable& table,
                                const std::vector<LiveRequest>& active, int E, int top_k,
                                const SparseRunBatchOptions& run,
                                std::vector<const float*>* rows, ObservedDecodeStep* observe) {
  using detail::ThrowOnError;
  SparseBatchCudaResult result;
  const auto t0 = Clock::now();
  const int B = static_cast<int>(active.size());
  float* queries = nullptr;
  ThrowOnError(dsd_sparse_staging(ctx.handle(), &queries, nullptr, nullptr, nullptr));
  std::vector<int> slots(static_cast<std::size_t>(B));
  rows->resize(static_cast<std::size_t>(B));
  for (int b = 0; b < B; ++b) {
    const LiveRequest& l = active[static_cast<std::size_t>(b)];
    slots[static_cast<std::size_t>(b)] = table.SlotOf(l.a.state.request_id);
    if (l.own) {
      float* row = queries + static_cast<std::size_t>(b) * E;
      std::memcpy(row, l.query_buf.data(), sizeof(float) * E);
      (*rows)[static_cast<std::size_t>(b)] = row;
    } else {
      (*rows)[static_cast<std::size_t>(b)] = l.query;
    }
  }
  const double layout_ms = Ms(t0, Clock::now());
  const bool timing = run.timing_mode == SparseBatchTimingMode::kKernelEvents;
  const bool outputs = run.output_mode != SparseBatchOutputMode::kNoOutputs || observe;
  dsd_step_timings t{};
  int* sel = nullptr;
  int* sel_counts = nullptr;
  if (observe != nullptr) {
    observe->queries.resize(static_cast<std::size_t>(B) * E);
    for (int b = 0; b < B; ++b) {
      std::memcpy(observe->queries.data() + static_cast<std::size_t>(b) * E,
                  (*rows)[static_cast<std::size_t>(b)], sizeof(float) * E);
    }
    observe->selected.assign(static_cast<std::size_t>(B) * std::max(1, top_k), 0);
    observe->selected_counts.assign(static_cast<std::size_t>(B), 0);
    sel = observe->selected.data();
    sel_counts = observe->selected_counts.data();
  }
  ThrowOnError(dsd_sparse_run_table(ctx.handle(), table.get(), B, slots.data(), nullptr,
                                    rows->data(), outputs ? DSD_OUTPUT_OUTPUTS : DSD_OUTPUT_NONE,
                                    timing ? DSD_TIMING_EVENTS : DSD_TIMING_NONE, nullptr, sel,
                                    sel_counts, &t));
  if (observe != nullptr) ObserveTableStep(ctx, table, slots, E, observe);
  if (timing) {
    result.aggregate_timings.page_scoring_ms = t.score_ms;
    result.aggregate_timings.topk_ms = t.topk_ms;
    result.aggregate_timings.attention_ms = t.attention_ms;
    result.aggregate_timings.gather_ms = 0.0;  // fused into attention
    result.aggregate_timings.total_ms = t.score_ms + t.topk_ms + t.attention_ms;
    result.kernel_ms = result.aggregate_timings.total_ms;
    result.runtime_overheads.time_prepare_sparse_layout_ms = layout_ms;
    result.runtime_overheads.time_memcpy_h2d_ms = t.h2d_ms;
    result.runtime_overheads.time_memcpy_d2h_ms = t.d2h_ms;
    result.runtime_overheads.time_kernel_launch_ms = t.launch_ms;
    result.runtime_overheads.time_sync_ms = t.sync_ms;
  }
  return result;
}

// One step of the pipelined table loop (PipelineEnabled): every query row
// lies in pinned memory that stays unchanged until the step has completed
// (the payload store or a payload slab).  The step is enqueued and not
// waited for, unless it is observed; its device times are collected at the
// end of the loop (CollectPipelinedSteps).
SparseBatchCudaResult PipelinedTableStep(SparseCudaContext& ctx, const LoopTable& table,
                                         const std::vector<LiveRequest>& active, int E,
                                         int top_k, const SparseRunBatchOptions& run,
                                         std::vector<const float*>* rows,
                                         ObservedDecodeStep* observe, long long* ticket) {
  using detail::ThrowOnError;
  SparseBatchCudaResult result;
  const auto t0 = Clock::now();
  const int B = static_cast<int>(active.size());
  std::vector<int> slots(static_cast<std::size_t>(B));
  rows->resize(static_cast<std::size_t>(B));
  for (int b = 0; b < B; ++b) {
    const LiveRequest& l = active[static_cast<std::size_t>(b)];
    if (l.own) throw std::logic_error("a pipelined step's query is not in pinned memory");
    slots[static_cast<std::size_t>(b)] = table.SlotOf(l.a.state.request_id);
    (*rows)[static_cast<std::size_t>(b)] = l.device_query != nullptr ? l.device_query : l.query;
  }
  const double layout_ms = Ms(t0, Clock::now());
  const bool timing = run.timing_mode == SparseBatchTimingMode::kKernelEvents;
  const bool outputs = run.output_mode != SparseBatchOutputMode::kNoOutputs || observe;
  dsd_step_timings t{};
  ThrowOnError(dsd_sparse_run_table_async(
      ctx.handle(), table.get(), B, slots.data(), nullptr, rows->data(),
      outputs ? DSD_OUTPUT_OUTPUTS : DSD_OUTPUT_NONE,
      timing ? DSD_TIMING_EVENTS : DSD_TIMING_NONE, ticket, &t));
  if (observe != nullptr) {
    ThrowOnError(dsd_sparse_async_wait(ctx.handle(), *ticket));
    observe->queries.resize(static_cast<std::size_t>(B) * E);
    for (int b = 0; b < B; ++b) {  // (the host rows)
      std::memcpy(observe->queries.data() + static_cast<std::size_t>(b) * E,
                  active[static_cast<std::size_t>(b)].Query(), sizeof(float) * E);
    }
    observe->selected.assign(static_cast<std::size_t>(B) * std::max(1, top_k), 0);
    observe->selected_counts.assign(static_cast<std::size_t>(B), 0);
    ThrowOnError(dsd_sparse_last_selection(ctx.handle(), B, observe->selected.data(),
                                           observe->selected_counts.data()));
    ObserveTableStep(ctx, table, slots, E, observe);
  }
  if (timing) {
    result.runtime_overheads.time_prepare_sparse_layout_ms = layout_ms;
    result.runtime_overheads.time_memcpy_h2d_ms = t.h2d_ms;
    result.runtime_overheads.time_kernel_launch_ms = t.launch_ms;
    result.runtime_overheads.time_sync_ms = t.sync_ms;  // waits for a free ring slot
  }
  return result;
}

// The pipelined loop's step records, once every step has completed: a
// step's time is its device time from its first command (the stage-in) to
// its last (the attention), as the device ran it -- gaps while the host was
// still enqueuing it included; the stage times are the kernel events'.
void CollectPipelinedSteps(SparseCudaContext& ctx, bool timing, std::vector<double>* step_ms,
                           StageTimings* timings) {
  step_ms->clear();
  std::vector<dsd_async_step> recs(256);
  for (;;) {
    int n = 0;
    detail::ThrowOnError(
        dsd_sparse_async_collect(ctx.handle(), recs.data(), static_cast<int>(recs.size()), &n));
    if (n == 0) return;
    for (int i = 0; i < n; ++i) {
      const dsd_async_step& r = recs[static_cast<std::size_t>(i)];
      step_ms->push_back(r.done_ms - r.start_ms);
      if (timing) {
        timings->page_scoring_ms += r.score_ms;
        timings->topk_ms += r.topk_ms;
        timings->attention_ms += r.attention_ms;
        timings->total_ms += r.score_ms + r.topk_ms + r.attention_ms;
      }
    }
  }
}

// Verification of a table step (DSD_VERIFY_STAGED): the device's candidate
// lists must be the host cache's (kept beside the table), and the step's
// outputs RunBatch's on those lists.
void VerifyTableStep(SparseCudaContext& ctx, const PagedKvCache& mirror,
                     const std::vector<LiveRequest>& active, int E) {
  using detail::ThrowOnError;
  const int B = static_cast<int>(active.size());
  std::vector<int> offs(static_cast<std::size_t>(B) + 1, 0);
  std::vector<int> want;
  for (const auto& l : active) {
    const auto& pages = mirror.GetRequestPages(l.a.state.request_id);
    want.insert(want.end(), pages.begin(), pages.end());
  }
  std::vector<int> ids(std::max<std::size_t>(1, want.size()));
  ThrowOnError(dsd_sparse_last_csr(ctx.handle(), B, offs.data(), ids.data(),
                                   static_cast<int>(ids.size())));
  ids.resize(static_cast<std::size_t>(offs[static_cast<std::size_t>(B)]));
  if (ids != want) {
    throw std::runtime_error("device page table differs from the host cache's page lists");
  }
  VerifyStagedStep(ctx, mirror, active, E);
}

void FinishStats(ContinuousBatchStats* stats, Clock::time_point wall_start,
                 const std::vector<double>& step_ms, const StageTimings& timings,
                 const RuntimeOverheadTimings& overheads, int steps, int batch_sum) {
  stats->total_wall_ms = Ms(wall_start, Clock::now());
  stats->tokens_per_second = stats->total_wall_ms > 0.0
                                 ? stats->total_generated_tokens / (stats->total_wall_ms / 1e3)
                                 : 0.0;
  stats->outside_run_batch_ms = std::max(0.0, stats->total_wall_ms - stats->run_batch_wall_ms);
  stats->serving_loop_other_ms =
      std::max(0.0, stats->total_wall_ms - stats->run_batch_wall_ms -
                        stats->runtime_admission_ms - stats->append_sync_ms -
                        stats->release_sync_ms);
  stats->measured_end_to_end_ms =
      stats->decode_payload_prep_ms + stats->prompt_preadmit_ms + stats->total_wall_ms;
  stats->avg_step_ms =
      step_ms.empty() ? 0.0
                      : std::accumulate(step_ms.begin(), step_ms.end(), 0.0) /
                            static_cast<double>(step_ms.size());
  stats->p50_step_ms = Percentile(step_ms, 0.50);
  stats->p95_step_ms = Percentile(step_ms, 0.95);
  stats->avg_active_batch_size =
      steps > 0 ? static_cast<double>(batch_sum) / static_cast<double>(steps) : 0.0;
  if (steps > 0) {
    stats->avg_sparse_timings = timings;
    Scale(&stats->avg_sparse_timings, 1.0 / steps);
    stats->avg_runtime_overheads = overheads;
    Scale(&stats->avg_runtime_overheads, 1.0 / steps);
  }
}

}  // namespace

std::vector<float> ContinuousTokenVector(int count, int request_id, int decode_step, int stream) {
  return TokenVector(count, request_id, decode_step, stream);
}

void SetContinuousStepObserver(ContinuousStepObserver observer, int every) {
  g_observer = std::move(observer);
  g_observe_every = g_observer ? every : 0;
}

std::vector<ContinuousRequestSpec> BuildSyntheticContinuousWorkload(
    const ModelConfig& config, int num_requests, int arrival_window, int min_prompt_tokens,
    int max_prompt_tokens, int min_decode_steps, int max_decode_steps, int seed) {
  if (num_requests < 0 || arrival_window < 0 || min_prompt_tokens < 0 ||
      max_prompt_tokens < min_prompt_tokens || min_decode_steps < 0 ||
      max_decode_steps < min_decode_steps) {
    throw std::invalid_argument("invalid continuous workload parameters");
  }
  std::mt19937 rng(static_cast<std::mt19937::result_type>(seed));
  std::uniform_int_distribution<int> arrival(0, std::max(0, arrival_window));
  std::uniform_int_distribution<int> prompt(min_prompt_tokens, max_prompt_tokens);
  std::uniform_int_distribution<int> decode(min_decode_steps, max_decode_steps);
  const int E = Ept(config);
  std::vector<ContinuousRequestSpec> specs;
  specs.reserve(static_cast<std::size_t>(num_requests));
  for (int id = 0; id < num_requests; ++id) {
    ContinuousRequestSpec s;
    s.request_id = id;
    s.arrival_step = arrival(rng);
    s.prompt_tokens = prompt(rng);
    s.decode_steps = decode(rng);
    if (NormalPayloads()) {
      // The reference stream advances past the payload's draws (one per
      // float) as in the U(-1, 1) mode, so arrivals and lengths stay the
      // reference's; the N(0, 1) payloads are drawn below.
      rng.discard(2ull * static_cast<unsigned long long>(s.prompt_tokens) * E + E);
    } else {
      s.prompt_keys = Uniform(s.prompt_tokens * E, rng);
      s.prompt_values = Uniform(s.prompt_tokens * E, rng);
      s.initial_query = Uniform(E, rng);
    }
    specs.push_back(std::move(s));
  }
  if (NormalPayloads()) {
    // Request r's prompt keys, values and initial query, in that order, from
    // its own engine std::mt19937(StepSeed(r, seed, 3)) (stream 3: the
    // decode tokens use 0-2), so the host workers draw them in parallel.
    dsd_host::Workers::Get().ParallelFor(static_cast<int>(specs.size()), [&](int i) {
      ContinuousRequestSpec& s = specs[static_cast<std::size_t>(i)];
      std::mt19937 prng(StepSeed(s.request_id, seed, 3));
      s.prompt_keys = Normal(s.prompt_tokens * E, prng);
      s.prompt_values = Normal(s.prompt_tokens * E, prng);
      s.initial_query = Normal(E, prng);
    });
  }
  std::sort(specs.begin(), specs.end(),
            [](const ContinuousRequestSpec& a, const ContinuousRequestSpec& b) {
              if (a.arrival_step == b.arrival_step) return a.request_id < b.request_id;
              return a.arrival_step < b.arrival_step;
            });
  return specs;
}

ContinuousBatchStats RunContinuousSparseDecode(const ModelConfig& config,
                                               const std::vector<ContinuousRequestSpec>& specs,
                                               int max_active_requests) {
  ContinuousDecodeOptions options;
  options.max_active_requests = max_active_requests;
  return RunContinuousSparseDecode(config, specs, options);
}

ContinuousBatchStats RunContinuousSparseDecode(const ModelConfig& config,
                                               const std::vector<ContinuousRequestSpec>& specs,
                                               const ContinuousDecodeOptions& options) {
  if (options.max_active_requests <= 0) {
    throw std::invalid_argument("max_active_requests must be positive");
  }
  if (!SparseAttentionCudaAvailable()) {
    throw std::runtime_error("continuous sparse decode requires a visible gfx950 GPU");
  }
  if (options.gpu_synthetic_decode_append &&
      options.prompt_admission_mode == ContinuousPromptAdmissionMode::kCpuCache) {
    throw std::invalid_argument(
        "gpu_synthetic_decode_append requires a GPU-resident prompt admission mode");
  }
  Validate(config, specs);
  const int E = Ept(config);
  const int total_pages = CapacityFor(config, specs);
  const int max_pages = MaxPagesPerRequest(config, specs);
  const int window_pages = std::max(1, options.max_active_requests * max_pages);
  const int capacity =
      options.preadmit_prompts ? total_pages : std::min(total_pages, window_pages);
  const int max_candidates = options.max_active_requests * max_pages;
  const int max_selected =
      options.max_active_requests * std::min(config.top_k_pages, max_pages);
  const bool metadata_only =
      options.prompt_admission_mode != ContinuousPromptAdmissionMode::kCpuCache;
  PagedKvCache cache(config, capacity, !metadata_only);
  SparseCudaContext ctx(cache, config, options.max_active_requests, max_candidates,
                        max_selected);
  ctx.ResetDeviceTransferStats();
  const bool debug_outputs = options.run_batch_output_mode == SparseBatchOutputMode::kDebugTensors;
  // GPU-resident admission: page lists in a device table (the host cache
  // then only mirrors them when steps are verified).
  const bool use_table = metadata_only && !debug_outputs && DeviceTableEnabled();
  const bool mirror = !use_table || VerifyStagedSteps();
  const bool pipelined = use_table && !VerifyStagedSteps() && PipelineEnabled();
  std::unique_ptr<LoopTable> table;
  if (use_table) {
    const int slots = options.preadmit_prompts ? static_cast<int>(specs.size())
                                               : options.max_active_requests;
    table = std::make_unique<LoopTable>(ctx.pool_handle(), std::max(1, slots), max_pages);
  }
  // Direct uploads at runtime admission overlap the steps (DSD_PREFETCH=0:
  // synchronous uploads at admission, as the reference).
  std::unique_ptr<PromptPrefetcher> prefetch;
  if (use_table && !options.preadmit_prompts &&
      options.prompt_admission_mode == ContinuousPromptAdmissionMode::kDirectGpuUpload &&
      PrefetchEnabled()) {
    prefetch = std::make_unique<PromptPrefetcher>(table->get(), specs, kPrefetchDepth);
  }
  auto admit = [&](std::size_t i) {
    if (use_table) {
      AdmitToTable(config, specs[i], i, options.prompt_admission_mode, table.get(),
                   mirror ? &cache : nullptr, prefetch.get());
    } else {
      AdmitPrompt(config, specs[i], options.prompt_admission_mode, &cache, &ctx);
    }
  };

  ContinuousBatchStats stats;
  DecodePayloads payloads;
  if (options.precompute_decode_payloads) {
    const auto t0 = Clock::now();
    payloads = BuildPayloads(config, specs, !options.gpu_synthetic_decode_append);
    if (pipelined && DeviceQueryStore()) {
      payloads.device_queries =
          DeviceFloats(payloads.queries.data(), payloads.query_rows * static_cast<std::size_t>(E));
    }
    stats.decode_payload_prep_ms = Ms(t0, Clock::now());
  }
  std::vector<double> step_ms;
  StageTimings timings;
  RuntimeOverheadTimings overheads;
  int steps_run = 0;
  int batch_sum = 0;
  std::deque<std::size_t> pending;
  std::vector<LiveRequest> active;
  active.reserve(static_cast<std::size_t>(options.max_active_requests));
  std::vector<const float*> step_rows;
  std::vector<const RequestState*> batch;
  std::vector<std::uint8_t> admitted(specs.size(), 0);
  // The pipelined loop's pinned payload rows and its step tickets; the
  // tickets' scope ends first, waiting for every enqueued step before the
  // rows those steps read are freed.
  std::unique_ptr<PayloadSlabs> slabs;
  if (pipelined) {
    slabs = std::make_unique<PayloadSlabs>(options.max_active_requests, E,
                                           !options.gpu_synthetic_decode_append);
  }
  StepTickets tickets(ctx.handle());
  int admitted_this_step = 0;

  if (options.preadmit_prompts) {
    for (std::size_t i = 0; i < specs.size(); ++i) {
      const auto t0 = Clock::now();
      admit(i);
      const double ms = Ms(t0, Clock::now());
      stats.admission_ms += ms;
      stats.prompt_preadmit_ms += ms;
      admitted[i] = 1;
    }
    stats.admission_device_transfer_stats = ctx.DeviceTransfers();
    ctx.ResetDeviceTransferStats();
  }

  std::size_t next = 0;
  int step = 0;
  const auto wall_start = Clock::now();
  while (next < specs.size() || !pending.empty() || !active.empty()) {
    if (active.empty() && pending.empty() && next < specs.size() &&
        step < specs[next].arrival_step) {
      step = specs[next].arrival_step;
    }
    while (next < specs.size() && specs[next].arrival_step <= step) pending.push_back(next++);
    while (static_cast<int>(active.size()) < options.max_active_requests && !pending.empty()) {
      const std::size_t i = pending.front();
      pending.pop_front();
      const auto& s = specs[i];
      if (!admitted[i]) {
        const auto t0 = Clock::now();
        admit(i);
        const double ms = Ms(t0, Clock::now());
        stats.admission_ms += ms;
        stats.runtime_admission_ms += ms;
        admitted[i] = 1;
      }
      if (s.decode_steps > 0) {
        LiveRequest l;
        if (mirror) {
          l.a.state =
              MakeRequestState(s.request_id, std::vector<float>(), cache, s.prompt_tokens);
        } else {
          l.a.state.request_id = s.request_id;
          l.a.state.context_tokens = s.prompt_tokens;
        }
        l.a.remaining_decode_steps = s.decode_steps;
        l.a.spec_index = i;
        if (pipelined) {
          // Into the step's query slab (rows the step reads in place).
          if (admitted_this_step == 0) tickets.WaitFor(steps_run - PayloadSlabs::kSlabs);
          float* row = slabs->Admitted(steps_run, admitted_this_step++);
          std::memcpy(row, s.initial_query.data(), sizeof(float) * E);
          l.query = row;
          l.own = false;
        } else {
          l.query_buf = s.initial_query;
          l.own = true;
        }
        active.push_back(std::move(l));
      } else if (use_table) {
        table->Release({s.request_id}, !options.lazy_release);
        if (mirror) cache.ReleaseRequest(s.request_id);
      } else {
        const auto freed = cache.ReleaseRequest(s.request_id);
        if (!options.lazy_release) ctx.SyncFreedPages(freed);
      }
    }
    if (active.empty()) {
      ++step;
      continue;
    }

    const auto t_step = Clock::now();
    SparseRunBatchOptions run;
    run.output_mode = options.run_batch_output_mode;
    run.timing_mode = options.run_batch_timing_mode;
    SparseBatchCudaResult result;
    const bool observe = g_observer && g_observe_every > 0 && steps_run % g_observe_every == 0;
    ObservedDecodeStep seen;
    if (debug_outputs) {
      // Debug tensors come back per request through RunBatch.
      batch.clear();
      for (auto& l : active) {
        l.a.state.query.assign(l.Query(), l.Query() + E);
        l.a.state.candidate_page_ids = cache.GetRequestPages(l.a.state.request_id);
        batch.push_back(&l.a.state);
      }
      result = ctx.RunBatch(batch, run);
      if (observe) {
        seen.cand_offsets.push_back(0);
        for (std::size_t b = 0; b < active.size(); ++b) {
          const RequestState& st = active[b].a.state;
          seen.cand_ids.insert(seen.cand_ids.end(), st.candidate_page_ids.begin(),
                               st.candidate_page_ids.end());
          seen.cand_offsets.push_back(static_cast<int>(seen.cand_ids.size()));
          seen.queries.insert(seen.queries.end(), st.query.begin(), st.query.end());
          const auto& pr = result.per_request[b];
          seen.selected_counts.push_back(static_cast<int>(pr.selected_page_ids.size()));
          seen.selected.insert(seen.selected.end(), pr.selected_page_ids.begin(),
                               pr.selected_page_ids.end());
          seen.outputs.insert(seen.outputs.end(), pr.output.output.begin(),
                              pr.output.output.end());
        }
      }
    } else if (pipelined) {
      long long ticket = 0;
      result = PipelinedTableStep(ctx, *table, active, E, config.top_k_pages, run, &step_rows,
                                  observe ? &seen : nullptr, &ticket);
      tickets.Push(ticket);
      admitted_this_step = 0;
    } else if (use_table) {
      result = TableStep(ctx, *table, active, E, config.top_k_pages, run, &step_rows,
                         observe ? &seen : nullptr);
      if (VerifyStagedSteps()) VerifyTableStep(ctx, cache, active, E);
    } else {
      result = StagedStep(ctx, cache, active, E, config.top_k_pages,
                          options.max_active_requests, max_candidates, max_selected, run,
                          &step_rows, observe ? &seen : nullptr);
    }
    if (observe) {
      seen.step = step;
      seen.elements = E;
      for (const auto& l : active) {
        seen.request_ids.push_back(l.a.state.request_id);
        seen.decode_steps.push_back(l.a.decode_step_index);
        seen.context_tokens.push_back(l.a.state.context_tokens);
      }
    }
    const double ms = Ms(t_step, Clock::now());
    stats.run_batch_wall_ms += ms;
    step_ms.push_back(ms);
    Add(&timings, result.aggregate_timings);
    Add(&overheads, result.runtime_overheads);
    ++steps_run;
    batch_sum += static_cast<int>(active.size());
    if (observe) g_observer(seen);

    // Payloads generated during the loop (not precomputed): every vector has
    // its own seed, so the host threads form them in any order with the
    // same values as the reference's in-loop generation (:596-633).
    const bool gen_kv =
        !options.gpu_synthetic_decode_append && !options.precompute_decode_payloads;
    const bool gen_q = !options.precompute_decode_payloads;
    std::vector<std::vector<float>> gen_k(gen_kv && !pipelined ? active.size() : 0);
    std::vector<std::vector<float>> gen_v(gen_kv && !pipelined ? active.size() : 0);
    // The pipelined loop writes the step's uploaded K/V rows (batch order,
    // up_row) and the next step's queries straight into their slabs, once
    // the steps that read those slabs last have completed.
    const long long this_step = steps_run - 1;
    const bool kv_rows = pipelined && !options.gpu_synthetic_decode_append;
    std::vector<int> up_row(active.size(), -1);
    float* kv_keys = nullptr;
    float* kv_values = nullptr;
    if (kv_rows) {
      int m = 0;
      for (std::size_t li = 0; li < active.size(); ++li) {
        if (active[li].a.remaining_decode_steps > 1) up_row[li] = m++;
      }
      tickets.WaitFor(this_step - PayloadSlabs::kSlabs + 1);
      kv_keys = slabs->Keys(this_step);
      kv_values = slabs->Values(this_step);
    }
    if (pipelined && gen_q) tickets.WaitFor(steps_run - PayloadSlabs::kSlabs);
    if (gen_kv || gen_q) {
      const int per = (gen_kv ? 2 : 0) + (gen_q ? 1 : 0);
      const std::size_t row_bytes = sizeof(float) * static_cast<std::size_t>(E);
      dsd_host::Workers::Get().ParallelFor(
          static_cast<int>(active.size()) * per, [&](int t) {
            const int i = t / per;
            const int which = t - i * per;
            LiveRequest& l = active[static_cast<std::size_t>(i)];
            const int id = l.a.state.request_id;
            const int dstep = l.a.decode_step_index;
            const int up = up_row[static_cast<std::size_t>(i)];
            if (gen_kv && which < 2) {
              std::vector<float> kv = TokenVector(E, id, dstep, which + 1);
              if (!pipelined) {
                (which == 0 ? gen_k : gen_v)[static_cast<std::size_t>(i)] = std::move(kv);
              } else if (up >= 0) {
                float* dst = (which == 0 ? kv_keys : kv_values) + static_cast<std::size_t>(up) * E;
                std::memcpy(dst, kv.data(), row_bytes);
              }
            } else if (pipelined) {
              const std::vector<float> q = TokenVector(E, id, dstep + 1, 0);
              std::memcpy(slabs->Query(steps_run, i), q.data(), row_bytes);
            } else {
              l.query_buf = TokenVector(E, id, dstep + 1, 0);  // the next step's query
            }
          });
    }
    std::vector<AppendTokenResult> appended;
    std::vector<float> keys, values;
    std::vector<int> synth_requests, synth_steps;
    // the table's append: every active request, batch order
    std::vector<int> t_slots, t_requests, t_steps;
    std::vector<unsigned char> t_fresh, t_upload;
    for (std::size_t li = 0; li < active.size(); ++li) {
      LiveRequest& l = active[li];
      auto& a = l.a;
      const int id = a.state.request_id;
      const int dstep = a.decode_step_index;
      const float* k = nullptr;
      const float* v = nullptr;
      if (!options.gpu_synthetic_decode_append) {
        if (options.precompute_decode_payloads) {
          k = Row(payloads.keys[a.spec_index], dstep, E);
          v = Row(payloads.values[a.spec_index], dstep, E);
        } else if (!pipelined) {
          k = gen_k[li].data();
          v = gen_v[li].data();
        }
        // (pipelined, generated: the rows are already in the K/V slab; no
        // host cache mirrors a pipelined loop)
      }
      // Decode tokens of GPU-admitted prompts start a fresh page (:614-616).
      const bool force_new = metadata_only && dstep == 0;
      AppendTokenResult r{};
      if (mirror) {
        r = options.gpu_synthetic_decode_append
                ? cache.AppendTokenMetadataOnly(id, force_new)
                : (metadata_only ? cache.AppendTokenMetadataOnly(id, k, force_new)
                                 : cache.AppendToken(id, k, v, force_new));
      }
      if (use_table) {
        t_slots.push_back(table->SlotOf(id));
        t_requests.push_back(id);
        t_steps.push_back(dstep);
        t_fresh.push_back(force_new ? 1 : 0);
        t_upload.push_back(a.remaining_decode_steps > 1 ? 1 : 0);
      }
      // The last decode token is never attended to, so it is not uploaded.
      if (a.remaining_decode_steps > 1) {
        appended.push_back(r);
        if (options.gpu_synthetic_decode_append) {
          synth_requests.push_back(id);
          synth_steps.push_back(dstep);
        } else if (kv_rows) {
          if (k != nullptr) {  // precomputed rows into the slab
            const std::size_t at = static_cast<std::size_t>(up_row[li]) * E;
            std::memcpy(kv_keys + at, k, sizeof(float) * E);
            std::memcpy(kv_values + at, v, sizeof(float) * E);
          }
        } else if (metadata_only) {
          keys.insert(keys.end(), k, k + E);
          values.insert(values.end(), v, v + E);
        }
      }
      ++a.state.context_tokens;
      // The next step's query; its candidate list is the cache's page list,
      // read when the step is staged.
      if (options.precompute_decode_payloads) {
        l.query = payloads.NextQuery(a.spec_index, dstep, E);
        l.device_query = payloads.NextQueryDevice(a.spec_index, dstep, E);
        l.own = false;
      } else if (pipelined) {
        l.query = slabs->Query(steps_run, static_cast<int>(li));  // generated above
        l.own = false;
      } else {
        l.own = true;  // query_buf already holds it (generated above)
      }
      ++a.decode_step_index;
      --a.remaining_decode_steps;
      ++stats.total_generated_tokens;
    }
    const auto t_append = Clock::now();
    if (use_table) {
      const bool rows = !options.gpu_synthetic_decode_append;
      const float* k_rows = kv_rows ? kv_keys : keys.data();
      const float* v_rows = kv_rows ? kv_values : values.data();
      detail::ThrowOnError(dsd_table_append(
          table->get(), static_cast<int>(t_slots.size()), t_slots.data(), t_fresh.data(),
          t_upload.data(), rows ? k_rows : nullptr, rows ? v_rows : nullptr,
          t_requests.data(), t_steps.data()));
    } else if (options.gpu_synthetic_decode_append) {
      ctx.AppendSyntheticTokens(cache, appended, synth_requests, synth_steps);
    } else if (metadata_only) {
      ctx.SyncAppendedTokensDirect(cache, appended, keys, values);
    } else {
      ctx.SyncAppendedTokens(cache, appended);
    }
    stats.append_sync_ms += Ms(t_append, Clock::now());

    std::vector<PageId> freed;
    std::vector<int> finished;
    active.erase(std::remove_if(active.begin(), active.end(),
                                [&](const LiveRequest& l) {
                                  const ActiveDecodeRequest& a = l.a;
                                  if (a.remaining_decode_steps > 0) return false;
                                  finished.push_back(a.state.request_id);
                                  if (mirror) {
                                    const auto ids = cache.ReleaseRequest(a.state.request_id);
                                    freed.insert(freed.end(), ids.begin(), ids.end());
                                  }
                                  return true;
                                }),
                 active.end());
    const auto t_release = Clock::now();
    if (use_table) {
      table->Release(finished, !options.lazy_release);
    } else if (!options.lazy_release) {
      ctx.SyncFreedPages(freed);
    }
    stats.release_sync_ms += Ms(t_release, Clock::now());
    ++step;
  }
  if (pipelined) {
    CollectPipelinedSteps(ctx, options.run_batch_timing_mode == SparseBatchTimingMode::kKernelEvents,
                          &step_ms, &timings);
  }
  FinishStats(&stats, wall_start, step_ms, timings, overheads, steps_run, batch_sum);
  Add(&stats.device_transfer_stats, ctx.DeviceTransfers());
  if (VerifyStagedSteps()) {
    std::fprintf(stderr, "dsd: %lld staged steps verified against RunBatch\n", g_verified_steps);
  }
  return stats;
}

ContinuousBatchStats RunContinuousDenseGpuDecode(
    const ModelConfig& config, const std::vector<ContinuousRequestSpec>& specs,
    int max_active_requests) {
  ContinuousDecodeOptions options;
  options.max_active_requests = max_active_requests;
  return RunContinuousDenseGpuDecode(config, specs, options);
}

ContinuousBatchStats RunContinuousDenseGpuDecode(
    const ModelConfig& config, const std::vector<ContinuousRequestSpec>& specs,
    const ContinuousDecodeOptions& options) {
  if (options.max_active_requests <= 0) {
    throw std::invalid_argument("max_active_requests must be positive");
  }
  if (!DenseAttentionCudaAvailable()) {
    throw std::runtime_error("continuous dense decode requires a visible gfx950 GPU");
  }
  Validate(config, specs);
  const int E = Ept(config);
  PagedKvCache cache(config, CapacityFor(config, specs), true);
  DenseCudaContext ctx(cache, config);
  ContinuousBatchStats stats;
  DecodePayloads payloads;
  if (options.precompute_decode_payloads) {
    const auto t0 = Clock::now();
    payloads = BuildPayloads(config, specs, true);
    stats.decode_payload_prep_ms = Ms(t0, Clock::now());
  }
  std::vector<double> step_ms;
  StageTimings timings;
  RuntimeOverheadTimings overheads;
  int steps_run = 0;
  int batch_sum = 0;
  std::deque<std::size_t> pending;
  std::vector<ActiveDecodeRequest> active;
  std::vector<RequestState> batch;
  std::vector<std::uint8_t> admitted(specs.size(), 0);
  auto admit = [&](std::size_t i, double* sink) {
    const auto t0 = Clock::now();
    ctx.SyncPagesFromCache(cache, AdmitToCache(config, specs[i], &cache));
    const double ms = Ms(t0, Clock::now());
    stats.admission_ms += ms;
    *sink += ms;
    admitted[i] = 1;
  };
  if (options.preadmit_prompts) {
    for (std::size_t i = 0; i < specs.size(); ++i) admit(i, &stats.prompt_preadmit_ms);
  }
  std::size_t next = 0;
  int step = 0;
  const auto wall_start = Clock::now();
  while (next < specs.size() || !pending.empty() || !active.empty()) {
    if (active.empty() && pending.empty() && next < specs.size() &&
        step < specs[next].arrival_step) {
      step = specs[next].arrival_step;
    }
    while (next < specs.size() && specs[next].arrival_step <= step) pending.push_back(next++);
    while (static_cast<int>(active.size()) < options.max_active_requests && !pending.empty()) {
      const std::size_t i = pending.front();
      pending.pop_front();
      if (!admitted[i]) admit(i, &stats.runtime_admission_ms);
      const auto& s = specs[i];
      if (s.decode_steps > 0) {
        ActiveDecodeRequest a;
        a.state = MakeRequestState(s.request_id, s.initial_query, cache, s.prompt_tokens);
        a.remaining_decode_steps = s.decode_steps;
        a.spec_index = i;
        active.push_back(std::move(a));
      } else {
        const auto freed = cache.ReleaseRequest(s.request_id);
        if (!options.lazy_release) ctx.SyncFreedPages(freed);
      }
    }
    if (active.empty()) {
      ++step;
      continue;
    }
    const auto t_step = Clock::now();
    batch.clear();
    for (const auto& a : active) batch.push_back(a.state);
    const auto result = ctx.RunBatch(batch);
    const double ms = Ms(t_step, Clock::now());
    stats.run_batch_wall_ms += ms;
    step_ms.push_back(ms);
    timings.attention_ms += result.kernel_ms;
    timings.total_ms += result.kernel_ms;
    Add(&overheads, result.runtime_overheads);
    ++steps_run;
    batch_sum += static_cast<int>(active.size());

    // In-loop payloads on the host threads, as in the sparse loop.
    const bool gen = !options.precompute_decode_payloads;
    std::vector<std::vector<float>> gen_k(gen ? active.size() : 0);
    std::vector<std::vector<float>> gen_v(gen ? active.size() : 0);
    std::vector<std::vector<float>> gen_q(gen ? active.size() : 0);
    if (gen) {
      dsd_host::Workers::Get().ParallelFor(static_cast<int>(active.size()) * 3, [&](int t) {
        const std::size_t i = static_cast<std::size_t>(t / 3);
        const int id = active[i].state.request_id;
        const int dstep = active[i].decode_step_index;
        switch (t % 3) {
          case 0: gen_k[i] = TokenVector(E, id, dstep, 1); break;
          case 1: gen_v[i] = TokenVector(E, id, dstep, 2); break;
          default: gen_q[i] = TokenVector(E, id, dstep + 1, 0); break;
        }
      });
    }
    std::vector<AppendTokenResult> appended;
    for (std::size_t ai = 0; ai < active.size(); ++ai) {
      auto& a = active[ai];
      const int id = a.state.request_id;
      const int dstep = a.decode_step_index;
      const float* k;
      const float* v;
      if (options.precompute_decode_payloads) {
        k = Row(payloads.keys[a.spec_index], dstep, E);
        v = Row(payloads.values[a.spec_index], dstep, E);
      } else {
        k = gen_k[ai].data();
        v = gen_v[ai].data();
      }
      const auto r = cache.AppendToken(id, k, v, false);
      if (a.remaining_decode_steps > 1) appended.push_back(r);
      ++a.state.context_tokens;
      const auto& pages = cache.GetRequestPages(id);
      a.state.candidate_page_ids.assign(pages.begin(), pages.end());
      if (options.precompute_decode_payloads) {
        const float* q = payloads.NextQuery(a.spec_index, dstep, E);
        a.state.query.assign(q, q + E);
      } else {
        a.state.query = std::move(gen_q[ai]);
      }
      ++a.decode_step_index;
      --a.remaining_decode_steps;
      ++stats.total_generated_tokens;
    }
    const auto t_append = Clock::now();
    ctx.SyncAppendedTokens(cache, appended);
    stats.append_sync_ms += Ms(t_append, Clock::now());
    std::vector<PageId> freed;
    active.erase(std::remove_if(active.begin(), active.end(),
                                [&](const ActiveDecodeRequest& a) {
                                  if (a.remaining_decode_steps > 0) return false;
                                  const auto ids = cache.ReleaseRequest(a.state.request_id);
                                  freed.insert(freed.end(), ids.begin(), ids.end());
                                  return true;
                                }),
                 active.end());
    const auto t_release = Clock::now();
    if (!options.lazy_release) ctx.SyncFreedPages(freed);
    stats.release_sync_ms += Ms(t_release, Clock::now());
    ++step;
  }
  FinishStats(&stats, wall_start, step_ms, timings, overheads, steps_run, batch_sum);
  return stats;
}

ContinuousBenchmarkResult RunContinuousSparseBenchmark(
    const ModelConfig& config, const std::vector<ContinuousRequestSpec>& specs,
    int max_active_requests) {
  ContinuousDecodeOptions options;
  options.max_active_requests = max_active_requests;
  return RunContinuousSparseBenchmark(config, specs, options);
}

ContinuousBenchmarkResult RunContinuousSparseBenchmark(
    const ModelConfig& config, const std::vector<ContinuousRequestSpec>& specs,
    const ContinuousDecodeOptions& options) {
  ContinuousBenchmarkResult result;
  result.continuous_sparse = RunContinuousSparseDecode(config, specs, options);
  ContinuousDecodeOptions serial = options;
  serial.max_active_requests = 1;
  result.serial_sparse = RunContinuousSparseDecode(config, specs, serial);
  result.continuous_vs_serial_speedup =
      result.serial_sparse.tokens_per_second > 0.0
          ? result.continuous_sparse.tokens_per_second / result.serial_sparse.tokens_per_second
          : 0.0;
  return result;
}

}  // namespace dsd
