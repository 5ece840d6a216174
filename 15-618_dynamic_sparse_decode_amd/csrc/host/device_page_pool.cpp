// device_page_pool.cpp -- DevicePagePool over the libdsd_hip.so C ABI.
// Argument checks and messages follow reference src/device_page_pool.cpp
// (:304-366 UploadPage, :408-489 UploadPagesFromCache, :491-624
// UploadPromptDirect, :626-679 PrefillPromptSynthetic, :700-983 token
// uploads, :989-1091 free/download).  Summary rows are copied from the cache
// when uploading cache pages/tokens (so the device holds exactly what
// sparse_cpu scores against) and computed on the device by the same host
// rules for direct uploads.
#include "dsd/device_page_pool.h"

#include <algorithm>
#include <cstring>
#include <stdexcept>

#include "dsd_hip.h"
#include "status.h"

namespace dsd {

using detail::ThrowOnError;

DevicePagePool::DevicePagePool(ModelConfig config, int capacity_pages)
    : config_(config), capacity_pages_(capacity_pages) {
  if (capacity_pages < 0) throw std::invalid_argument("capacity_pages must be non-negative");
  ThrowOnError(dsd_pool_create(config.num_heads, config.head_dim, config.page_size,
                               capacity_pages, &pool_));
}

DevicePagePool::~DevicePagePool() {
  if (pool_ != nullptr) dsd_pool_destroy(pool_);
}

DevicePagePool::DevicePagePool(DevicePagePool&& other) noexcept
    : config_(other.config_),
      capacity_pages_(other.capacity_pages_),
      pool_(other.pool_),
      stats_(other.stats_) {
  other.pool_ = nullptr;
}

DevicePagePool& DevicePagePool::operator=(DevicePagePool&& other) noexcept {
  if (this != &other) {
    if (pool_ != nullptr) dsd_pool_destroy(pool_);
    config_ = other.config_;
    capacity_pages_ = other.capacity_pages_;
    pool_ = other.pool_;
    stats_ = other.stats_;
    other.pool_ = nullptr;
  }
  return *this;
}

void DevicePagePool::CheckCache(const PagedKvCache& cache) const {
  if (cache.CapacityPages() != capacity_pages_) {
    throw std::invalid_argument("cache capacity does not match device page pool");
  }
}

void DevicePagePool::CheckId(PageId page_id) const {
  if (page_id < 0 || page_id >= capacity_pages_) throw std::out_of_range("invalid page id");
}

void DevicePagePool::Reset() { ThrowOnError(dsd_pool_reset(pool_)); }

void DevicePagePool::UploadPage(PageId page_id, const float* host_keys,
                                const float* host_values, int token_count) {
  CheckId(page_id);
  if (token_count <= 0 || token_count > config_.page_size) {
    throw std::invalid_argument("token_count must be in (0, page_size]");
  }
  if (host_keys == nullptr || host_values == nullptr) {
    throw std::invalid_argument("host page payload pointers must be non-null");
  }
  const int64_t offset = 0;
  ThrowOnError(dsd_pool_upload_pages(pool_, 1, &page_id, &token_count, &offset, host_keys,
                                     host_values, nullptr));
}

void DevicePagePool::UploadPageFromCache(const PagedKvCache& cache, PageId page_id) {
  UploadPagesFromCache(cache, std::vector<PageId>{page_id});
}

void DevicePagePool::UploadPagesFromCache(const PagedKvCache& cache,
                                          const std::vector<PageId>& page_ids) {
  CheckCache(cache);
  if (page_ids.empty()) return;
  std::vector<PageId> ids = page_ids;
  std::sort(ids.begin(), ids.end());
  ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
  const int E = elements_per_token();
  std::vector<int> counts(ids.size());
  std::vector<int64_t> offsets(ids.size());
  std::vector<float> rows(ids.size() * static_cast<std::size_t>(E));
  for (std::size_t i = 0; i < ids.size(); ++i) {
    CheckId(ids[i]);
    const auto& page = cache.GetPage(ids[i]);
    if (page.request_id == -1 || page.token_count == 0) {
      throw std::invalid_argument("cannot upload a free or empty page from cache");
    }
    counts[i] = page.token_count;
    offsets[i] = static_cast<int64_t>(ids[i]) * elements_per_page();
    std::memcpy(rows.data() + i * E,
                cache.PageSummaryPool().data() + static_cast<std::size_t>(ids[i]) * E,
                sizeof(float) * E);
  }
  if (!cache.HasKvStorage()) {
    throw std::invalid_argument("cache holds no K/V storage to upload");
  }
  ThrowOnError(dsd_pool_upload_pages(pool_, static_cast<int>(ids.size()), ids.data(),
                                     counts.data(), offsets.data(), cache.KeyPool().data(),
                                     cache.ValuePool().data(), rows.data()));
}

void DevicePagePool::UploadActivePagesFromCache(const PagedKvCache& cache) {
  std::vector<PageId> ids;
  for (const auto& page : cache.Pages()) {
    if (page.request_id != -1 && page.token_count > 0) ids.push_back(page.id);
  }
  UploadPagesFromCache(cache, ids);
}

void DevicePagePool::UploadAllFromCache(const PagedKvCache& cache) {
  CheckCache(cache);
  Reset();
  UploadActivePagesFromCache(cache);
}

void DevicePagePool::UploadPromptDirect(const PagedKvCache& cache,
                                        const std::vector<PageId>& page_ids,
                                        const std::vector<int>& token_counts,
                                        const float* prompt_keys, const float* prompt_values) {
  CheckCache(cache);
  if (page_ids.size() != token_counts.size()) {
    throw std::invalid_argument("page_ids and token_counts sizes must match");
  }
  if (page_ids.empty()) return;
  const int E = elements_per_token();
  std::vector<int64_t> offsets(page_ids.size());
  int64_t token = 0;
  for (std::size_t i = 0; i < page_ids.size(); ++i) {
    CheckId(page_ids[i]);
    if (token_counts[i] <= 0 || token_counts[i] > config_.page_size) {
      throw std::invalid_argument("token_count must be in (0, page_size]");
    }
    const auto& page = cache.GetPage(page_ids[i]);
    if (page.request_id == -1 || page.token_count != token_counts[i]) {
      throw std::invalid_argument("reserved prompt page metadata is inconsistent");
    }
    offsets[i] = token * E;
    token += token_counts[i];
  }
  if (token > 0 && (prompt_keys == nullptr || prompt_values == nullptr)) {
    throw std::invalid_argument("prompt payload pointers must be non-null");
  }
  ThrowOnError(dsd_pool_upload_pages(pool_, static_cast<int>(page_ids.size()), page_ids.data(),
                                     token_counts.data(), offsets.data(), prompt_keys,
                                     prompt_values, nullptr));
}

void DevicePagePool::PrefillPromptSynthetic(const PagedKvCache& cache,
                                            const std::vector<PageId>& page_ids,
                                            const std::vector<int>& token_counts,
                                            int request_id) {
  CheckCache(cache);
  if (page_ids.size() != token_counts.size()) {
    throw std::invalid_argument("page_ids and token_counts sizes must match");
  }
  if (page_ids.empty()) return;
  for (std::size_t i = 0; i < page_ids.size(); ++i) {
    CheckId(page_ids[i]);
    if (token_counts[i] <= 0 || token_counts[i] > config_.page_size) {
      throw std::invalid_argument("token_count must be in (0, page_size]");
    }
    const auto& page = cache.GetPage(page_ids[i]);
    if (page.request_id == -1 || page.token_count != token_counts[i]) {
      throw std::invalid_argument("reserved prompt page metadata is inconsistent");
    }
  }
  ThrowOnError(dsd_pool_prefill_synthetic(pool_, static_cast<int>(page_ids.size()),
                                          page_ids.data(), token_counts.data(), request_id));
}

void DevicePagePool::UploadTokenFromCache(const PagedKvCache& cache, PageId page_id,
                                          int token_offset) {
  UploadTokensFromCache(cache, {AppendTokenResult{page_id, token_offset, false}});
}

void DevicePagePool::UploadTokensFromCache(const PagedKvCache& cache,
                                           const std::vector<AppendTokenResult>& results) {
  CheckCache(cache);
  if (results.empty()) return;
  const int E = elements_per_token();
  const std::size_t n = results.size();
  std::vector<int> ids(n), offsets(n), counts(n);
  std::vector<float> keys(n * E), values(n * E), rows(n * E);
  for (std::size_t i = 0; i < n; ++i) {
    const auto& r = results[i];
    CheckId(r.page_id);
    const auto& page = cache.GetPage(r.page_id);
    if (page.request_id == -1 || page.token_count == 0) {
      throw std::invalid_argument("cannot upload a token from a free cache page");
    }
    if (r.token_offset < 0 || r.token_offset >= page.token_count) {
      throw std::out_of_range("token_offset is outside the valid page prefix");
    }
    if (!cache.HasKvStorage()) {
      throw std::invalid_argument("cache holds no K/V storage to upload");
    }
    ids[i] = r.page_id;
    offsets[i] = r.token_offset;
    counts[i] = page.token_count;
    const std::size_t src = static_cast<std::size_t>(r.page_id) * elements_per_page() +
                            static_cast<std::size_t>(r.token_offset) * E;
    std::memcpy(keys.data() + i * E, cache.KeyPool().data() + src, sizeof(float) * E);
    std::memcpy(values.data() + i * E, cache.ValuePool().data() + src, sizeof(float) * E);
    std::memcpy(rows.data() + i * E,
                cache.PageSummaryPool().data() + static_cast<std::size_t>(r.page_id) * E,
                sizeof(float) * E);
  }
  ThrowOnError(dsd_pool_upload_tokens(pool_, static_cast<int>(n), ids.data(), offsets.data(),
                                      counts.data(), keys.data(), values.data(), rows.data()));
}

void DevicePagePool::UploadTokensDirect(const PagedKvCache& cache,
                                        const std::vector<AppendTokenResult>& results,
                                        const std::vector<float>& token_keys,
                                        const std::vector<float>& token_values) {
  CheckCache(cache);
  if (results.empty()) return;
  const int E = elements_per_token();
  const std::size_t n = results.size();
  if (token_keys.size() != n * E || token_values.size() != n * E) {
    throw std::invalid_argument("direct token payload size does not match results");
  }
  std::vector<int> ids(n), offsets(n), counts(n);
  for (std::size_t i = 0; i < n; ++i) {
    const auto& r = results[i];
    CheckId(r.page_id);
    const auto& page = cache.GetPage(r.page_id);
    if (page.request_id == -1 || page.token_count == 0) {
      throw std::invalid_argument("cannot upload a token to a free cache page");
    }
    if (r.token_offset < 0 || r.token_offset >= page.token_count) {
      throw std::out_of_range("token_offset is outside the valid page prefix");
    }
    ids[i] = r.page_id;
    offsets[i] = r.token_offset;
    counts[i] = page.token_count;
  }
  // Summaries: the running-mean update applied on the device.
  ThrowOnError(dsd_pool_upload_tokens(pool_, static_cast<int>(n), ids.data(), offsets.data(),
                                      counts.data(), token_keys.data(), token_values.data(),
                                      nullptr));
}

void DevicePagePool::AppendTokensSynthetic(const PagedKvCache& cache,
                                           const std::vector<AppendTokenResult>& results,
                                           const std::vector<int>& request_ids,
                                           const std::vector<int>& decode_steps) {
  CheckCache(cache);
  if (results.empty()) return;
  if (request_ids.size() != results.size() || decode_steps.size() != results.size()) {
    throw std::invalid_argument("synthetic append metadata size mismatch");
  }
  const std::size_t n = results.size();
  std::vector<int> ids(n), offsets(n), counts(n);
  for (std::size_t i = 0; i < n; ++i) {
    const auto& r = results[i];
    CheckId(r.page_id);
    const auto& page = cache.GetPage(r.page_id);
    if (page.request_id == -1 || page.token_count == 0) {
      throw std::invalid_argument("cannot append a synthetic token to a free page");
    }
    if (r.token_offset < 0 || r.token_offset >= page.token_count) {
      throw std::out_of_range("token_offset is outside the valid page prefix");
    }
    if (page.request_id != request_ids[i]) {
      throw std::invalid_argument("synthetic append request_id mismatch");
    }
    ids[i] = r.page_id;
    offsets[i] = r.token_offset;
    counts[i] = page.token_count;
  }
  ThrowOnError(dsd_pool_append_synthetic(pool_, static_cast<int>(n), ids.data(),
                                         offsets.data(), counts.data(), request_ids.data(),
                                         decode_steps.data()));
}

void DevicePagePool::MarkPageFree(PageId page_id) { MarkPagesFree(std::vector<PageId>{page_id}); }

void DevicePagePool::MarkPagesFree(const std::vector<PageId>& page_ids) {
  if (page_ids.empty()) return;
  ThrowOnError(dsd_pool_mark_free(pool_, static_cast<int>(page_ids.size()), page_ids.data()));
}

void DevicePagePool::DownloadPage(PageId page_id, std::vector<float>* host_keys,
                                  std::vector<float>* host_values) const {
  if (host_keys == nullptr || host_values == nullptr) {
    throw std::invalid_argument("download outputs must be non-null");
  }
  CheckId(page_id);
  std::vector<float> k(static_cast<std::size_t>(elements_per_page()));
  std::vector<float> v(k.size());
  int count = 0;
  ThrowOnError(dsd_pool_download_page(pool_, page_id, k.data(), v.data(), &count));
  k.resize(static_cast<std::size_t>(count) * elements_per_token());
  v.resize(k.size());
  *host_keys = std::move(k);
  *host_values = std::move(v);
}

void DevicePagePool::DownloadMetadata(std::vector<int>* token_counts,
                                      std::vector<std::uint8_t>* live_mask) const {
  if (token_counts == nullptr || live_mask == nullptr) {
    throw std::invalid_argument("metadata outputs must be non-null");
  }
  token_counts->resize(static_cast<std::size_t>(capacity_pages_));
  live_mask->resize(static_cast<std::size_t>(capacity_pages_));
  ThrowOnError(dsd_pool_download_meta(pool_, token_counts->data(), live_mask->data()));
}

void DevicePagePool::ResetTransferStats() {
  ThrowOnError(dsd_pool_reset_transfer_stats(pool_));
  stats_ = DeviceTransferStats{};
}

const DeviceTransferStats& DevicePagePool::transfer_stats() const {
  dsd_transfer_stats s{};
  ThrowOnError(dsd_pool_transfer_stats(pool_, &s));
  stats_ = DeviceTransferStats{s.h2d_bytes,       s.d2h_bytes,      s.h2d_calls,
                               s.d2h_calls,       s.h2d_large_calls, s.d2h_large_calls};
  return stats_;
}

int DevicePagePool::elements_per_token() const { return config_.num_heads * config_.head_dim; }

int DevicePagePool::elements_per_page() const { return config_.page_size * elements_per_token(); }

namespace {
dsd_pool_arrays Arrays(const ::dsd_pool* pool) {
  dsd_pool_arrays a{};
  ThrowOnError(dsd_pool_device_arrays(pool, &a));
  return a;
}
}  // namespace

const float* DevicePagePool::key_base_device() const { return Arrays(pool_).keys; }
const float* DevicePagePool::value_base_device() const { return Arrays(pool_).values; }
const float* DevicePagePool::page_summary_base_device() const { return Arrays(pool_).summaries; }
const int* DevicePagePool::page_token_counts_device() const { return Arrays(pool_).token_counts; }
const std::uint8_t* DevicePagePool::page_live_mask_device() const { return Arrays(pool_).live; }
const std::uint64_t* DevicePagePool::page_k_offsets_device() const {
  return reinterpret_cast<const std::uint64_t*>(Arrays(pool_).k_offsets);
}
const std::uint64_t* DevicePagePool::page_v_offsets_device() const {
  return reinterpret_cast<const std::uint64_t*>(Arrays(pool_).v_offsets);
}

}  // namespace dsd
