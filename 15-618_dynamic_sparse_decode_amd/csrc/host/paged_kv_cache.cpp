// paged_kv_cache.cpp -- host paged KV cache (behaviour of reference
// src/paged_kv_cache.cpp:18-515).  Summary rules (bit-exact, no FMA):
//   AppendPage:  s = 0; s += k[t] in token order; s *= fl(1/count)   (:87-99)
//   AppendToken: s = (s*old + k) / (old+1)                           (:231-238)
#include "dsd/paged_kv_cache.h"

#include <algorithm>
#include <stdexcept>

namespace dsd {

namespace {
const std::vector<PageId>& NoPages() {
  static const std::vector<PageId> empty;
  return empty;
}
}  // namespace

PagedKvCache::PagedKvCache(ModelConfig config, int capacity_pages, bool allocate_kv_storage)
    : config_(config),
      pool_(config, capacity_pages, allocate_kv_storage),
      summaries_(static_cast<std::size_t>(capacity_pages) *
                     static_cast<std::size_t>(config.num_heads * config.head_dim),
                 0.0f) {
  pages_.reserve(static_cast<std::size_t>(capacity_pages));
  for (PageId id = 0; id < capacity_pages; ++id) pages_.push_back(FreeDescriptor(id));
  summary_written_.assign(static_cast<std::size_t>(std::max(capacity_pages, 0)), 0);
}

PageId PagedKvCache::AppendPage(int request_id, const std::vector<float>& keys,
                                const std::vector<float>& values, int token_count) {
  if (token_count <= 0 || token_count > config_.page_size) {
    throw std::invalid_argument("token_count must be in (0, page_size]");
  }
  const std::size_t n = static_cast<std::size_t>(token_count) * ElementsPerToken();
  if (keys.size() != n || values.size() != n) {
    throw std::invalid_argument("page payload does not match expected size");
  }
  return AppendPage(request_id, keys.data(), values.data(), token_count, true);
}

PageId PagedKvCache::AppendPage(int request_id, const float* keys, const float* values,
                                int token_count) {
  return AppendPage(request_id, keys, values, token_count, true);
}

PageId PagedKvCache::AppendPage(int request_id, const float* keys, const float* values,
                                int token_count, bool compute_summary) {
  if (token_count <= 0 || token_count > config_.page_size) {
    throw std::invalid_argument("token_count must be in (0, page_size]");
  }
  const int E = ElementsPerToken();
  const std::size_t n = static_cast<std::size_t>(token_count) * E;
  if (n == 0) throw std::invalid_argument("page payload does not match expected size");
  if (keys == nullptr || values == nullptr) {
    throw std::invalid_argument("page payload pointers must be non-null");
  }
  if (!pool_.has_storage()) throw std::runtime_error("page pool KV storage is disabled");

  const PageId id = pool_.allocate_page();
  const int start = NextStartToken(request_id);
  std::copy(keys, keys + n, pool_.get_k_page_ptr(id));
  std::copy(values, values + n, pool_.get_v_page_ptr(id));
  ClearSummary(id);
  float* s = SummaryRow(id);
  if (compute_summary) {
    summary_written_[static_cast<std::size_t>(id)] = 1;
    for (int t = 0; t < token_count; ++t) {
      const float* row = keys + static_cast<std::size_t>(t) * E;
      for (int i = 0; i < E; ++i) s[i] += row[i];
    }
    const float inv = 1.0f / static_cast<float>(token_count);
    for (int i = 0; i < E; ++i) s[i] *= inv;
  }
  const std::size_t offset = static_cast<std::size_t>(id) * ElementsPerPage();
  pages_[static_cast<std::size_t>(id)] =
      PageDescriptor{id, request_id, start, token_count, offset, offset};
  request_pages_[request_id].push_back(id);
  ++live_pages_;
  return id;
}

std::vector<PageId> PagedKvCache::ReservePagesForRequest(int request_id,
                                                         const std::vector<int>& token_counts) {
  std::vector<PageId> ids;
  if (token_counts.empty()) return ids;
  for (int c : token_counts) {
    if (c <= 0 || c > config_.page_size) {
      throw std::invalid_argument("token_count must be in (0, page_size]");
    }
  }
  ids.reserve(token_counts.size());
  for (std::size_t i = 0; i < token_counts.size(); ++i) ids.push_back(pool_.allocate_page());
  std::sort(ids.begin(), ids.end());
  int start = NextStartToken(request_id);
  auto& list = request_pages_[request_id];
  for (std::size_t i = 0; i < ids.size(); ++i) {
    const PageId id = ids[i];
    ClearSummary(id);
    const std::size_t offset = static_cast<std::size_t>(id) * ElementsPerPage();
    pages_[static_cast<std::size_t>(id)] =
        PageDescriptor{id, request_id, start, token_counts[i], offset, offset};
    list.push_back(id);
    start += token_counts[i];
    ++live_pages_;
  }
  return ids;
}

PageDescriptor& PagedKvCache::TailForAppend(int request_id, bool force_new_page,
                                            bool* allocated) {
  auto& list = request_pages_[request_id];
  *allocated = false;
  PageId id;
  if (force_new_page || list.empty() ||
      pages_[static_cast<std::size_t>(list.back())].token_count >= config_.page_size) {
    id = pool_.allocate_page();
    const std::size_t offset = static_cast<std::size_t>(id) * ElementsPerPage();
    pages_[static_cast<std::size_t>(id)] =
        PageDescriptor{id, request_id, NextStartToken(request_id), 0, offset, offset};
    ClearSummary(id);
    list.push_back(id);
    ++live_pages_;
    *allocated = true;
  } else {
    id = list.back();
  }
  PageDescriptor& page = pages_[static_cast<std::size_t>(id)];
  if (page.request_id != request_id || page.token_count < 0 ||
      page.token_count >= config_.page_size) {
    throw std::runtime_error("request tail page is inconsistent");
  }
  return page;
}

AppendTokenResult PagedKvCache::AppendToken(int request_id, const std::vector<float>& key,
                                            const std::vector<float>& value) {
  return AppendToken(request_id, key, value, false);
}

AppendTokenResult PagedKvCache::AppendToken(int request_id, const std::vector<float>& key,
                                            const std::vector<float>& value,
                                            bool force_new_page) {
  const int E = ElementsPerToken();
  if (static_cast<int>(key.size()) != E || static_cast<int>(value.size()) != E) {
    throw std::invalid_argument("token payload does not match expected size");
  }
  return AppendToken(request_id, key.data(), value.data(), force_new_page);
}

AppendTokenResult PagedKvCache::AppendToken(int request_id, const float* key,
                                            const float* value, bool force_new_page) {
  if (key == nullptr || value == nullptr) {
    throw std::invalid_argument("token payload pointers must be non-null");
  }
  bool allocated = false;
  PageDescriptor& page = TailForAppend(request_id, force_new_page, &allocated);
  const int E = ElementsPerToken();
  const int offset = page.token_count;
  const std::size_t row = static_cast<std::size_t>(offset) * E;
  std::copy(key, key + E, pool_.get_k_page_ptr(page.id) + row);
  std::copy(value, value + E, pool_.get_v_page_ptr(page.id) + row);
  float* s = SummaryRow(page.id);
  summary_written_[static_cast<std::size_t>(page.id)] = 1;
  const float old_count = static_cast<float>(page.token_count);
  const float new_count = old_count + 1.0f;
  for (int i = 0; i < E; ++i) s[i] = (s[i] * old_count + key[i]) / new_count;
  ++page.token_count;
  return AppendTokenResult{page.id, offset, allocated};
}

AppendTokenResult PagedKvCache::AppendTokenMetadataOnly(int request_id,
                                                        const std::vector<float>& key,
                                                        bool force_new_page) {
  if (static_cast<int>(key.size()) != ElementsPerToken()) {
    throw std::invalid_argument("token payload does not match expected size");
  }
  return AppendTokenMetadataOnly(request_id, key.data(), force_new_page);
}

AppendTokenResult PagedKvCache::AppendTokenMetadataOnly(int request_id, const float* key,
                                                        bool force_new_page) {
  if (key == nullptr) throw std::invalid_argument("token payload pointer must be non-null");
  bool allocated = false;
  PageDescriptor& page = TailForAppend(request_id, force_new_page, &allocated);
  const int E = ElementsPerToken();
  const int offset = page.token_count;
  float* s = SummaryRow(page.id);
  summary_written_[static_cast<std::size_t>(page.id)] = 1;
  const float old_count = static_cast<float>(page.token_count);
  const float new_count = old_count + 1.0f;
  for (int i = 0; i < E; ++i) s[i] = (s[i] * old_count + key[i]) / new_count;
  ++page.token_count;
  return AppendTokenResult{page.id, offset, allocated};
}

AppendTokenResult PagedKvCache::AppendTokenMetadataOnly(int request_id, bool force_new_page) {
  bool allocated = false;
  PageDescriptor& page = TailForAppend(request_id, force_new_page, &allocated);
  const int offset = page.token_count;
  ++page.token_count;
  return AppendTokenResult{page.id, offset, allocated};
}

std::vector<PageId> PagedKvCache::ReleaseRequest(int request_id) {
  const auto it = request_pages_.find(request_id);
  if (it == request_pages_.end()) return {};
  std::vector<PageId> released = it->second;
  for (PageId id : released) {
    if (pages_[static_cast<std::size_t>(id)].request_id != request_id) {
      throw std::runtime_error("request page mapping is inconsistent");
    }
    ClearSummary(id);
    pages_[static_cast<std::size_t>(id)] = FreeDescriptor(id);
    pool_.free_page(id);
    --live_pages_;
  }
  request_pages_.erase(it);
  return released;
}

void PagedKvCache::Reset() {
  request_pages_.clear();
  live_pages_ = 0;
  pool_.reset_pool();
  std::fill(summaries_.begin(), summaries_.end(), 0.0f);
  std::fill(summary_written_.begin(), summary_written_.end(), 0);
  for (PageId id = 0; id < static_cast<PageId>(pages_.size()); ++id) {
    pages_[static_cast<std::size_t>(id)] = FreeDescriptor(id);
  }
}

const PageDescriptor& PagedKvCache::GetPage(PageId page_id) const {
  if (page_id < 0 || page_id >= static_cast<PageId>(pages_.size())) {
    throw std::out_of_range("invalid page id");
  }
  return pages_[static_cast<std::size_t>(page_id)];
}

const std::vector<PageId>& PagedKvCache::GetRequestPages(int request_id) const {
  const auto it = request_pages_.find(request_id);
  return it == request_pages_.end() ? NoPages() : it->second;
}

std::vector<float> PagedKvCache::CopyPageKeys(PageId page_id) const {
  const auto& page = GetPage(page_id);
  const std::size_t n = static_cast<std::size_t>(page.token_count) * ElementsPerToken();
  if (n == 0) return {};
  const float* p = pool_.get_k_page_ptr(page_id);
  return std::vector<float>(p, p + n);
}

std::vector<float> PagedKvCache::CopyPageValues(PageId page_id) const {
  const auto& page = GetPage(page_id);
  const std::size_t n = static_cast<std::size_t>(page.token_count) * ElementsPerToken();
  if (n == 0) return {};
  const float* p = pool_.get_v_page_ptr(page_id);
  return std::vector<float>(p, p + n);
}

void PagedKvCache::CopyPageToken(PageId page_id, int token_offset, std::vector<float>* key,
                                 std::vector<float>* value) const {
  if (key == nullptr || value == nullptr) {
    throw std::invalid_argument("token copy outputs must be non-null");
  }
  const auto& page = GetPage(page_id);
  if (page.request_id == -1 || page.token_count == 0) {
    throw std::invalid_argument("cannot copy a token from a free page");
  }
  if (token_offset < 0 || token_offset >= page.token_count) {
    throw std::out_of_range("token_offset is outside the valid page prefix");
  }
  const int E = ElementsPerToken();
  const std::size_t row = static_cast<std::size_t>(token_offset) * E;
  const float* k = pool_.get_k_page_ptr(page_id) + row;
  const float* v = pool_.get_v_page_ptr(page_id) + row;
  key->assign(k, k + E);
  value->assign(v, v + E);
}

std::vector<float> PagedKvCache::BuildPageSummary(PageId page_id) const {
  return CopyPageSummary(page_id);
}

std::vector<float> PagedKvCache::CopyPageSummary(PageId page_id) const {
  const auto& page = GetPage(page_id);
  const int E = ElementsPerToken();
  if (page.token_count == 0) return std::vector<float>(static_cast<std::size_t>(E), 0.0f);
  const float* s = SummaryRow(page_id);
  return std::vector<float>(s, s + E);
}

int PagedKvCache::TotalPages() const { return live_pages_; }

int PagedKvCache::ElementsPerToken() const { return config_.num_heads * config_.head_dim; }

int PagedKvCache::ElementsPerPage() const { return config_.page_size * ElementsPerToken(); }

PageDescriptor PagedKvCache::FreeDescriptor(PageId page_id) const {
  const std::size_t offset = static_cast<std::size_t>(page_id) * ElementsPerPage();
  return PageDescriptor{page_id, -1, 0, 0, offset, offset};
}

int PagedKvCache::NextStartToken(int request_id) const {
  const auto it = request_pages_.find(request_id);
  if (it == request_pages_.end() || it->second.empty()) return 0;
  const auto& last = GetPage(it->second.back());
  return last.start_token + last.token_count;
}

// A summary row holds nonzero values only once written; rows never written
// since their last clear are zero already, so clearing them is skipped (a
// request released from GPU-side admission owns hundreds of such rows).
void PagedKvCache::ClearSummary(PageId page_id) {
  float* s = SummaryRow(page_id);
  std::uint8_t& written = summary_written_[static_cast<std::size_t>(page_id)];
  if (written) std::fill(s, s + ElementsPerToken(), 0.0f);
  written = 0;
}

float* PagedKvCache::SummaryRow(PageId page_id) {
  if (page_id < 0 || page_id >= static_cast<PageId>(pages_.size())) {
    throw std::out_of_range("invalid page id");
  }
  return summaries_.data() + static_cast<std::size_t>(page_id) * ElementsPerToken();
}

const float* PagedKvCache::SummaryRow(PageId page_id) const {
  if (page_id < 0 || page_id >= static_cast<PageId>(pages_.size())) {
    throw std::out_of_range("invalid page id");
  }
  return summaries_.data() + static_cast<std::size_t>(page_id) * ElementsPerToken();
}

}  // namespace dsd
