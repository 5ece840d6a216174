// paged_kv_cache.h -- host paged KV cache and per-page key summaries
// (reference include/dsd/paged_kv_cache.h:13-122).  The summary of a page is
// the per-element mean of its keys: built as sum-in-token-order times
// fl(1/count) by AppendPage, updated as (s*old + k)/(old+1) by AppendToken.
// These two rules are part of the parity contract: the device pool
// reproduces them bit for bit.
#pragma once

#include <cstddef>
#include <cstdint>
#include <unordered_map>
#include <vector>

#include "dsd/config.h"
#include "dsd/page_pool.h"
#include "dsd/types.h"

namespace dsd {

struct PageDescriptor {
  PageId id = -1;
  int request_id = -1;
  int start_token = 0;
  int token_count = 0;
  std::size_t k_offset = 0;
  std::size_t v_offset = 0;
};

class PagedKvCache {
 public:
  explicit PagedKvCache(ModelConfig config, int capacity_pages = 1024,
                        bool allocate_kv_storage = true);

  PageId AppendPage(int request_id, const std::vector<float>& keys,
                    const std::vector<float>& values, int token_count);
  PageId AppendPage(int request_id, const float* keys, const float* values, int token_count);
  PageId AppendPage(int request_id, const float* keys, const float* values, int token_count,
                    bool compute_summary);

  std::vector<PageId> ReservePagesForRequest(int request_id,
                                             const std::vector<int>& token_counts);

  AppendTokenResult AppendToken(int request_id, const std::vector<float>& key,
                                const std::vector<float>& value);
  AppendTokenResult AppendToken(int request_id, const std::vector<float>& key,
                                const std::vector<float>& value, bool force_new_page);
  AppendTokenResult AppendToken(int request_id, const float* key, const float* value,
                                bool force_new_page);

  AppendTokenResult AppendTokenMetadataOnly(int request_id, const std::vector<float>& key,
                                            bool force_new_page);
  AppendTokenResult AppendTokenMetadataOnly(int request_id, const float* key,
                                            bool force_new_page);
  AppendTokenResult AppendTokenMetadataOnly(int request_id, bool force_new_page);

  std::vector<PageId> ReleaseRequest(int request_id);

  void Reset();

  const PageDescriptor& GetPage(PageId page_id) const;
  const std::vector<PageId>& GetRequestPages(int request_id) const;
  const std::vector<PageDescriptor>& Pages() const { return pages_; }
  const std::vector<float>& KeyPool() const { return pool_.key_storage(); }
  const std::vector<float>& ValuePool() const { return pool_.value_storage(); }
  const std::vector<float>& PageSummaryPool() const { return summaries_; }

  std::vector<float> CopyPageKeys(PageId page_id) const;
  std::vector<float> CopyPageValues(PageId page_id) const;
  void CopyPageToken(PageId page_id, int token_offset, std::vector<float>* key,
                     std::vector<float>* value) const;
  std::vector<float> CopyPageSummary(PageId page_id) const;
  std::vector<float> BuildPageSummary(PageId page_id) const;

  int TotalPages() const;
  int CapacityPages() const { return pool_.capacity_pages(); }
  int ElementsPerToken() const;
  int ElementsPerPage() const;
  bool HasKvStorage() const { return pool_.has_storage(); }

 private:
  // Tail page of the request that receives the next token (allocating one
  // when forced, absent or full), then validates it.
  PageDescriptor& TailForAppend(int request_id, bool force_new_page, bool* allocated);
  PageDescriptor FreeDescriptor(PageId page_id) const;
  int NextStartToken(int request_id) const;
  float* SummaryRow(PageId page_id);
  const float* SummaryRow(PageId page_id) const;
  void ClearSummary(PageId page_id);

  ModelConfig config_;
  PagePool pool_;
  std::vector<PageDescriptor> pages_;
  std::vector<float> summaries_;
  std::vector<std::uint8_t> summary_written_;  // per page: summary row nonzero
  std::unordered_map<int, std::vector<PageId>> request_pages_;
  int live_pages_ = 0;
};

}  // namespace dsd
