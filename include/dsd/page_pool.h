// page_pool.h -- host page allocator (reference include/dsd/page_pool.h:11-48).
// LIFO free list: the first page handed out is capacity-1.  Optional host K/V
// storage [capacity][page_size][E].  Errors: std::runtime_error on exhaustion,
// double free or missing storage; std::out_of_range on an invalid id.
#pragma once

#include <cstdint>
#include <vector>

#include "dsd/config.h"
#include "dsd/types.h"

namespace dsd {

class PagePool {
 public:
  PagePool(ModelConfig config, int capacity_pages, bool allocate_storage = true);

  PageId allocate_page();
  void free_page(PageId page_id);

  float* get_k_page_ptr(PageId page_id);
  const float* get_k_page_ptr(PageId page_id) const;

  float* get_v_page_ptr(PageId page_id);
  const float* get_v_page_ptr(PageId page_id) const;

  void reset_pool();

  int capacity_pages() const { return capacity_pages_; }
  bool is_allocated(PageId page_id) const;
  int elements_per_token() const;
  int elements_per_page() const;

  const std::vector<float>& key_storage() const { return keys_; }
  const std::vector<float>& value_storage() const { return values_; }
  bool has_storage() const { return has_storage_; }

 private:
  void CheckId(PageId page_id) const;
  void CheckLive(PageId page_id) const;
  void CheckStorage() const;
  std::size_t Offset(PageId page_id) const;

  ModelConfig config_;
  int capacity_pages_ = 0;
  std::vector<PageId> free_stack_;
  std::vector<std::uint8_t> live_;
  std::vector<float> keys_;
  std::vector<float> values_;
  bool has_storage_ = true;
};

}  // namespace dsd
