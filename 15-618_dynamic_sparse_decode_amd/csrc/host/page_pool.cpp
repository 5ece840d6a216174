// page_pool.cpp -- host page allocator (behaviour of reference
// src/page_pool.cpp:18-128: LIFO ids, allocation bitmap, optional storage).
#include "dsd/page_pool.h"

#include <algorithm>
#include <numeric>
#include <stdexcept>

namespace dsd {

PagePool::PagePool(ModelConfig config, int capacity_pages, bool allocate_storage)
    : config_(config), capacity_pages_(capacity_pages), has_storage_(allocate_storage) {
  if (capacity_pages < 0) {
    throw std::invalid_argument("capacity_pages must be non-negative");
  }
  live_.assign(static_cast<std::size_t>(capacity_pages_), 0);
  if (has_storage_) {
    const std::size_t n = static_cast<std::size_t>(capacity_pages_) * elements_per_page();
    keys_.assign(n, 0.0f);
    values_.assign(n, 0.0f);
  }
  reset_pool();
}

PageId PagePool::allocate_page() {
  if (free_stack_.empty()) throw std::runtime_error("page pool is exhausted");
  const PageId id = free_stack_.back();
  free_stack_.pop_back();
  live_[static_cast<std::size_t>(id)] = 1;
  return id;
}

void PagePool::free_page(PageId page_id) {
  CheckId(page_id);
  CheckLive(page_id);
  live_[static_cast<std::size_t>(page_id)] = 0;
  free_stack_.push_back(page_id);
}

float* PagePool::get_k_page_ptr(PageId page_id) {
  CheckId(page_id);
  CheckLive(page_id);
  CheckStorage();
  return keys_.data() + Offset(page_id);
}

const float* PagePool::get_k_page_ptr(PageId page_id) const {
  CheckId(page_id);
  CheckLive(page_id);
  CheckStorage();
  return keys_.data() + Offset(page_id);
}

float* PagePool::get_v_page_ptr(PageId page_id) {
  CheckId(page_id);
  CheckLive(page_id);
  CheckStorage();
  return values_.data() + Offset(page_id);
}

const float* PagePool::get_v_page_ptr(PageId page_id) const {
  CheckId(page_id);
  CheckLive(page_id);
  CheckStorage();
  return values_.data() + Offset(page_id);
}

void PagePool::reset_pool() {
  std::fill(live_.begin(), live_.end(), 0);
  // Popped from the back: ids come out capacity-1, capacity-2, ...
  free_stack_.resize(static_cast<std::size_t>(capacity_pages_));
  std::iota(free_stack_.begin(), free_stack_.end(), 0);
}

bool PagePool::is_allocated(PageId page_id) const {
  CheckId(page_id);
  return live_[static_cast<std::size_t>(page_id)] != 0;
}

int PagePool::elements_per_token() const { return config_.num_heads * config_.head_dim; }

int PagePool::elements_per_page() const { return config_.page_size * elements_per_token(); }

void PagePool::CheckId(PageId page_id) const {
  if (page_id < 0 || page_id >= capacity_pages_) throw std::out_of_range("invalid page id");
}

void PagePool::CheckLive(PageId page_id) const {
  if (!live_[static_cast<std::size_t>(page_id)]) {
    throw std::runtime_error("page is not currently allocated");
  }
}

void PagePool::CheckStorage() const {
  if (!has_storage_) throw std::runtime_error("page pool KV storage is disabled");
}

std::size_t PagePool::Offset(PageId page_id) const {
  return static_cast<std::size_t>(page_id) * static_cast<std::size_t>(elements_per_page());
}

}  // namespace dsd
