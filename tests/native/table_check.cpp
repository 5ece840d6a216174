// table_check.cpp -- the device request -> page table (dsd_table_*) against
// the host paged KV cache of the reference API (dsd::PagedKvCache, the
// reference's PagePool / PagedKvCache order: src/page_pool.cpp,
// src/paged_kv_cache.cpp:114-160, 312-373).
//
// A seeded random sequence of the serving loop's operations runs on both:
// prompt admission (ReservePagesForRequest / dsd_table_admit_synthetic), one
// decode token for a batch of requests (AppendTokenMetadataOnly in batch
// order / dsd_table_append, fresh pages forced now and then, a request's
// last token not uploaded, as the loop does) and releases in batch order
// (ReleaseRequest / dsd_table_release).  After every operation each live
// request's page list downloaded from the device must equal the cache's,
// and each of its pages' device token count the cache's count.  At the end
// the remaining free pages are drained one at a time through both (forced
// fresh pages), which compares the whole free stack in pop order.
//
// usage: table_check <capacity> <max_slots> <operations> <seed>
// prints "table_check ok ..." and exits 0, or names the first mismatch and
// exits 1.
#include <algorithm>
#include <cstdio>
#include <exception>
#include <cstdlib>
#include <random>
#include <vector>

#include "dsd/paged_kv_cache.h"
#include "dsd_hip.h"

namespace {

int Fail(const char* what, int op, int request, int detail) {
  std::printf("table_check MISMATCH: %s at operation %d (request %d, %d): %s\n", what, op,
              request, detail, dsd_last_error());
  return 1;
}

#define CHECK_OK(expr)                                                         \
  do {                                                                         \
    if ((expr) != 0) {                                                         \
      std::printf("table_check ERROR: %s -> %s\n", #expr, dsd_last_error());  \
      return 2;                                                                \
    }                                                                          \
  } while (0)

}  // namespace

int main(int argc, char** argv) {
  if (argc != 5) {
    std::printf("usage: table_check <capacity> <max_slots> <operations> <seed>\n");
    return 2;
  }
  const int capacity = std::atoi(argv[1]);
  const int max_slots = std::atoi(argv[2]);
  const int operations = std::atoi(argv[3]);
  const int seed = std::atoi(argv[4]);
  dsd::ModelConfig config;
  config.num_heads = 2;
  config.head_dim = 32;
  config.page_size = 4;
  const int ps = config.page_size;
  const int max_pages = capacity;  // one request may take every page
  std::printf("table_check capacity %d slots %d operations %d seed %d\n", capacity, max_slots,
              operations, seed);
  std::fflush(stdout);

  dsd_pool* pool = nullptr;
  CHECK_OK(dsd_pool_create(config.num_heads, config.head_dim, ps, capacity, &pool));
  dsd_table* table = nullptr;
  CHECK_OK(dsd_table_create(pool, max_slots, max_pages, &table));
  dsd::PagedKvCache cache(config, capacity, false);

  struct Live {
    int request = -1;
    int decode_step = 0;
    bool closing = false;  // its last token was appended without upload
  };
  std::vector<Live> slot(max_slots);
  std::vector<int> free_slots;
  for (int s = max_slots - 1; s >= 0; --s) free_slots.push_back(s);
  std::mt19937 rng(static_cast<std::mt19937::result_type>(seed));
  auto uniform = [&](int lo, int hi) { return std::uniform_int_distribution<int>(lo, hi)(rng); };
  int next_request = 0;
  int free_pages = capacity;
  std::vector<int> dev_pages(capacity);
  std::vector<int> dev_counts(capacity);
  std::vector<unsigned char> dev_live(capacity);
  long long compared_lists = 0;

  // The cache's list of a request (empty before its first page).
  auto host_pages = [&](int request) -> std::vector<dsd::PageId> {
    try {
      return cache.GetRequestPages(request);
    } catch (const std::exception&) {
      return {};
    }
  };

  auto compare = [&](int op) -> int {
    CHECK_OK(dsd_pool_download_meta(pool, dev_counts.data(), dev_live.data()));
    for (int s = 0; s < max_slots; ++s) {
      if (slot[s].request < 0) continue;
      const auto want = host_pages(slot[s].request);
      int n = 0;
      CHECK_OK(dsd_table_download(table, s, dev_pages.data(), capacity, &n));
      if (n != static_cast<int>(want.size())) return Fail("page count", op, slot[s].request, n);
      for (int j = 0; j < n; ++j) {
        if (dev_pages[j] != want[j]) return Fail("page id", op, slot[s].request, j);
        // A request closing has one token the device never received.
        const int host = cache.GetPage(want[j]).token_count;
        const int dev = dev_counts[want[j]];
        const bool last = j == n - 1 && slot[s].closing;
        if (!last && dev != host) return Fail("token count", op, slot[s].request, j);
      }
      ++compared_lists;
    }
    int dev_free = 0;
    CHECK_OK(dsd_table_free_pages(table, &dev_free));
    if (dev_free != free_pages) return Fail("free pages", op, -1, dev_free);
    return 0;
  };

  for (int op = 0; op < operations; ++op) {
    const int kind = uniform(0, 9);
    std::vector<int> live;
    for (int s = 0; s < max_slots; ++s) {
      if (slot[s].request >= 0) live.push_back(s);
    }
    if (kind <= 2 && !free_slots.empty()) {
      // admission
      const int tokens = uniform(0, std::max(1, std::min(free_pages, 3 * ps + 8) * ps / 2));
      const int pages = (tokens + ps - 1) / ps;
      if (pages > free_pages) continue;
      const int s = free_slots.back();
      free_slots.pop_back();
      const int id = next_request++;
      std::vector<int> counts;
      for (int t = 0; t < tokens; t += ps) counts.push_back(std::min(ps, tokens - t));
      cache.ReservePagesForRequest(id, counts);
      CHECK_OK(dsd_table_admit_synthetic(table, s, tokens, id));
      slot[s] = Live{id, 0, false};
      free_pages -= pages;
    } else if (kind <= 7 && !live.empty()) {
      // one decode token for a batch of live requests (random order)
      std::shuffle(live.begin(), live.end(), rng);
      live.resize(static_cast<size_t>(uniform(1, static_cast<int>(live.size()))));
      std::vector<int> slots, req, steps;
      std::vector<unsigned char> fresh, upload;
      int need = 0;
      for (int s : live) {
        if (slot[s].closing) continue;
        const auto pages = host_pages(slot[s].request);
        const bool force = uniform(0, 15) == 0 || (slot[s].decode_step == 0 && uniform(0, 1));
        const bool full =
            pages.empty() || cache.GetPage(pages.back()).token_count >= ps;
        need += (force || full) ? 1 : 0;
        slots.push_back(s);
        req.push_back(slot[s].request);
        steps.push_back(slot[s].decode_step);
        fresh.push_back(force ? 1 : 0);
        upload.push_back(uniform(0, 9) == 0 ? 0 : 1);  // no upload: the request's last token
      }
      if (slots.empty() || need > free_pages) continue;
      for (size_t i = 0; i < slots.size(); ++i) {
        cache.AppendTokenMetadataOnly(req[i], fresh[i] != 0);
        Live& l = slot[slots[i]];
        ++l.decode_step;
        if (upload[i] == 0) l.closing = true;
      }
      CHECK_OK(dsd_table_append(table, static_cast<int>(slots.size()), slots.data(),
                                fresh.data(), upload.data(), nullptr, nullptr, req.data(),
                                steps.data()));
      free_pages -= need;
    } else if (!live.empty()) {
      // release a batch (closing requests always, others at random)
      std::shuffle(live.begin(), live.end(), rng);
      std::vector<int> rel;
      for (int s : live) {
        if (slot[s].closing || uniform(0, 2) == 0) rel.push_back(s);
      }
      if (rel.empty()) continue;
      for (int s : rel) {
        const auto freed = cache.ReleaseRequest(slot[s].request);
        free_pages += static_cast<int>(freed.size());
      }
      CHECK_OK(dsd_table_release(table, static_cast<int>(rel.size()), rel.data(), 1));
      for (int s : rel) {
        slot[s] = Live{};
        free_slots.push_back(s);
      }
    } else {
      continue;
    }
    if (int rc = compare(op)) return rc;
  }

  // Drain: every free page through a forced fresh page on one new request,
  // in pop order on both sides.
  if (!free_slots.empty()) {
    const int s = free_slots.back();
    const int id = next_request++;
    cache.ReservePagesForRequest(id, {});
    CHECK_OK(dsd_table_admit_synthetic(table, s, 0, id));
    slot[s] = Live{id, 0, false};
    const int drain = free_pages;
    for (int k = 0; k < drain; ++k) {
      cache.AppendTokenMetadataOnly(id, true);
      const unsigned char fresh = 1, up = 1;
      const int step = k;
      CHECK_OK(dsd_table_append(table, 1, &s, &fresh, &up, nullptr, nullptr, &id, &step));
      --free_pages;
    }
    if (int rc = compare(operations)) return rc;
    std::printf("table_check drained %d free pages in stack order\n", drain);
  }
  std::printf("table_check ok: %lld page lists compared, %d requests\n", compared_lists,
              next_request);
  CHECK_OK(dsd_table_destroy(table));
  CHECK_OK(dsd_pool_destroy(pool));
  return 0;
}
