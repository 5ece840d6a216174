// Checks dsd_host::Workers (15-618_dynamic_sparse_decode_amd/csrc/host_workers.h):
// every index runs exactly once, calls are reusable, calls from several
// threads are serialised, and the pool works with one thread.
#include <atomic>
#include <cstdio>
#include <thread>
#include <vector>

#include "host_workers.h"

static int Fail(const char* what, int a, int b) {
  std::printf("FAIL %s: %d vs %d\n", what, a, b);
  return 1;
}

int main() {
  auto& w = dsd_host::Workers::Get();
  for (int n : {0, 1, 2, 3, 17, 100, 4096}) {
    for (int rep = 0; rep < 20; ++rep) {
      std::vector<std::atomic<int>> hits(static_cast<std::size_t>(n));
      for (auto& h : hits) h.store(0);
      w.ParallelFor(n, [&](int i) { hits[static_cast<std::size_t>(i)].fetch_add(1); });
      for (int i = 0; i < n; ++i) {
        if (hits[static_cast<std::size_t>(i)].load() != 1) return Fail("hits", i, hits[i].load());
      }
    }
  }
  // Several callers at once: each call must still see all of its indices.
  std::atomic<int> bad{0};
  std::vector<std::thread> callers;
  for (int c = 0; c < 4; ++c) {
    callers.emplace_back([&, c] {
      for (int rep = 0; rep < 50; ++rep) {
        const int n = 37 + c;
        std::atomic<long> sum{0};
        w.ParallelFor(n, [&](int i) { sum.fetch_add(i + 1); });
        if (sum.load() != static_cast<long>(n) * (n + 1) / 2) bad.fetch_add(1);
      }
    });
  }
  for (auto& t : callers) t.join();
  if (bad.load() != 0) return Fail("concurrent callers", bad.load(), 0);
  std::printf("host workers ok: %d threads\n", w.size());
  return 0;
}
