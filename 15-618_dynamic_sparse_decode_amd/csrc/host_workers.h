// host_workers.h -- a fixed set of host threads for the host-side halves of
// the path: payload generation in the serving loop and the staging copies of
// large uploads.  Header-only; each library that includes it owns one pool,
// created on first use.  Size: DSD_HOST_THREADS if set (1 = run inline),
// else min(hardware threads, 16).
#pragma once

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <cstdlib>
#include <functional>
#include <mutex>
#include <thread>
#include <vector>

namespace dsd_host {

class Workers {
 public:
  static Workers& Get() {
    static Workers pool;
    return pool;
  }

  int size() const { return static_cast<int>(threads_.size()) + 1; }

  // fn(i) for every i in [0, n), spread over the workers and the calling
  // thread; returns when all are done.  Calls from several threads run one
  // after another.  fn must not call ParallelFor.
  void ParallelFor(int n, const std::function<void(int)>& fn) {
    if (n <= 0) return;
    if (threads_.empty() || n == 1) {
      for (int i = 0; i < n; ++i) fn(i);
      return;
    }
    std::lock_guard<std::mutex> serial(call_);
    {
      std::lock_guard<std::mutex> lock(mu_);
      job_ = &fn;
      count_ = n;
      next_.store(0);
      pending_ = static_cast<int>(threads_.size());
      ++generation_;
    }
    wake_.notify_all();
    Drain();
    std::unique_lock<std::mutex> lock(mu_);
    done_.wait(lock, [&] { return pending_ == 0; });
    job_ = nullptr;
  }

  Workers(const Workers&) = delete;
  Workers& operator=(const Workers&) = delete;

 private:
  Workers() {
    int n = static_cast<int>(std::thread::hardware_concurrency());
    if (n <= 0) n = 1;
    n = std::min(n, 16);
    if (const char* env = std::getenv("DSD_HOST_THREADS")) {
      const int v = std::atoi(env);
      if (v >= 1) n = std::min(v, 64);
    }
    for (int i = 1; i < n; ++i) threads_.emplace_back([this] { Loop(); });
  }

  ~Workers() {
    {
      std::lock_guard<std::mutex> lock(mu_);
      stop_ = true;
    }
    wake_.notify_all();
    for (auto& t : threads_) t.join();
  }

  void Drain() {
    for (int i = next_.fetch_add(1); i < count_; i = next_.fetch_add(1)) (*job_)(i);
  }

  void Loop() {
    unsigned long long seen = 0;
    for (;;) {
      {
        std::unique_lock<std::mutex> lock(mu_);
        wake_.wait(lock, [&] { return stop_ || generation_ != seen; });
        if (stop_) return;
        seen = generation_;
      }
      Drain();
      {
        std::lock_guard<std::mutex> lock(mu_);
        if (--pending_ == 0) done_.notify_one();
      }
    }
  }

  std::vector<std::thread> threads_;
  std::mutex call_;
  std::mutex mu_;
  std::condition_variable wake_;
  std::condition_variable done_;
  const std::function<void(int)>* job_ = nullptr;
  int count_ = 0;
  std::atomic<int> next_{0};
  int pending_ = 0;
  unsigned long long generation_ = 0;
  bool stop_ = false;
};

}  // namespace dsd_host
