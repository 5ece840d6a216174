// capi.hip -- the extern "C" boundary of libdsd_hip.so (declared in
// include/dsd_hip.h).  Host-side orchestration only: argument checks with the
// reference's error semantics, HBM allocation, copies, kernel launches and
// timing.  All math runs in the kernels of pool_kernels.hip / step_kernels.hip.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <numeric>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "dsd_hip.h"
#include "dsd_internal.h"
#include "host_workers.h"

using dsdk::PoolView;

namespace {

thread_local std::string g_last_error;

// Runs f and maps the reference's exception types onto status codes.
template <typename F>
int Guard(F&& f) {
  try {
    f();
    return DSD_OK;
  } catch (const std::invalid_argument& e) {
    g_last_error = e.what();
    return DSD_ERR_INVALID_ARGUMENT;
  } catch (const std::out_of_range& e) {
    g_last_error = e.what();
    return DSD_ERR_OUT_OF_RANGE;
  } catch (const dsdk::HipError& e) {
    g_last_error = e.what();
    return DSD_ERR_HIP;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return DSD_ERR_RUNTIME;
  } catch (...) {
    g_last_error = "unknown error";
    return DSD_ERR_RUNTIME;
  }
}

void Require(bool ok, const char* message) {
  if (!ok) throw std::invalid_argument(message);
}

using Clock = std::chrono::steady_clock;
double MsSince(Clock::time_point t0) {
  return std::chrono::duration<double, std::milli>(Clock::now() - t0).count();
}

// Spins until *word >= target: a progress word the device stores with a
// system-scope release (dsdk::ProgressMark, dsdk::LaunchStepMark).  Every
// few thousand polls it asks `stream` for an error, so a failed launch or a
// device fault is reported rather than spun on.
void AwaitWord(const unsigned long long* word, unsigned long long target, hipStream_t stream) {
  for (unsigned long it = 1;; ++it) {
    if (__hip_atomic_load(word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) >= target) return;
    if (it % 4096 == 0) {
      const hipError_t e = hipStreamQuery(stream);
      if (e == hipSuccess) {
        if (__hip_atomic_load(word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) >= target) {
          return;
        }
        throw std::runtime_error("the stream is idle but an awaited progress mark never came");
      }
      if (e != hipErrorNotReady) DSD_HIP_CHECK(e);
      std::this_thread::yield();
    }
  }
}

// Grow-only device buffer.
template <typename T>
struct DeviceBuffer {
  T* ptr = nullptr;
  size_t count = 0;
  DeviceBuffer() = default;
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer() { Release(); }
  void Release() {
    if (ptr != nullptr) (void)hipFree(ptr);
    ptr = nullptr;
    count = 0;
  }
  void Reserve(size_t n) {
    if (n <= count) return;
    Release();
    DSD_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&ptr), n * sizeof(T)));
    count = n;
  }
};

// Grow-only pinned host buffer (allocated pinned; never registered).
template <typename T>
struct PinnedBuffer {
  T* ptr = nullptr;
  size_t count = 0;
  PinnedBuffer() = default;
  PinnedBuffer(const PinnedBuffer&) = delete;
  PinnedBuffer& operator=(const PinnedBuffer&) = delete;
  ~PinnedBuffer() { Release(); }
  void Release() {
    if (ptr != nullptr) (void)hipHostFree(ptr);
    ptr = nullptr;
    count = 0;
  }
  // hipHostMallocCoherent for buffers that kernels read or write directly
  // (no GPU caching of host lines, so no stale data across steps).
  void Reserve(size_t n, unsigned flags = hipHostMallocDefault) {
    if (n <= count) return;
    Release();
    DSD_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&ptr), n * sizeof(T), flags));
    count = n;
  }
};

constexpr uint64_t kLargeCopyBytes = 1ull << 20;  // src/device_page_pool.cpp:13

// Polls of a cross-workgroup wait of the single-launch step before it gives
// up (each poll is a sleep plus a coherent read, about 1-2 us).  A wait
// normally ends within microseconds; the limit, about 0.1-0.3 s, only
// bounds a step whose workgroups cannot all get a compute unit (another
// process holding them), which then fails instead of hanging.
constexpr unsigned kDefaultSpinLimit = 1u << 17;

// Uploads from pageable memory of at least kStageMinBytes go through pinned
// staging: the host threads copy one chunk while the DMA engine moves the
// previous one (the runtime's own pageable path copies at about 27 GB/s on
// the MI355X boxes, bound by one host thread).
constexpr size_t kStageMinBytes = 4u << 20;
constexpr size_t kStageChunkBytes = 16u << 20;
constexpr int kStageBuffers = 3;
constexpr size_t kStagePieceBytes = 1u << 20;  // per host thread task

// True for memory the device reads directly (hipHostMalloc'd or registered).
bool IsPinnedHost(const void* p) {
  hipPointerAttribute_t attr{};
  if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
    (void)hipGetLastError();  // pageable memory may report an error: clear it
    return false;
  }
  return attr.type == hipMemoryTypeHost;
}

// The blocks handed out by dsd_host_alloc (pinned) and dsd_device_alloc
// (start -> bytes), so a step that reads query rows in place can check that
// every row lies inside memory the device may read.
class RowBlocks {
 public:
  static RowBlocks& Host() {
    static RowBlocks blocks;
    return blocks;
  }
  static RowBlocks& Device() {
    static RowBlocks blocks;
    return blocks;
  }
  // Whether [p, p + bytes) lies inside one block.
  bool Holds(const void* p, size_t bytes) {
    const float* row = static_cast<const float*>(p);
    return FirstOutside(&row, 1, bytes) < 0;
  }
  void Add(void* p, size_t bytes) {
    std::lock_guard<std::mutex> lock(mu_);
    blocks_[reinterpret_cast<uintptr_t>(p)] = bytes;
  }
  bool Remove(void* p) {
    std::lock_guard<std::mutex> lock(mu_);
    return blocks_.erase(reinterpret_cast<uintptr_t>(p)) == 1;
  }
  // Index of the first of rows[0..n) that does not lie whole inside one
  // block, or -1 when all do.
  int FirstOutside(const float* const* rows, int n, size_t row_bytes) {
    std::lock_guard<std::mutex> lock(mu_);
    for (int r = 0; r < n; ++r) {
      const uintptr_t a = reinterpret_cast<uintptr_t>(rows[r]);
      auto it = blocks_.upper_bound(a);
      if (it == blocks_.begin()) return r;
      --it;
      const uintptr_t off = a - it->first;
      if (off > it->second || row_bytes > it->second - off) return r;
    }
    return -1;
  }

 private:
  std::mutex mu_;
  std::map<uintptr_t, size_t> blocks_;
};

// memcpy on the host threads, in pieces of kStagePieceBytes.
void ParallelCopy(void* dst, const void* src, size_t bytes) {
  const int pieces = static_cast<int>((bytes + kStagePieceBytes - 1) / kStagePieceBytes);
  dsd_host::Workers::Get().ParallelFor(pieces, [&](int i) {
    const size_t off = static_cast<size_t>(i) * kStagePieceBytes;
    const size_t n = std::min(kStagePieceBytes, bytes - off);
    std::memcpy(static_cast<char*>(dst) + off, static_cast<const char*>(src) + off, n);
  });
}

}  // namespace

// ---------------------------------------------------------------------------
// Pool
// ---------------------------------------------------------------------------
struct dsd_pool {
  PoolView view;
  std::vector<int> host_counts;
  std::vector<uint8_t> host_live;
  mutable dsd_transfer_stats stats{};
  hipStream_t stream = nullptr;
  // staging for metadata / token uploads
  DeviceBuffer<int> stage_ids, stage_counts, stage_offsets, stage_order, stage_segs;
  DeviceBuffer<float> stage_rows, stage_keys, stage_values;
  // dense-path scratch: device inputs, and coherent pinned staging that the
  // stage-in kernel reads and the attention writes its outputs into
  DeviceBuffer<float> dense_q;
  DeviceBuffer<int> dense_offsets, dense_ids;
  PinnedBuffer<float> h_dense_q, h_dense_out;
  PinnedBuffer<int> h_dense_offsets, h_dense_ids;
  hipEvent_t dense_start = nullptr, dense_stop = nullptr;
  uint64_t* k_offsets = nullptr;  // [capacity] element offset of each page
  uint64_t* v_offsets = nullptr;
  // The synthetic append returns once enqueued: `done` marks its end, its
  // metadata travels from pinned staging, and every other pool call (and
  // every step on a context using the pool) is ordered after it.
  hipEvent_t done = nullptr;
  mutable bool pending = false;
  PinnedBuffer<int> h_meta;
  // Pinned chunks for large pageable uploads; stage_ev[b] marks the end of
  // the last DMA out of chunk b.
  PinnedBuffer<char> stage_host[kStageBuffers];
  hipEvent_t stage_ev[kStageBuffers] = {};
  bool stage_busy[kStageBuffers] = {};
  int stage_next = 0;

  ~dsd_pool() {
    if (pending && done) (void)hipEventSynchronize(done);
    if (done) (void)hipEventDestroy(done);
    for (int b = 0; b < kStageBuffers; ++b) {
      if (stage_ev[b]) {
        if (stage_busy[b]) (void)hipEventSynchronize(stage_ev[b]);
        (void)hipEventDestroy(stage_ev[b]);
      }
    }
    if (k_offsets) (void)hipFree(k_offsets);
    if (v_offsets) (void)hipFree(v_offsets);
    if (view.keys) (void)hipFree(view.keys);
    if (view.values) (void)hipFree(view.values);
    if (view.summaries) (void)hipFree(view.summaries);
    if (view.token_counts) (void)hipFree(view.token_counts);
    if (view.live) (void)hipFree(view.live);
    if (dense_start) (void)hipEventDestroy(dense_start);
    if (dense_stop) (void)hipEventDestroy(dense_stop);
    if (stream) (void)hipStreamDestroy(stream);
  }

  void H2D(void* dst, const void* src, size_t bytes) {
    if (bytes == 0) return;
    if (bytes >= kStageMinBytes && !IsPinnedHost(src)) {
      StagedH2D(dst, src, bytes);
    } else {
      DSD_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, stream));
    }
    CountH2D(bytes);
  }
  // One host -> device transfer of the reference's accounting
  // (src/device_page_pool.cpp:1137-1150).
  void CountH2D(size_t bytes) {
    stats.h2d_bytes += bytes;
    ++stats.h2d_calls;
    if (bytes >= kLargeCopyBytes) ++stats.h2d_large_calls;
  }
  void D2H(void* dst, const void* src, size_t bytes) const {
    if (bytes == 0) return;
    DSD_HIP_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, stream));
    stats.d2h_bytes += bytes;
    ++stats.d2h_calls;
    if (bytes >= kLargeCopyBytes) ++stats.d2h_large_calls;
  }
  // A pageable upload in chunks through the pinned staging ring.  The
  // caller's buffer may be reused as soon as this returns (every byte has
  // been copied out of it); the DMA of the last chunks may still run.
  void StagedH2D(void* dst, const void* src, size_t bytes) {
    for (int b = 0; b < kStageBuffers; ++b) {
      if (stage_host[b].ptr == nullptr) {
        stage_host[b].Reserve(kStageChunkBytes);
        DSD_HIP_CHECK(hipEventCreateWithFlags(&stage_ev[b], hipEventDisableTiming));
      }
    }
    for (size_t off = 0; off < bytes; off += kStageChunkBytes) {
      const size_t n = std::min(kStageChunkBytes, bytes - off);
      const int b = stage_next;
      stage_next = (b + 1) % kStageBuffers;
      if (stage_busy[b]) DSD_HIP_CHECK(hipEventSynchronize(stage_ev[b]));
      ParallelCopy(stage_host[b].ptr, static_cast<const char*>(src) + off, n);
      DSD_HIP_CHECK(hipMemcpyAsync(static_cast<char*>(dst) + off, stage_host[b].ptr, n,
                                   hipMemcpyHostToDevice, stream));
      DSD_HIP_CHECK(hipEventRecord(stage_ev[b], stream));
      stage_busy[b] = true;
    }
  }
  void Sync() const { DSD_HIP_CHECK(hipStreamSynchronize(stream)); }
  // The host waits for an enqueued append (before reusing its staging).
  void WaitPending() const {
    if (pending) {
      DSD_HIP_CHECK(hipEventSynchronize(done));
      pending = false;
    }
  }
  // Work enqueued on another stream starts after an enqueued append (on
  // the pool's own stream, stream order does it).
  void OrderAfterPending(hipStream_t s) const {
    if (pending && s != stream) DSD_HIP_CHECK(hipStreamWaitEvent(s, done, 0));
  }

  void ValidatePage(int page_id) const {
    if (page_id < 0 || page_id >= view.capacity) {
      throw std::out_of_range("invalid page id");
    }
  }
  void ValidateTokenCount(int count) const {
    if (count <= 0 || count > view.page_size) {
      throw std::invalid_argument("token_count must be in (0, page_size]");
    }
  }
};

extern "C" {

const char* dsd_last_error(void) { return g_last_error.c_str(); }

int dsd_gpu_available(void) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) return 0;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int dsd_device_synchronize(void) {
  return Guard([&] { DSD_HIP_CHECK(hipDeviceSynchronize()); });
}

int dsd_pool_create(int num_heads, int head_dim, int page_size,
                    int capacity_pages, dsd_pool** out_pool) {
  return Guard([&] {
    Require(out_pool != nullptr, "out_pool must be non-null");
    *out_pool = nullptr;
    if (capacity_pages < 0) {
      throw std::invalid_argument("capacity_pages must be non-negative");
    }
    Require(num_heads > 0 && head_dim > 0 && page_size > 0,
            "num_heads, head_dim and page_size must be positive");
    if (!dsd_gpu_available()) {
      throw std::runtime_error("no visible gfx950 GPU");
    }
    auto pool = std::make_unique<dsd_pool>();
    PoolView& v = pool->view;
    v.num_heads = num_heads;
    v.head_dim = head_dim;
    v.page_size = page_size;
    v.elements = num_heads * head_dim;
    v.capacity = capacity_pages;
    v.page_elems = static_cast<int64_t>(page_size) * v.elements;
    DSD_HIP_CHECK(hipStreamCreateWithFlags(&pool->stream, hipStreamNonBlocking));
    DSD_HIP_CHECK(hipEventCreateWithFlags(&pool->done, hipEventDisableTiming));
    DSD_HIP_CHECK(hipEventCreate(&pool->dense_start));
    DSD_HIP_CHECK(hipEventCreate(&pool->dense_stop));
    pool->host_counts.assign(static_cast<size_t>(capacity_pages), 0);
    pool->host_live.assign(static_cast<size_t>(capacity_pages), 0);
    if (capacity_pages > 0) {
      const size_t kv_bytes = static_cast<size_t>(capacity_pages) *
                              static_cast<size_t>(v.page_elems) * sizeof(float);
      const size_t sum_bytes = static_cast<size_t>(capacity_pages) *
                               static_cast<size_t>(v.elements) * sizeof(float);
      DSD_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&v.keys), kv_bytes));
      DSD_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&v.values), kv_bytes));
      DSD_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&v.summaries), sum_bytes));
      DSD_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&v.token_counts),
                              sizeof(int) * static_cast<size_t>(capacity_pages)));
      DSD_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&v.live),
                              static_cast<size_t>(capacity_pages)));
      DSD_HIP_CHECK(hipMemsetAsync(v.summaries, 0, sum_bytes, pool->stream));
      DSD_HIP_CHECK(hipMemsetAsync(v.token_counts, 0,
                                   sizeof(int) * static_cast<size_t>(capacity_pages),
                                   pool->stream));
      DSD_HIP_CHECK(hipMemsetAsync(v.live, 0, static_cast<size_t>(capacity_pages),
                                   pool->stream));
      std::vector<uint64_t> offsets(static_cast<size_t>(capacity_pages));
      for (int p = 0; p < capacity_pages; ++p) {
        offsets[p] = static_cast<uint64_t>(p) * static_cast<uint64_t>(v.page_elems);
      }
      const size_t off_bytes = sizeof(uint64_t) * offsets.size();
      DSD_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&pool->k_offsets), off_bytes));
      DSD_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&pool->v_offsets), off_bytes));
      DSD_HIP_CHECK(hipMemcpy(pool->k_offsets, offsets.data(), off_bytes, hipMemcpyHostToDevice));
      DSD_HIP_CHECK(hipMemcpy(pool->v_offsets, offsets.data(), off_bytes, hipMemcpyHostToDevice));
      pool->Sync();
    }
    *out_pool = pool.release();
  });
}

int dsd_pool_destroy(dsd_pool* pool) {
  return Guard([&] {
    if (pool != nullptr) {
      (void)hipStreamSynchronize(pool->stream);
      pool->pending = false;
      delete pool;
    }
  });
}

int dsd_pool_capacity(const dsd_pool* pool) {
  return pool == nullptr ? 0 : pool->view.capacity;
}

int dsd_pool_reset(dsd_pool* pool) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    const PoolView& v = pool->view;
    std::fill(pool->host_counts.begin(), pool->host_counts.end(), 0);
    std::fill(pool->host_live.begin(), pool->host_live.end(), 0);
    if (v.capacity > 0) {
      DSD_HIP_CHECK(hipMemsetAsync(v.summaries, 0,
                                   sizeof(float) * static_cast<size_t>(v.capacity) *
                                       static_cast<size_t>(v.elements),
                                   pool->stream));
      DSD_HIP_CHECK(hipMemsetAsync(v.token_counts, 0,
                                   sizeof(int) * static_cast<size_t>(v.capacity),
                                   pool->stream));
      DSD_HIP_CHECK(hipMemsetAsync(v.live, 0, static_cast<size_t>(v.capacity),
                                   pool->stream));
    }
    pool->Sync();
  });
}

int dsd_pool_upload_pages(dsd_pool* pool, int n, const int* page_ids,
                          const int* token_counts, const int64_t* src_offsets,
                          const float* keys, const float* values,
                          const float* summaries) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    Require(n >= 0, "page count must be non-negative");
    if (n == 0) return;
    Require(page_ids != nullptr && token_counts != nullptr && src_offsets != nullptr,
            "page metadata pointers must be non-null");
    Require(keys != nullptr && values != nullptr,
            "host page payload pointers must be non-null");
    const PoolView& v = pool->view;
    const int E = v.elements;
    for (int i = 0; i < n; ++i) {
      pool->ValidatePage(page_ids[i]);
      pool->ValidateTokenCount(token_counts[i]);
      Require(src_offsets[i] >= 0, "source offsets must be non-negative");
    }
    // Payload copies: merge runs of full pages that are consecutive both in
    // the pool and in the source into one copy each.
    int i = 0;
    while (i < n) {
      int run_end = i + 1;
      if (token_counts[i] == v.page_size) {
        while (run_end < n && token_counts[run_end] == v.page_size &&
               page_ids[run_end] == page_ids[run_end - 1] + 1 &&
               src_offsets[run_end] == src_offsets[run_end - 1] + v.page_elems) {
          ++run_end;
        }
      }
      const int pages = run_end - i;
      const size_t elems = pages == 1
                               ? static_cast<size_t>(token_counts[i]) * E
                               : static_cast<size_t>(pages) * v.page_elems;
      const size_t dst = static_cast<size_t>(page_ids[i]) * v.page_elems;
      pool->H2D(v.keys + dst, keys + src_offsets[i], elems * sizeof(float));
      pool->H2D(v.values + dst, values + src_offsets[i], elems * sizeof(float));
      i = run_end;
    }
    // Metadata + summaries: one entry per distinct page, the last occurrence
    // winning (its payload copy was also enqueued last).
    std::vector<int> last(n, 1);
    {
      std::vector<int> idx(n);
      std::iota(idx.begin(), idx.end(), 0);
      std::stable_sort(idx.begin(), idx.end(),
                       [&](int a, int b) { return page_ids[a] < page_ids[b]; });
      for (int q = 0; q + 1 < n; ++q) {
        if (page_ids[idx[q]] == page_ids[idx[q + 1]]) last[idx[q]] = 0;
      }
    }
    std::vector<int> ids, counts, rows_src;
    ids.reserve(n);
    counts.reserve(n);
    for (int q = 0; q < n; ++q) {
      if (!last[q]) continue;
      ids.push_back(page_ids[q]);
      counts.push_back(token_counts[q]);
      rows_src.push_back(q);
      pool->host_counts[page_ids[q]] = token_counts[q];
      pool->host_live[page_ids[q]] = 1;
    }
    const int m = static_cast<int>(ids.size());
    pool->stage_ids.Reserve(m);
    pool->stage_counts.Reserve(m);
    pool->H2D(pool->stage_ids.ptr, ids.data(), sizeof(int) * m);
    pool->H2D(pool->stage_counts.ptr, counts.data(), sizeof(int) * m);
    const float* d_rows = nullptr;
    if (summaries != nullptr) {
      std::vector<float> rows(static_cast<size_t>(m) * E);
      for (int q = 0; q < m; ++q) {
        std::memcpy(rows.data() + static_cast<size_t>(q) * E,
                    summaries + static_cast<size_t>(rows_src[q]) * E,
                    sizeof(float) * E);
      }
      pool->stage_rows.Reserve(rows.size());
      pool->H2D(pool->stage_rows.ptr, rows.data(), sizeof(float) * rows.size());
      d_rows = pool->stage_rows.ptr;
    }
    dsdk::LaunchFinishPageUpload(v, pool->stage_ids.ptr, pool->stage_counts.ptr,
                                 d_rows, m, pool->stream);
    pool->Sync();
  });
}

int dsd_pool_upload_tokens(dsd_pool* pool, int n, const int* page_ids,
                           const int* token_offsets,
                           const int* page_token_counts, const float* keys,
                           const float* values, const float* summaries) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    Require(n >= 0, "token count must be non-negative");
    if (n == 0) return;
    Require(page_ids != nullptr && token_offsets != nullptr &&
                page_token_counts != nullptr,
            "token metadata pointers must be non-null");
    Require(keys != nullptr && values != nullptr,
            "token payload pointers must be non-null");
    const PoolView& v = pool->view;
    const int E = v.elements;
    for (int i = 0; i < n; ++i) {
      pool->ValidatePage(page_ids[i]);
      pool->ValidateTokenCount(page_token_counts[i]);
      if (token_offsets[i] < 0 || token_offsets[i] >= page_token_counts[i]) {
        throw std::out_of_range("token_offset is outside the valid page prefix");
      }
    }
    // Segments: tokens sorted by (page, offset), one segment per page.
    std::vector<int> order(n);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
      if (page_ids[a] != page_ids[b]) return page_ids[a] < page_ids[b];
      return token_offsets[a] < token_offsets[b];
    });
    std::vector<int> segs;
    segs.push_back(0);
    for (int q = 1; q < n; ++q) {
      if (page_ids[order[q]] != page_ids[order[q - 1]]) segs.push_back(q);
    }
    segs.push_back(n);
    const int nseg = static_cast<int>(segs.size()) - 1;
    if (summaries == nullptr) {
      // Device running mean: each page's tokens must extend its current prefix.
      for (int s = 0; s < nseg; ++s) {
        const int page = page_ids[order[segs[s]]];
        int expect = token_offsets[order[segs[s]]] == 0 ? 0 : pool->host_counts[page];
        for (int q = segs[s]; q < segs[s + 1]; ++q) {
          if (token_offsets[order[q]] != expect) {
            throw std::invalid_argument(
                "device summary update needs tokens that extend the page prefix");
          }
          ++expect;
        }
      }
    }
    for (int q = 0; q < n; ++q) {
      pool->host_counts[page_ids[q]] = page_token_counts[q];
      pool->host_live[page_ids[q]] = 1;
    }
    const size_t row_elems = static_cast<size_t>(n) * E;
    pool->stage_keys.Reserve(row_elems);
    pool->stage_values.Reserve(row_elems);
    pool->stage_ids.Reserve(n);
    pool->stage_offsets.Reserve(n);
    pool->stage_counts.Reserve(n);
    pool->stage_order.Reserve(n);
    pool->stage_segs.Reserve(nseg + 1);
    pool->H2D(pool->stage_keys.ptr, keys, sizeof(float) * row_elems);
    pool->H2D(pool->stage_values.ptr, values, sizeof(float) * row_elems);
    pool->H2D(pool->stage_ids.ptr, page_ids, sizeof(int) * n);
    pool->H2D(pool->stage_offsets.ptr, token_offsets, sizeof(int) * n);
    pool->H2D(pool->stage_counts.ptr, page_token_counts, sizeof(int) * n);
    pool->H2D(pool->stage_order.ptr, order.data(), sizeof(int) * n);
    pool->H2D(pool->stage_segs.ptr, segs.data(), sizeof(int) * (nseg + 1));
    const float* d_rows = nullptr;
    if (summaries != nullptr) {
      pool->stage_rows.Reserve(row_elems);
      pool->H2D(pool->stage_rows.ptr, summaries, sizeof(float) * row_elems);
      d_rows = pool->stage_rows.ptr;
    }
    dsdk::LaunchAppendTokens(v, pool->stage_segs.ptr, pool->stage_order.ptr,
                             pool->stage_ids.ptr, pool->stage_offsets.ptr,
                             pool->stage_counts.ptr, pool->stage_keys.ptr,
                             pool->stage_values.ptr, d_rows, nseg, pool->stream);
    pool->Sync();
  });
}

int dsd_pool_mark_free(dsd_pool* pool, int n, const int* page_ids) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    Require(n >= 0, "page count must be non-negative");
    if (n == 0) return;
    Require(page_ids != nullptr, "page ids must be non-null");
    std::vector<int> ids(page_ids, page_ids + n);
    std::sort(ids.begin(), ids.end());
    ids.erase(std::unique(ids.begin(), ids.end()), ids.end());
    for (int id : ids) pool->ValidatePage(id);
    for (int id : ids) {
      pool->host_counts[id] = 0;
      pool->host_live[id] = 0;
    }
    const int m = static_cast<int>(ids.size());
    pool->stage_ids.Reserve(m);
    pool->H2D(pool->stage_ids.ptr, ids.data(), sizeof(int) * m);
    dsdk::LaunchMarkFree(pool->view, pool->stage_ids.ptr, m, pool->stream);
    pool->Sync();
  });
}

int dsd_pool_download_page(const dsd_pool* pool, int page_id, float* keys,
                           float* values, int* token_count) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    Require(keys != nullptr && values != nullptr, "download outputs must be non-null");
    pool->ValidatePage(page_id);
    // The device's metadata (pages handed out by a dsd_table are not in the
    // host mirror).
    int count = 0;
    uint8_t live = 0;
    DSD_HIP_CHECK(hipMemcpyAsync(&count, pool->view.token_counts + page_id, sizeof(int),
                                 hipMemcpyDeviceToHost, pool->stream));
    DSD_HIP_CHECK(hipMemcpyAsync(&live, pool->view.live + page_id, 1, hipMemcpyDeviceToHost,
                                 pool->stream));
    pool->Sync();
    if (live == 0 || count == 0) {
      throw std::runtime_error("cannot download a free device page");
    }
    const PoolView& v = pool->view;
    const size_t elems = static_cast<size_t>(count) * v.elements;
    const size_t off = static_cast<size_t>(page_id) * v.page_elems;
    pool->D2H(keys, v.keys + off, elems * sizeof(float));
    pool->D2H(values, v.values + off, elems * sizeof(float));
    pool->Sync();
    if (token_count != nullptr) *token_count = count;
  });
}

int dsd_pool_download_meta(const dsd_pool* pool, int* token_counts,
                           uint8_t* live) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    Require(token_counts != nullptr && live != nullptr,
            "metadata outputs must be non-null");
    const PoolView& v = pool->view;
    pool->D2H(token_counts, v.token_counts, sizeof(int) * static_cast<size_t>(v.capacity));
    pool->D2H(live, v.live, static_cast<size_t>(v.capacity));
    pool->Sync();
  });
}

int dsd_pool_download_summaries(const dsd_pool* pool, int n,
                                const int* page_ids, float* out) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    Require(n >= 0, "page count must be non-negative");
    if (n == 0) return;
    Require(page_ids != nullptr && out != nullptr, "pointers must be non-null");
    const PoolView& v = pool->view;
    for (int i = 0; i < n; ++i) pool->ValidatePage(page_ids[i]);
    for (int i = 0; i < n; ++i) {
      pool->D2H(out + static_cast<size_t>(i) * v.elements,
                v.summaries + static_cast<size_t>(page_ids[i]) * v.elements,
                sizeof(float) * v.elements);
    }
    pool->Sync();
  });
}

int dsd_pool_device_arrays(const dsd_pool* pool, dsd_pool_arrays* out) {
  return Guard([&] {
    Require(pool != nullptr && out != nullptr, "pointers must be non-null");
    pool->WaitPending();
    out->keys = pool->view.keys;
    out->values = pool->view.values;
    out->summaries = pool->view.summaries;
    out->token_counts = pool->view.token_counts;
    out->live = pool->view.live;
    out->k_offsets = pool->k_offsets;
    out->v_offsets = pool->v_offsets;
  });
}

int dsd_pool_prefill_synthetic(dsd_pool* pool, int n, const int* page_ids,
                               const int* token_counts, int request_id) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    Require(n >= 0, "page count must be non-negative");
    if (n == 0) return;
    Require(page_ids != nullptr && token_counts != nullptr, "pointers must be non-null");
    for (int i = 0; i < n; ++i) {
      pool->ValidatePage(page_ids[i]);
      pool->ValidateTokenCount(token_counts[i]);
    }
    for (int i = 0; i < n; ++i) {
      pool->host_counts[page_ids[i]] = token_counts[i];
      pool->host_live[page_ids[i]] = 1;
    }
    pool->stage_ids.Reserve(n);
    pool->stage_counts.Reserve(n);
    pool->H2D(pool->stage_ids.ptr, page_ids, sizeof(int) * n);
    pool->H2D(pool->stage_counts.ptr, token_counts, sizeof(int) * n);
    dsdk::LaunchPrefillSynthetic(pool->view, pool->stage_ids.ptr, pool->stage_counts.ptr, n,
                                 request_id, pool->stream);
    pool->Sync();
  });
}

int dsd_pool_append_synthetic(dsd_pool* pool, int n, const int* page_ids,
                              const int* token_offsets, const int* page_token_counts,
                              const int* request_ids, const int* decode_steps) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    Require(n >= 0, "token count must be non-negative");
    if (n == 0) return;
    Require(page_ids != nullptr && token_offsets != nullptr && page_token_counts != nullptr &&
                request_ids != nullptr && decode_steps != nullptr,
            "pointers must be non-null");
    for (int i = 0; i < n; ++i) {
      pool->ValidatePage(page_ids[i]);
      pool->ValidateTokenCount(page_token_counts[i]);
      if (token_offsets[i] < 0 || token_offsets[i] >= page_token_counts[i]) {
        throw std::out_of_range("token_offset is outside the valid page prefix");
      }
    }
    std::vector<int> order(n);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
      if (page_ids[a] != page_ids[b]) return page_ids[a] < page_ids[b];
      return token_offsets[a] < token_offsets[b];
    });
    std::vector<int> segs{0};
    for (int q = 1; q < n; ++q) {
      if (page_ids[order[q]] != page_ids[order[q - 1]]) segs.push_back(q);
    }
    segs.push_back(n);
    const int nseg = static_cast<int>(segs.size()) - 1;
    for (int q = 0; q < n; ++q) {
      pool->host_counts[page_ids[q]] = page_token_counts[q];
      pool->host_live[page_ids[q]] = 1;
    }
    // The metadata goes into coherent pinned staging that the kernel reads
    // directly (the previous append has finished with it: WaitPending
    // above): segment starts, then the tokens' five fields in page / offset
    // order.  The call returns once the kernel is enqueued.  The transfer
    // count is the reference's: five copies of n ints.
    const size_t un = static_cast<size_t>(n);
    pool->h_meta.Reserve(5 * un + static_cast<size_t>(nseg) + 1, hipHostMallocCoherent);
    int* m = pool->h_meta.ptr;
    std::memcpy(m, segs.data(), sizeof(int) * (static_cast<size_t>(nseg) + 1));
    int* f = m + nseg + 1;
    for (int q = 0; q < n; ++q) {
      const int t = order[q];
      f[q] = page_ids[t];
      f[un + q] = token_offsets[t];
      f[2 * un + q] = page_token_counts[t];
      f[3 * un + q] = request_ids[t];
      f[4 * un + q] = decode_steps[t];
    }
    for (int c = 0; c < 5; ++c) pool->CountH2D(sizeof(int) * un);
    dsdk::LaunchAppendSynthetic(pool->view, m, n, nseg, pool->stream);
    DSD_HIP_CHECK(hipEventRecord(pool->done, pool->stream));
    pool->pending = true;
  });
}

int dsd_pool_transfer_stats(const dsd_pool* pool, dsd_transfer_stats* out) {
  return Guard([&] {
    Require(pool != nullptr && out != nullptr, "pointers must be non-null");
    *out = pool->stats;
  });
}

int dsd_pool_reset_transfer_stats(dsd_pool* pool) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->stats = dsd_transfer_stats{};
  });
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Request -> page table (device resident; kernels in page_table.hip)
// ---------------------------------------------------------------------------
namespace {
// Pinned argument blocks that the table's kernels read directly; a block is
// rewritten only after the work that read it is done (ring of kArgBlocks).
constexpr int kArgBlocks = 8;
}  // namespace

struct dsd_table {
  dsd_pool* pool = nullptr;
  dsdk::TableView view;
  DeviceBuffer<int> pages, npages, stack, top;
  // Host mirror of the device counts: pages per slot, device tokens in each
  // slot's tail page, free pages.  Page ids stay on the device.
  std::vector<int> h_npages, h_tail;
  int h_free = 0;
  // staging
  DeviceBuffer<float> d_keys, d_values;  // prompt / appended rows
  DeviceBuffer<int> d_plan, d_order;
  PinnedBuffer<int> h_args[kArgBlocks];
  hipEvent_t args_ev[kArgBlocks] = {};
  bool args_busy[kArgBlocks] = {};
  // A block whose reader stores a progress mark instead (the per-step
  // append and release): the mark's sequence number, 0 when none pending.
  unsigned long long args_seq[kArgBlocks] = {};
  PinnedBuffer<unsigned long long> h_progress;  // the marks' word
  unsigned long long progress_seq = 0;
  int args_next = 0;
  // Prompt staging ahead of admission (dsd_table_staging_init): device
  // buffers filled on a copy stream of their own, from a pinned ring; a
  // buffer is ready when stg_ready fires and free again when the admission
  // that read it has finished (stg_free).
  hipStream_t copy_stream = nullptr;
  int stg_tokens = 0;
  std::vector<std::unique_ptr<DeviceBuffer<float>>> stg_k, stg_v;
  std::vector<hipEvent_t> stg_ready, stg_free;
  std::vector<char> stg_freed;  // stg_free recorded since the last staging
  PinnedBuffer<char> ring[kStageBuffers];
  hipEvent_t ring_ev[kStageBuffers] = {};
  bool ring_busy[kStageBuffers] = {};
  int ring_next = 0;

  ~dsd_table() {
    if (progress_seq != 0) (void)hipStreamSynchronize(pool->stream);
    for (int b = 0; b < kArgBlocks; ++b) {
      if (args_ev[b]) {
        if (args_busy[b]) (void)hipEventSynchronize(args_ev[b]);
        (void)hipEventDestroy(args_ev[b]);
      }
    }
    if (copy_stream != nullptr) (void)hipStreamSynchronize(copy_stream);
    for (int b = 0; b < kStageBuffers; ++b) {
      if (ring_ev[b]) (void)hipEventDestroy(ring_ev[b]);
    }
    for (hipEvent_t e : stg_ready) (void)hipEventDestroy(e);
    for (hipEvent_t e : stg_free) {
      (void)hipEventSynchronize(e);
      (void)hipEventDestroy(e);
    }
    if (copy_stream != nullptr) (void)hipStreamDestroy(copy_stream);
  }
  // A pageable host block into device memory on the copy stream, through
  // the pinned ring (host threads fill one chunk while the DMA moves the
  // previous one).
  void CopyIn(float* dst, const float* src, size_t bytes) {
    const char* s = reinterpret_cast<const char*>(src);
    char* d = reinterpret_cast<char*>(dst);
    for (size_t off = 0; off < bytes; off += kStageChunkBytes) {
      const size_t n = std::min(kStageChunkBytes, bytes - off);
      const int b = ring_next;
      ring_next = (b + 1) % kStageBuffers;
      if (ring_busy[b]) DSD_HIP_CHECK(hipEventSynchronize(ring_ev[b]));
      ParallelCopy(ring[b].ptr, s + off, n);
      DSD_HIP_CHECK(hipMemcpyAsync(d + off, ring[b].ptr, n, hipMemcpyHostToDevice, copy_stream));
      DSD_HIP_CHECK(hipEventRecord(ring_ev[b], copy_stream));
      ring_busy[b] = true;
    }
  }
  // A pinned block of at least n ints that no enqueued kernel still reads;
  // Done(block) after the launches that read it.
  int Acquire(size_t n) {
    const int b = args_next;
    args_next = (b + 1) % kArgBlocks;
    if (args_busy[b]) {
      DSD_HIP_CHECK(hipEventSynchronize(args_ev[b]));
      args_busy[b] = false;
    }
    if (args_seq[b] != 0) {
      AwaitWord(h_progress.ptr, args_seq[b], pool->stream);
      args_seq[b] = 0;
    }
    h_args[b].Reserve(std::max<size_t>(n, 64), hipHostMallocCoherent);
    return b;
  }
  void Done(int b) {
    DSD_HIP_CHECK(hipEventRecord(args_ev[b], pool->stream));
    args_busy[b] = true;
  }
  // Done(b) by a progress mark the launch's last kernel stores (no event
  // barrier on the stream).
  dsdk::ProgressMark Mark(int b) {
    args_seq[b] = ++progress_seq;
    return dsdk::ProgressMark{h_progress.ptr, args_seq[b]};
  }
  void CheckSlot(int slot) const {
    if (slot < 0 || slot >= view.max_slots) throw std::out_of_range("table slot out of range");
  }
  int PagesFor(int tokens) const {
    return (tokens + pool->view.page_size - 1) / pool->view.page_size;
  }
  // Reserves a prompt's pages for an empty slot (mirror + kernel).
  int Reserve(int slot, int tokens) {
    CheckSlot(slot);
    Require(tokens >= 0, "prompt tokens must be non-negative");
    if (h_npages[slot] != 0) throw std::invalid_argument("table slot is not empty");
    const int n = PagesFor(tokens);
    if (n > view.max_pages) throw std::invalid_argument("prompt exceeds the table's max_pages");
    if (n > h_free) throw std::runtime_error("page pool is exhausted");
    // The mirror follows the device only once the kernel is enqueued.
    dsdk::LaunchTableReserve(view, slot, n, pool->stream);
    h_npages[slot] = n;
    h_tail[slot] = n == 0 ? 0 : tokens - (n - 1) * pool->view.page_size;
    h_free -= n;
    return n;
  }
  const int* SlotPages(int slot) const {
    return view.pages + static_cast<size_t>(slot) * view.max_pages;
  }
  // The token counts of a prompt's n pages in a pinned block the upload
  // kernels read (the admission's metadata transfer); Done(block) after.
  int PromptCounts(int tokens, int n, const int** counts) {
    const int b = Acquire(static_cast<size_t>(n));
    int* c = h_args[b].ptr;
    const int ps = pool->view.page_size;
    for (int j = 0; j < n; ++j) c[j] = std::min(ps, tokens - j * ps);
    pool->CountH2D(sizeof(int) * static_cast<size_t>(n));
    *counts = c;
    return b;
  }
};

extern "C" {

int dsd_table_create(dsd_pool* pool, int max_slots, int max_pages, dsd_table** out) {
  return Guard([&] {
    Require(out != nullptr, "out must be non-null");
    *out = nullptr;
    Require(pool != nullptr, "pool must be non-null");
    Require(max_slots > 0 && max_pages > 0, "table sizes must be positive");
    Require(pool->view.elements % 4 == 0, "the table needs E % 4 == 0");
    {
      // Admission ranks a prompt's popped page ids in LDS (4 bytes a page).
      int device = 0, lds = 0;
      DSD_HIP_CHECK(hipGetDevice(&device));
      DSD_HIP_CHECK(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device));
      if (static_cast<int64_t>(max_pages) * static_cast<int64_t>(sizeof(int)) > lds) {
        throw std::invalid_argument("table max_pages exceeds what one admission can rank in LDS (" +
                                    std::to_string(lds / static_cast<int>(sizeof(int))) +
                                    " pages)");
      }
    }
    auto t = std::make_unique<dsd_table>();
    t->pool = pool;
    t->pages.Reserve(static_cast<size_t>(max_slots) * max_pages);
    t->npages.Reserve(max_slots);
    t->stack.Reserve(std::max(1, pool->view.capacity));
    t->top.Reserve(1);
    t->view.pages = t->pages.ptr;
    t->view.npages = t->npages.ptr;
    t->view.free_stack = t->stack.ptr;
    t->view.free_top = t->top.ptr;
    t->view.max_slots = max_slots;
    t->view.max_pages = max_pages;
    t->h_npages.assign(max_slots, 0);
    t->h_tail.assign(max_slots, 0);
    t->h_free = pool->view.capacity;
    // The argument blocks' events only tell the host that the kernels which
    // read a block have finished: no system-scope fence (a cache writeback
    // and invalidate that stalls the stream for microseconds).
    for (hipEvent_t& e : t->args_ev) {
      DSD_HIP_CHECK(
          hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventDisableSystemFence));
    }
    t->h_progress.Reserve(1, hipHostMallocCoherent);
    t->h_progress.ptr[0] = 0;
    for (PinnedBuffer<int>& b : t->h_args) b.Reserve(256, hipHostMallocCoherent);
    dsdk::PreloadTableKernels();
    pool->WaitPending();
    dsdk::LaunchTableReset(t->view, pool->view.capacity, pool->stream);
    pool->Sync();
    *out = t.release();
  });
}

int dsd_table_destroy(dsd_table* table) {
  return Guard([&] {
    if (table == nullptr) return;
    table->pool->Sync();
    delete table;
  });
}

int dsd_table_reset(dsd_table* table) {
  return Guard([&] {
    Require(table != nullptr, "table must be non-null");
    table->pool->WaitPending();
    std::fill(table->h_npages.begin(), table->h_npages.end(), 0);
    std::fill(table->h_tail.begin(), table->h_tail.end(), 0);
    table->h_free = table->pool->view.capacity;
    dsdk::LaunchTableReset(table->view, table->pool->view.capacity, table->pool->stream);
    table->pool->Sync();
  });
}

int dsd_table_slot_pages(const dsd_table* table, int slot, int* count) {
  return Guard([&] {
    Require(table != nullptr && count != nullptr, "pointers must be non-null");
    table->CheckSlot(slot);
    *count = table->h_npages[slot];
  });
}

int dsd_table_free_pages(const dsd_table* table, int* count) {
  return Guard([&] {
    Require(table != nullptr && count != nullptr, "pointers must be non-null");
    *count = table->h_free;
  });
}

int dsd_table_download(dsd_table* table, int slot, int* page_ids, int capacity, int* count) {
  return Guard([&] {
    Require(table != nullptr && count != nullptr, "pointers must be non-null");
    table->CheckSlot(slot);
    const int n = table->h_npages[slot];
    *count = n;
    if (n == 0) return;
    Require(page_ids != nullptr && capacity >= n, "page_ids must hold the slot's pages");
    DSD_HIP_CHECK(hipMemcpyAsync(page_ids, table->SlotPages(slot), sizeof(int) * n,
                                 hipMemcpyDeviceToHost, table->pool->stream));
    table->pool->Sync();
  });
}

int dsd_table_free_stack(dsd_table* table, int* page_ids, int capacity, int* count) {
  return Guard([&] {
    Require(table != nullptr && count != nullptr, "pointers must be non-null");
    const int n = table->h_free;
    *count = n;
    if (n == 0) return;
    Require(page_ids != nullptr && capacity >= n, "page_ids must hold the free pages");
    DSD_HIP_CHECK(hipMemcpyAsync(page_ids, table->view.free_stack, sizeof(int) * n,
                                 hipMemcpyDeviceToHost, table->pool->stream));
    table->pool->Sync();
  });
}

int dsd_table_admit_prompt(dsd_table* table, int slot, int tokens, const float* keys,
                           const float* values) {
  return Guard([&] {
    Require(table != nullptr, "table must be non-null");
    dsd_pool* pool = table->pool;
    pool->WaitPending();
    if (tokens > 0) Require(keys != nullptr && values != nullptr, "prompt rows must be non-null");
    const int n = table->Reserve(slot, tokens);
    if (n == 0) return;
    const size_t elems = static_cast<size_t>(tokens) * pool->view.elements;
    table->d_keys.Reserve(elems);
    table->d_values.Reserve(elems);
    pool->H2D(table->d_keys.ptr, keys, sizeof(float) * elems);
    pool->H2D(table->d_values.ptr, values, sizeof(float) * elems);
    dsdk::LaunchTableScatter(pool->view, table->view, slot, tokens, table->d_keys.ptr,
                             table->d_values.ptr, pool->stream);
    const int* counts = nullptr;
    const int b = table->PromptCounts(tokens, n, &counts);
    dsdk::LaunchFinishPageUpload(pool->view, table->SlotPages(slot), counts, nullptr, n,
                                 pool->stream);
    table->Done(b);
  });
}

int dsd_table_staging_init(dsd_table* table, int buffers, int max_tokens) {
  return Guard([&] {
    Require(table != nullptr, "table must be non-null");
    Require(buffers > 0 && max_tokens > 0, "staging sizes must be positive");
    Require(table->copy_stream == nullptr, "the table's staging is already set up");
    DSD_HIP_CHECK(hipStreamCreateWithFlags(&table->copy_stream, hipStreamNonBlocking));
    const size_t elems = static_cast<size_t>(max_tokens) * table->pool->view.elements;
    table->stg_tokens = max_tokens;
    for (int b = 0; b < buffers; ++b) {
      table->stg_k.push_back(std::make_unique<DeviceBuffer<float>>());
      table->stg_v.push_back(std::make_unique<DeviceBuffer<float>>());
      table->stg_k.back()->Reserve(elems);
      table->stg_v.back()->Reserve(elems);
      hipEvent_t ready = nullptr, freed = nullptr;
      DSD_HIP_CHECK(hipEventCreateWithFlags(&ready, hipEventDisableTiming));
      DSD_HIP_CHECK(hipEventCreateWithFlags(&freed, hipEventDisableTiming));
      table->stg_ready.push_back(ready);
      table->stg_free.push_back(freed);
      table->stg_freed.push_back(0);
    }
    for (int b = 0; b < kStageBuffers; ++b) {
      table->ring[b].Reserve(kStageChunkBytes);
      DSD_HIP_CHECK(hipEventCreateWithFlags(&table->ring_ev[b], hipEventDisableTiming));
    }
  });
}

int dsd_table_stage_prompt(dsd_table* table, int buffer, int tokens, const float* keys,
                           const float* values) {
  return Guard([&] {
    Require(table != nullptr, "table must be non-null");
    Require(table->copy_stream != nullptr, "call dsd_table_staging_init first");
    Require(buffer >= 0 && buffer < static_cast<int>(table->stg_k.size()),
            "staging buffer out of range");
    Require(tokens >= 0 && tokens <= table->stg_tokens, "prompt exceeds the staging buffers");
    if (tokens > 0) Require(keys != nullptr && values != nullptr, "prompt rows must be non-null");
    // The last admission from this buffer has read it.
    if (table->stg_freed[buffer]) DSD_HIP_CHECK(hipEventSynchronize(table->stg_free[buffer]));
    const size_t bytes =
        sizeof(float) * static_cast<size_t>(tokens) * table->pool->view.elements;
    table->CopyIn(table->stg_k[buffer]->ptr, keys, bytes);
    table->CopyIn(table->stg_v[buffer]->ptr, values, bytes);
    DSD_HIP_CHECK(hipEventRecord(table->stg_ready[buffer], table->copy_stream));
  });
}

int dsd_table_admit_staged(dsd_table* table, int slot, int buffer, int tokens) {
  return Guard([&] {
    Require(table != nullptr, "table must be non-null");
    Require(table->copy_stream != nullptr, "call dsd_table_staging_init first");
    Require(buffer >= 0 && buffer < static_cast<int>(table->stg_k.size()),
            "staging buffer out of range");
    Require(tokens <= table->stg_tokens, "prompt exceeds the staging buffers");
    dsd_pool* pool = table->pool;
    pool->WaitPending();
    const int n = table->Reserve(slot, tokens);
    if (n == 0) return;
    // The admission's bytes crossed PCIe on the copy stream.
    const size_t bytes = sizeof(float) * static_cast<size_t>(tokens) * pool->view.elements;
    pool->CountH2D(bytes);
    pool->CountH2D(bytes);
    DSD_HIP_CHECK(hipStreamWaitEvent(pool->stream, table->stg_ready[buffer], 0));
    dsdk::LaunchTableScatter(pool->view, table->view, slot, tokens, table->stg_k[buffer]->ptr,
                             table->stg_v[buffer]->ptr, pool->stream);
    const int* counts = nullptr;
    const int b = table->PromptCounts(tokens, n, &counts);
    dsdk::LaunchFinishPageUpload(pool->view, table->SlotPages(slot), counts, nullptr, n,
                                 pool->stream);
    table->Done(b);
    DSD_HIP_CHECK(hipEventRecord(table->stg_free[buffer], pool->stream));
    table->stg_freed[buffer] = 1;
  });
}

int dsd_table_admit_synthetic(dsd_table* table, int slot, int tokens, int request_id) {
  return Guard([&] {
    Require(table != nullptr, "table must be non-null");
    dsd_pool* pool = table->pool;
    pool->WaitPending();
    const int n = table->Reserve(slot, tokens);
    if (n == 0) return;
    const int* counts = nullptr;
    const int b = table->PromptCounts(tokens, n, &counts);
    dsdk::LaunchPrefillSynthetic(pool->view, table->SlotPages(slot), counts, n, request_id,
                                 pool->stream);
    table->Done(b);
  });
}

int dsd_table_append(dsd_table* table, int n, const int* slots, const unsigned char* fresh_page,
                     const unsigned char* upload, const float* keys, const float* values,
                     const int* request_ids, const int* decode_steps) {
  return Guard([&] {
    Require(table != nullptr, "table must be non-null");
    dsd_pool* pool = table->pool;
    Require(n >= 0, "token count must be non-negative");
    if (n == 0) return;
    Require(slots != nullptr && upload != nullptr, "slots and upload flags must be non-null");
    const bool rows = keys != nullptr || values != nullptr;
    if (rows) Require(keys != nullptr && values != nullptr, "keys and values go together");
    if (!rows) {
      Require(request_ids != nullptr && decode_steps != nullptr,
              "synthetic payloads need request ids and decode steps");
    }
    pool->WaitPending();
    const int ps = pool->view.page_size;
    // Mirror first (all checks before anything is enqueued or changed).
    int fresh_pages = 0, m = 0;
    {
      std::vector<int> seen;
      for (int i = 0; i < n; ++i) {
        table->CheckSlot(slots[i]);
        seen.push_back(slots[i]);
      }
      std::sort(seen.begin(), seen.end());
      if (std::adjacent_find(seen.begin(), seen.end()) != seen.end()) {
        throw std::invalid_argument("a slot appears twice in one append");
      }
      for (int i = 0; i < n; ++i) {
        const int s = slots[i];
        const bool fresh = (fresh_page != nullptr && fresh_page[i] != 0) ||
                           table->h_npages[s] == 0 || table->h_tail[s] >= ps;
        if (fresh && table->h_npages[s] >= table->view.max_pages) {
          throw std::invalid_argument("a request exceeds the table's max_pages");
        }
        fresh_pages += fresh ? 1 : 0;
        m += upload[i] != 0 ? 1 : 0;
      }
      if (fresh_pages > table->h_free) throw std::runtime_error("page pool is exhausted");
    }
    const int b = table->Acquire(4 * static_cast<size_t>(n));
    int* args = table->h_args[b].ptr;
    for (int i = 0; i < n; ++i) {
      args[i] = slots[i];
      args[n + i] = ((fresh_page != nullptr && fresh_page[i] != 0) ? 1 : 0) |
                    (upload[i] != 0 ? 2 : 0);
      args[2 * n + i] = request_ids != nullptr ? request_ids[i] : 0;
      args[3 * n + i] = decode_steps != nullptr ? decode_steps[i] : 0;
    }
    pool->CountH2D(sizeof(int) * 4 * static_cast<size_t>(n));  // the kernel reads the block
    table->d_plan.Reserve(6 * static_cast<size_t>(m) + 1);
    table->d_order.Reserve(std::max(1, m));
    dsdk::LaunchTablePlanAppend(pool->view, table->view, args, n, m, table->d_plan.ptr,
                                table->d_order.ptr, pool->stream, table->Mark(b));
    // The plan kernel is enqueued: the device pops the fresh pages, so the
    // mirror follows now (before the payload kernels).
    for (int i = 0; i < n; ++i) {
      const int s = slots[i];
      const bool fresh = (fresh_page != nullptr && fresh_page[i] != 0) ||
                         table->h_npages[s] == 0 || table->h_tail[s] >= ps;
      if (fresh) {
        ++table->h_npages[s];
        table->h_tail[s] = 0;
      }
      if (upload[i] != 0) ++table->h_tail[s];
    }
    table->h_free -= fresh_pages;
    if (m == 0) return;
    if (rows) {
      const size_t elems = static_cast<size_t>(m) * pool->view.elements;
      table->d_keys.Reserve(elems);
      table->d_values.Reserve(elems);
      pool->H2D(table->d_keys.ptr, keys, sizeof(float) * elems);
      pool->H2D(table->d_values.ptr, values, sizeof(float) * elems);
      int* plan = table->d_plan.ptr;
      dsdk::LaunchAppendTokens(pool->view, plan, table->d_order.ptr, plan + m + 1,
                               plan + 2 * m + 1, plan + 3 * m + 1, table->d_keys.ptr,
                               table->d_values.ptr, nullptr, m, pool->stream);
    } else {
      dsdk::LaunchAppendSynthetic(pool->view, table->d_plan.ptr, m, m, pool->stream);
    }
  });
}

int dsd_table_release(dsd_table* table, int n, const int* slots, int clear) {
  return Guard([&] {
    Require(table != nullptr, "table must be non-null");
    Require(n >= 0, "slot count must be non-negative");
    if (n == 0) return;
    Require(slots != nullptr, "slots must be non-null");
    dsd_pool* pool = table->pool;
    pool->WaitPending();
    std::vector<int> seen(slots, slots + n);
    for (int s : seen) table->CheckSlot(s);
    std::sort(seen.begin(), seen.end());
    if (std::adjacent_find(seen.begin(), seen.end()) != seen.end()) {
      throw std::invalid_argument("a slot appears twice in one release");
    }
    constexpr int kChunk = 1024;
    for (int c0 = 0; c0 < n; c0 += kChunk) {
      const int c = std::min(kChunk, n - c0);
      int pages = 0;
      for (int i = 0; i < c; ++i) pages += table->h_npages[slots[c0 + i]];
      const int b = table->Acquire(static_cast<size_t>(c));
      std::memcpy(table->h_args[b].ptr, slots + c0, sizeof(int) * c);
      pool->CountH2D(sizeof(int) * static_cast<size_t>(c));
      dsdk::LaunchTableRelease(pool->view, table->view, table->h_args[b].ptr, c, pages,
                               clear != 0, pool->stream, table->Mark(b));
      for (int i = 0; i < c; ++i) {
        table->h_npages[slots[c0 + i]] = 0;
        table->h_tail[slots[c0 + i]] = 0;
      }
      table->h_free += pages;
    }
  });
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Sparse decode step
// ---------------------------------------------------------------------------
namespace {

// One decode step's launch: inputs and outputs, the scratch its kernels use
// (score intervals, publication words, counters) and the launch parameters.
// A context fills it with its own scratch; the allocation-free entry point
// with the library's static scratch.
struct StepLaunch {
  bool valid = false;
  bool certified = false;
  bool fused = false;
  bool wide = false;  // the wide single launch (requests beyond the fused step's 256)
  // A batch the wide step takes, whether or not it runs (DSD_WIDE_STEP=0,
  // graph capture): three-kernel steps split its heads as the wide step
  // does, so both forms give the same outputs.
  bool wide_shape = false;
  int batch = 0, total = 0, max_n = 0;
  int top_k = 0;
  int compute_units = 256;
  float scale = 0.0f;
  const float* queries = nullptr;
  const int* offsets = nullptr;
  const int* ids = nullptr;
  float* outputs = nullptr;
  float* scores = nullptr;  // exact scores, or the certified midpoints
  int* selected = nullptr;  // [batch][max(1, top_k)]
  int* counts = nullptr;
  float* lo = nullptr;
  float* hi = nullptr;
  unsigned long long* rec = nullptr;  // [3 * total] publication words
  unsigned long long* refined = nullptr;  // [batch][8][3] refined-interval words
  unsigned long long* sel_rec = nullptr;  // wide step: tagged ids, then counts
  unsigned long long* cnt_rec = nullptr;
  unsigned* wide_counters = nullptr;  // two sets of wide_counter_words (eager launches),
                                      // then two for captured ones
  unsigned* wide_seq = nullptr;       // device: captured wide launches so far
  int wide_counter_words = 0;
  unsigned* wide_launches = nullptr;  // host: wide launches so far (picks the set)
  int* exact_pages = nullptr;         // may be null
  unsigned long long* fail_word = nullptr;
  unsigned epoch = 0;  // fresh (non-zero, below 2^30) for every launch
  const unsigned* epoch_src = nullptr;  // captured launches: the device epoch counter
  unsigned spin_limit = kDefaultSpinLimit;
  bool never_ready = false;
  dsdk::FailReport Fail() const {
    dsdk::FailReport f;
    f.word = fail_word;
    f.epoch = epoch;
    return f;
  }
};

// Whether work enqueued on `s` is being captured into a graph.  A captured
// step cannot take its epoch from the host (every replay would reuse it) nor
// wait on events recorded outside the capture.
bool StreamCapturing(hipStream_t s) {
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  DSD_HIP_CHECK(hipStreamIsCapturing(s, &status));
  return status == hipStreamCaptureStatusActive;
}

float StepScale(const PoolView& v) {
  return 1.0f / std::sqrt(static_cast<float>(v.head_dim));
}

// Certified scoring unless exact scores are requested or the shape is
// outside what the certified kernels handle; the single-launch step for
// certified selection on the hot shape.
bool StepCertified(const PoolView& v, int score_mode, int max_n, bool need_exact_scores) {
  return score_mode == DSD_SCORE_CERTIFIED && !need_exact_scores &&
         dsdk::CertifiedScoringSupported(v.elements, max_n);
}
bool StepFused(const PoolView& v, bool certified, bool enabled, int max_n, int top_k) {
  return certified && enabled && dsdk::FusedStepSupported(v, max_n, top_k);
}

void EnqueueScoreStage(const PoolView& v, const StepLaunch& L, hipStream_t s) {
  if (L.total <= 0) return;
  if (L.certified) {
    dsdk::LaunchScoreBounds(v, L.queries, L.offsets, L.ids, L.batch, L.total, L.max_n, L.scale,
                            L.scores, L.lo, L.hi, L.Fail(), s);
  } else {
    dsdk::LaunchScoreExact(v, L.queries, L.offsets, L.ids, L.batch, L.total, L.max_n, L.scale,
                           L.scores, L.Fail(), s);
  }
}

void EnqueueSelectStage(const PoolView& v, const StepLaunch& L, hipStream_t s) {
  if (L.certified) {
    dsdk::LaunchSelectCertified(v, L.scores, L.lo, L.hi, L.queries, L.offsets, L.ids, L.batch,
                                L.total, L.max_n, L.scale, L.top_k, L.selected, L.counts,
                                L.exact_pages, L.Fail(), s);
  } else {
    dsdk::LaunchSelectTopK(L.scores, L.offsets, L.ids, L.batch, L.total, L.max_n, L.top_k,
                           L.selected, L.counts, L.Fail(), s);
  }
}

void EnqueueAttentionStage(const PoolView& v, const StepLaunch& L, hipStream_t s) {
  dsdk::AttentionArgs a;
  a.queries = L.queries;
  a.list_ids = L.selected;
  a.list_counts = L.counts;
  a.list_stride = L.top_k > 0 ? L.top_k : 1;
  a.batch = L.batch;
  a.scale = L.scale;
  a.outputs = L.outputs;
  a.wide_partition = L.wide_shape;
  dsdk::LaunchAttention(v, a, s);
}

dsdk::FusedArgs FusedStepArgs(const PoolView& v, const StepLaunch& L) {
  dsdk::FusedArgs a;
  a.queries = L.queries;
  a.cand_offsets = L.offsets;
  a.cand_ids = L.ids;
  a.batch = L.batch;
  a.total = L.total;
  a.top_k = L.top_k;
  a.sel_stride = L.top_k > 0 ? L.top_k : 1;
  a.heads_per_group = dsdk::FusedStepHeadsPerGroup(v, L.batch, L.compute_units);
  a.max_candidates = L.max_n;
  a.scale = L.scale;
  a.mid = L.scores;
  a.lo = L.lo;
  a.hi = L.hi;
  a.selected = L.selected;
  a.counts = L.counts;
  a.outputs = L.outputs;
  a.rec = L.rec;
  a.refined = L.refined;
  a.epoch = L.epoch;
  a.wait_mask = L.never_ready ? 0x80000000u : 0u;
  a.wait_tag = L.epoch | a.wait_mask;
  a.epoch_src = L.epoch_src;
  a.spin_limit = L.spin_limit;
  a.exact_pages = L.exact_pages;
  a.fail = L.Fail();
  return a;
}

// The wide step's arguments (dsdk::WideArgs): the fused step's, the score
// slices of the stand-alone score kernel, and its scratch.
dsdk::WideArgs WideStepArgs(const PoolView& v, const StepLaunch& L) {
  dsdk::WideArgs w;
  w.a = FusedStepArgs(v, L);
  w.sel_rec = L.sel_rec;
  w.cnt_rec = L.cnt_rec;
  w.counters = L.wide_counters;
  w.pages_per_group = dsdk::ScorePagesPerGroup(L.total);
  w.groups = (L.max_n + w.pages_per_group - 1) / w.pages_per_group;
  // Every score slice ahead of every attention item.  An attention item
  // whose id falls in the first dispatch round occupies a CU from the
  // launch on while it waits for its request's select; on 32 requests of
  // 2048 pages the step spanned 379 us with all slices first and 427-489 us
  // with 4 to 16 requests between a request's slices and its attention.
  // (DSD_WIDE_LAG and DSD_WIDE_TICKETS=0, tuning switches read once per
  // process, give the other orders)
  static const int lag_env = [] {
    const char* env = std::getenv("DSD_WIDE_LAG");
    return env != nullptr ? std::atoi(env) : -1;
  }();
  static const bool tickets = [] {
    const char* env = std::getenv("DSD_WIDE_TICKETS");
    return env == nullptr || std::atoi(env) != 0;
  }();
  const int lag = lag_env >= 0 ? lag_env : L.batch;
  w.lag = std::max(0, std::min(lag, L.batch));
  w.tickets = tickets;
  w.items = dsdk::WideStepItems(v, L.batch, w.groups);
  return w;
}

// The counter set of the next launch: launches alternate between the two
// sets, and each zeroes the other for the one after it.  The count advances
// only once a launch was enqueued (LaunchWideCounted), so a launch that
// throws leaves the sets in turn.
void UseWideCounters(dsdk::WideArgs* w, const StepLaunch& L) {
  const unsigned n = *L.wide_launches;
  w->counter_words = L.wide_counter_words;
  // (a captured launch picks one of the other two sets on the device)
  w->seq_src = L.wide_seq;
  w->capture_counters = L.wide_counters + 2 * static_cast<size_t>(L.wide_counter_words);
  w->counters = L.wide_counters + (n & 1u) * static_cast<size_t>(L.wide_counter_words);
  w->next_counters = L.wide_counters + ((n + 1u) & 1u) * static_cast<size_t>(L.wide_counter_words);
}

void LaunchWideCounted(const PoolView& v, dsdk::WideArgs* w, const StepLaunch& L,
                       hipStream_t s) {
  UseWideCounters(w, L);
  dsdk::LaunchWideStep(v, *w, s);
  if (w->a.epoch_src == nullptr) ++*L.wide_launches;
}

// The whole step: one launch (fused) or score, select and attention.
void EnqueueStep(const PoolView& v, const StepLaunch& L, hipStream_t s) {
  if (L.wide) {
    dsdk::WideArgs w = WideStepArgs(v, L);
    LaunchWideCounted(v, &w, L, s);
    return;
  }
  if (L.fused) {
    dsdk::LaunchFusedStep(v, FusedStepArgs(v, L), s);
    return;
  }
  EnqueueScoreStage(v, L, s);
  EnqueueSelectStage(v, L, s);
  EnqueueAttentionStage(v, L, s);
}

// One in-flight asynchronous table step: the pinned words its stage-in
// kernel reads (slot ids, query row pointers, a copied query block), its
// progress words and, when timed, its fused-step stamps or stage events.
// A slot is reused only after the step that last used it has completed and
// been harvested.  The step records no event unless it is a timed
// three-kernel step: each event's barrier idles the stream for microseconds.
struct AsyncSlot {
  PinnedBuffer<int> slots;
  PinnedBuffer<const float*> rows;
  PinnedBuffer<float> queries;
  PinnedBuffer<unsigned long long> stamps;
  // words[0]: the ticket, stored by the step-mark kernel after the step;
  // words[1]: the device clock then; words[2]: the clock as the stage-in
  // started.
  PinnedBuffer<unsigned long long> words;
  // k[0..3] around score / select / attention (timed three-kernel steps)
  hipEvent_t k[4] = {};
  bool busy = false;
  bool timed = false;
  bool fused = false;
  bool wide = false;
  bool new_timeline = false;  // the first step of a timeline
  int batch = 0;
  int stamp_grid = 0;
  unsigned epoch = 0;
  long long ticket = 0;
};
constexpr int kAsyncDepth = 4;

}  // namespace

struct dsd_sparse_ctx {
  dsd_pool* pool = nullptr;
  int top_k = 0;
  int max_batch = 0;
  int max_cand = 0;
  int max_sel = 0;
  hipStream_t stream = nullptr;  // the pool's stream (not owned)
  hipEvent_t ev[6] = {};
  DeviceBuffer<float> d_queries, d_scores, d_lo, d_hi;
  DeviceBuffer<int> d_offsets, d_ids, d_selected, d_counts, d_exact_pages;
  // fused-step publication words (see fused_step.hip)
  DeviceBuffer<unsigned long long> d_rec;
  DeviceBuffer<unsigned long long> d_refined;
  // The epoch counter of captured fused launches (advanced on the device).
  DeviceBuffer<unsigned> d_epoch;
  // The wide step's tagged selections ([max_batch][k] ids, then
  // [max_batch] counts) and counters ([2 + max_batch], zero between
  // launches).
  DeviceBuffer<unsigned long long> d_sel_rec;
  DeviceBuffer<unsigned> d_wide_counters;
  DeviceBuffer<unsigned> d_wide_seq;
  mutable unsigned wide_launches = 0;  // host count of wide launches (picks the counter set)
  // The epoch of the step being enqueued: it tags the fused step's
  // publication words and every failure report of the step's kernels.
  unsigned epoch = 0;
  unsigned spin_limit = kDefaultSpinLimit;
  bool never_ready = false;  // test hook: every fused-step wait gives up
  // The stream of the last launch that used the context's scratch, and the
  // event that orders a launch on another stream after it.
  hipStream_t last_stream = nullptr;
  hipEvent_t ev_switch = nullptr;
  double wall_khz = 0.0;  // wall_clock64() rate
  int compute_units = 256;
  int score_mode = DSD_SCORE_CERTIFIED;
  bool fused_enabled = true;
  bool wide_enabled = true;
  PinnedBuffer<float> h_queries, h_scores, h_outputs;
  PinnedBuffer<int> h_offsets, h_ids, h_selected, h_counts;
  // The step kernels' failure word: (epoch << 32) | code, pinned, coherent.
  PinnedBuffer<unsigned long long> h_fail;
  // per-workgroup clock stamps of a timed fused launch
  PinnedBuffer<unsigned long long> h_stamps;
  PinnedBuffer<const float*> h_rows;  // row pointers of a row-gather step
  int stamp_grid = 0;  // workgroups stamped by the last timed fused launch

  StepLaunch last;  // the last step's launch (replays re-enqueue its stages)

  // Asynchronous table steps (dsd_sparse_run_table_async): a ring of
  // in-flight slots, the tickets handed out and harvested, the timeline's
  // base (the device clock as its first step started: a timeline starts
  // whenever nothing is in flight and every record has been collected) and
  // the harvested records, oldest first.
  AsyncSlot async[kAsyncDepth];
  int async_next = 0;
  long long async_issued = 0;
  long long async_harvested = 0;
  unsigned long long async_base = 0;
  std::deque<dsd_async_step> async_records;

  ~dsd_sparse_ctx() {
    // (dsd_sparse_destroy has waited for the device)
    for (AsyncSlot& a : async) {
      for (hipEvent_t e : a.k) {
        if (e) (void)hipEventDestroy(e);
      }
    }
    for (hipEvent_t& e : ev) {
      if (e) (void)hipEventDestroy(e);
    }
    if (ev_switch) (void)hipEventDestroy(ev_switch);
  }

  // A fresh epoch for the next launch (never 0: the words start at 0; below
  // 2^30, where the device epochs of captured launches never are).
  void NextEpoch() {
    if (++epoch >= 0x40000000u) epoch = 1;
  }
  // Every launch shares the context's scratch (intervals, publication words,
  // ids).  Launches on one stream are ordered by it; a launch on another
  // stream first waits for everything enqueued on the previous one.
  void OrderOn(hipStream_t s) {
    if (last_stream != nullptr && last_stream != s) {
      DSD_HIP_CHECK(hipEventRecord(ev_switch, last_stream));
      DSD_HIP_CHECK(hipStreamWaitEvent(s, ev_switch, 0));
    }
    last_stream = s;
  }
  // After the launches of interest have finished: throws the failure a step
  // reported, if any -- only one of `only_epoch`'s when that is non-zero --
  // and clears the word.  A failure of another epoch is left in place.
  void CheckFailure(unsigned only_epoch) {
    const unsigned long long w =
        __hip_atomic_load(h_fail.ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    const int code = static_cast<int>(w & 0xffffffffull);
    const unsigned at = static_cast<unsigned>(w >> 32);
    if (code == 0 || (only_epoch != 0 && at != only_epoch)) return;
    h_fail.ptr[0] = 0;
    if (code == dsdk::kFailShape) {
      throw std::invalid_argument(
          "a request's candidate list does not fit the step's max_candidates / "
          "total_candidates (or its offsets are malformed): nothing was selected for it");
    }
    if (code == dsdk::kFailPageId) {
      throw std::out_of_range("a candidate page id of the step is outside the pool");
    }
    if (code == dsdk::kFailSelect) {
      throw std::runtime_error(
          "decode step: a selection slot held an id that is not one of the request's "
          "candidates (written as -1, not attended)");
    }
    throw std::runtime_error("fused decode step: wait for page selection timed out");
  }

  // A launch over the context's scratch; the caller fills inputs and
  // outputs.
  StepLaunch Plan(int batch, int total, int max_n, bool need_exact_scores) const {
    StepLaunch L;
    const PoolView& v = pool->view;
    L.valid = true;
    L.certified = StepCertified(v, score_mode, max_n, need_exact_scores);
    L.fused = StepFused(v, L.certified, fused_enabled, max_n, top_k);
    // The wide step takes the batches the single launch cannot (a request
    // beyond 256 candidates); DSD_FUSED_STEP=0 alone keeps three kernels.
    L.wide_shape = !L.fused && L.certified && batch > 0 &&
                   !dsdk::FusedStepSupported(v, max_n, top_k) &&
                   dsdk::WideStepSupported(v, max_n, top_k);
    L.wide = L.wide_shape && wide_enabled;
    L.batch = batch;
    L.total = total;
    L.max_n = max_n;
    L.top_k = top_k;
    L.compute_units = compute_units;
    L.scale = StepScale(v);
    L.sel_rec = d_sel_rec.ptr;
    L.cnt_rec = d_sel_rec.ptr + static_cast<size_t>(max_batch) * std::max(1, top_k);
    L.wide_counters = d_wide_counters.ptr;
    L.wide_counter_words = static_cast<int>(d_wide_counters.count / 4);
    L.wide_seq = d_wide_seq.ptr;
    L.wide_launches = &wide_launches;
    L.scores = d_scores.ptr;
    L.selected = d_selected.ptr;
    L.counts = d_counts.ptr;
    L.lo = d_lo.ptr;
    L.hi = d_hi.ptr;
    L.rec = d_rec.ptr;
    L.refined = d_refined.ptr;
    L.exact_pages = d_exact_pages.ptr;
    L.fail_word = h_fail.ptr;
    return L;
  }
  // Stamps the launch with a fresh epoch and the current wait settings.
  void Fresh(StepLaunch* L) {
    NextEpoch();
    L->epoch = epoch;
    L->spin_limit = spin_limit;
    L->never_ready = never_ready;
  }

  // The single-launch step with per-workgroup clock stamps written straight
  // into pinned host memory (timing mode); returns the stamped grid.
  int EnqueueFusedStamped(const StepLaunch& L, hipStream_t s,
                          PinnedBuffer<unsigned long long>* stamps) {
    dsdk::FusedArgs a = FusedStepArgs(pool->view, L);
    const int grid = dsdk::FusedStepGrid(pool->view, L.batch, a.heads_per_group);
    if (static_cast<size_t>(grid) * dsdk::FusedStepStampsPerGroup() > stamps->count) {
      throw std::runtime_error("fused step stamps exceed their buffer");
    }
    a.stamps = stamps->ptr;
    dsdk::LaunchFusedStep(pool->view, a, s);
    return grid;
  }
  // Phase split of a timed fused launch from its workgroup stamps (start,
  // slice scored, counter ready, records read, ranked, selected, end):
  // first start -> last slice scored -> last selection -> last end.
  void FusedPhases(const unsigned long long* st, int grid, double* score_ms,
                   double* select_ms, double* attention_ms) const {
    *score_ms = *select_ms = *attention_ms = 0.0;
    if (grid <= 0 || wall_khz <= 0.0) return;
    const int per = dsdk::FusedStepStampsPerGroup();
    unsigned long long t0 = ~0ull, t_score = 0, t_select = 0, t_end = 0;
    for (int g = 0; g < grid; ++g) {
      t0 = std::min(t0, st[per * g + 0]);
      t_score = std::max(t_score, st[per * g + 1]);
      t_select = std::max(t_select, st[per * g + 5]);
      t_end = std::max(t_end, st[per * g + 6]);
    }
    t_score = std::max(t_score, t0);
    t_select = std::max(t_select, t_score);
    t_end = std::max(t_end, t_select);
    *score_ms = static_cast<double>(t_score - t0) / wall_khz;
    *select_ms = static_cast<double>(t_select - t_score) / wall_khz;
    *attention_ms = static_cast<double>(t_end - t_select) / wall_khz;
  }
  // Enqueues a step (fresh epoch); with timing, events k[0] .. k[3] around
  // the stages (a fused launch: k[0] and k[3]) and, for the fused step, the
  // workgroup stamps into `stamps` (their grid in *stamped).
  void Enqueue(StepLaunch* L, hipStream_t s, bool timing, hipEvent_t* k = nullptr,
               PinnedBuffer<unsigned long long>* stamps = nullptr, int* stamped = nullptr) {
    Fresh(L);
    const PoolView& v = pool->view;
    if (!timing) {
      EnqueueStep(v, *L, s);
      return;
    }
    if (k == nullptr) k = ev;
    if (stamps == nullptr) stamps = &h_stamps;
    if (stamped == nullptr) stamped = &stamp_grid;
    DSD_HIP_CHECK(hipEventRecord(k[0], s));
    if (L->wide) {
      // One launch whose stages overlap: its whole time, and per-workgroup
      // stamps.
      dsdk::WideArgs w = WideStepArgs(v, *L);
      if (static_cast<size_t>(w.items) * dsdk::WideStepStampsPerGroup() <= stamps->count) {
        w.a.stamps = stamps->ptr;
        *stamped = w.items;
      } else {
        *stamped = 0;
      }
      LaunchWideCounted(v, &w, *L, s);
      DSD_HIP_CHECK(hipEventRecord(k[3], s));
      return;
    }
    if (L->fused) {
      *stamped = EnqueueFusedStamped(*L, s, stamps);
      DSD_HIP_CHECK(hipEventRecord(k[3], s));
      return;
    }
    EnqueueScoreStage(v, *L, s);
    DSD_HIP_CHECK(hipEventRecord(k[1], s));
    EnqueueSelectStage(v, *L, s);
    DSD_HIP_CHECK(hipEventRecord(k[2], s));
    EnqueueAttentionStage(v, *L, s);
    DSD_HIP_CHECK(hipEventRecord(k[3], s));
  }
};

extern "C" {

int dsd_sparse_create(dsd_pool* pool, int top_k, int max_batch,
                      int max_total_candidates, int max_total_selected,
                      dsd_sparse_ctx** out_ctx) {
  return Guard([&] {
    Require(out_ctx != nullptr, "out_ctx must be non-null");
    *out_ctx = nullptr;
    Require(pool != nullptr, "pool must be non-null");
    if (pool->view.head_dim <= 0 || pool->view.head_dim > 128) {
      throw std::invalid_argument("sparse decode supports head_dim in (0, 128]");
    }
    if (max_batch < 0 || max_total_candidates < 0 || max_total_selected < 0) {
      throw std::invalid_argument("sparse context capacities must be non-negative");
    }
    Require(top_k >= 0, "top_k must be non-negative");
    auto ctx = std::make_unique<dsd_sparse_ctx>();
    ctx->pool = pool;
    ctx->top_k = top_k;
    ctx->max_batch = max_batch;
    ctx->max_cand = max_total_candidates;
    ctx->max_sel = max_total_selected;
    // Steps run on the pool's stream: stream order then places them after
    // an enqueued append and before any later pool work, with no cross-
    // stream waits (each costs several microseconds of host time per step).
    ctx->stream = pool->stream;
    // Timing events only (the host waits on the stream itself): no
    // system-scope fence, which would stall the stream between the stages.
    for (hipEvent_t& e : ctx->ev) {
      DSD_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    }
    DSD_HIP_CHECK(hipEventCreateWithFlags(&ctx->ev_switch, hipEventDisableTiming));
    const size_t E = static_cast<size_t>(pool->view.elements);
    const size_t B = static_cast<size_t>(std::max(1, max_batch));
    const size_t P = static_cast<size_t>(std::max(1, max_total_candidates));
    const size_t K = static_cast<size_t>(std::max(1, top_k));
    ctx->d_queries.Reserve(B * E);
    ctx->d_scores.Reserve(P);
    ctx->d_offsets.Reserve(B + 1);
    ctx->d_ids.Reserve(P);
    ctx->d_selected.Reserve(B * K);
    ctx->d_counts.Reserve(B);
    ctx->d_lo.Reserve(P);
    ctx->d_hi.Reserve(P);
    ctx->d_exact_pages.Reserve(1);
    DSD_HIP_CHECK(hipMemset(ctx->d_exact_pages.ptr, 0, sizeof(int)));
    ctx->d_epoch.Reserve(1);
    DSD_HIP_CHECK(hipMemset(ctx->d_epoch.ptr, 0, sizeof(unsigned)));
    ctx->d_sel_rec.Reserve(B * K + B);
    DSD_HIP_CHECK(hipMemset(ctx->d_sel_rec.ptr, 0, (B * K + B) * sizeof(unsigned long long)));
    ctx->d_wide_counters.Reserve(4 * (B + 1));
    DSD_HIP_CHECK(hipMemset(ctx->d_wide_counters.ptr, 0, 4 * (B + 1) * sizeof(unsigned)));
    ctx->d_wide_seq.Reserve(1);
    DSD_HIP_CHECK(hipMemset(ctx->d_wide_seq.ptr, 0, sizeof(unsigned)));
    {
      const size_t rec = 3 * P;
      // The largest fused grid: one head per workgroup.
      const size_t stamps =
          static_cast<size_t>(dsdk::FusedStepGrid(pool->view, static_cast<int>(B), 1)) *
          dsdk::FusedStepStampsPerGroup();
      ctx->d_rec.Reserve(rec);
      ctx->h_stamps.Reserve(stamps, hipHostMallocCoherent);
      DSD_HIP_CHECK(hipMemset(ctx->d_rec.ptr, 0, rec * sizeof(unsigned long long)));
      const size_t refined = 3 * dsdk::kFRefineSlots * B;
      ctx->d_refined.Reserve(refined);
      DSD_HIP_CHECK(hipMemset(ctx->d_refined.ptr, 0, refined * sizeof(unsigned long long)));
    }
    ctx->h_fail.Reserve(1, hipHostMallocCoherent);
    ctx->h_fail.ptr[0] = 0;
    {
      int device = 0, khz = 0;
      DSD_HIP_CHECK(hipGetDevice(&device));
      DSD_HIP_CHECK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device));
      ctx->wall_khz = static_cast<double>(khz);
      int cus = 0;
      DSD_HIP_CHECK(
          hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device));
      if (cus > 0) ctx->compute_units = cus;
    }
    if (const char* env = std::getenv("DSD_FUSED_STEP")) {
      ctx->fused_enabled = std::strcmp(env, "0") != 0;
    }
    if (const char* env = std::getenv("DSD_WIDE_STEP")) {
      ctx->wide_enabled = std::strcmp(env, "0") != 0;
    }
    // The host step's staging: the step's kernels read the inputs from here
    // and write the outputs here directly (no DMA copies).
    ctx->h_queries.Reserve(B * E, hipHostMallocCoherent);
    ctx->h_rows.Reserve(B, hipHostMallocCoherent);
    ctx->h_outputs.Reserve(B * E, hipHostMallocCoherent);
    ctx->h_scores.Reserve(P);
    ctx->h_offsets.Reserve(B + 1, hipHostMallocCoherent);
    ctx->h_ids.Reserve(P, hipHostMallocCoherent);
    ctx->h_selected.Reserve(B * K);
    ctx->h_counts.Reserve(B);
    // The asynchronous steps' ring slots (a copied query block is reserved
    // at its first use), so the first steps pay no pinned allocation.
    for (AsyncSlot& a : ctx->async) {
      a.slots.Reserve(B + 1, hipHostMallocCoherent);
      a.rows.Reserve(B + 1, hipHostMallocCoherent);
      a.stamps.Reserve(std::max<size_t>(1, ctx->h_stamps.count), hipHostMallocCoherent);
      a.words.Reserve(4, hipHostMallocCoherent);
      for (int i = 0; i < 4; ++i) a.words.ptr[i] = 0;
      for (hipEvent_t& e : a.k) {
        DSD_HIP_CHECK(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
      }
    }
    dsdk::PreloadStepKernels();
    dsdk::PreloadFusedKernels();
    dsdk::PreloadPoolKernels();
    *out_ctx = ctx.release();
  });
}

int dsd_sparse_destroy(dsd_sparse_ctx* ctx) {
  return Guard([&] {
    if (ctx != nullptr) {
      // A device-buffer step may still run on a caller's stream: wait for
      // every stream before the scratch it uses is freed.
      (void)hipDeviceSynchronize();
      delete ctx;
    }
  });
}

void* dsd_sparse_stream(dsd_sparse_ctx* ctx) {
  return ctx == nullptr ? nullptr : reinterpret_cast<void*>(ctx->stream);
}

namespace {

// Waits for an asynchronous step, frees its ring slot and appends its
// record (device times from the timeline's base event).  A failure the step
// reported is thrown here (its outputs are then zeros for the request
// concerned), and the record is dropped.
void HarvestAsync(dsd_sparse_ctx* ctx, AsyncSlot& a) {
  AwaitWord(a.words.ptr, static_cast<unsigned long long>(a.ticket), ctx->stream);
  a.busy = false;
  ctx->async_harvested = std::max(ctx->async_harvested, a.ticket);
  ctx->CheckFailure(a.epoch);
  dsd_async_step r{};
  r.ticket = a.ticket;
  r.batch = a.batch;
  r.fused = a.fused ? 1 : 0;
  r.wide = a.wide ? 1 : 0;
  const unsigned long long start =
      __hip_atomic_load(a.words.ptr + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  const unsigned long long end =
      __hip_atomic_load(a.words.ptr + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  if (a.new_timeline) ctx->async_base = start;
  const double khz = ctx->wall_khz > 0.0 ? ctx->wall_khz : 1.0e5;
  r.start_ms = static_cast<double>(static_cast<long long>(start - ctx->async_base)) / khz;
  r.done_ms = static_cast<double>(static_cast<long long>(end - ctx->async_base)) / khz;
  if (a.timed && a.fused) {
    ctx->FusedPhases(a.stamps.ptr, a.stamp_grid, &r.score_ms, &r.topk_ms, &r.attention_ms);
    r.kernel_ms = r.score_ms + r.topk_ms + r.attention_ms;
  } else if (a.timed && a.wide) {
    DSD_HIP_CHECK(hipEventSynchronize(a.k[3]));
    float k = 0.f;
    DSD_HIP_CHECK(hipEventElapsedTime(&k, a.k[0], a.k[3]));
    r.kernel_ms = k;  // (its stages overlap: no split)
  } else if (a.timed) {
    // (the stream has passed them; the runtime reports them complete once
    // it has seen that)
    DSD_HIP_CHECK(hipEventSynchronize(a.k[3]));
    float x = 0.f, y = 0.f, z = 0.f;
    DSD_HIP_CHECK(hipEventElapsedTime(&x, a.k[0], a.k[1]));
    DSD_HIP_CHECK(hipEventElapsedTime(&y, a.k[1], a.k[2]));
    DSD_HIP_CHECK(hipEventElapsedTime(&z, a.k[2], a.k[3]));
    r.score_ms = x;
    r.topk_ms = y;
    r.attention_ms = z;
    r.kernel_ms = static_cast<double>(x) + y + z;
  }
  ctx->async_records.push_back(r);
}

// Harvests, oldest first, every in-flight asynchronous step whose ticket is
// at most `ticket`.
void HarvestThrough(dsd_sparse_ctx* ctx, long long ticket) {
  for (;;) {
    AsyncSlot* oldest = nullptr;
    for (AsyncSlot& a : ctx->async) {
      if (a.busy && (oldest == nullptr || a.ticket < oldest->ticket)) oldest = &a;
    }
    if (oldest == nullptr || oldest->ticket > ticket) return;
    HarvestAsync(ctx, *oldest);
  }
}

// One host-buffer step.  Inputs are copied into the context's pinned
// staging unless `staged` (the caller wrote them there); outputs land in the
// pinned staging and are copied to `outputs` when it is non-null.  With
// `rows`, request r's query is read from rows[r] (pinned memory the device
// reads directly) instead of from `queries`.
// With `table`, request r's candidate list is the page list of table slot
// slots[r] (cand_offsets / cand_ids unused): the stage-in kernel builds the
// CSR on the device, and only the queries and the slot ids cross PCIe.
// With `async` (table steps only), the step's pinned inputs go to that ring
// slot instead of the context's staging, its events are recorded there, and
// the call returns once the step is enqueued: no wait, no results (the
// outputs stay in the staging; the slot is harvested later).
void HostStep(dsd_sparse_ctx* ctx, int batch, bool staged, const float* queries,
              const float* const* rows, const int* cand_offsets, const int* cand_ids,
              int output_mode, int timing_mode, float* outputs, float* scores, int* selected,
              int* selected_counts, dsd_step_timings* timings,
              const dsd_table* table = nullptr, const int* slots = nullptr,
              AsyncSlot* async = nullptr) {
    Require(ctx != nullptr, "context must be non-null");
    Require(batch >= 0, "batch must be non-negative");
    Require(output_mode >= DSD_OUTPUT_NONE && output_mode <= DSD_OUTPUT_DEBUG,
            "unknown output mode");
    dsd_step_timings t{};
    if (timings != nullptr) *timings = t;
    if (batch == 0) return;
    Require(queries != nullptr || rows != nullptr, "inputs must be non-null");
    if (table != nullptr) {
      Require(slots != nullptr, "slots must be non-null");
      Require(table->pool == ctx->pool, "the table belongs to another pool");
    } else {
      Require(cand_offsets != nullptr, "inputs must be non-null");
      Require(async == nullptr, "only table steps run asynchronously");
    }
    const bool want_outputs = output_mode != DSD_OUTPUT_NONE;
    const bool debug = output_mode == DSD_OUTPUT_DEBUG;
    // Ids are returned in debug mode, or in outputs mode when buffers are given.
    const bool want_ids =
        debug || (want_outputs && selected != nullptr && selected_counts != nullptr);
    const bool timing = timing_mode == DSD_TIMING_EVENTS;
    if (want_outputs && !staged && table == nullptr) {
      Require(outputs != nullptr, "outputs must be non-null");
    }
    if (debug) {
      Require(scores != nullptr && selected != nullptr && selected_counts != nullptr,
              "debug outputs must be non-null");
    }
    const dsd_pool& pool = *ctx->pool;
    const int E = pool.view.elements;

    // Shape checks (the reference's PackSparseBatchInto + capacity checks,
    // src/cuda/sparse_batched_attention.cu:24-96,600-608); a table's counts
    // come from its host mirror.
    if (table == nullptr) Require(cand_offsets[0] == 0, "cand_offsets[0] must be 0");
    int max_n = 0;
    int total_sel = 0;
    int total = 0;
    for (int r = 0; r < batch; ++r) {
      int n = 0;
      if (table != nullptr) {
        table->CheckSlot(slots[r]);
        n = table->h_npages[slots[r]];
      } else {
        n = cand_offsets[r + 1] - cand_offsets[r];
        Require(n >= 0, "cand_offsets must be non-decreasing");
      }
      max_n = std::max(max_n, n);
      total_sel += std::min(ctx->top_k, n);
      total += n;
    }
    if (table == nullptr) total = cand_offsets[batch];
    if (batch > ctx->max_batch) {
      throw std::invalid_argument("request batch exceeds sparse context capacity");
    }
    if (total > ctx->max_cand) {
      throw std::invalid_argument("candidate page count exceeds sparse context capacity");
    }
    if (total_sel > ctx->max_sel) {
      throw std::invalid_argument("selected page count exceeds sparse context capacity");
    }
    if (table == nullptr) {
      if (total > 0) Require(cand_ids != nullptr, "cand_ids must be non-null");
      for (int c = 0; c < total; ++c) ctx->pool->ValidatePage(cand_ids[c]);
    }
    if (rows != nullptr) {
      // Each row: non-null, 16-byte aligned, and inside a dsd_host_alloc
      // block or the context's own query staging (its row r).
      Require(E % 4 == 0, "query rows need a multiple of 4 elements");
      const size_t row_bytes = sizeof(float) * static_cast<size_t>(E);
      for (int r = 0; r < batch; ++r) {
        Require(rows[r] != nullptr, "query rows must be non-null");
        Require(reinterpret_cast<uintptr_t>(rows[r]) % 16 == 0,
                "query rows must be 16-byte aligned");
      }
      // (An asynchronous step may not read the staging, which the next
      // synchronous step rewrites.)
      std::vector<const float*> foreign;
      std::vector<int> foreign_at;
      for (int r = 0; r < batch; ++r) {
        if (async != nullptr || rows[r] != ctx->h_queries.ptr + static_cast<size_t>(r) * E) {
          foreign.push_back(rows[r]);
          foreign_at.push_back(r);
        }
      }
      for (size_t f = 0; f < foreign.size(); ++f) {
        if (RowBlocks::Host().Holds(foreign[f], row_bytes) ||
            RowBlocks::Device().Holds(foreign[f], row_bytes)) {
          continue;
        }
        throw std::invalid_argument("query row " + std::to_string(foreign_at[f]) +
                                    " is not in dsd_host_alloc or dsd_device_alloc memory");
      }
    }

    // Host -> device through pinned staging (an asynchronous step's ring
    // slot, or the context's staging).
    auto t0 = Clock::now();
    const size_t qn = static_cast<size_t>(batch) * E;
    int* stage_slots = ctx->h_offsets.ptr;
    const float** stage_rows = ctx->h_rows.ptr;
    float* stage_queries = ctx->h_queries.ptr;
    if (async != nullptr) {
      async->slots.Reserve(static_cast<size_t>(ctx->max_batch) + 1, hipHostMallocCoherent);
      async->rows.Reserve(static_cast<size_t>(ctx->max_batch) + 1, hipHostMallocCoherent);
      stage_slots = async->slots.ptr;
      stage_rows = async->rows.ptr;
      if (rows == nullptr) {
        async->queries.Reserve(static_cast<size_t>(ctx->max_batch) * E, hipHostMallocCoherent);
        stage_queries = async->queries.ptr;
      }
    }
    if (table != nullptr) {
      if (rows == nullptr && queries != stage_queries) {
        std::memcpy(stage_queries, queries, sizeof(float) * qn);
      }
      std::memcpy(stage_slots, slots, sizeof(int) * batch);  // the slot ids
    } else if (!staged) {
      if (rows == nullptr) std::memcpy(ctx->h_queries.ptr, queries, sizeof(float) * qn);
      std::memcpy(ctx->h_offsets.ptr, cand_offsets, sizeof(int) * (batch + 1));
      if (total > 0) std::memcpy(ctx->h_ids.ptr, cand_ids, sizeof(int) * total);
    }
    ctx->pool->OrderAfterPending(ctx->stream);
    ctx->OrderOn(ctx->stream);
    {
      // One kernel on the step's stream copies the staged inputs to the
      // device: DMA copies would each cost a copy-engine hand-off.
      dsdk::StageSegments seg;
      if (async != nullptr) seg.start_stamp = async->words.ptr + 2;
      if (table != nullptr) {
        seg.table = table->view;
        seg.table_slots = stage_slots;
        seg.table_batch = batch;
        seg.csr_offsets = ctx->d_offsets.ptr;
        seg.csr_ids = ctx->d_ids.ptr;
      } else {
        seg.src[0] = reinterpret_cast<const uint32_t*>(ctx->h_offsets.ptr);
        seg.dst[0] = reinterpret_cast<uint32_t*>(ctx->d_offsets.ptr);
        seg.words[0] = batch + 1;
        seg.src[1] = reinterpret_cast<const uint32_t*>(ctx->h_ids.ptr);
        seg.dst[1] = reinterpret_cast<uint32_t*>(ctx->d_ids.ptr);
        seg.words[1] = total;
        seg.count = 2;
      }
      if (rows != nullptr) {
        std::memcpy(stage_rows, rows, sizeof(const float*) * batch);
        seg.rows = stage_rows;
        seg.rows_dst = ctx->d_queries.ptr;
        seg.nrows = batch;
        seg.row_words = E;
      } else {
        seg.src[seg.count] = reinterpret_cast<const uint32_t*>(stage_queries);
        seg.dst[seg.count] = reinterpret_cast<uint32_t*>(ctx->d_queries.ptr);
        seg.words[seg.count] = static_cast<int>(qn);
        ++seg.count;
      }
      dsdk::LaunchStageIn(seg, ctx->stream);
    }
    t.h2d_ms = MsSince(t0);

    StepLaunch L = ctx->Plan(batch, total, max_n, debug);
    L.queries = ctx->d_queries.ptr;
    L.offsets = ctx->d_offsets.ptr;
    L.ids = ctx->d_ids.ptr;
    // The attention writes the outputs straight into the pinned staging.
    L.outputs = ctx->h_outputs.ptr;
    t0 = Clock::now();
    if (async != nullptr) {
      async->stamps.Reserve(std::max<size_t>(1, ctx->h_stamps.count), hipHostMallocCoherent);
      async->stamp_grid = 0;
      if (timing && L.fused) {
        // Timed by its workgroup stamps alone (no events).
        ctx->Fresh(&L);
        async->stamp_grid = ctx->EnqueueFusedStamped(L, ctx->stream, &async->stamps);
      } else {
        ctx->Enqueue(&L, ctx->stream, timing, async->k, &async->stamps, &async->stamp_grid);
      }
      dsdk::LaunchStepMark(async->words.ptr, static_cast<unsigned long long>(async->ticket),
                           ctx->stream);
      ctx->last = L;
      async->busy = true;
      async->timed = timing;
      async->fused = L.fused;
      async->wide = L.wide;
      async->batch = batch;
      async->epoch = L.epoch;
      t.launch_ms = MsSince(t0);
      if (timings != nullptr) *timings = t;
      return;
    }
    ctx->Enqueue(&L, ctx->stream, timing);
    ctx->last = L;
    t.launch_ms = MsSince(t0);

    if (want_outputs) {
      t0 = Clock::now();
      if (debug && total > 0) {
        DSD_HIP_CHECK(hipMemcpyAsync(ctx->h_scores.ptr, ctx->d_scores.ptr,
                                     sizeof(float) * total, hipMemcpyDeviceToHost,
                                     ctx->stream));
      }
      if (want_ids) {
        const size_t kk = static_cast<size_t>(std::max(1, ctx->top_k));
        DSD_HIP_CHECK(hipMemcpyAsync(ctx->h_selected.ptr, ctx->d_selected.ptr,
                                     sizeof(int) * kk * batch, hipMemcpyDeviceToHost,
                                     ctx->stream));
        DSD_HIP_CHECK(hipMemcpyAsync(ctx->h_counts.ptr, ctx->d_counts.ptr,
                                     sizeof(int) * batch, hipMemcpyDeviceToHost,
                                     ctx->stream));
      }
      t.d2h_ms = MsSince(t0);
    }
    t0 = Clock::now();
    DSD_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    t.sync_ms = MsSince(t0);
    // A failure this step reported (its outputs are then zeros for the
    // request concerned); failures of earlier device-buffer steps are left
    // for dsd_sparse_device_status.
    ctx->CheckFailure(ctx->epoch);
    if (timing && L.fused) {
      // One kernel: its event time, split at the workgroup clock stamps.
      float k = 0.f;
      DSD_HIP_CHECK(hipEventElapsedTime(&k, ctx->ev[0], ctx->ev[3]));
      ctx->FusedPhases(ctx->h_stamps.ptr, ctx->stamp_grid, &t.score_ms, &t.topk_ms,
                       &t.attention_ms);
      t.kernel_ms = k;
    } else if (timing && L.wide) {
      // The wide step's stages overlap: only its whole time (kernel_ms).
      float k = 0.f;
      DSD_HIP_CHECK(hipEventElapsedTime(&k, ctx->ev[0], ctx->ev[3]));
      t.kernel_ms = k;
    } else if (timing) {
      float a = 0.f, b = 0.f, c = 0.f;
      DSD_HIP_CHECK(hipEventElapsedTime(&a, ctx->ev[0], ctx->ev[1]));
      DSD_HIP_CHECK(hipEventElapsedTime(&b, ctx->ev[1], ctx->ev[2]));
      DSD_HIP_CHECK(hipEventElapsedTime(&c, ctx->ev[2], ctx->ev[3]));
      t.score_ms = a;
      t.topk_ms = b;
      t.attention_ms = c;
      t.kernel_ms = static_cast<double>(a) + b + c;
    }
    if (want_outputs) {
      if (outputs != nullptr) std::memcpy(outputs, ctx->h_outputs.ptr, sizeof(float) * qn);
      if (debug && total > 0) std::memcpy(scores, ctx->h_scores.ptr, sizeof(float) * total);
      if (want_ids) {
        int w = 0;
        const int kk = std::max(1, ctx->top_k);
        for (int r = 0; r < batch; ++r) {
          const int cnt = ctx->h_counts.ptr[r];
          selected_counts[r] = cnt;
          for (int q = 0; q < cnt; ++q) selected[w++] = ctx->h_selected.ptr[r * kk + q];
        }
      }
    }
    if (timings != nullptr) *timings = t;
}

}  // namespace

int dsd_sparse_run_batch(dsd_sparse_ctx* ctx, int batch, const float* queries,
                         const int* cand_offsets, const int* cand_ids,
                         int output_mode, int timing_mode, float* outputs,
                         float* scores, int* selected, int* selected_counts,
                         dsd_step_timings* timings) {
  return Guard([&] {
    HostStep(ctx, batch, false, queries, nullptr, cand_offsets, cand_ids, output_mode,
             timing_mode, outputs, scores, selected, selected_counts, timings);
  });
}

int dsd_sparse_run_table(dsd_sparse_ctx* ctx, dsd_table* table, int batch, const int* slots,
                         const float* queries, const float* const* query_rows, int output_mode,
                         int timing_mode, float* outputs, int* selected, int* selected_counts,
                         dsd_step_timings* timings) {
  return Guard([&] {
    Require(ctx != nullptr && table != nullptr, "context and table must be non-null");
    Require(output_mode != DSD_OUTPUT_DEBUG, "the table step has no debug mode");
    Require(batch <= ctx->max_batch, "request batch exceeds sparse context capacity");
    Require(queries == nullptr || query_rows == nullptr, "give queries or query_rows, not both");
    HostStep(ctx, batch, false, queries, query_rows, nullptr, nullptr, output_mode, timing_mode,
             outputs, nullptr, selected, selected_counts, timings, table, slots);
  });
}

int dsd_sparse_run_table_async(dsd_sparse_ctx* ctx, dsd_table* table, int batch,
                               const int* slots, const float* queries,
                               const float* const* query_rows, int output_mode, int timing_mode,
                               long long* ticket, dsd_step_timings* host_timings) {
  return Guard([&] {
    Require(ticket != nullptr, "ticket must be non-null");
    *ticket = 0;
    if (host_timings != nullptr) *host_timings = dsd_step_timings{};
    Require(ctx != nullptr && table != nullptr, "context and table must be non-null");
    Require(output_mode != DSD_OUTPUT_DEBUG, "the table step has no debug mode");
    Require(batch >= 0 && batch <= ctx->max_batch,
            "request batch exceeds sparse context capacity");
    Require(queries == nullptr || query_rows == nullptr, "give queries or query_rows, not both");
    if (batch == 0) return;
    // The ring slot this step takes: its previous step must have completed.
    AsyncSlot& a = ctx->async[ctx->async_next];
    const auto t0 = Clock::now();
    if (a.busy) HarvestThrough(ctx, a.ticket);
    const double wait_ms = MsSince(t0);
    bool in_flight = false;
    for (const AsyncSlot& o : ctx->async) in_flight = in_flight || o.busy;
    a.new_timeline = !in_flight && ctx->async_records.empty();
    a.ticket = ctx->async_issued + 1;
    dsd_step_timings t{};
    HostStep(ctx, batch, false, queries, query_rows, nullptr, nullptr, output_mode, timing_mode,
             nullptr, nullptr, nullptr, nullptr, &t, table, slots, &a);
    ctx->async_issued = a.ticket;
    ctx->async_next = (ctx->async_next + 1) % kAsyncDepth;
    *ticket = a.ticket;
    t.sync_ms = wait_ms;
    if (host_timings != nullptr) *host_timings = t;
  });
}

int dsd_sparse_async_wait(dsd_sparse_ctx* ctx, long long ticket) {
  return Guard([&] {
    Require(ctx != nullptr, "context must be non-null");
    Require(ticket <= ctx->async_issued, "the ticket was not issued by this context");
    HarvestThrough(ctx, ticket);
  });
}

int dsd_sparse_async_collect(dsd_sparse_ctx* ctx, dsd_async_step* steps, int capacity,
                             int* count) {
  return Guard([&] {
    Require(ctx != nullptr && count != nullptr, "context and count must be non-null");
    *count = 0;
    Require(capacity >= 0, "capacity must be non-negative");
    Require(capacity == 0 || steps != nullptr, "steps must be non-null");
    HarvestThrough(ctx, ctx->async_issued);
    const int n = static_cast<int>(
        std::min<size_t>(static_cast<size_t>(capacity), ctx->async_records.size()));
    for (int i = 0; i < n; ++i) {
      steps[i] = ctx->async_records.front();
      ctx->async_records.pop_front();
    }
    *count = n;
  });
}

int dsd_sparse_last_selection(dsd_sparse_ctx* ctx, int batch, int* selected,
                              int* selected_counts) {
  return Guard([&] {
    Require(ctx != nullptr && selected != nullptr && selected_counts != nullptr,
            "pointers must be non-null");
    Require(batch >= 0 && batch <= ctx->max_batch, "batch out of range");
    if (batch == 0) return;
    const size_t kk = static_cast<size_t>(std::max(1, ctx->top_k));
    DSD_HIP_CHECK(hipMemcpyAsync(ctx->h_selected.ptr, ctx->d_selected.ptr,
                                 sizeof(int) * kk * batch, hipMemcpyDeviceToHost, ctx->stream));
    DSD_HIP_CHECK(hipMemcpyAsync(ctx->h_counts.ptr, ctx->d_counts.ptr, sizeof(int) * batch,
                                 hipMemcpyDeviceToHost, ctx->stream));
    DSD_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    int w = 0;
    for (int r = 0; r < batch; ++r) {
      const int cnt = ctx->h_counts.ptr[r];
      Require(cnt >= 0 && static_cast<size_t>(cnt) <= kk, "the last step's counts are malformed");
      selected_counts[r] = cnt;
      for (int q = 0; q < cnt; ++q) selected[w++] = ctx->h_selected.ptr[r * kk + q];
    }
  });
}

int dsd_sparse_last_csr(dsd_sparse_ctx* ctx, int batch, int* cand_offsets, int* cand_ids,
                        int capacity) {
  return Guard([&] {
    Require(ctx != nullptr && cand_offsets != nullptr, "pointers must be non-null");
    Require(batch >= 0 && batch <= ctx->max_batch, "batch out of range");
    DSD_HIP_CHECK(hipMemcpyAsync(cand_offsets, ctx->d_offsets.ptr, sizeof(int) * (batch + 1),
                                 hipMemcpyDeviceToHost, ctx->stream));
    DSD_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    const int total = cand_offsets[batch];
    Require(total >= 0 && total <= ctx->max_cand, "the last step's CSR is malformed");
    if (total == 0) return;
    Require(cand_ids != nullptr && capacity >= total, "cand_ids must hold the candidates");
    DSD_HIP_CHECK(hipMemcpyAsync(cand_ids, ctx->d_ids.ptr, sizeof(int) * total,
                                 hipMemcpyDeviceToHost, ctx->stream));
    DSD_HIP_CHECK(hipStreamSynchronize(ctx->stream));
  });
}

int dsd_sparse_staging(dsd_sparse_ctx* ctx, float** queries, int** cand_offsets, int** cand_ids,
                       float** outputs) {
  return Guard([&] {
    Require(ctx != nullptr, "context must be non-null");
    if (queries != nullptr) *queries = ctx->h_queries.ptr;
    if (cand_offsets != nullptr) *cand_offsets = ctx->h_offsets.ptr;
    if (cand_ids != nullptr) *cand_ids = ctx->h_ids.ptr;
    if (outputs != nullptr) *outputs = ctx->h_outputs.ptr;
  });
}

int dsd_sparse_run_staged(dsd_sparse_ctx* ctx, int batch, int output_mode, int timing_mode,
                          int* selected, int* selected_counts, dsd_step_timings* timings) {
  return Guard([&] {
    Require(ctx != nullptr, "context must be non-null");
    Require(output_mode != DSD_OUTPUT_DEBUG, "the staged step has no debug mode");
    // Before the staging's offsets are read: it holds max_batch + 1 of them.
    Require(batch <= ctx->max_batch, "request batch exceeds sparse context capacity");
    HostStep(ctx, batch, true, ctx->h_queries.ptr, nullptr, ctx->h_offsets.ptr,
             ctx->h_ids.ptr, output_mode, timing_mode, nullptr, nullptr, selected,
             selected_counts, timings);
  });
}

int dsd_sparse_run_staged_rows(dsd_sparse_ctx* ctx, int batch, const float* const* query_rows,
                               int output_mode, int timing_mode, int* selected,
                               int* selected_counts, dsd_step_timings* timings) {
  return Guard([&] {
    Require(ctx != nullptr, "context must be non-null");
    Require(output_mode != DSD_OUTPUT_DEBUG, "the staged step has no debug mode");
    if (batch > 0) Require(query_rows != nullptr, "query_rows must be non-null");
    // Before the staging's offsets are read: it holds max_batch + 1 of them.
    Require(batch <= ctx->max_batch, "request batch exceeds sparse context capacity");
    HostStep(ctx, batch, true, nullptr, query_rows, ctx->h_offsets.ptr, ctx->h_ids.ptr,
             output_mode, timing_mode, nullptr, nullptr, selected, selected_counts, timings);
  });
}

int dsd_synthetic_batch(int num_heads, int head_dim, int page_size, int batch,
                        int min_context_tokens, int max_context_tokens, int seed,
                        int distribution, int capacity_pages, int* context_tokens,
                        float* key_pool, float* value_pool, float* queries) {
  return Guard([&] {
    Require(num_heads > 0 && head_dim > 0 && page_size > 0, "model shape must be positive");
    Require(batch >= 0, "batch must be non-negative");
    Require(min_context_tokens >= 0 && min_context_tokens <= max_context_tokens,
            "context range must be 0 <= min <= max");
    Require(distribution == DSD_SYNTHETIC_UNIFORM || distribution == DSD_SYNTHETIC_NORMAL,
            "unknown distribution");
    Require(context_tokens != nullptr, "context_tokens must be non-null");
    // The reference's draw order (src/synthetic_data.cpp:23-68): one engine;
    // every context length first, then per request and page the keys, then
    // the values, then the request's query; one distribution object per
    // vector, as the reference's Uniform() makes.
    std::mt19937 rng(static_cast<std::mt19937::result_type>(seed));
    std::uniform_int_distribution<int> length(min_context_tokens, max_context_tokens);
    long long pages = 0;
    for (int r = 0; r < batch; ++r) {
      context_tokens[r] = length(rng);
      pages += (context_tokens[r] + page_size - 1) / page_size;
    }
    if (key_pool == nullptr && value_pool == nullptr && queries == nullptr) return;
    Require(key_pool != nullptr && value_pool != nullptr && queries != nullptr,
            "key_pool, value_pool and queries go together");
    Require(pages <= capacity_pages, "the batch's pages exceed capacity_pages");
    const size_t E = static_cast<size_t>(num_heads) * static_cast<size_t>(head_dim);
    const size_t page_floats = static_cast<size_t>(page_size) * E;
    auto fill = [&](float* out, size_t n) {
      if (distribution == DSD_SYNTHETIC_UNIFORM) {
        std::uniform_real_distribution<float> dist(-1.0f, 1.0f);
        for (size_t i = 0; i < n; ++i) out[i] = dist(rng);
      } else {
        std::normal_distribution<float> dist(0.0f, 1.0f);
        for (size_t i = 0; i < n; ++i) out[i] = dist(rng);
      }
    };
    long long g = 0;  // the batch's page g is pool page capacity - 1 - g (LIFO)
    for (int r = 0; r < batch; ++r) {
      const int n = context_tokens[r];
      const int count = (n + page_size - 1) / page_size;
      for (int j = 0; j < count; ++j, ++g) {
        const size_t row = static_cast<size_t>(capacity_pages - 1 - g) * page_floats;
        const size_t tokens = static_cast<size_t>(std::min(page_size, n - j * page_size));
        std::fill(key_pool + row, key_pool + row + page_floats, 0.0f);
        std::fill(value_pool + row, value_pool + row + page_floats, 0.0f);
        fill(key_pool + row, tokens * E);
        fill(value_pool + row, tokens * E);
      }
      fill(queries + static_cast<size_t>(r) * E, E);
    }
  });
}

int dsd_host_alloc(size_t bytes, void** out) {
  return Guard([&] {
    Require(out != nullptr, "out must be non-null");
    Require(bytes > 0, "bytes must be positive");
    *out = nullptr;
    void* p = nullptr;
    DSD_HIP_CHECK(hipHostMalloc(&p, bytes, hipHostMallocCoherent));
    RowBlocks::Host().Add(p, bytes);
    *out = p;
  });
}

int dsd_host_free(void* p) {
  return Guard([&] {
    if (p == nullptr) return;
    Require(RowBlocks::Host().Remove(p), "pointer was not returned by dsd_host_alloc");
    DSD_HIP_CHECK(hipHostFree(p));
  });
}

int dsd_device_alloc(size_t bytes, void** out) {
  return Guard([&] {
    Require(out != nullptr, "out must be non-null");
    Require(bytes > 0, "bytes must be positive");
    *out = nullptr;
    void* p = nullptr;
    DSD_HIP_CHECK(hipMalloc(&p, bytes));
    RowBlocks::Device().Add(p, bytes);
    *out = p;
  });
}

int dsd_device_upload(void* dst, const void* src, size_t bytes) {
  return Guard([&] {
    if (bytes == 0) return;
    Require(dst != nullptr && src != nullptr, "pointers must be non-null");
    Require(RowBlocks::Device().Holds(dst, bytes),
            "the destination is not inside one dsd_device_alloc block");
    DSD_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
  });
}

int dsd_device_free(void* p) {
  return Guard([&] {
    if (p == nullptr) return;
    Require(RowBlocks::Device().Remove(p), "pointer was not returned by dsd_device_alloc");
    // Steps enqueued without a wait may still read it.
    DSD_HIP_CHECK(hipDeviceSynchronize());
    DSD_HIP_CHECK(hipFree(p));
  });
}

int dsd_sparse_run_batch_device(dsd_sparse_ctx* ctx, int batch,
                                int total_candidates, int max_candidates,
                                const float* d_queries,
                                const int* d_cand_offsets,
                                const int* d_cand_ids, float* d_outputs,
                                float* d_scores, int* d_selected,
                                int* d_selected_counts, void* stream) {
  return Guard([&] {
    Require(ctx != nullptr, "context must be non-null");
    Require(batch >= 0 && total_candidates >= 0 && max_candidates >= 0,
            "sizes must be non-negative");
    if (batch == 0) return;
    if (batch > ctx->max_batch) {
      throw std::invalid_argument("request batch exceeds sparse context capacity");
    }
    if (total_candidates > ctx->max_cand) {
      throw std::invalid_argument("candidate page count exceeds sparse context capacity");
    }
    Require(d_queries != nullptr && d_cand_offsets != nullptr && d_outputs != nullptr,
            "device inputs must be non-null");
    if (total_candidates > 0) Require(d_cand_ids != nullptr, "cand_ids must be non-null");
    StepLaunch L = ctx->Plan(batch, total_candidates, max_candidates, false);
    L.queries = d_queries;
    L.offsets = d_cand_offsets;
    L.ids = d_cand_ids;
    L.outputs = d_outputs;
    if (d_scores != nullptr) L.scores = d_scores;
    if (d_selected != nullptr) L.selected = d_selected;
    if (d_selected_counts != nullptr) L.counts = d_selected_counts;
    hipStream_t s = stream != nullptr ? reinterpret_cast<hipStream_t>(stream) : ctx->stream;
    if (StreamCapturing(s)) {
      // Captured into a graph: the epoch comes from the device, and the
      // caller orders the graph's replays against the context's other work.
      if (ctx->pool->pending) {
        throw std::invalid_argument(
            "a pool append is still pending: synchronise before capturing a step");
      }
      L.epoch_src = ctx->d_epoch.ptr;
      ctx->last_stream = nullptr;
    } else {
      ctx->pool->OrderAfterPending(s);
      ctx->OrderOn(s);
    }
    ctx->Enqueue(&L, s, false);
    ctx->last = L;
  });
}

int dsd_sparse_replay_stage(dsd_sparse_ctx* ctx, int stage, void* stream) {
  return Guard([&] {
    Require(ctx != nullptr, "context must be non-null");
    Require(ctx->last.valid, "no previous step to replay");
    hipStream_t s = stream != nullptr ? reinterpret_cast<hipStream_t>(stream) : ctx->stream;
    Require(stage >= 0 && stage <= 3, "stage must be 0, 1, 2 or 3");
    if (stage == 3) {
      Require(ctx->last.fused || ctx->last.wide,
              "the last step did not use a single-launch kernel");
    }
    ctx->pool->OrderAfterPending(s);
    ctx->OrderOn(s);
    StepLaunch L = ctx->last;
    ctx->Fresh(&L);
    const PoolView& v = ctx->pool->view;
    switch (stage) {
      case 0: EnqueueScoreStage(v, L, s); break;
      case 1: EnqueueSelectStage(v, L, s); break;
      case 2: EnqueueAttentionStage(v, L, s); break;
      default: EnqueueStep(v, L, s); break;
    }
  });
}

int dsd_sparse_set_score_mode(dsd_sparse_ctx* ctx, int mode) {
  return Guard([&] {
    Require(ctx != nullptr, "context must be non-null");
    Require(mode == DSD_SCORE_CERTIFIED || mode == DSD_SCORE_EXACT, "unknown score mode");
    ctx->score_mode = mode;
  });
}

int dsd_sparse_score_bounds(dsd_sparse_ctx* ctx, int n, float* mid, float* lo, float* hi) {
  return Guard([&] {
    Require(ctx != nullptr, "context must be non-null");
    Require(ctx->last.valid && ctx->last.certified,
            "the last step did not use certified scoring");
    Require(n >= 0 && n <= ctx->last.total, "n exceeds the last step's candidate count");
    Require(mid != nullptr && lo != nullptr && hi != nullptr, "outputs must be non-null");
    DSD_HIP_CHECK(hipStreamSynchronize(ctx->stream));
    DSD_HIP_CHECK(hipMemcpy(mid, ctx->last.scores, sizeof(float) * n, hipMemcpyDeviceToHost));
    DSD_HIP_CHECK(hipMemcpy(lo, ctx->d_lo.ptr, sizeof(float) * n, hipMemcpyDeviceToHost));
    DSD_HIP_CHECK(hipMemcpy(hi, ctx->d_hi.ptr, sizeof(float) * n, hipMemcpyDeviceToHost));
  });
}

int dsd_sparse_exact_rescored_pages(dsd_sparse_ctx* ctx, int reset, int* out) {
  return Guard([&] {
    Require(ctx != nullptr && out != nullptr, "pointers must be non-null");
    DSD_HIP_CHECK(hipDeviceSynchronize());
    ctx->CheckFailure(0);
    DSD_HIP_CHECK(hipMemcpy(out, ctx->d_exact_pages.ptr, sizeof(int), hipMemcpyDeviceToHost));
    if (reset) DSD_HIP_CHECK(hipMemset(ctx->d_exact_pages.ptr, 0, sizeof(int)));
  });
}

int dsd_sparse_last_launch(const dsd_sparse_ctx* ctx, dsd_launch_info* out) {
  return Guard([&] {
    Require(ctx != nullptr && out != nullptr, "pointers must be non-null");
    Require(ctx->last.valid, "no step has been launched on this context");
    const auto& L = ctx->last;
    const dsdk::PoolView& v = ctx->pool->view;
    *out = dsd_launch_info{};
    out->fused = L.fused ? 1 : 0;
    out->wide = L.wide ? 1 : 0;
    out->certified = L.certified ? 1 : 0;
    if (L.wide) {
      const dsdk::WideArgs w = WideStepArgs(v, L);
      out->score_pages_per_group = w.pages_per_group;
      out->grid = dsdk::WideStepGrid(w.items, w.tickets);
    } else if (L.fused) {
      const int hpw = dsdk::FusedStepHeadsPerGroup(v, L.batch, ctx->compute_units);
      out->heads_per_group = hpw;
      out->multi_pass = dsdk::FusedStepMultiPass(v, L.max_n, hpw) ? 1 : 0;
      out->grid = dsdk::FusedStepGrid(v, L.batch, hpw);
    } else if (L.certified && v.elements == 4096) {
      const int per = dsdk::ScorePagesPerGroup(L.total);
      out->score_pages_per_group = per;
      out->grid = L.batch * ((L.max_n + per - 1) / per);
    }
  });
}

int dsd_sparse_step_stamps(const dsd_sparse_ctx* ctx, int* grid, int* per_group, double* khz,
                           uint64_t* out, size_t capacity) {
  return Guard([&] {
    Require(ctx != nullptr && grid != nullptr && per_group != nullptr && khz != nullptr,
            "pointers must be non-null");
    *grid = ctx->stamp_grid;
    *per_group = ctx->last.wide ? dsdk::WideStepStampsPerGroup()
                                : dsdk::FusedStepStampsPerGroup();
    *khz = ctx->wall_khz;
    if (out == nullptr) return;
    const size_t n = static_cast<size_t>(ctx->stamp_grid) * static_cast<size_t>(*per_group);
    Require(capacity >= n, "stamp buffer too small");
    std::memcpy(out, ctx->h_stamps.ptr, sizeof(uint64_t) * n);
  });
}

int dsd_sparse_device_status(dsd_sparse_ctx* ctx) {
  return Guard([&] {
    Require(ctx != nullptr, "context must be non-null");
    DSD_HIP_CHECK(hipDeviceSynchronize());
    ctx->CheckFailure(0);
  });
}

int dsd_sparse_set_wait_limit(dsd_sparse_ctx* ctx, unsigned spin_limit, int never_ready) {
  return Guard([&] {
    Require(ctx != nullptr, "context must be non-null");
    Require(spin_limit > 0, "spin_limit must be positive");
    ctx->spin_limit = spin_limit;
    ctx->never_ready = never_ready != 0;
  });
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free device step
// ---------------------------------------------------------------------------
namespace {

// Limits of one call of dsd_sparse_run_batch_device_static, set by the size
// of the static scratch below.
constexpr int kStaticMaxBatch = 1024;
constexpr int kStaticMaxCandidates = 65536;  // total candidates per call
constexpr int kStaticMaxSelected = 65536;    // batch * max(1, top_k) held for
                                             // a caller that passes no ids
constexpr size_t Align256(size_t bytes) { return (bytes + 255) / 256 * 256; }
// Byte offsets of the scratch's parts: publication words (3 per candidate),
// midpoints, lower and upper bounds, selected ids, selected counts, the
// device epoch, refined-interval words (3 per flagged-page slot of each
// request).
constexpr size_t kStaticRec = 0;
constexpr size_t kStaticMid =
    Align256(kStaticRec + sizeof(unsigned long long) * 3 * kStaticMaxCandidates);
constexpr size_t kStaticLo = Align256(kStaticMid + sizeof(float) * kStaticMaxCandidates);
constexpr size_t kStaticHi = Align256(kStaticLo + sizeof(float) * kStaticMaxCandidates);
constexpr size_t kStaticSel = Align256(kStaticHi + sizeof(float) * kStaticMaxCandidates);
constexpr size_t kStaticCounts = Align256(kStaticSel + sizeof(int) * kStaticMaxSelected);
constexpr size_t kStaticEpoch = Align256(kStaticCounts + sizeof(int) * kStaticMaxBatch);
constexpr size_t kStaticRefined = Align256(kStaticEpoch + sizeof(unsigned));
constexpr size_t kStaticBytes = Align256(
    kStaticRefined + sizeof(unsigned long long) * 3 * dsdk::kFRefineSlots * kStaticMaxBatch);

}  // namespace

// The scratch of dsd_sparse_run_batch_device_static (2.7 MiB): one copy per
// GPU, held until the process ends, shared by every call on that GPU.  Host
// code never names it except to look up its device address.
static __device__ __align__(256) unsigned char scratch[kStaticBytes];

namespace {

constexpr int kStaticMaxDevices = 64;

// Per GPU: the device address of `scratch` (looked up once, with that GPU
// current) and the epoch counter of the calls on it.
struct StaticScratch {
  std::once_flag once;
  hipError_t status = hipSuccess;
  unsigned char* ptr = nullptr;
  int compute_units = 256;
  unsigned epoch = 0;
};
StaticScratch g_static_scratch[kStaticMaxDevices];

StaticScratch& StaticScratchOn(int device) {
  StaticScratch& st = g_static_scratch[device];
  std::call_once(st.once, [&] {
    void* p = nullptr;
    st.status = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (st.status != hipSuccess) return;
    st.ptr = static_cast<unsigned char*>(p);
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) ==
            hipSuccess &&
        cus > 0) {
      st.compute_units = cus;
    }
  });
  DSD_HIP_CHECK(st.status);
  return st;
}

}  // namespace

extern "C" {

int dsd_sparse_run_batch_device_static(dsd_pool* pool, int top_k, int batch,
                                       int total_candidates, int max_candidates,
                                       const float* d_queries, const int* d_cand_offsets,
                                       const int* d_cand_ids, float* d_outputs, float* d_scores,
                                       int* d_selected, int* d_selected_counts,
                                       unsigned long long* d_fail, void* stream) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    Require(top_k >= 0, "top_k must be non-negative");
    Require(batch >= 0 && total_candidates >= 0 && max_candidates >= 0,
            "sizes must be non-negative");
    if (pool->view.head_dim <= 0 || pool->view.head_dim > 128) {
      throw std::invalid_argument("sparse decode supports head_dim in (0, 128]");
    }
    if (batch == 0) return;
    if (batch > kStaticMaxBatch) {
      throw std::invalid_argument(
          "dsd_sparse_run_batch_device_static: batch exceeds the static scratch's 1024 "
          "requests");
    }
    if (total_candidates > kStaticMaxCandidates) {
      throw std::invalid_argument(
          "dsd_sparse_run_batch_device_static: total_candidates exceeds the static scratch's "
          "65536 candidates");
    }
    if (d_selected == nullptr &&
        static_cast<int64_t>(batch) * std::max(1, top_k) > kStaticMaxSelected) {
      throw std::invalid_argument(
          "dsd_sparse_run_batch_device_static: batch * top_k exceeds the static scratch's 65536 "
          "selected ids (pass d_selected)");
    }
    Require(d_queries != nullptr && d_cand_offsets != nullptr && d_outputs != nullptr,
            "device inputs must be non-null");
    if (total_candidates > 0) Require(d_cand_ids != nullptr, "cand_ids must be non-null");
    int device = 0;
    DSD_HIP_CHECK(hipGetDevice(&device));
    Require(device >= 0 && device < kStaticMaxDevices, "device ordinal beyond 64");
    StaticScratch& st = StaticScratchOn(device);
    if (++st.epoch >= 0x40000000u) st.epoch = 1;
    const PoolView& v = pool->view;
    StepLaunch L;
    L.valid = true;
    L.certified = StepCertified(v, DSD_SCORE_CERTIFIED, max_candidates, false);
    L.fused = StepFused(v, L.certified, true, max_candidates, top_k);
    // (three kernels where a context would run the wide step, with its
    // attention partition: the same outputs)
    L.wide_shape = !L.fused && L.certified && batch > 0 &&
                   !dsdk::FusedStepSupported(v, max_candidates, top_k) &&
                   dsdk::WideStepSupported(v, max_candidates, top_k);
    L.batch = batch;
    L.total = total_candidates;
    L.max_n = max_candidates;
    L.top_k = top_k;
    L.compute_units = st.compute_units;
    L.scale = StepScale(v);
    L.queries = d_queries;
    L.offsets = d_cand_offsets;
    L.ids = d_cand_ids;
    L.outputs = d_outputs;
    L.rec = reinterpret_cast<unsigned long long*>(st.ptr + kStaticRec);
    L.refined = reinterpret_cast<unsigned long long*>(st.ptr + kStaticRefined);
    L.scores = d_scores != nullptr ? d_scores : reinterpret_cast<float*>(st.ptr + kStaticMid);
    L.lo = reinterpret_cast<float*>(st.ptr + kStaticLo);
    L.hi = reinterpret_cast<float*>(st.ptr + kStaticHi);
    L.selected = d_selected != nullptr ? d_selected : reinterpret_cast<int*>(st.ptr + kStaticSel);
    L.counts = d_selected_counts != nullptr ? d_selected_counts
                                            : reinterpret_cast<int*>(st.ptr + kStaticCounts);
    L.exact_pages = nullptr;
    L.fail_word = d_fail;
    L.epoch = st.epoch;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    if (StreamCapturing(s)) {
      // Captured into a graph: the epoch comes from the device (a word of
      // the static scratch, zero at load).
      if (pool->pending) {
        throw std::invalid_argument(
            "a pool append is still pending: synchronise before capturing a step");
      }
      L.epoch_src = reinterpret_cast<const unsigned*>(st.ptr + kStaticEpoch);
    } else {
      pool->OrderAfterPending(s);
    }
    EnqueueStep(v, L, s);
  });
}

// ---------------------------------------------------------------------------
// Dense decode (DenseCudaContext::RunBatch, src/cuda/kernels.cu:197-292).
// ---------------------------------------------------------------------------
int dsd_dense_run_batch(dsd_pool* pool, int batch, const float* queries,
                        const int* cand_offsets, const int* cand_ids,
                        float* outputs, double* kernel_ms) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    Require(batch >= 0, "batch must be non-negative");
    if (kernel_ms != nullptr) *kernel_ms = 0.0;
    if (batch == 0) return;
    Require(queries != nullptr && cand_offsets != nullptr && outputs != nullptr,
            "inputs must be non-null");
    Require(pool->view.head_dim > 0 && pool->view.head_dim <= 256,
            "head_dim must be in (0, 256]");
    Require(cand_offsets[0] == 0, "cand_offsets[0] must be 0");
    for (int r = 0; r < batch; ++r) {
      Require(cand_offsets[r + 1] >= cand_offsets[r], "cand_offsets must be non-decreasing");
    }
    const int total = cand_offsets[batch];
    if (total > 0) Require(cand_ids != nullptr, "cand_ids must be non-null");
    for (int c = 0; c < total; ++c) pool->ValidatePage(cand_ids[c]);
    const size_t qn = static_cast<size_t>(batch) * pool->view.elements;
    pool->dense_q.Reserve(qn);
    pool->dense_offsets.Reserve(batch + 1);
    pool->dense_ids.Reserve(std::max(1, total));
    pool->h_dense_q.Reserve(qn, hipHostMallocCoherent);
    pool->h_dense_out.Reserve(qn, hipHostMallocCoherent);
    pool->h_dense_offsets.Reserve(batch + 1, hipHostMallocCoherent);
    pool->h_dense_ids.Reserve(std::max(1, total), hipHostMallocCoherent);
    // As the sparse host step: inputs through pinned staging and one
    // stage-in kernel, outputs written by the attention into pinned memory
    // (no DMA copies, so no copy-engine hand-offs).
    std::memcpy(pool->h_dense_q.ptr, queries, sizeof(float) * qn);
    std::memcpy(pool->h_dense_offsets.ptr, cand_offsets, sizeof(int) * (batch + 1));
    if (total > 0) std::memcpy(pool->h_dense_ids.ptr, cand_ids, sizeof(int) * total);
    {
      dsdk::StageSegments seg;
      seg.src[0] = reinterpret_cast<const uint32_t*>(pool->h_dense_q.ptr);
      seg.dst[0] = reinterpret_cast<uint32_t*>(pool->dense_q.ptr);
      seg.words[0] = static_cast<int>(qn);
      seg.src[1] = reinterpret_cast<const uint32_t*>(pool->h_dense_offsets.ptr);
      seg.dst[1] = reinterpret_cast<uint32_t*>(pool->dense_offsets.ptr);
      seg.words[1] = batch + 1;
      seg.src[2] = reinterpret_cast<const uint32_t*>(pool->h_dense_ids.ptr);
      seg.dst[2] = reinterpret_cast<uint32_t*>(pool->dense_ids.ptr);
      seg.words[2] = total;
      seg.count = 3;
      dsdk::LaunchStageIn(seg, pool->stream);
    }
    dsdk::AttentionArgs a;
    a.queries = pool->dense_q.ptr;
    a.list_ids = pool->dense_ids.ptr;
    a.list_offsets = pool->dense_offsets.ptr;
    a.list_stride = 0;
    a.batch = batch;
    a.scale = 1.0f / std::sqrt(static_cast<float>(pool->view.head_dim));
    a.outputs = pool->h_dense_out.ptr;
    DSD_HIP_CHECK(hipEventRecord(pool->dense_start, pool->stream));
    dsdk::LaunchAttention(pool->view, a, pool->stream);
    DSD_HIP_CHECK(hipEventRecord(pool->dense_stop, pool->stream));
    pool->Sync();
    std::memcpy(outputs, pool->h_dense_out.ptr, sizeof(float) * qn);
    if (kernel_ms != nullptr) {
      float ms = 0.f;
      DSD_HIP_CHECK(hipEventElapsedTime(&ms, pool->dense_start, pool->dense_stop));
      *kernel_ms = ms;
    }
  });
}

int dsd_dense_run_batch_device(dsd_pool* pool, int batch,
                               const float* d_queries,
                               const int* d_cand_offsets,
                               const int* d_cand_ids, float* d_outputs,
                               void* stream) {
  return Guard([&] {
    Require(pool != nullptr, "pool must be non-null");
    pool->WaitPending();
    Require(batch >= 0, "batch must be non-negative");
    if (batch == 0) return;
    Require(d_queries != nullptr && d_cand_offsets != nullptr && d_outputs != nullptr,
            "device inputs must be non-null");
    dsdk::AttentionArgs a;
    a.queries = d_queries;
    a.list_ids = d_cand_ids;
    a.list_offsets = d_cand_offsets;
    a.list_stride = 0;
    a.batch = batch;
    a.scale = 1.0f / std::sqrt(static_cast<float>(pool->view.head_dim));
    a.outputs = d_outputs;
    dsdk::LaunchAttention(pool->view, a, reinterpret_cast<hipStream_t>(stream));
  });
}

}  // extern "C"
