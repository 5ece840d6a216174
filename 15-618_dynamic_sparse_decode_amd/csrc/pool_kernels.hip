// pool_kernels.hip -- device page pool maintenance kernels (gfx950).
//
// Summaries follow the reference's host rule exactly (no FMA contraction, no
// division shortcut): upload = sum in token order then times fl(1/count)
// (src/paged_kv_cache.cpp:87-99); append = (s*old + k)/(old+1)
// (src/paged_kv_cache.cpp:231-238).  The reference's device kernel instead
// divides by the count (src/device_page_pool.cpp:89-99), which can differ by
// an ulp; this pool reproduces the host cache bit for bit.
#include <algorithm>

#include "dsd_internal.h"

namespace dsdk {
namespace {

constexpr int kPoolThreads = 256;

// One workgroup per uploaded page; threads stride the E summary elements so
// each token row is read with contiguous, coalesced loads.
__global__ __launch_bounds__(kPoolThreads) void FinishPageUploadKernel(
    PoolView pool, const int* __restrict__ page_ids,
    const int* __restrict__ token_counts, const float* __restrict__ rows,
    int n) {
  const int i = blockIdx.x;
  if (i >= n) return;
  const int page = page_ids[i];
  const int count = token_counts[i];
  const int E = pool.elements;
  float* summary = pool.summaries + static_cast<size_t>(page) * E;
  if (rows != nullptr) {
    const float* src = rows + static_cast<size_t>(i) * E;
    for (int e = threadIdx.x; e < E; e += blockDim.x) summary[e] = src[e];
  } else {
    const float* keys = pool.keys + static_cast<size_t>(page) * pool.page_elems;
    const float inv = __fdiv_rn(1.0f, static_cast<float>(count));
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      float acc = 0.0f;
      for (int t = 0; t < count; ++t) {
        acc = __fadd_rn(acc, keys[static_cast<size_t>(t) * E + e]);
      }
      summary[e] = __fmul_rn(acc, inv);
    }
  }
  if (threadIdx.x == 0) {
    pool.token_counts[page] = count;
    pool.live[page] = 1;
  }
}

// One workgroup per page segment; tokens of a segment are applied in offset
// order so the running mean matches the host's sequence of updates.
__global__ __launch_bounds__(kPoolThreads) void AppendTokensKernel(
    PoolView pool, const int* __restrict__ seg_start,
    const int* __restrict__ order, const int* __restrict__ page_ids,
    const int* __restrict__ offsets, const int* __restrict__ counts,
    const float* __restrict__ keys, const float* __restrict__ values,
    const float* __restrict__ rows, int num_segments) {
  const int seg = blockIdx.x;
  if (seg >= num_segments) return;
  const int begin = seg_start[seg];
  const int end = seg_start[seg + 1];
  const int E = pool.elements;
  const int page = page_ids[order[begin]];
  const size_t page_base = static_cast<size_t>(page) * pool.page_elems;

  for (int q = begin; q < end; ++q) {
    const int tok = order[q];
    const size_t dst = page_base + static_cast<size_t>(offsets[tok]) * E;
    const size_t src = static_cast<size_t>(tok) * E;
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      pool.keys[dst + e] = keys[src + e];
      pool.values[dst + e] = values[src + e];
    }
  }

  float* summary = pool.summaries + static_cast<size_t>(page) * E;
  if (rows != nullptr) {
    const float* src = rows + static_cast<size_t>(order[end - 1]) * E;
    for (int e = threadIdx.x; e < E; e += blockDim.x) summary[e] = src[e];
  } else {
    const bool fresh = offsets[order[begin]] == 0;
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
      float s = fresh ? 0.0f : summary[e];
      for (int q = begin; q < end; ++q) {
        const int tok = order[q];
        const float old_count = static_cast<float>(offsets[tok]);
        const float new_count = __fadd_rn(old_count, 1.0f);
        s = __fdiv_rn(__fadd_rn(__fmul_rn(s, old_count),
                                keys[static_cast<size_t>(tok) * E + e]),
                      new_count);
      }
      summary[e] = s;
    }
  }
  if (threadIdx.x == 0) {
    pool.token_counts[page] = counts[order[end - 1]];
    pool.live[page] = 1;
  }
}

__global__ __launch_bounds__(kPoolThreads) void MarkFreeKernel(
    PoolView pool, const int* __restrict__ page_ids, int n) {
  const int i = blockIdx.x;
  if (i >= n) return;
  const int page = page_ids[i];
  float* summary = pool.summaries + static_cast<size_t>(page) * pool.elements;
  for (int e = threadIdx.x; e < pool.elements; e += blockDim.x) summary[e] = 0.0f;
  if (threadIdx.x == 0) {
    pool.token_counts[page] = 0;
    pool.live[page] = 0;
  }
}

// Integer-hash synthetic payloads for the GPU-resident admission modes.  The
// mixing sequence and the value map (x % 2001 - 1000) / 1000 follow
// src/device_page_pool.cpp:102-138 so that a workload generated here is the
// same workload the reference generates.
__device__ __forceinline__ uint32_t HashMix(uint32_t x, int v, uint32_t salt) {
  return x ^ (static_cast<uint32_t>(v) + salt + (x << 6) + (x >> 2));
}

__device__ __forceinline__ float HashValue(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return static_cast<float>(static_cast<int>(x % 2001u) - 1000) / 1000.0f;
}

__device__ __forceinline__ float PromptValue(int request_id, int page_idx, int token,
                                             int element, int stream) {
  uint32_t x = 0x9e3779b9u;
  x = HashMix(x, request_id, 0x85ebca6bu);
  x = HashMix(x, page_idx, 0xc2b2ae35u);
  x = HashMix(x, token, 0x27d4eb2fu);
  x = HashMix(x, element, 0x165667b1u);
  x = HashMix(x, stream, 0xd3a2646cu);
  return HashValue(x);
}

__device__ __forceinline__ float DecodeValue(int request_id, int decode_step, int element,
                                             int stream) {
  uint32_t x = 0x9e3779b9u;
  x = HashMix(x, request_id, 0x85ebca6bu);
  x = HashMix(x, decode_step, 0xc2b2ae35u);
  x = HashMix(x, element, 0x165667b1u);
  x = HashMix(x, stream, 0xd3a2646cu);
  return HashValue(x);
}

// One workgroup per prompt page: K/V from the hash, summary by the host rule.
__global__ __launch_bounds__(kPoolThreads) void PrefillSyntheticKernel(
    PoolView pool, const int* __restrict__ page_ids, const int* __restrict__ token_counts,
    int n, int request_id) {
  const int i = blockIdx.x;
  if (i >= n) return;
  const int page = page_ids[i];
  const int count = token_counts[i];
  const int E = pool.elements;
  const size_t base = static_cast<size_t>(page) * pool.page_elems;
  const float inv = __fdiv_rn(1.0f, static_cast<float>(count));
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    float acc = 0.0f;
    for (int t = 0; t < count; ++t) {
      const float k = PromptValue(request_id, i, t, e, 1);
      const float v = PromptValue(request_id, i, t, e, 2);
      pool.keys[base + static_cast<size_t>(t) * E + e] = k;
      pool.values[base + static_cast<size_t>(t) * E + e] = v;
      acc = __fadd_rn(acc, k);
    }
    pool.summaries[static_cast<size_t>(page) * E + e] = __fmul_rn(acc, inv);
  }
  if (threadIdx.x == 0) {
    pool.token_counts[page] = count;
    pool.live[page] = 1;
  }
}

// One workgroup per (page segment, kPoolThreads elements of the token row),
// summary by the running mean s = (s*old + k)/new, each operation rounded
// separately (the host rule).  A page's single token of the call uses the
// reference's counts: old = the page's token count - 1, new = that count
// (src/device_page_pool.cpp:219-231; the serving loop appends one token per
// page per step, so this is every real call).  The reference runs one block
// per token, so several tokens of one page in one call race there; here
// they apply in offset order with old = offset, the host cache's sequence
// (src/paged_kv_cache.cpp:231-238).  The metadata is read straight from the
// caller's pinned staging (layout at LaunchAppendSynthetic), so the append
// is one launch with no copies.
__global__ __launch_bounds__(kPoolThreads) void AppendSyntheticKernel(PoolView pool,
                                                                      const int* __restrict__ meta,
                                                                      int n, int num_segments) {
  const int seg = blockIdx.x;
  if (seg >= num_segments) return;
  const int* page_ids = meta + num_segments + 1;
  const int* offsets = page_ids + n;
  const int* counts = offsets + n;
  const int* request_ids = counts + n;
  const int* decode_steps = request_ids + n;
  const int begin = meta[seg];
  const int end = meta[seg + 1];
  const int E = pool.elements;
  const int page = page_ids[begin];
  const size_t base = static_cast<size_t>(page) * pool.page_elems;
  float* summary = pool.summaries + static_cast<size_t>(page) * E;
  const int e = static_cast<int>(blockIdx.y * kPoolThreads + threadIdx.x);
  if (e < E) {
    float s = summary[e];
    const bool single = end - begin == 1;
    for (int q = begin; q < end; ++q) {
      const int off = offsets[q];
      const float k = DecodeValue(request_ids[q], decode_steps[q], e, 1);
      const float v = DecodeValue(request_ids[q], decode_steps[q], e, 2);
      const size_t dst = base + static_cast<size_t>(off) * E + e;
      pool.keys[dst] = k;
      pool.values[dst] = v;
      const int old = single ? counts[q] - 1 : off;
      // A page's first token: whatever the row held before (a lazily freed
      // page keeps its old summary) is multiplied by 0, i.e. dropped.
      if (old == 0) s = 0.0f;
      s = __fdiv_rn(__fadd_rn(__fmul_rn(s, static_cast<float>(old)), k),
                    static_cast<float>(old + 1));
    }
    summary[e] = s;
  }
  if (blockIdx.y == 0 && threadIdx.x == 0) {
    pool.token_counts[page] = counts[end - 1];
    pool.live[page] = 1;
  }
}

}  // namespace

void LaunchFinishPageUpload(const PoolView& pool, const int* d_page_ids,
                            const int* d_token_counts, const float* d_rows,
                            int n, hipStream_t stream) {
  if (n <= 0) return;
  hipLaunchKernelGGL(FinishPageUploadKernel, dim3(n), dim3(kPoolThreads), 0,
                     stream, pool, d_page_ids, d_token_counts, d_rows, n);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchAppendTokens(const PoolView& pool, const int* d_seg_start,
                        const int* d_order, const int* d_page_ids,
                        const int* d_offsets, const int* d_counts,
                        const float* d_keys, const float* d_values,
                        const float* d_rows, int num_segments,
                        hipStream_t stream) {
  if (num_segments <= 0) return;
  hipLaunchKernelGGL(AppendTokensKernel, dim3(num_segments), dim3(kPoolThreads),
                     0, stream, pool, d_seg_start, d_order, d_page_ids,
                     d_offsets, d_counts, d_keys, d_values, d_rows,
                     num_segments);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchPrefillSynthetic(const PoolView& pool, const int* d_page_ids,
                            const int* d_token_counts, int n, int request_id,
                            hipStream_t stream) {
  if (n <= 0) return;
  hipLaunchKernelGGL(PrefillSyntheticKernel, dim3(n), dim3(kPoolThreads), 0, stream, pool,
                     d_page_ids, d_token_counts, n, request_id);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchAppendSynthetic(const PoolView& pool, const int* meta, int n, int num_segments,
                           hipStream_t stream) {
  if (num_segments <= 0) return;
  const unsigned slices = static_cast<unsigned>((pool.elements + kPoolThreads - 1) / kPoolThreads);
  hipLaunchKernelGGL(AppendSyntheticKernel, dim3(static_cast<unsigned>(num_segments), slices),
                     dim3(kPoolThreads), 0, stream, pool, meta, n, num_segments);
  DSD_HIP_CHECK(hipGetLastError());
}

// The host step's inputs, from the context's pinned (device-visible,
// coherent) staging into device buffers, on the step's stream: one small
// kernel instead of DMA copies, each of which costs a hand-off between the
// copy engine and the compute queue (tens of microseconds per step).
// Exclusive prefix sum of one int per thread of a kPoolThreads workgroup;
// *total gets the sum.  Every thread calls.
__device__ int PoolBlockScan(int x, int* scratch, int* total) {
  constexpr int kWaves = kPoolThreads / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  int incl = x;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) scratch[wave] = incl;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const int v = scratch[w];
    before += w < wave ? v : 0;
    all += v;
  }
  __syncthreads();
  *total = all;
  return before + incl - x;
}

__global__ __launch_bounds__(kPoolThreads) void StageInKernel(StageSegments s) {
  if (s.start_stamp != nullptr && blockIdx.x == 0 && threadIdx.x == 0) {
    __hip_atomic_store(s.start_stamp, static_cast<unsigned long long>(wall_clock64()),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  const int tid = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  const int stride = static_cast<int>(gridDim.x * blockDim.x);
  for (int k = 0; k < s.count; ++k) {
    const int words = s.words[k];
    const int n4 = words / 4;
    const uint4* src4 = reinterpret_cast<const uint4*>(s.src[k]);
    uint4* dst4 = reinterpret_cast<uint4*>(s.dst[k]);
    for (int i = tid; i < n4; i += stride) dst4[i] = src4[i];
    for (int i = 4 * n4 + tid; i < words; i += stride) s.dst[k][i] = s.src[k][i];
  }
  if (s.nrows > 0) {
    // One chunk of blockDim.x float4s per workgroup turn, so each workgroup
    // reads its row pointer once (a uniform load) and the rows stream
    // straight from host memory.
    const int per_row = s.row_words / 4;
    const int chunks = (per_row + kPoolThreads - 1) / kPoolThreads;
    const int items = s.nrows * chunks;
    for (int item = static_cast<int>(blockIdx.x); item < items;
         item += static_cast<int>(gridDim.x)) {
      const int row = item / chunks;
      const int i = (item - row * chunks) * kPoolThreads + static_cast<int>(threadIdx.x);
      if (i < per_row) {
        const float4* src = reinterpret_cast<const float4*>(s.rows[row]);
        reinterpret_cast<float4*>(s.rows_dst)[static_cast<size_t>(row) * per_row + i] = src[i];
      }
    }
  }
  if (s.table_batch > 0) {
    // The batch's candidate lists from the page table.  Every workgroup
    // forms the same offsets (a scan of the slots' page counts, in chunks
    // of kPoolThreads requests); workgroup 0 writes them, and request b's
    // list is copied by workgroup b mod gridDim.x.
    __shared__ int scan[kPoolThreads / 64];
    __shared__ int pos_s[kPoolThreads], np_s[kPoolThreads], slot_s[kPoolThreads];
    int base = 0;
    for (int b0 = 0; b0 < s.table_batch; b0 += kPoolThreads) {
      const int b = b0 + static_cast<int>(threadIdx.x);
      const bool in = b < s.table_batch;
      const int slot = in ? s.table_slots[b] : 0;
      const int np = in ? s.table.npages[slot] : 0;
      int total = 0;
      const int pos = base + PoolBlockScan(np, scan, &total);
      if (in && blockIdx.x == 0) s.csr_offsets[b] = pos;
      pos_s[threadIdx.x] = pos;
      np_s[threadIdx.x] = np;
      slot_s[threadIdx.x] = slot;
      __syncthreads();
      const int chunk = min(kPoolThreads, s.table_batch - b0);
      for (int k = 0; k < chunk; ++k) {
        if ((b0 + k) % static_cast<int>(gridDim.x) != static_cast<int>(blockIdx.x)) continue;
        const int* list = s.table.pages + static_cast<size_t>(slot_s[k]) * s.table.max_pages;
        for (int j = threadIdx.x; j < np_s[k]; j += kPoolThreads) s.csr_ids[pos_s[k] + j] = list[j];
      }
      __syncthreads();
      base += total;
    }
    if (blockIdx.x == 0 && threadIdx.x == 0) s.csr_offsets[s.table_batch] = base;
  }
}

__global__ __launch_bounds__(64) void StepMarkKernel(unsigned long long* words,
                                                     unsigned long long ticket) {
  if (threadIdx.x == 0) {
    __hip_atomic_store(words + 1, static_cast<unsigned long long>(wall_clock64()),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(words, ticket, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
  }
}

void LaunchStepMark(unsigned long long* words, unsigned long long ticket, hipStream_t stream) {
  if (words == nullptr) throw std::invalid_argument("step mark needs its words");
  hipLaunchKernelGGL(StepMarkKernel, dim3(1), dim3(64), 0, stream, words, ticket);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchStageIn(const StageSegments& s, hipStream_t stream) {
  size_t words = 0;
  for (int k = 0; k < s.count; ++k) {
    if (s.words[k] < 0) throw std::invalid_argument("negative staging segment");
    if ((reinterpret_cast<uintptr_t>(s.src[k]) | reinterpret_cast<uintptr_t>(s.dst[k])) % 16 != 0) {
      throw std::invalid_argument("staging segments must be 16-byte aligned");
    }
    words += static_cast<size_t>(s.words[k]);
  }
  if (s.nrows > 0) {
    if (s.rows == nullptr || s.rows_dst == nullptr || s.row_words % 4 != 0 ||
        reinterpret_cast<uintptr_t>(s.rows_dst) % 16 != 0) {
      throw std::invalid_argument("row gather needs 16-byte aligned rows of 4k words");
    }
    words += static_cast<size_t>(s.nrows) * static_cast<size_t>(s.row_words);
  }
  if (s.table_batch > 0) {
    if (s.table_slots == nullptr || s.csr_offsets == nullptr || s.csr_ids == nullptr ||
        s.table.pages == nullptr) {
      throw std::invalid_argument("table staging needs slots, a table and CSR buffers");
    }
    words += static_cast<size_t>(s.table_batch) * 64;  // at least a workgroup per 4 requests
  }
  if (words == 0) return;
  size_t groups = (words / 4 + kPoolThreads - 1) / kPoolThreads + 1;
  if (s.nrows > 0) {
    const size_t per_row = static_cast<size_t>(s.row_words) / 4;
    groups = std::max(groups, static_cast<size_t>(s.nrows) *
                                  ((per_row + kPoolThreads - 1) / kPoolThreads));
  }
  groups = std::min<size_t>(groups, 256);
  hipLaunchKernelGGL(StageInKernel, dim3(static_cast<unsigned>(groups)), dim3(kPoolThreads), 0,
                     stream, s);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchMarkFree(const PoolView& pool, const int* d_page_ids, int n,
                    hipStream_t stream) {
  if (n <= 0) return;
  hipLaunchKernelGGL(MarkFreeKernel, dim3(n), dim3(kPoolThreads), 0, stream,
                     pool, d_page_ids, n);
  DSD_HIP_CHECK(hipGetLastError());
}

void PreloadPoolKernels() {
  PreloadKernel(StageInKernel);
  PreloadKernel(StepMarkKernel);
  PreloadKernel(AppendSyntheticKernel);
  PreloadKernel(AppendTokensKernel);
}

}  // namespace dsdk
