// page_table.hip -- the request -> page table and the free-page stack of a
// device page pool, resident in HBM (gfx950).
//
// The reference keeps both on the host: PagedKvCache::request_to_pages_
// (include/dsd/paged_kv_cache.h:120) and PagePool's free list
// (src/page_pool.cpp:36-44, 121-127).  Here they live next to the pool so
// that admission, token append, release and the per-step packing of the
// candidate lists run as kernels: per step only the queries and the batch's
// slot ids cross PCIe.  The operations keep the reference's page-id order
// exactly:
//   * the stack starts as [0, 1, ..., capacity-1] and pops from the top, so
//     the first page handed out is capacity-1 (PagePool::allocate_page);
//   * admission pops n pages and keeps them sorted ascending
//     (PagedKvCache::ReservePagesForRequest, src/paged_kv_cache.cpp:114-160);
//   * an append pops one page for each request, in batch order, whose tail
//     page is full or that asks for a fresh page (AppendTokenMetadataOnly,
//     src/paged_kv_cache.cpp:312-351);
//   * a release pushes the request's pages in list order, requests in batch
//     order (ReleaseRequest, src/paged_kv_cache.cpp:354-373).
// The host mirrors only the counts (pages per slot, tokens in the tail page,
// stack depth), so it can size launches and reject exhaustion without
// reading the device; page ids never leave HBM unless downloaded.
#include <algorithm>

#include "dsd_internal.h"

namespace dsdk {
namespace {

constexpr int kTableThreads = 1024;
constexpr int kTableWaves = kTableThreads / 64;

// Block-wide exclusive prefix sum of one int per thread (every thread
// calls); `scratch` holds kTableWaves + 1 ints of LDS.  Returns the sum of
// the values of the threads below; *total gets the block's sum.
__device__ int BlockExclusiveScan(int x, int* scratch, int* total) {
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
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < kTableWaves; ++w) {
      const int v = scratch[w];
      scratch[w] = run;
      run += v;
    }
    scratch[kTableWaves] = run;
  }
  __syncthreads();
  const int excl = scratch[wave] + incl - x;
  *total = scratch[kTableWaves];
  __syncthreads();
  return excl;
}

__global__ void TableResetKernel(TableView t, int capacity) {
  const int i = static_cast<int>(blockIdx.x * blockDim.x + threadIdx.x);
  const int stride = static_cast<int>(gridDim.x * blockDim.x);
  for (int p = i; p < capacity; p += stride) t.free_stack[p] = p;
  for (int s = i; s < t.max_slots; s += stride) t.npages[s] = 0;
  if (i == 0) *t.free_top = capacity;
}

// Admission of slot `slot`: pops n pages (n <= max_pages, checked by the
// host against its mirror of the stack depth), keeps them ascending.
__global__ __launch_bounds__(kTableThreads) void TableReserveKernel(TableView t, int slot, int n) {
  extern __shared__ int ids[];  // n
  const int top = *t.free_top;
  for (int j = threadIdx.x; j < n; j += blockDim.x) ids[j] = t.free_stack[top - 1 - j];
  __syncthreads();
  int* list = t.pages + static_cast<size_t>(slot) * t.max_pages;
  // The popped ids are distinct: a page's place is the count of smaller ones.
  for (int j = threadIdx.x; j < n; j += blockDim.x) {
    const int id = ids[j];
    int rank = 0;
    for (int k = 0; k < n; ++k) rank += ids[k] < id ? 1 : 0;
    list[rank] = id;
  }
  if (threadIdx.x == 0) {
    t.npages[slot] = n;
    *t.free_top = top - n;
  }
}

// Prompt rows (tokens x E, keys then values staged contiguously on the
// device) into the pages of `slot`, token i to page i / page_size at row
// i % page_size; one float4 per thread, grid-stride.
__global__ void TableScatterKernel(PoolView pool, TableView t, int slot, int tokens,
                                   const float4* __restrict__ keys,
                                   const float4* __restrict__ values) {
  const int* list = t.pages + static_cast<size_t>(slot) * t.max_pages;
  const int e4 = pool.elements / 4;
  const size_t total = static_cast<size_t>(tokens) * e4;
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t x = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; x < total;
       x += stride) {
    const int tok = static_cast<int>(x / e4);
    const int c = static_cast<int>(x - static_cast<size_t>(tok) * e4);
    const int page = list[tok / pool.page_size];
    const size_t dst = (static_cast<size_t>(page) * pool.page_elems +
                        static_cast<size_t>(tok % pool.page_size) * pool.elements) / 4 + c;
    reinterpret_cast<float4*>(pool.keys)[dst] = keys[x];
    reinterpret_cast<float4*>(pool.values)[dst] = values[x];
  }
}

// One token for each of n slots (batch order).  args: slots[n], then
// flags[n] (bit 0: start a fresh page; bit 1: the payload is uploaded),
// request_ids[n], decode_steps[n] -- pinned host memory read directly.
// Pops the fresh pages in batch order and writes, for the m uploaded tokens
// (batch order; m is the host's count of bit 1), the append kernels' plan:
//   plan: seg_start[m+1] | page ids[m] | offsets[m] | counts[m] |
//         request ids[m] | decode steps[m]
// (AppendSyntheticKernel's metadata layout; AppendTokensKernel takes the
// first four arrays and order[m] = 0..m-1).  Each token is its page's only
// one in the call, so every segment holds one token.  The payload's count is
// the device count plus one; a token that is not uploaded (a request's
// last) leaves the device count alone, as the reference's pool never
// receives it, and a fresh page it opened keeps no tokens.
__global__ __launch_bounds__(kTableThreads) void TablePlanAppendKernel(
    PoolView pool, TableView t, const int* __restrict__ args, int n, int m, int* plan,
    int* order, ProgressMark mark) {
  __shared__ int scan[kTableWaves + 1];
  const int* slots = args;
  const int* flags = args + n;
  const int* request_ids = flags + n;
  const int* decode_steps = request_ids + n;
  int* page_ids = plan + m + 1;
  int* offsets = page_ids + m;
  int* counts = offsets + m;
  int* req = counts + m;
  int* steps = req + m;
  const int top = *t.free_top;
  int new_base = 0, up_base = 0;
  for (int b0 = 0; b0 < n; b0 += blockDim.x) {
    const int i = b0 + static_cast<int>(threadIdx.x);
    const bool in = i < n;
    int slot = 0, np = 0, tail = -1, count = 0, flag = 0;
    if (in) {
      slot = slots[i];
      flag = flags[i];
      np = t.npages[slot];
      if (np > 0) {
        tail = t.pages[static_cast<size_t>(slot) * t.max_pages + np - 1];
        count = pool.token_counts[tail];
      }
    }
    const bool fresh = in && ((flag & 1) != 0 || np == 0 || count >= pool.page_size);
    const bool up = in && (flag & 2) != 0;
    int tot_new = 0, tot_up = 0;
    const int my_new = BlockExclusiveScan(fresh ? 1 : 0, scan, &tot_new);
    const int my_up = BlockExclusiveScan(up ? 1 : 0, scan, &tot_up);
    if (in) {
      int page = tail;
      int offset = count;
      if (fresh) {
        page = t.free_stack[top - 1 - (new_base + my_new)];
        t.pages[static_cast<size_t>(slot) * t.max_pages + np] = page;
        t.npages[slot] = np + 1;
        offset = 0;
        if (!up) pool.token_counts[page] = 0;
      }
      const int q = up_base + my_up;
      if (up && q < m) {
        order[q] = q;
        plan[q] = q;
        page_ids[q] = page;
        offsets[q] = offset;
        counts[q] = offset + 1;
        req[q] = request_ids[i];
        steps[q] = decode_steps[i];
      }
    }
    new_base += tot_new;
    up_base += tot_up;
  }
  if (threadIdx.x == 0) {
    plan[m] = m;  // seg_start[m]
    *t.free_top = top - new_base;
  }
  __syncthreads();  // every thread has read its arguments
  if (threadIdx.x == 0) StoreProgress(mark);
}

// Release of n <= 1024 slots (batch order): their pages go back on the stack
// in list order, slots in batch order; when `clear`, each page's token
// count, live flag and summary are cleared (the reference's device
// MarkPagesFree).  slots: pinned.  Every workgroup forms the same prefix of
// the slots' page counts (the stack top and the counts are read before any
// workgroup writes them: TableReleaseFinishKernel resets the counts and
// moves the top afterwards); workgroup 0 pushes, the grid clears one page
// per workgroup at a time.
__global__ __launch_bounds__(kTableThreads) void TableReleaseKernel(
    PoolView pool, TableView t, const int* __restrict__ slots, int n, int clear) {
  __shared__ int scan[kTableWaves + 1];
  __shared__ int pos_s[kTableThreads], slot_s[kTableThreads];
  const int top = *t.free_top;
  const int i = static_cast<int>(threadIdx.x);
  const int slot = i < n ? slots[i] : 0;
  const int np = i < n ? t.npages[slot] : 0;
  int total = 0;
  const int pos = BlockExclusiveScan(np, scan, &total);
  pos_s[i] = i < n ? pos : total;
  slot_s[i] = slot;
  __syncthreads();
  // The slot holding released page g: the last s with pos_s[s] <= g.
  auto find = [&](int g) {
    int lo = 0, hi = n;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (pos_s[mid] <= g) lo = mid + 1; else hi = mid;
    }
    return lo - 1;
  };
  if (blockIdx.x == 0) {
    for (int g = i; g < total; g += blockDim.x) {
      const int s = find(g);
      t.free_stack[top + g] = t.pages[static_cast<size_t>(slot_s[s]) * t.max_pages + (g - pos_s[s])];
    }
  }
  if (clear) {
    for (int g = static_cast<int>(blockIdx.x); g < total; g += gridDim.x) {
      const int s = find(g);
      const int page = t.pages[static_cast<size_t>(slot_s[s]) * t.max_pages + (g - pos_s[s])];
      float4* sum = reinterpret_cast<float4*>(pool.summaries +
                                              static_cast<size_t>(page) * pool.elements);
      for (int e = i; e < pool.elements / 4; e += blockDim.x) {
        sum[e] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      }
      if (i == 0) {
        pool.token_counts[page] = 0;
        pool.live[page] = 0;
      }
    }
  }
}

__global__ __launch_bounds__(kTableThreads) void TableReleaseFinishKernel(
    TableView t, const int* __restrict__ slots, int n, ProgressMark mark) {
  __shared__ int scan[kTableWaves + 1];
  const int i = static_cast<int>(threadIdx.x);
  const int slot = i < n ? slots[i] : 0;
  const int np = i < n ? t.npages[slot] : 0;
  int total = 0;
  (void)BlockExclusiveScan(np, scan, &total);  // reads every count first
  if (i < n) t.npages[slot] = 0;
  if (i == 0) *t.free_top += total;
  // (the scan's barriers follow every thread's read of slots; the release
  // kernel before this one has finished reading them)
  if (i == 0) StoreProgress(mark);
}

}  // namespace

void LaunchTableReset(const TableView& t, int capacity, hipStream_t stream) {
  const int n = std::max(capacity, t.max_slots);
  const int groups = std::max(1, std::min(1024, (n + 255) / 256));
  hipLaunchKernelGGL(TableResetKernel, dim3(groups), dim3(256), 0, stream, t, capacity);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchTableReserve(const TableView& t, int slot, int n, hipStream_t stream) {
  if (n <= 0) return;
  hipLaunchKernelGGL(TableReserveKernel, dim3(1), dim3(kTableThreads),
                     static_cast<size_t>(n) * sizeof(int), stream, t, slot, n);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchTableScatter(const PoolView& pool, const TableView& t, int slot, int tokens,
                        const float* d_keys, const float* d_values, hipStream_t stream) {
  if (tokens <= 0) return;
  const size_t total = static_cast<size_t>(tokens) * (pool.elements / 4);
  const int groups = static_cast<int>(std::min<size_t>(2048, (total + 255) / 256));
  hipLaunchKernelGGL(TableScatterKernel, dim3(groups), dim3(256), 0, stream, pool, t, slot,
                     tokens, reinterpret_cast<const float4*>(d_keys),
                     reinterpret_cast<const float4*>(d_values));
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchTablePlanAppend(const PoolView& pool, const TableView& t, const int* args, int n,
                           int m, int* d_plan, int* d_order, hipStream_t stream,
                           ProgressMark mark) {
  if (n <= 0) return;
  hipLaunchKernelGGL(TablePlanAppendKernel, dim3(1), dim3(kTableThreads), 0, stream, pool, t,
                     args, n, m, d_plan, d_order, mark);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchTableRelease(const PoolView& pool, const TableView& t, const int* slots, int n,
                        int released_pages, bool clear, hipStream_t stream, ProgressMark mark) {
  if (n <= 0) return;
  if (n > kTableThreads) throw std::invalid_argument("at most 1024 slots per release launch");
  const int groups = clear ? std::max(1, std::min(256, released_pages)) : 1;
  hipLaunchKernelGGL(TableReleaseKernel, dim3(groups), dim3(kTableThreads), 0, stream, pool, t,
                     slots, n, clear ? 1 : 0);
  DSD_HIP_CHECK(hipGetLastError());
  hipLaunchKernelGGL(TableReleaseFinishKernel, dim3(1), dim3(kTableThreads), 0, stream, t, slots,
                     n, mark);
  DSD_HIP_CHECK(hipGetLastError());
}

void PreloadTableKernels() {
  PreloadKernel(TablePlanAppendKernel);
  PreloadKernel(TableReleaseKernel);
  PreloadKernel(TableReleaseFinishKernel);
  PreloadKernel(TableReserveKernel);
  PreloadKernel(TableScatterKernel);
}

}  // namespace dsdk
