// pcie_peak.cpp -- the host link's measured copy rates (test infrastructure):
// the roofline a PCIe-bound serving loop is measured against.  Large copies
// of `mib` MiB each way, timed with events over `reps` repetitions after one
// warm-up: host -> device from pinned memory (hipHostMalloc) and from
// pageable memory (malloc, every page touched first), and device -> host
// into pinned memory.  Prints key=value lines, best and mean GB/s (1e9 B/s).
//
//   pcie_peak [mib=256] [reps=10]
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace {

void Check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    std::fprintf(stderr, "%s failed: %s\n", what, hipGetErrorString(e));
    std::exit(1);
  }
}

void Measure(const char* name, void* dst, const void* src, size_t bytes, hipMemcpyKind kind,
             int reps, hipStream_t s) {
  hipEvent_t a, b;
  Check(hipEventCreate(&a), "hipEventCreate");
  Check(hipEventCreate(&b), "hipEventCreate");
  Check(hipMemcpyAsync(dst, src, bytes, kind, s), "warm-up copy");
  Check(hipStreamSynchronize(s), "hipStreamSynchronize");
  std::vector<double> gbps;
  for (int r = 0; r < reps; ++r) {
    Check(hipEventRecord(a, s), "hipEventRecord");
    Check(hipMemcpyAsync(dst, src, bytes, kind, s), "copy");
    Check(hipEventRecord(b, s), "hipEventRecord");
    Check(hipEventSynchronize(b), "hipEventSynchronize");
    float ms = 0.f;
    Check(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
    gbps.push_back(static_cast<double>(bytes) / (ms * 1e-3) / 1e9);
  }
  double mean = 0.0;
  for (double g : gbps) mean += g;
  mean /= static_cast<double>(gbps.size());
  std::printf("%s_best_gbps=%.2f\n%s_mean_gbps=%.2f\n", name,
              *std::max_element(gbps.begin(), gbps.end()), name, mean);
  Check(hipEventDestroy(a), "hipEventDestroy");
  Check(hipEventDestroy(b), "hipEventDestroy");
}

}  // namespace

int main(int argc, char** argv) {
  const size_t mib = argc > 1 ? static_cast<size_t>(std::atol(argv[1])) : 256;
  const int reps = argc > 2 ? std::atoi(argv[2]) : 10;
  const size_t bytes = mib << 20;
  std::printf("copy_bytes=%zu\nreps=%d\n", bytes, reps);
  hipStream_t s;
  Check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  void* dev = nullptr;
  void* pinned = nullptr;
  Check(hipMalloc(&dev, bytes), "hipMalloc");
  Check(hipHostMalloc(&pinned, bytes, hipHostMallocDefault), "hipHostMalloc");
  std::memset(pinned, 1, bytes);
  char* pageable = static_cast<char*>(std::malloc(bytes));
  if (pageable == nullptr) return 1;
  std::memset(pageable, 1, bytes);
  Measure("h2d_pinned", dev, pinned, bytes, hipMemcpyHostToDevice, reps, s);
  Measure("h2d_pageable", dev, pageable, bytes, hipMemcpyHostToDevice, reps, s);
  Measure("d2h_pinned", pinned, dev, bytes, hipMemcpyDeviceToHost, reps, s);
  std::free(pageable);
  Check(hipHostFree(pinned), "hipHostFree");
  Check(hipFree(dev), "hipFree");
  Check(hipStreamDestroy(s), "hipStreamDestroy");
  return 0;
}
