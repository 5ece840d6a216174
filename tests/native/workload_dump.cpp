// workload_dump.cpp -- prints this build's BuildSyntheticContinuousWorkload
// (libdsd.so) as one line per request: request_id arrival_step prompt_tokens
// decode_steps, then FNV-1a (64-bit) of the prompt keys, prompt values and
// initial query bytes.  The CPU suite compares it with the reference's own
// generator compiled in oracle/_ref (ref_workload_hashes).
//
// With a twelfth argument "tokens" it then prints, for a fixed set of
// (request, decode step, stream), "T id step stream" and the FNV-1a of the
// loop's decode payload (ContinuousTokenVector) of one token row.  The
// payload distribution follows DSD_PAYLOAD_DIST, as in the loop.
//
//   workload_dump heads head_dim page_size top_k requests window min_prompt
//                 max_prompt min_decode max_decode seed [tokens]
#include <cinttypes>
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "dsd/continuous_batching.h"
#include "dsd/step_observer.h"

namespace {

std::uint64_t Fnv1a(const std::vector<float>& v) {
  std::uint64_t h = 1469598103934665603ull;
  const auto* p = reinterpret_cast<const unsigned char*>(v.data());
  for (std::size_t i = 0; i < v.size() * sizeof(float); ++i) {
    h ^= p[i];
    h *= 1099511628211ull;
  }
  return h;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc != 12 && argc != 13) {
    std::fprintf(stderr, "usage: %s heads head_dim page_size top_k requests window "
                         "min_prompt max_prompt min_decode max_decode seed\n", argv[0]);
    return 2;
  }
  int v[11];
  for (int i = 0; i < 11; ++i) v[i] = std::atoi(argv[i + 1]);
  dsd::ModelConfig config;
  config.num_heads = v[0];
  config.head_dim = v[1];
  config.page_size = v[2];
  config.top_k_pages = v[3];
  const auto specs =
      dsd::BuildSyntheticContinuousWorkload(config, v[4], v[5], v[6], v[7], v[8], v[9], v[10]);
  for (const auto& s : specs) {
    std::printf("%d %d %d %d %" PRIu64 " %" PRIu64 " %" PRIu64 "\n", s.request_id,
                s.arrival_step, s.prompt_tokens, s.decode_steps, Fnv1a(s.prompt_keys),
                Fnv1a(s.prompt_values), Fnv1a(s.initial_query));
  }
  if (argc == 13) {
    const int E = v[0] * v[1];
    const int probes[][3] = {{0, 0, 0}, {0, 1, 1}, {5, 3, 2}, {127, 63, 0}, {3, 64, 1}};
    for (const auto& p : probes) {
      std::printf("T %d %d %d %" PRIu64 "\n", p[0], p[1], p[2],
                  Fnv1a(dsd::ContinuousTokenVector(E, p[0], p[1], p[2])));
    }
  }
  return 0;
}
