// ref_loop_harness.cpp -- extern "C" probe of the reference's serving-loop
// generators.
//
// TEST INFRASTRUCTURE ONLY.  The reference's src/continuous_batching.cpp is
// compiled as part of this translation unit (oracle/Makefile passes its path
// as REF_CONTINUOUS_SRC; nothing is copied), so that the helpers it keeps in
// an unnamed namespace -- MixSeed and DeterministicTokenVector (:44-59), the
// per-step decode payloads of the loop (:294-306, :596-633) -- can be
// called.  Tests pin the oracle's restatement (oracle_mix_seed,
// oracle_token_vector) and the product's workload generator against them.
#include <cstdint>
#include <cstring>
#include <vector>

#include REF_CONTINUOUS_SRC

namespace {

// FNV-1a (64-bit) over the bytes of a float vector: a fingerprint that
// changes with any bit of any value.
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

extern "C" {

unsigned ref_mix_seed(int request_id, int decode_step, int stream) {
  return dsd::MixSeed(request_id, decode_step, stream);
}

void ref_token_vector(int count, int request_id, int decode_step, int stream, float* out) {
  const auto v = dsd::DeterministicTokenVector(count, request_id, decode_step, stream);
  std::memcpy(out, v.data(), sizeof(float) * v.size());
}

// BuildSyntheticContinuousWorkload (:336-381) in its sorted order: meta is
// [n][4] = request_id, arrival_step, prompt_tokens, decode_steps; hashes is
// [n][3] = FNV-1a of the prompt keys, prompt values and initial query.
int ref_workload_hashes(int heads, int head_dim, int page_size, int top_k, int num_requests,
                        int window, int min_prompt, int max_prompt, int min_decode,
                        int max_decode, int seed, int* meta, std::uint64_t* hashes) {
  dsd::ModelConfig config;
  config.num_heads = heads;
  config.head_dim = head_dim;
  config.page_size = page_size;
  config.top_k_pages = top_k;
  const auto specs = dsd::BuildSyntheticContinuousWorkload(
      config, num_requests, window, min_prompt, max_prompt, min_decode, max_decode, seed);
  for (std::size_t i = 0; i < specs.size(); ++i) {
    const auto& s = specs[i];
    meta[4 * i + 0] = s.request_id;
    meta[4 * i + 1] = s.arrival_step;
    meta[4 * i + 2] = s.prompt_tokens;
    meta[4 * i + 3] = s.decode_steps;
    hashes[3 * i + 0] = Fnv1a(s.prompt_keys);
    hashes[3 * i + 1] = Fnv1a(s.prompt_values);
    hashes[3 * i + 2] = Fnv1a(s.initial_query);
  }
  return static_cast<int>(specs.size());
}

}  // extern "C"
