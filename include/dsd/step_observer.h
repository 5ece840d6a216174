// step_observer.h -- a verification hook into the continuous-batching
// serving loop: after each sampled decode step the loop hands the step's
// inputs (requests, their decode-step indices, page lists and queries) and
// what the device returned (selected page ids, outputs) to a callback.
//
// No reference counterpart: the reference's RunContinuousSparseDecode
// (src/continuous_batching.cpp:392-741) returns statistics only, so a loop's
// per-step results could not otherwise be checked against sparse_cpu.
#pragma once

#include <functional>
#include <vector>

#include "dsd/types.h"

namespace dsd {

struct ObservedDecodeStep {
  int step = 0;                      // the loop's step counter
  int elements = 0;                  // E = num_heads * head_dim
  std::vector<int> request_ids;      // [B], in batch order
  std::vector<int> decode_steps;     // [B]: decode_step_index of this step
  std::vector<int> context_tokens;   // [B]
  std::vector<int> cand_offsets;     // [B + 1]
  std::vector<PageId> cand_ids;      // each request's pages, logical order
  std::vector<float> queries;        // [B][E]
  std::vector<int> selected_counts;  // [B]
  std::vector<PageId> selected;      // compact, in rank order
  std::vector<float> outputs;        // [B][E]
};

using ContinuousStepObserver = std::function<void(const ObservedDecodeStep&)>;

// RunContinuousSparseDecode calls `observer` after every `every`-th decode
// step (its 0th, every-th, ...) of loops started afterwards; an empty
// observer or every <= 0 turns it off.  Observed steps return their outputs
// and ids even in the no-outputs mode.  Not thread-safe: set it before the
// loop starts.
void SetContinuousStepObserver(ContinuousStepObserver observer, int every);

// The decode payload the serving loop generates for (request, decode step,
// stream): stream 0 = the query after that step, 1 = the appended key, 2 =
// the appended value.  The reference's DeterministicTokenVector
// (src/continuous_batching.cpp:53-59), U(-1, 1) on std::mt19937(MixSeed);
// N(0, 1) by Box-Muller on the same engine when DSD_PAYLOAD_DIST=normal.
std::vector<float> ContinuousTokenVector(int count, int request_id, int decode_step, int stream);

}  // namespace dsd
