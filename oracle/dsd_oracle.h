/*
 * dsd_oracle.h -- CPU oracle for the batched page-level sparse decode step.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * CPU path (`sparse_cpu` / `dense_cpu`), used by tests/, by
 * __graft_entry__.smoke() and by the cpu_baseline leg of bench.py as the
 * checker.  Nothing in the product library links, loads or calls it.
 *
 * Build: gcc -O3 -ffp-contract=off (no -march), so every float multiply and
 * add rounds separately, exactly as the reference's default x86-64 build
 * does (no FMA in the baseline ISA, no reassociation without -ffast-math).
 *
 * Layout (reference src/page_pool.cpp:58-59, src/paged_kv_cache.cpp:24-27):
 *   key_pool / value_pool  float[capacity][page_size][E], E = heads*head_dim
 *   summaries              float[capacity][E]
 *   token_counts           int[capacity]
 */
#ifndef DSD_ORACLE_H_
#define DSD_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 1.0f / sqrtf((float)head_dim)  (src/reference_kernels.cpp:70). */
float oracle_scale(int head_dim);

/* Page summary, host rule: s = 0; s += k[t] in token order; s *= fl(1/c).
 * (src/paged_kv_cache.cpp:87-99; src/device_page_pool.cpp:332-349).
 * token_count == 0 gives an all-zero summary. */
void oracle_page_summary(const float* keys, int token_count, int elements,
                         float* summary);

/* Running-mean update for one appended token:
 *   s[i] = (s[i] * old + k[i]) / (old + 1)   (src/paged_kv_cache.cpp:231-238). */
void oracle_append_summary(float* summary, const float* key, int old_count,
                           int elements);

/* Sequential dot product, acc += a[i]*b[i] (src/reference_kernels.cpp:13-19). */
float oracle_dot(const float* a, const float* b, int count);

/* Page scoring (src/reference_kernels.cpp:59-80):
 *   scores[c] = Dot(query, summary[page_ids[c]], E) * scale.
 * A candidate page whose token_count is 0 scores against an all-zero summary
 * (CopyPageSummary, src/paged_kv_cache.cpp:457-459). */
void oracle_score_pages(const float* query, const float* summaries,
                        const int* token_counts, const int* page_ids,
                        int num_candidates, int elements, float scale,
                        float* scores);

/* Top-k (src/reference_kernels.cpp:82-107): the first min(k, n) page ids in
 * (score descending, page id ascending) order; -0.0 == +0.0 is a tie.
 * k <= 0 or n == 0 selects nothing.  Returns the number written. */
int oracle_select_topk(const float* scores, const int* page_ids,
                       int num_candidates, int top_k, int* selected);

/* Gather + attention for one request (src/reference_kernels.cpp:109-194):
 * gathers the listed pages in order (token_count tokens each), then per head
 * logits = Dot(q_h, k_t, D) * scale, softmax with max subtraction and a
 * sequential sum, out += w * v.  No tokens gives an all-zero output. */
void oracle_attention(const float* query, const float* key_pool,
                      const float* value_pool, const int* token_counts,
                      const int* page_ids, int num_pages, int num_heads,
                      int head_dim, int page_size, float* output);

/* One full sparse_cpu step for one request (src/decode_pipeline.cpp:13-46):
 * score, select, gather+attend.  scores (num_candidates) and selected
 * (min(k, n)) may be NULL.  Returns the number of selected pages. */
int oracle_sparse_step(const float* query, const float* key_pool,
                       const float* value_pool, const float* summaries,
                       const int* token_counts, const int* candidate_ids,
                       int num_candidates, int num_heads, int head_dim,
                       int page_size, int top_k, float* scores, int* selected,
                       float* output);

/* Batched sparse_cpu over CSR candidates (src/decode_pipeline.cpp:89-107).
 * selected is laid out [B][top_k] (unused slots untouched); counts[B]
 * receives min(k, n_r).  Per-stage wall times (ms) are accumulated into
 * stage_ms[0..3] = score, top-k, gather, attention when stage_ms != NULL. */
void oracle_sparse_batch(const float* queries, const float* key_pool,
                         const float* value_pool, const float* summaries,
                         const int* token_counts, const int* cand_offsets,
                         const int* cand_ids, int batch, int num_heads,
                         int head_dim, int page_size, int top_k, float* scores,
                         int* selected, int* counts, float* outputs,
                         double* stage_ms);

/* dense_cpu for one request (src/reference_kernels.cpp:196-203). */
void oracle_dense_step(const float* query, const float* key_pool,
                       const float* value_pool, const int* token_counts,
                       const int* candidate_ids, int num_candidates,
                       int num_heads, int head_dim, int page_size,
                       float* output);

/* Max-abs difference; +inf if sizes differ (src/reference_kernels.cpp:205-217). */
float oracle_max_abs_diff(const float* a, int64_t na, const float* b,
                          int64_t nb);

/* ---- the serving loop's decode payloads (src/continuous_batching.cpp) -- */

/* The first `count` outputs of std::mt19937 seeded with `seed` (MT19937,
 * Matsumoto and Nishimura 1998). */
void oracle_mt19937_draws(uint32_t seed, int count, uint32_t* out);

/* MixSeed(request_id, decode_step, stream) (src/continuous_batching.cpp:44-51). */
uint32_t oracle_mix_seed(int request_id, int decode_step, int stream);

/* DeterministicTokenVector (src/continuous_batching.cpp:53-59): `count`
 * draws of std::uniform_real_distribution<float>(-1, 1) (as libstdc++
 * evaluates it) from std::mt19937(MixSeed(request_id, decode_step, stream)).
 * Stream 0 = the next query (decode_step + 1 for the query after step
 * decode_step), 1 = the appended key, 2 = the appended value
 * (:294-306, :596-633). */
void oracle_token_vector(int count, int request_id, int decode_step, int stream,
                         float* out);

/* The serving loop's N(0, 1) payload mode (DSD_PAYLOAD_DIST=normal; no
 * reference counterpart): Box-Muller on pairs of std::mt19937 draws
 * (u1 = (a + 1/2) 2^-32, u2 = b 2^-32, r = sqrt(-2 ln u1), r cos / r sin of
 * 2 pi u2, in double).  Decode tokens: from mt19937(MixSeed(request_id,
 * decode_step, stream)), as oracle_token_vector.  Prompt payloads of request
 * r: keys (prompt_tokens * elements), values, then the initial query, from
 * one mt19937(MixSeed(r, seed, 3)). */
void oracle_token_vector_normal(int count, int request_id, int decode_step, int stream,
                                float* out);
void oracle_prompt_normal(int seed, int request_id, int prompt_tokens, int elements,
                          float* keys, float* values, float* query);

#ifdef __cplusplus
}
#endif

#endif /* DSD_ORACLE_H_ */
