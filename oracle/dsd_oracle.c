/*
 * dsd_oracle.c -- CPU oracle (test infrastructure only; see dsd_oracle.h).
 *
 * Each function restates the reference's CPU algorithm in plain C and cites
 * the reference file:line it follows.  Built with -O3 -ffp-contract=off and no
 * -march so that float arithmetic rounds exactly as the reference build does.
 */
#include "dsd_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static double now_ms(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec * 1e3 + (double)ts.tv_nsec * 1e-6;
}

/* src/reference_kernels.cpp:70 */
float oracle_scale(int head_dim) {
  return 1.0f / sqrtf((float)head_dim);
}

/* src/paged_kv_cache.cpp:87-99 (same rule in src/device_page_pool.cpp:332-349) */
void oracle_page_summary(const float* keys, int token_count, int elements,
                         float* summary) {
  int i, t;
  for (i = 0; i < elements; ++i) summary[i] = 0.0f;
  if (token_count <= 0) return;
  for (t = 0; t < token_count; ++t) {
    const float* row = keys + (size_t)t * (size_t)elements;
    for (i = 0; i < elements; ++i) summary[i] += row[i];
  }
  {
    const float inv = 1.0f / (float)token_count;
    for (i = 0; i < elements; ++i) summary[i] *= inv;
  }
}

/* src/paged_kv_cache.cpp:231-238 (AppendToken; AppendTokenMetadataOnly
 * :299-306 is the same loop).  Pinned bit for bit against the reference's own
 * PagedKvCache compiled in oracle/_ref (tests/test_oracle.py,
 * test_append_summary_matches_compiled_reference). */
void oracle_append_summary(float* summary, const float* key, int old_count,
                           int elements) {
  const float old_c = (float)old_count;
  const float new_c = old_c + 1.0f;
  int i;
  for (i = 0; i < elements; ++i) {
    summary[i] = (summary[i] * old_c + key[i]) / new_c;
  }
}

/* src/reference_kernels.cpp:13-19 */
float oracle_dot(const float* a, const float* b, int count) {
  float acc = 0.0f;
  int i;
  for (i = 0; i < count; ++i) acc += a[i] * b[i];
  return acc;
}

/* src/reference_kernels.cpp:59-80; zero-count pages read as all-zero
 * summaries (src/paged_kv_cache.cpp:457-459). */
void oracle_score_pages(const float* query, const float* summaries,
                        const int* token_counts, const int* page_ids,
                        int num_candidates, int elements, float scale,
                        float* scores) {
  int c;
  for (c = 0; c < num_candidates; ++c) {
    const int page = page_ids[c];
    float dot;
    if (token_counts[page] == 0) {
      /* Dot against zeros: every product is +/-0 and acc stays +0 unless
       * q holds -0 products only; reproduce the sequence literally. */
      float acc = 0.0f;
      int i;
      for (i = 0; i < elements; ++i) acc += query[i] * 0.0f;
      dot = acc;
    } else {
      dot = oracle_dot(query, summaries + (size_t)page * (size_t)elements,
                       elements);
    }
    scores[c] = dot * scale;
  }
}

/* Comparator of src/reference_kernels.cpp:94-99: score descending, then
 * page id ascending; float == treats -0.0 and +0.0 as equal. */
static int better(float sa, int ia, float sb, int ib) {
  if (sa == sb) return ia < ib;
  return sa > sb;
}

/* src/reference_kernels.cpp:82-107.  std::partial_sort leaves the first
 * min(k, n) positions holding the smallest elements under the comparator in
 * sorted order; that prefix is fully determined by the strict weak order, so
 * an insertion-based top-k gives the same ids. */
int oracle_select_topk(const float* scores, const int* page_ids,
                       int num_candidates, int top_k, int* selected) {
  int kk, c, filled = 0;
  float* best_s;
  if (top_k <= 0 || num_candidates <= 0) return 0;
  kk = top_k < num_candidates ? top_k : num_candidates;
  best_s = (float*)malloc(sizeof(float) * (size_t)kk);
  for (c = 0; c < num_candidates; ++c) {
    const float s = scores[c];
    const int id = page_ids[c];
    int pos;
    if (filled == kk && !better(s, id, best_s[kk - 1], selected[kk - 1])) {
      continue;
    }
    pos = filled < kk ? filled : kk - 1;
    while (pos > 0 && better(s, id, best_s[pos - 1], selected[pos - 1])) {
      best_s[pos] = best_s[pos - 1];
      selected[pos] = selected[pos - 1];
      --pos;
    }
    best_s[pos] = s;
    selected[pos] = id;
    if (filled < kk) ++filled;
  }
  free(best_s);
  return kk;
}

/* src/reference_kernels.cpp:109-143 (gather) + :145-194 (attention) with
 * Softmax from :21-40. */
void oracle_attention(const float* query, const float* key_pool,
                      const float* value_pool, const int* token_counts,
                      const int* page_ids, int num_pages, int num_heads,
                      int head_dim, int page_size, float* output) {
  const int elements = num_heads * head_dim;
  const size_t page_elems = (size_t)page_size * (size_t)elements;
  const float scale = oracle_scale(head_dim);
  int total_tokens = 0, p, h, t, d;
  const float** krow;
  const float** vrow;
  float *logits, *weights;

  for (d = 0; d < elements; ++d) output[d] = 0.0f;
  for (p = 0; p < num_pages; ++p) total_tokens += token_counts[page_ids[p]];
  if (total_tokens == 0) return;

  /* The gather stage copies rows in (page order, token order); indexing the
   * pool rows in that order reads the same values. */
  krow = (const float**)malloc(sizeof(float*) * (size_t)total_tokens);
  vrow = (const float**)malloc(sizeof(float*) * (size_t)total_tokens);
  logits = (float*)malloc(sizeof(float) * (size_t)total_tokens);
  weights = (float*)malloc(sizeof(float) * (size_t)total_tokens);
  t = 0;
  for (p = 0; p < num_pages; ++p) {
    const int page = page_ids[p];
    const int count = token_counts[page];
    int j;
    for (j = 0; j < count; ++j) {
      krow[t] = key_pool + (size_t)page * page_elems + (size_t)j * elements;
      vrow[t] = value_pool + (size_t)page * page_elems + (size_t)j * elements;
      ++t;
    }
  }

  for (h = 0; h < num_heads; ++h) {
    const float* qh = query + (size_t)h * head_dim;
    float max_logit, sum = 0.0f;
    for (t = 0; t < total_tokens; ++t) {
      logits[t] = oracle_dot(qh, krow[t] + (size_t)h * head_dim, head_dim) *
                  scale;
    }
    /* std::max_element: the first maximal value. */
    max_logit = logits[0];
    for (t = 1; t < total_tokens; ++t) {
      if (max_logit < logits[t]) max_logit = logits[t];
    }
    for (t = 0; t < total_tokens; ++t) {
      weights[t] = expf(logits[t] - max_logit);
      sum += weights[t];
    }
    for (t = 0; t < total_tokens; ++t) weights[t] /= sum;
    for (t = 0; t < total_tokens; ++t) {
      const float w = weights[t];
      const float* v = vrow[t] + (size_t)h * head_dim;
      float* out = output + (size_t)h * head_dim;
      for (d = 0; d < head_dim; ++d) out[d] += w * v[d];
    }
  }
  free(krow);
  free(vrow);
  free(logits);
  free(weights);
}

/* src/decode_pipeline.cpp:13-46 */
int oracle_sparse_step(const float* query, const float* key_pool,
                       const float* value_pool, const float* summaries,
                       const int* token_counts, const int* candidate_ids,
                       int num_candidates, int num_heads, int head_dim,
                       int page_size, int top_k, float* scores, int* selected,
                       float* output) {
  const int elements = num_heads * head_dim;
  float* sc = scores;
  int* sel = selected;
  int kk;
  const int cap = top_k < num_candidates ? top_k : num_candidates;
  if (sc == NULL) sc = (float*)malloc(sizeof(float) * (size_t)(num_candidates + 1));
  if (sel == NULL) sel = (int*)malloc(sizeof(int) * (size_t)(cap > 0 ? cap : 1));
  oracle_score_pages(query, summaries, token_counts, candidate_ids,
                     num_candidates, elements, oracle_scale(head_dim), sc);
  kk = oracle_select_topk(sc, candidate_ids, num_candidates, top_k, sel);
  oracle_attention(query, key_pool, value_pool, token_counts, sel, kk,
                   num_heads, head_dim, page_size, output);
  if (scores == NULL) free(sc);
  if (selected == NULL) free(sel);
  return kk;
}

/* src/decode_pipeline.cpp:89-107 with the per-stage timers of :21-42. */
void oracle_sparse_batch(const float* queries, const float* key_pool,
                         const float* value_pool, const float* summaries,
                         const int* token_counts, const int* cand_offsets,
                         const int* cand_ids, int batch, int num_heads,
                         int head_dim, int page_size, int top_k, float* scores,
                         int* selected, int* counts, float* outputs,
                         double* stage_ms) {
  const int elements = num_heads * head_dim;
  const float scale = oracle_scale(head_dim);
  int r, max_n = 0;
  float* tmp_scores;
  int* tmp_sel;
  for (r = 0; r < batch; ++r) {
    const int n = cand_offsets[r + 1] - cand_offsets[r];
    if (n > max_n) max_n = n;
  }
  tmp_scores = (float*)malloc(sizeof(float) * (size_t)(max_n + 1));
  tmp_sel = (int*)malloc(sizeof(int) * (size_t)(top_k > 0 ? top_k : 1));
  for (r = 0; r < batch; ++r) {
    const int begin = cand_offsets[r];
    const int n = cand_offsets[r + 1] - begin;
    const float* q = queries + (size_t)r * elements;
    float* sc = scores ? scores + begin : tmp_scores;
    int kk;
    double t0 = now_ms(), t1, t2, t3;
    oracle_score_pages(q, summaries, token_counts, cand_ids + begin, n,
                       elements, scale, sc);
    t1 = now_ms();
    kk = oracle_select_topk(sc, cand_ids + begin, n, top_k, tmp_sel);
    t2 = now_ms();
    /* The gather stage is folded into oracle_attention, which reads the pool
     * rows in gather order; its time is reported under attention. */
    oracle_attention(q, key_pool, value_pool, token_counts, tmp_sel, kk,
                     num_heads, head_dim, page_size,
                     outputs + (size_t)r * elements);
    t3 = now_ms();
    if (selected && kk > 0) {
      memcpy(selected + (size_t)r * (size_t)top_k, tmp_sel,
             sizeof(int) * (size_t)kk);
    }
    if (counts) counts[r] = kk;
    if (stage_ms) {
      stage_ms[0] += t1 - t0;
      stage_ms[1] += t2 - t1;
      stage_ms[3] += t3 - t2;
    }
  }
  free(tmp_scores);
  free(tmp_sel);
}

/* src/reference_kernels.cpp:196-203 */
void oracle_dense_step(const float* query, const float* key_pool,
                       const float* value_pool, const int* token_counts,
                       const int* candidate_ids, int num_candidates,
                       int num_heads, int head_dim, int page_size,
                       float* output) {
  oracle_attention(query, key_pool, value_pool, token_counts, candidate_ids,
                   num_candidates, num_heads, head_dim, page_size, output);
}

/* src/reference_kernels.cpp:205-217 */
float oracle_max_abs_diff(const float* a, int64_t na, const float* b,
                          int64_t nb) {
  float diff = 0.0f;
  int64_t i;
  if (na != nb) return INFINITY;
  for (i = 0; i < na; ++i) {
    const float d = fabsf(a[i] - b[i]);
    if (d > diff) diff = d;
  }
  return diff;
}

/* ---- the serving loop's decode payloads --------------------------------- */

/* MT19937 (Matsumoto and Nishimura, ACM TOMACS 8(1), 1998), the engine of
 * std::mt19937: seeding by x_i = 1812433253 (x_{i-1} ^ (x_{i-1} >> 30)) + i,
 * then the twist and tempering of the paper. */
typedef struct {
  uint32_t mt[624];
  int next;
} oracle_mt;

static void oracle_mt_seed(oracle_mt* g, uint32_t seed) {
  int i;
  g->mt[0] = seed;
  for (i = 1; i < 624; ++i) {
    g->mt[i] = 1812433253u * (g->mt[i - 1] ^ (g->mt[i - 1] >> 30)) + (uint32_t)i;
  }
  g->next = 624;
}

static uint32_t oracle_mt_draw(oracle_mt* g) {
  uint32_t y;
  if (g->next >= 624) {
    int k;
    for (k = 0; k < 624; ++k) {
      y = (g->mt[k] & 0x80000000u) | (g->mt[(k + 1) % 624] & 0x7fffffffu);
      g->mt[k] = g->mt[(k + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908b0dfu : 0u);
    }
    g->next = 0;
  }
  y = g->mt[g->next++];
  y ^= y >> 11;
  y ^= (y << 7) & 0x9d2c5680u;
  y ^= (y << 15) & 0xefc60000u;
  y ^= y >> 18;
  return y;
}

void oracle_mt19937_draws(uint32_t seed, int count, uint32_t* out) {
  oracle_mt g;
  int i;
  oracle_mt_seed(&g, seed);
  for (i = 0; i < count; ++i) out[i] = oracle_mt_draw(&g);
}

/* src/continuous_batching.cpp:44-51 (MixSeed). */
uint32_t oracle_mix_seed(int request_id, int decode_step, int stream) {
  uint32_t x = 0x9e3779b9u;
  x ^= ((uint32_t)request_id + 0x85ebca6bu) + (x << 6) + (x >> 2);
  x ^= ((uint32_t)decode_step + 0xc2b2ae35u) + (x << 6) + (x >> 2);
  x ^= ((uint32_t)stream + 0x27d4eb2fu) + (x << 6) + (x >> 2);
  return x;
}

/* std::uniform_real_distribution<float>(-1, 1) on std::mt19937 as libstdc++
 * evaluates it: generate_canonical<float, 24> takes one 32-bit draw g and
 * returns fl(fl(g) / 2^32) (clamped below 1), and the distribution returns
 * fl(fl(u * 2) + -1) (src/continuous_batching.cpp:35-42 uses it). */
static float oracle_uniform_pm1(oracle_mt* g) {
  float u = (float)oracle_mt_draw(g) / 4294967296.0f;
  if (u >= 1.0f) u = nextafterf(1.0f, 0.0f);
  return u * 2.0f + -1.0f;
}

/* N(0, 1) floats by the Box-Muller transform on consecutive draw pairs
 * (a, b): u1 = (a + 1/2) 2^-32, u2 = b 2^-32, r = sqrt(-2 ln u1),
 * z0 = (float)(r cos(2 pi u2)), z1 = (float)(r sin(2 pi u2)), in double; an
 * odd count ends with a pair's z0.  The serving loop's N(0, 1) payload mode
 * (DSD_PAYLOAD_DIST=normal; the reference has no such mode, so this is the
 * restatement the loop's generator is checked against). */
static void oracle_normals(oracle_mt* g, int count, float* out) {
  int i;
  for (i = 0; i < count; i += 2) {
    const double u1 = ((double)oracle_mt_draw(g) + 0.5) * 0x1p-32;
    const double u2 = (double)oracle_mt_draw(g) * 0x1p-32;
    const double r = sqrt(-2.0 * log(u1));
    const double t = 6.283185307179586476925 * u2;
    out[i] = (float)(r * cos(t));
    if (i + 1 < count) out[i + 1] = (float)(r * sin(t));
  }
}

void oracle_token_vector_normal(int count, int request_id, int decode_step, int stream,
                                float* out) {
  oracle_mt g;
  oracle_mt_seed(&g, oracle_mix_seed(request_id, decode_step, stream));
  oracle_normals(&g, count, out);
}

void oracle_prompt_normal(int seed, int request_id, int prompt_tokens, int elements,
                          float* keys, float* values, float* query) {
  oracle_mt g;
  const int n = prompt_tokens * elements;
  oracle_mt_seed(&g, oracle_mix_seed(request_id, seed, 3));
  oracle_normals(&g, n, keys);
  oracle_normals(&g, n, values);
  oracle_normals(&g, elements, query);
}

/* DeterministicTokenVector (src/continuous_batching.cpp:53-59). */
void oracle_token_vector(int count, int request_id, int decode_step, int stream,
                         float* out) {
  oracle_mt g;
  int i;
  oracle_mt_seed(&g, oracle_mix_seed(request_id, decode_step, stream));
  for (i = 0; i < count; ++i) out[i] = oracle_uniform_pm1(&g);
}
