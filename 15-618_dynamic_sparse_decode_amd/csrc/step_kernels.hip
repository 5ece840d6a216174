// step_kernels.hip -- the three kernels of one sparse decode step (gfx950):
//   1. exact-order page scoring   (reference ScorePagesCpu, src/reference_kernels.cpp:59-80)
//   2. per-request top-k select   (reference SelectTopKPagesCpu, :82-107)
//   3. fused gather + attention   (reference GatherPagesCpu + SparseAttentionCpu, :109-194)
// Dense attention (reference DenseAttentionCpu, :196-203) reuses kernel 3
// with every candidate page as the list.
#include <cmath>

#include "dsd_internal.h"

namespace dsdk {
namespace {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// 1. Exact-order scoring.
//
// The reference scores a page as acc = 0; acc = fl(acc + fl(q[i]*s[i])) for
// i = 0..E-1, then fl(acc*scale).  That chain must be reproduced in order to
// keep page selection bit-exact, so one lane owns one candidate page and
// walks its summary row sequentially with separately rounded multiply and
// add (__fmul_rn / __fadd_rn; never contracted to FMA).  A wave covers 64
// candidates of one request, so the query operand is wave-uniform and is
// fetched through the scalar cache.
// ---------------------------------------------------------------------------
template <bool kVec4>
__global__ __launch_bounds__(kWave) void ScoreExactKernel(
    const float* __restrict__ queries, const float* __restrict__ summaries,
    const int* __restrict__ token_counts, const int* __restrict__ cand_offsets,
    const int* __restrict__ cand_ids, int E, float scale,
    float* __restrict__ scores) {
  const int r = blockIdx.y;
  const int begin = cand_offsets[r];
  const int end = cand_offsets[r + 1];
  const int first = begin + blockIdx.x * kWave;
  if (first >= end) return;
  const int c = first + static_cast<int>(threadIdx.x);
  const bool active = c < end;
  const int page = active ? cand_ids[c] : cand_ids[first];
  // A page holding no tokens reads as an all-zero summary
  // (src/paged_kv_cache.cpp:457-459); the products q*0 are still formed.
  const bool zero = !active || token_counts[page] == 0;
  const float* __restrict__ q = queries + static_cast<size_t>(r) * E;
  const float* __restrict__ s = summaries + static_cast<size_t>(page) * E;

  float acc = 0.0f;
  if constexpr (kVec4) {
#pragma unroll 8
    for (int i = 0; i < E; i += 4) {
      const float4 qv = *reinterpret_cast<const float4*>(q + i);
      float4 sv = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (!zero) sv = *reinterpret_cast<const float4*>(s + i);
      acc = __fadd_rn(acc, __fmul_rn(qv.x, sv.x));
      acc = __fadd_rn(acc, __fmul_rn(qv.y, sv.y));
      acc = __fadd_rn(acc, __fmul_rn(qv.z, sv.z));
      acc = __fadd_rn(acc, __fmul_rn(qv.w, sv.w));
    }
  } else {
    for (int i = 0; i < E; ++i) {
      const float sv = zero ? 0.0f : s[i];
      acc = __fadd_rn(acc, __fmul_rn(q[i], sv));
    }
  }
  if (active) scores[c] = __fmul_rn(acc, scale);
}

// ---------------------------------------------------------------------------
// 2. Top-k select.
//
// Each candidate becomes one 64-bit key whose unsigned order is the
// reference's comparator: high word = order-preserving image of the score
// (-0.0 folded onto +0.0, since the reference compares with ==), low word =
// ~page_id so that a smaller id wins a tie.  One workgroup bitonic-sorts a
// request's keys descending in LDS and emits the first min(k, n) ids.
// ---------------------------------------------------------------------------
constexpr int kSelectMaxKeys = 8192;  // 64 KiB of LDS

__device__ __forceinline__ uint64_t SelectKey(float score, int page_id) {
  uint32_t bits = __float_as_uint(score);
  if (bits == 0x80000000u) bits = 0u;
  const uint32_t ord = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
  return (static_cast<uint64_t>(ord) << 32) |
         static_cast<uint64_t>(0xFFFFFFFFu - static_cast<uint32_t>(page_id));
}

__device__ __forceinline__ int KeyPage(uint64_t key) {
  return static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(key & 0xFFFFFFFFull));
}

__global__ __launch_bounds__(256) void SelectTopKKernel(
    const float* __restrict__ scores, const int* __restrict__ cand_offsets,
    const int* __restrict__ cand_ids, int top_k, int* __restrict__ selected,
    int* __restrict__ counts) {
  extern __shared__ uint64_t keys[];
  const int r = blockIdx.x;
  const int begin = cand_offsets[r];
  const int n = cand_offsets[r + 1] - begin;
  const int kk = top_k <= 0 ? 0 : (top_k < n ? top_k : n);
  if (kk == 0) {
    if (threadIdx.x == 0) counts[r] = 0;
    return;
  }
  int m = 1;
  int log_m = 0;
  while (m < n) {
    m <<= 1;
    ++log_m;
  }
  for (int i = threadIdx.x; i < m; i += blockDim.x) {
    keys[i] = i < n ? SelectKey(scores[begin + i], cand_ids[begin + i]) : 0ull;
  }
  __syncthreads();
  const int half = m >> 1;
  for (int log_size = 1; log_size <= log_m; ++log_size) {
    const int size = 1 << log_size;
    for (int log_stride = log_size - 1; log_stride >= 0; --log_stride) {
      const int stride = 1 << log_stride;
      for (int i = threadIdx.x; i < half; i += blockDim.x) {
        const int lo = ((i >> log_stride) << (log_stride + 1)) | (i & (stride - 1));
        const int hi = lo + stride;
        const bool descending = (lo & size) == 0;
        const uint64_t a = keys[lo];
        const uint64_t b = keys[hi];
        if ((a < b) == descending) {
          keys[lo] = b;
          keys[hi] = a;
        }
      }
      __syncthreads();
    }
  }
  int* out = selected + static_cast<size_t>(r) * top_k;
  for (int i = threadIdx.x; i < kk; i += blockDim.x) out[i] = KeyPage(keys[i]);
  if (threadIdx.x == 0) counts[r] = kk;
}

// ---------------------------------------------------------------------------
// 3. Fused gather + softmax attention (flash-decoding inside a workgroup).
//
// Workgroup = (head h, request r); its waves stride over 16-token chunks of
// the request's page list.  Lane (g, j) = (lane/4, lane%4) owns token slot g
// of the chunk and the j-th quarter of the head's dims, so a 4-lane group
// reads one 4*DQ-float K row and one V row (contiguous, vectorised).  Each
// lane keeps its own online-softmax stream (m, l, acc[DQ]) over the tokens
// it sees: the only per-token cross-lane traffic is the 2-step dot-product
// reduction within the group.  Streams are merged once at the end: across
// the 16 token slots with xor shuffles, across waves through LDS.  Logits
// live in the log2 domain (q pre-scaled by scale*log2 e) so each exponential
// is one v_exp_f32.
// ---------------------------------------------------------------------------
constexpr int kAttnWaves = 4;
constexpr int kAttnThreads = kAttnWaves * kWave;
constexpr int kChunk = 16;
constexpr float kLog2e = 1.4426950408889634f;

template <int DQ>
__device__ __forceinline__ void LoadDims(const float* __restrict__ p,
                                         float (&v)[DQ]) {
  if constexpr (DQ % 4 == 0) {
#pragma unroll
    for (int i = 0; i < DQ / 4; ++i) {
      const float4 x = reinterpret_cast<const float4*>(p)[i];
      v[4 * i + 0] = x.x;
      v[4 * i + 1] = x.y;
      v[4 * i + 2] = x.z;
      v[4 * i + 3] = x.w;
    }
  } else if constexpr (DQ % 2 == 0) {
#pragma unroll
    for (int i = 0; i < DQ / 2; ++i) {
      const float2 x = reinterpret_cast<const float2*>(p)[i];
      v[2 * i + 0] = x.x;
      v[2 * i + 1] = x.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < DQ; ++i) v[i] = p[i];
  }
}

__device__ __forceinline__ float Exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// DQ > 0: head_dim == 4*DQ, lane j covers dims [j*DQ, (j+1)*DQ).
// DQ == 0: generic head_dim <= 256, lane j covers dims j, j+4, j+8, ...
template <int DQ>
__global__ __launch_bounds__(kAttnThreads) void AttentionKernel(
    PoolView pool, AttentionArgs args) {
  constexpr int kRegs = DQ > 0 ? DQ : 64;
  const int h = blockIdx.x;
  const int r = blockIdx.y;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int g = lane >> 2;
  const int j = lane & 3;
  const int D = pool.head_dim;
  const int E = pool.elements;
  const int ps = pool.page_size;

  int start, count;
  if (args.list_stride > 0) {
    start = r * args.list_stride;
    count = args.list_counts[r];
  } else {
    start = args.list_offsets[r];
    count = args.list_offsets[r + 1] - start;
  }

  const int nd = DQ > 0 ? DQ : (D - j + 3) / 4;
  const int dim0 = DQ > 0 ? j * DQ : j;
  const int dstep = DQ > 0 ? 1 : 4;
  const int head_off = h * D + dim0;

  float q[kRegs];
  float acc[kRegs];
  {
    const float qscale = args.scale * kLog2e;
    const float* qp = args.queries + static_cast<size_t>(r) * E + head_off;
    if constexpr (DQ > 0) {
      LoadDims<DQ>(qp, q);
    } else {
#pragma unroll
      for (int i = 0; i < kRegs; ++i) q[i] = i < nd ? qp[i * dstep] : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < kRegs; ++i) {
      q[i] *= qscale;
      acc[i] = 0.0f;
    }
  }

  float m = -INFINITY;
  float l = 0.0f;
  const int total = count * ps;
  for (int base = wave * kChunk; base < total; base += kAttnWaves * kChunk) {
    const int f = base + g;
    bool valid = false;
    float kv[kRegs];
    float vv[kRegs];
    if (f < total) {
      const int slot = f / ps;
      const int t = f - slot * ps;
      const int page = args.list_ids[start + slot];
      valid = t < pool.token_counts[page];
      if (valid) {
        const size_t off = static_cast<size_t>(page) * pool.page_elems +
                           static_cast<size_t>(t) * E + head_off;
        if constexpr (DQ > 0) {
          LoadDims<DQ>(pool.keys + off, kv);
          LoadDims<DQ>(pool.values + off, vv);
        } else {
#pragma unroll
          for (int i = 0; i < kRegs; ++i) {
            kv[i] = i < nd ? pool.keys[off + i * dstep] : 0.0f;
            vv[i] = i < nd ? pool.values[off + i * dstep] : 0.0f;
          }
        }
      }
    }
    float dot = 0.0f;
    if (valid) {
#pragma unroll
      for (int i = 0; i < kRegs; ++i) dot = fmaf(q[i], kv[i], dot);
    }
    dot += __shfl_xor(dot, 1, kWave);
    dot += __shfl_xor(dot, 2, kWave);
    if (valid) {
      const float m_new = fmaxf(m, dot);
      const float alpha = Exp2(m - m_new);
      const float beta = Exp2(dot - m_new);
      l = fmaf(l, alpha, beta);
#pragma unroll
      for (int i = 0; i < kRegs; ++i) acc[i] = fmaf(acc[i], alpha, beta * vv[i]);
      m = m_new;
    }
  }

  // Merge the 16 token-slot streams of this wave (lanes differing in g).
  float wm = m;
#pragma unroll
  for (int o = 4; o < kWave; o <<= 1) wm = fmaxf(wm, __shfl_xor(wm, o, kWave));
  const float sc = (m == -INFINITY) ? 0.0f : Exp2(m - wm);
  float wl = l * sc;
#pragma unroll
  for (int i = 0; i < kRegs; ++i) acc[i] *= sc;
#pragma unroll
  for (int o = 4; o < kWave; o <<= 1) {
    wl += __shfl_xor(wl, o, kWave);
#pragma unroll
    for (int i = 0; i < kRegs; ++i) acc[i] += __shfl_xor(acc[i], o, kWave);
  }

  // Merge the waves through LDS: s_acc[wave][D], s_m/s_l[wave].
  extern __shared__ float smem[];
  float* s_m = smem;
  float* s_l = smem + kAttnWaves;
  float* s_acc = smem + 2 * kAttnWaves;
  if (g == 0) {
    if (j == 0) {
      s_m[wave] = wm;
      s_l[wave] = wl;
    }
#pragma unroll
    for (int i = 0; i < kRegs; ++i) {
      if (i < nd) s_acc[wave * D + dim0 + i * dstep] = acc[i];
    }
  }
  __syncthreads();
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < kAttnWaves; ++w) mx = fmaxf(mx, s_m[w]);
  float* out = args.outputs + static_cast<size_t>(r) * E + static_cast<size_t>(h) * D;
  for (int d = threadIdx.x; d < D; d += kAttnThreads) {
    float lt = 0.0f;
    float at = 0.0f;
    if (mx != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kAttnWaves; ++w) {
        const float s = (s_m[w] == -INFINITY) ? 0.0f : Exp2(s_m[w] - mx);
        lt = fmaf(s_l[w], s, lt);
        at = fmaf(s_acc[w * D + d], s, at);
      }
    }
    // No valid token at all: the reference returns zeros
    // (src/cuda/sparse_batched_attention.cu:364-369; CPU :159-161).
    out[d] = lt == 0.0f ? 0.0f : at / lt;
  }
}

template <int DQ>
void LaunchAttentionT(const PoolView& pool, const AttentionArgs& args,
                      hipStream_t stream) {
  const size_t lds = sizeof(float) * (2 * kAttnWaves + kAttnWaves * pool.head_dim);
  hipLaunchKernelGGL(AttentionKernel<DQ>, dim3(pool.num_heads, args.batch),
                     dim3(kAttnThreads), lds, stream, pool, args);
}

}  // namespace

void LaunchScoreExact(const PoolView& pool, const float* d_queries,
                      const int* d_cand_offsets, const int* d_cand_ids,
                      int batch, int max_candidates, float scale,
                      float* d_scores, hipStream_t stream) {
  if (batch <= 0 || max_candidates <= 0) return;
  const dim3 grid((max_candidates + kWave - 1) / kWave, batch);
  if (pool.elements % 4 == 0) {
    hipLaunchKernelGGL(ScoreExactKernel<true>, grid, dim3(kWave), 0, stream,
                       d_queries, pool.summaries, pool.token_counts,
                       d_cand_offsets, d_cand_ids, pool.elements, scale, d_scores);
  } else {
    hipLaunchKernelGGL(ScoreExactKernel<false>, grid, dim3(kWave), 0, stream,
                       d_queries, pool.summaries, pool.token_counts,
                       d_cand_offsets, d_cand_ids, pool.elements, scale, d_scores);
  }
  DSD_HIP_CHECK(hipGetLastError());
}

int SelectMaxCandidates() { return kSelectMaxKeys; }

void LaunchSelectTopK(const float* d_scores, const int* d_cand_offsets,
                      const int* d_cand_ids, int batch, int max_candidates,
                      int top_k, int* d_selected, int* d_counts,
                      hipStream_t stream) {
  if (batch <= 0) return;
  int m = 1;
  while (m < max_candidates) m <<= 1;
  if (m > kSelectMaxKeys) {
    throw std::invalid_argument(
        "candidate pages per request exceed the top-k select limit of " +
        std::to_string(kSelectMaxKeys));
  }
  int threads = m / 2;
  if (threads < kWave) threads = kWave;
  if (threads > 256) threads = 256;
  hipLaunchKernelGGL(SelectTopKKernel, dim3(batch), dim3(threads),
                     sizeof(uint64_t) * static_cast<size_t>(m), stream, d_scores,
                     d_cand_offsets, d_cand_ids, top_k, d_selected, d_counts);
  DSD_HIP_CHECK(hipGetLastError());
}

void LaunchAttention(const PoolView& pool, const AttentionArgs& args,
                     hipStream_t stream) {
  if (args.batch <= 0 || pool.num_heads <= 0) return;
  const int D = pool.head_dim;
  if (D <= 0 || D > 256) {
    throw std::invalid_argument("head_dim must be in (0, 256]");
  }
  switch (D % 4 == 0 ? D / 4 : 0) {
    case 1: LaunchAttentionT<1>(pool, args, stream); break;
    case 2: LaunchAttentionT<2>(pool, args, stream); break;
    case 4: LaunchAttentionT<4>(pool, args, stream); break;
    case 8: LaunchAttentionT<8>(pool, args, stream); break;
    case 16: LaunchAttentionT<16>(pool, args, stream); break;
    case 20: LaunchAttentionT<20>(pool, args, stream); break;
    case 32: LaunchAttentionT<32>(pool, args, stream); break;
    case 64: LaunchAttentionT<64>(pool, args, stream); break;
    default: LaunchAttentionT<0>(pool, args, stream); break;
  }
  DSD_HIP_CHECK(hipGetLastError());
}

}  // namespace dsdk
