// Ragged causal GQA attention over the paged KV cache.
//
// Work item = (packed row, KV head, context split). The G = Q/K query heads that share a
// KV head are handled together so every K/V element is read once per row. A split walks
// its positions in tiles of 256: K rows are scored by one thread each (G dot products),
// the tile's softmax statistics are reduced per head, and the value sum is accumulated by
// threads that own (head, dimension) pairs, reading V rows coalesced. Online softmax keeps
// (max, sum, acc) across tiles; the combine kernel merges splits and writes the
// O-projection operand (F-layout, hi and optional lo parts).
//
// Scores, softmax and accumulation are F32 (cpp/src/cpu/llama.cpp:67-112 semantics,
// cpp/src/cuda/stage.cpp:291-300: F32 scores and softmax); K/V are F16 or F32.
#include "kernels.hpp"

namespace hllm_rocm {
namespace {

constexpr int kThreads = 256;
constexpr int kTile = 256;
constexpr int kMaxPairs = 8;  // (head, dim) pairs per thread: G * D <= 2048

__device__ inline float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ inline float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ inline int split_length(int ctx, int max_splits, int unit) {
  int splits = (ctx + unit - 1) / unit;
  splits = splits < max_splits ? splits : max_splits;
  const int per = (ctx + splits - 1) / splits;
  return (per + 15) & ~15;
}

template <typename KV>
__global__ void __launch_bounds__(kThreads) attention_split_kernel(AttentionArgs a) {
  const int r = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;
  const int ctx = a.row_position[r] + 1;
  const int per = split_length(ctx, a.max_splits, a.split_unit);
  const int p0 = s * per;
  if (p0 >= ctx) return;
  const int p1 = min(ctx, p0 + per);
  const int D = a.head_dim, G = a.q_heads / a.kv_heads;
  const int seq = a.items[a.row_item[r]].sequence;
  const int32_t* table = a.block_table + (size_t)seq * a.table_width;
  const KV* pool = static_cast<const KV*>(a.kv.pool) + (uint64_t)a.layer * a.kv.layer_stride;
  const int bt = a.kv.block_tokens;
  const uint64_t head_stride = (uint64_t)bt * D;

  extern __shared__ float smem[];
  float* qs = smem;                 // [G][D]
  float* sc = qs + G * D;           // [G][kTile]
  float* stat = sc + G * kTile;     // [G] tile max, [G] rescale
  const int tid = threadIdx.x;
  for (int e = tid; e < G * D; e += kThreads) {
    qs[e] = a.q[((size_t)r * a.q_heads + kvh * G) * D + e];
  }
  // Thread-owned (head, dim) pairs: dim = tid % D, heads tid / D + k * (256 / D).
  const int my_d = tid % D;
  const int h_first = tid / D, h_step = kThreads / D > 0 ? kThreads / D : 1;
  float acc[kMaxPairs];
#pragma unroll
  for (int k = 0; k < kMaxPairs; ++k) acc[k] = 0.0f;
  float run_max[kMaxPairs], run_sum[kMaxPairs];
#pragma unroll
  for (int k = 0; k < kMaxPairs; ++k) {
    run_max[k] = -INFINITY;
    run_sum[k] = 0.0f;
  }
  __syncthreads();

  for (int t0 = p0; t0 < p1; t0 += kTile) {
    const int n = min(kTile, p1 - t0);
    if (tid < n) {
      const int p = t0 + tid;
      const KV* k = pool + ((uint64_t)table[p / bt] * 2 * a.kv_heads + kvh) * head_stride +
                    (uint64_t)(p % bt) * D;
      float dots[8];
#pragma unroll
      for (int g = 0; g < 8; ++g) dots[g] = 0.0f;
      for (int d = 0; d < D; ++d) {
        const float kv = (float)k[d];
#pragma unroll
        for (int g = 0; g < 8; ++g)
          if (g < G) dots[g] += qs[g * D + d] * kv;
      }
#pragma unroll
      for (int g = 0; g < 8; ++g)
        if (g < G) sc[g * kTile + tid] = dots[g] * a.scale;
    }
    __syncthreads();
    // Per-head tile maximum and exp: wave w handles heads w, w + 4, ...
    const int wave = tid >> 6, lane = tid & 63;
    for (int g = wave; g < G; g += kThreads / 64) {
      float m = -INFINITY;
      for (int i = lane; i < n; i += 64) m = fmaxf(m, sc[g * kTile + i]);
      m = wave_max(m);
      float sum = 0.0f;
      for (int i = lane; i < n; i += 64) {
        const float e = expf(sc[g * kTile + i] - m);
        sc[g * kTile + i] = e;
        sum += e;
      }
      sum = wave_sum(sum);
      if (lane == 0) {
        stat[g] = m;
        stat[G + g] = sum;
      }
    }
    __syncthreads();
    // Value accumulation with online rescaling.
#pragma unroll
    for (int k = 0; k < kMaxPairs; ++k) {
      const int g = h_first + k * h_step;
      if (tid < G * D && g < G && k * h_step * D + tid < G * D) {
        const float tile_max = stat[g];
        const float new_max = fmaxf(run_max[k], tile_max);
        const float old_scale = expf(run_max[k] - new_max);
        const float tile_scale = expf(tile_max - new_max);
        run_sum[k] = run_sum[k] * old_scale + stat[G + g] * tile_scale;
        run_max[k] = new_max;
        acc[k] *= old_scale;
        float part = 0.0f;
        for (int i = 0; i < n; ++i) {
          const int p = t0 + i;
          const KV* v = pool + (((uint64_t)table[p / bt] * 2 + 1) * a.kv_heads + kvh) * head_stride +
                        (uint64_t)(p % bt) * D;
          part += sc[g * kTile + i] * (float)v[my_d];
        }
        acc[k] += part * tile_scale;
      }
    }
    __syncthreads();
  }
  const int stride = D + 2;
#pragma unroll
  for (int k = 0; k < kMaxPairs; ++k) {
    const int g = h_first + k * h_step;
    if (tid < G * D && g < G && k * h_step * D + tid < G * D) {
      float* out = a.partial + (((size_t)r * a.q_heads + kvh * G + g) * a.max_splits + s) * stride;
      out[my_d] = acc[k];
      if (my_d == 0) {
        out[D] = run_max[k];
        out[D + 1] = run_sum[k];
      }
    }
  }
}

// One block per (row, query head): merge the splits, normalise, write the operand.
__global__ void attention_combine_kernel(AttentionArgs a) {
  const int r = blockIdx.x, qh = blockIdx.y;
  const int D = a.head_dim;
  const int ctx = a.row_position[r] + 1;
  const int per = split_length(ctx, a.max_splits, a.split_unit);
  const int splits = (ctx + per - 1) / per;
  const int stride = D + 2;
  const float* part = a.partial + ((size_t)r * a.q_heads + qh) * a.max_splits * stride;
  float m = -INFINITY;
  for (int s = 0; s < splits; ++s) m = fmaxf(m, part[s * stride + D]);
  float total = 0.0f;
  for (int s = 0; s < splits; ++s) total += part[s * stride + D + 1] * expf(part[s * stride + D] - m);
  const float inv = 1.0f / total;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float v = 0.0f;
    for (int s = 0; s < splits; ++s) v += part[s * stride + d] * expf(part[s * stride + D] - m);
    const float y = v * inv;
    const uint64_t at = flayout_index(r, (uint64_t)qh * D + d, a.out_cols_padded);
    const _Float16 hi = to_half(y);
    a.out_hi[at] = __builtin_bit_cast(uint16_t, hi);
    if (a.out_lo) a.out_lo[at] = __builtin_bit_cast(uint16_t, to_half((y - (float)hi) * kLoScale));
  }
  // Zero the operand's padded columns (their weights are zero; the values must be finite).
  if (qh == 0) {
    for (uint64_t c = (uint64_t)a.q_heads * D + threadIdx.x; c < a.out_cols_padded; c += blockDim.x) {
      const uint64_t at = flayout_index(r, c, a.out_cols_padded);
      a.out_hi[at] = 0;
      if (a.out_lo) a.out_lo[at] = 0;
    }
  }
}

}  // namespace

void launch_attention(hipStream_t stream, const AttentionArgs& a) {
  if (a.rows <= 0) return;
  const int G = a.q_heads / a.kv_heads;
  const size_t lds = ((size_t)G * a.head_dim + (size_t)G * kTile + 2 * G) * sizeof(float);
  dim3 grid(a.rows, a.kv_heads, a.max_splits);
  if (a.kv.f32)
    attention_split_kernel<float><<<grid, kThreads, lds, stream>>>(a);
  else
    attention_split_kernel<_Float16><<<grid, kThreads, lds, stream>>>(a);
  attention_combine_kernel<<<dim3(a.rows, a.q_heads), 128, 0, stream>>>(a);
}

}  // namespace hllm_rocm
