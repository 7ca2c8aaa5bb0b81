// Bandwidth-light kernels of a pass: ragged packing, embedding gather, F16 boundary
// codec, RMSNorm into GEMM operands, QK-norm + RoPE + paged KV append, greedy argmax,
// and checkpoint relayout. All are memory- or latency-bound; none reshapes work into GEMMs.
#include "kernels.hpp"

namespace hllm_rocm {

thread_local LaunchObserver* launch_observer = nullptr;
namespace {

constexpr int kBlock = 256;

__device__ inline float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ inline int wave_sum_int(int v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over the block's waves in a fixed order (deterministic); scratch holds a float per wave.
__device__ inline float block_sum(float v, float* scratch) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wave] = v;
  __syncthreads();
  float total = 0.0f;
  for (int w = 0; w < (int)(blockDim.x >> 6); ++w) total += scratch[w];
  __syncthreads();
  return total;
}

// ------------------------------------------------------------------ packing

// One block per item: its row offset and sampling rank are prefix sums over the items
// before it (item order = scheduler claim order).
__global__ void __launch_bounds__(kBlock) pack_kernel(const ItemMeta* items, int n_items,
                                                     const int32_t* host_tokens,
                                                     const int32_t* last_token,
                                                     const int32_t* block_table, int table_width,
                                                     int block_tokens, PackOut out) {
  __shared__ int scratch[4 * (2 + 2 * kAttnClasses)];
  const int i = blockIdx.x;
  // Prefix sums over the items before this one (rows, samples, attention work items per
  // dispatch class), and the attention work items of all items per class.
  int offset = 0, samples = 0, before[kAttnClasses] = {0, 0, 0}, all[kAttnClasses] = {0, 0, 0};
  for (int j = threadIdx.x; j < (out.attn_work ? n_items : i); j += blockDim.x) {
    int c[kAttnClasses] = {0, 0, 0};
    if (out.attn_work)
      attn_item_work_classes((int)items[j].query_tokens, (int)items[j].first_position, out.attn_group,
                             out.attn_max_splits, out.attn_decode_unit, out.attn_decode_split, c);
    for (int k = 0; k < kAttnClasses; ++k) all[k] += c[k];
    if (j < i) {
      offset += (int)items[j].query_tokens;
      samples += (items[j].flags & HLLM_ITEM_SAMPLE) ? 1 : 0;
      for (int k = 0; k < kAttnClasses; ++k) before[k] += c[k];
    }
  }
  int sums[2 + 2 * kAttnClasses] = {offset, samples, before[0], before[1], before[2], all[0], all[1], all[2]};
  const int wave = threadIdx.x >> 6;
  for (int k = 0; k < 2 + 2 * kAttnClasses; ++k) {
    sums[k] = wave_sum_int(sums[k]);
    if ((threadIdx.x & 63) == 0) scratch[4 * k + wave] = sums[k];
  }
  __syncthreads();
  for (int k = 0; k < 2 + 2 * kAttnClasses; ++k)
    sums[k] = scratch[4 * k] + scratch[4 * k + 1] + scratch[4 * k + 2] + scratch[4 * k + 3];
  offset = sums[0];
  samples = sums[1];
  // Next list slot of each class: the class's base (the classes before it, all items) plus
  // this class's work of the items before this one.
  int next[kAttnClasses] = {sums[2], sums[5] + sums[3], sums[5] + sums[6] + sums[4]};
  const int total = sums[5] + sums[6] + sums[7];
  const ItemMeta it = items[i];
  const bool sample = (it.flags & HLLM_ITEM_SAMPLE) != 0;
  if (threadIdx.x == 0) {
    if (i == 0) *out.flags = 0;
    out.cu_seqlens[i] = offset;
    if (sample) {
      out.sample_row[samples] = offset + (int)it.query_tokens - 1;
      out.sample_item[samples] = i;
    }
    if (i == n_items - 1) {
      out.cu_seqlens[n_items] = offset + (int)it.query_tokens;
      *out.sample_count = samples + (sample ? 1 : 0);
    }
  }
  const int32_t* table = block_table + (size_t)it.sequence * table_width;
  const int group = out.attn_group, qb = out.attn_work ? attn_block_rows(group) : 1;
  for (int j = threadIdx.x; j < (int)it.query_tokens; j += blockDim.x) {
    const int r = offset + j;
    const int position = (int)it.first_position + j;
    out.row_item[r] = i;
    out.row_position[r] = position;
    out.row_slot[r] = table[position / block_tokens] * block_tokens + position % block_tokens;
    out.row_token[r] = (it.flags & HLLM_ITEM_TOKEN_FROM_DEVICE) ? last_token[it.sequence]
                                                                 : host_tokens[r];
    if (out.attn_work) {
      // The key splits of the row's attention block (as the work items below count them).
      const int r0 = j / qb * qb, rows = min(qb, (int)it.query_tokens - r0);
      const int keys = (int)it.first_position + r0 + rows;
      const int per = attn_split_keys(keys, rows * group, out.attn_max_splits, out.attn_decode_unit, out.attn_decode_split);
      out.row_splits[r] = attn_merges_in_kernel(rows * group, out.attn_fold) ? 1 : (keys + per - 1) / per;
    }
  }
  // Attention blocks of this item: query rows [r0, r0 + rows) against keys [0, first + r0 + rows),
  // the last block (most keys) first (the rows' split counts are written above, one thread
  // per row). Wave 0 takes 64 blocks at a time, a lane per block in list order; a block's
  // first slot in its class is the class's next slot plus the splits of the lanes before
  // it in that class (a scan over the wave).
  if (out.attn_work && threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const int q = (int)it.query_tokens, first = (int)it.first_position;
    const int nblocks = (q + qb - 1) / qb;
    for (int k0 = 0; k0 < nblocks; k0 += 64) {
      const int k = k0 + lane;
      const bool valid = k < nblocks;
      const int r0 = valid ? (nblocks - 1 - k) * qb : 0;
      const int rows = min(qb, q - r0);
      const int keys = first + r0 + rows;
      const int per = attn_split_keys(keys, rows * group, out.attn_max_splits, out.attn_decode_unit, out.attn_decode_split);
      const int splits = valid ? (keys + per - 1) / per : 0;
      const int cls = attn_work_class(per, rows * group, out.attn_decode_unit);
#pragma unroll
      for (int c = 0; c < kAttnClasses; ++c) {
        const int mine = cls == c ? splits : 0;
        int incl = mine;
        for (int o = 1; o < 64; o <<= 1) {
          const int t = __shfl_up(incl, o, 64);
          if (lane >= o) incl += t;
        }
        if (mine > 0) {
          const int slot = next[c] + incl - mine;
          for (int sp = 0; sp < splits; ++sp)
            out.attn_work[slot + sp] = AttnWork{i, offset + r0, rows, first + r0, sp, splits, sp * per,
                                                min(keys, (sp + 1) * per)};
        }
        next[c] += __shfl(incl, 63, 64);
      }
    }
    if (i == n_items - 1 && lane == 0) *out.attn_count = total;
  }
}

// ------------------------------------------------------------------ embedding / boundary

__global__ void __launch_bounds__(kBlock) embed_kernel(const uint16_t* hi, const uint16_t* lo,
                                                      uint64_t cols_padded,
                                                      const int32_t* row_token, int hidden,
                                                      float* h) {
  const int r = blockIdx.x;
  const uint64_t id = (uint64_t)uniform_load(row_token + r);
  float* out = h + (size_t)r * hidden;
  for (int c = threadIdx.x * 8; c < hidden; c += blockDim.x * 8) {
    const uint64_t at = flayout_index(id, c, cols_padded);
    const half8 vh = *reinterpret_cast<const half8*>(hi + at);
    half8 vl = {};
    if (lo) vl = *reinterpret_cast<const half8*>(lo + at);
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (float)vh[j] + (float)vl[j] * kLoUnscale;
    if (c + 8 <= hidden && (hidden & 3) == 0) {  // two 16-byte stores
      *reinterpret_cast<floatx4*>(out + c) = floatx4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<floatx4*>(out + c + 4) = floatx4{v[4], v[5], v[6], v[7]};
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (c + j < hidden) out[c + j] = v[j];
    }
  }
}

__global__ void boundary_decode_kernel(const uint16_t* in, uint64_t n, float* h) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) h[i] = from_half_bits(in[i]);
}

__global__ void boundary_encode_kernel(const float* h, uint64_t n, uint16_t* out, int32_t* flags) {
  const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const uint16_t b = half_bits(h[i]);
  out[i] = b;
  if ((b & 0x7c00u) == 0x7c00u) atomicOr(flags, 4);
}

// ------------------------------------------------------------------ RMSNorm -> operand

__device__ inline void load8(const float* x, int c0, int hidden, bool vec, float* v) {
  if (vec && c0 < hidden) {
    const floatx4 a = *reinterpret_cast<const floatx4*>(x + c0);
    const floatx4 b = *reinterpret_cast<const floatx4*>(x + c0 + 4);
    v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
    v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = c0 + j < hidden ? x[c0 + j] : 0.0f;
  }
}
__device__ inline void load8_at(const float* x, float* v) {
  const floatx4 a = *reinterpret_cast<const floatx4*>(x);
  const floatx4 b = *reinterpret_cast<const floatx4*>(x + 4);
  v[0] = a[0]; v[1] = a[1]; v[2] = a[2]; v[3] = a[3];
  v[4] = b[0]; v[5] = b[1]; v[6] = b[2]; v[7] = b[3];
}

// One block per row; each thread owns Q chunks of 8 columns (blockDim = 64 * ceil(hidden /
// 512) threads, at most 1024; Q = 2 above 8192 columns) and keeps them in registers
// between the square sum and the scaled store. A row is a short chain of dependent steps,
// so the kernel is latency-bound:
// every load of a step (the chunks, or U K-split partials of every chunk) is issued
// unconditionally, at clamped addresses, before any is used; the launcher picks U for the
// partial count, so few clamped loads repeat the last partial.
template <int Q, int U>
__global__ void __launch_bounds__(1024) rmsnorm_flayout_kernel(
    float* h, int hidden, const int32_t* row_index, int rows, const int32_t* device_rows,
    const float* weight, float eps, uint16_t* out_hi, uint16_t* out_lo, uint64_t cols_padded,
    Partials residual) {
  __shared__ float scratch[16];
  const int r = blockIdx.x;
  // The row count and the row map were written by earlier launches: scalar loads.
  const int count = device_rows ? uniform_load(device_rows) : rows;
  if (r >= count) return;
  const int src = row_index ? uniform_load(row_index + r) : r;
  float* x = h + (size_t)src * hidden;
  float v[Q][8], wv[Q][8];
  int c0[Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) c0[q] = (threadIdx.x + q * blockDim.x) * 8;
  if ((hidden & 7) == 0) {
    int c[Q];  // clamped chunk columns
    // The norm weights first (they do not depend on the row), then the row.
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      c[q] = min(c0[q], hidden - 8);
      load8_at(weight + c[q], wv[q]);
    }
#pragma unroll
    for (int q = 0; q < Q; ++q) load8_at(x + c[q], v[q]);
    if (residual.parts > 0) {
      // The projection's K-split partials summed in split order from zero, then the
      // residual add (the order of the reduce kernel's residual epilogue), written back.
      float y[Q][8];
#pragma unroll
      for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int j = 0; j < 8; ++j) y[q][j] = 0.0f;
      const float* base = residual.data + (size_t)src * hidden;
      // U splits' loads in flight at once.
      for (int s0 = 0; s0 < residual.parts; s0 += U) {
        float p[U][Q][8];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int q = 0; q < Q; ++q)
            load8_at(base + (size_t)min(s0 + u, residual.parts - 1) * residual.stride + c[q], p[u][q]);
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int q = 0; q < Q; ++q)
#pragma unroll
            for (int j = 0; j < 8; ++j) y[q][j] = s0 + u < residual.parts ? y[q][j] + p[u][q][j] : y[q][j];
      }
#pragma unroll
      for (int q = 0; q < Q; ++q) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[q][j] += y[q][j];
        if (c0[q] < hidden) {
          *reinterpret_cast<floatx4*>(x + c0[q]) = floatx4{v[q][0], v[q][1], v[q][2], v[q][3]};
          *reinterpret_cast<floatx4*>(x + c0[q] + 4) = floatx4{v[q][4], v[q][5], v[q][6], v[q][7]};
        }
      }
    }
#pragma unroll
    for (int q = 0; q < Q; ++q)
      if (c0[q] >= hidden) {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[q][j] = 0.0f;
      }
  } else {
    // Hidden sizes that are not a multiple of 8 (test models): element-wise.
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
      for (int j = 0; j < 8; ++j) wv[q][j] = c0[q] + j < hidden ? weight[c0[q] + j] : 0.0f;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
      load8(x, c0[q], hidden, false, v[q]);
      if (residual.parts > 0 && c0[q] < hidden) {
        float y[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int s = 0; s < residual.parts; ++s) {
          float p[8];
          load8(residual.data + s * residual.stride + (size_t)src * hidden, c0[q], hidden, false, p);
#pragma unroll
          for (int j = 0; j < 8; ++j) y[j] += p[j];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          v[q][j] += y[j];
          if (c0[q] + j < hidden) x[c0[q] + j] = v[q][j];
        }
      }
    }
  }
  float squares = 0.0f;
#pragma unroll
  for (int q = 0; q < Q; ++q)
#pragma unroll
    for (int j = 0; j < 8; ++j) squares += v[q][j] * v[q][j];
  squares = block_sum(squares, scratch);
  const float inverse = 1.0f / sqrtf(squares / (float)hidden + eps);
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    if (c0[q] >= (int)cols_padded) continue;
    half8 vh, vl;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int cc = c0[q] + j;
      const float y = cc < hidden ? (v[q][j] * inverse) * wv[q][j] : 0.0f;
      vh[j] = to_half(y);
      vl[j] = to_half((y - (float)vh[j]) * kLoScale);
    }
    const uint64_t at = flayout_index(r, c0[q], cols_padded);
    *reinterpret_cast<half8*>(out_hi + at) = vh;
    if (out_lo) *reinterpret_cast<half8*>(out_lo + at) = vl;
  }
}

// ------------------------------------------------------------------ QK-norm + RoPE + KV append

__device__ inline uint64_t kv_index(const KvView& kv, int layer, int slot, int which, int head,
                                    int d) {
  const int block = slot / kv.block_tokens;
  const int offset = slot - block * kv.block_tokens;
  return which ? kv_value_index(kv, layer, (uint64_t)block, offset, head, d)
               : kv_key_index(kv, layer, (uint64_t)block, offset, head, d);
}

// A wave handles HB heads of a row at a time (heads head0 + k * stride). Lane l holds
// elements d = l + 64 j. Head dimensions are powers of two in [4, 256]: for D >= 128 both
// members of a rotate-half pair (d, d + D/2) sit in the same lane; for D <= 64 the partner
// is lane l ^ (D/2). PER: elements per lane, ceil(D / 64); U: K-split partials loaded per
// round. The kernel is a short latency-bound chain per head, so every load of the wave's HB
// heads (the partials of their first U K splits and their norm weights) and the row's RoPE
// factors are issued before any is used, unconditionally at valid addresses (lanes past D
// re-read element D - 1, heads past the last re-read the last head).
template <int PER, int U, int HB>
__global__ void __launch_bounds__(kBlock) qkv_rope_append_kernel(
    const float* qkv, int q_heads, int kv_heads, int head_dim, const float* q_norm,
    const float* k_norm, float eps, const float* rope_cos, const float* rope_sin,
    const int32_t* row_position, const int32_t* row_slot, KvView kv, int layer, float* q_out,
    Partials parts) {
  const int r = blockIdx.x;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, waves = blockDim.x >> 6;
  const int heads = q_heads + 2 * kv_heads;
  const int stride = waves * gridDim.y;
  const int head0 = blockIdx.y * waves + wave;
  const int D = head_dim, half = D / 2;
  constexpr int per_lane = PER;
  // The row's position and slot were written by the pack kernel: scalar loads.
  const int position = uniform_load(row_position + r);
  const int slot = uniform_load(row_slot + r);
  const float* row = qkv + (size_t)r * heads * D;
  const float* cos_row = rope_cos + (size_t)position * half;
  const float* sin_row = rope_sin + (size_t)position * half;
  int dd[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) dd[j] = min(lane + 64 * j, D - 1);
  // RoPE factors (the row's): for D >= 128 the lane's first-half elements lane + 64 j
  // (j < PER / 2), for D <= 64 element lane mod D / 2.
  float cr[PER], sr[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = D >= 128 ? min(lane + 64 * j, half - 1) : (lane & (half - 1));
    cr[j] = cos_row[e];
    sr[j] = sin_row[e];
  }
  for (int hb = head0; hb < heads; hb += HB * stride) {
    float p[HB][U][PER], wv[HB][PER];
#pragma unroll
    for (int k = 0; k < HB; ++k) {
      const int head = min(hb + k * stride, heads - 1);
      const size_t at = (size_t)r * heads * D + (size_t)head * D;
      if (parts.parts > 0) {
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int j = 0; j < PER; ++j)
            p[k][u][j] = parts.data[(size_t)min(u, parts.parts - 1) * parts.stride + at + dd[j]];
      } else {
#pragma unroll
        for (int j = 0; j < PER; ++j) p[k][0][j] = row[head * D + dd[j]];
      }
      const bool is_v = head >= q_heads + kv_heads;
      const float* w = head < q_heads ? q_norm : k_norm;
#pragma unroll
      for (int j = 0; j < PER; ++j) wv[k][j] = w && !is_v ? w[dd[j]] : 1.0f;
    }
#pragma unroll
    for (int k = 0; k < HB; ++k) {
      const int head = hb + k * stride;
      if (head >= heads) break;  // uniform over the wave
      const bool is_q = head < q_heads;
      const bool is_v = head >= q_heads + kv_heads;
      const float* w = is_q ? q_norm : k_norm;
      const size_t at = (size_t)r * heads * D + (size_t)head * D;
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      if (parts.parts > 0) {
        // K-split partials of the projection, summed in split order from zero (the reduce
        // kernel's order for a plain store).
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int j = 0; j < PER; ++j) v[j] = u < parts.parts ? v[j] + p[k][u][j] : v[j];
        for (int s0 = U; s0 < parts.parts; s0 += U) {  // splits past the first U
          float q[U][PER];
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int j = 0; j < PER; ++j)
              q[u][j] = parts.data[(size_t)min(s0 + u, parts.parts - 1) * parts.stride + at + dd[j]];
#pragma unroll
          for (int u = 0; u < U; ++u)
#pragma unroll
            for (int j = 0; j < PER; ++j) v[j] = s0 + u < parts.parts ? v[j] + q[u][j] : v[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < PER; ++j) v[j] = p[k][0][j];
      }
      float squares = 0.0f;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        if (lane + 64 * j >= D) v[j] = 0.0f;
        squares += v[j] * v[j];
      }
      if (!is_v) {
        if (w) {
          squares = wave_sum(squares);
          const float inverse = 1.0f / sqrtf(squares / (float)D + eps);
#pragma unroll
          for (int j = 0; j < PER; ++j) v[j] = v[j] * (inverse * wv[k][j]);  // lanes past D hold 0
        }
        if (D >= 128) {
          const int pairs = per_lane / 2;  // elements [0, pairs) are first halves
#pragma unroll
          for (int j = 0; j < 2; ++j) {
            if (j < pairs) {
              const float c = cr[j], s = sr[j];
              const float a = v[j], b = v[j + pairs];
              v[j] = a * c - b * s;
              v[j + pairs] = b * c + a * s;
            }
          }
        } else {
          const float partner = __shfl_xor(v[0], half, 64);
          if (lane < D) {
            const float c = cr[0], s = sr[0];
            if (lane < half)
              v[0] = v[0] * c - partner * s;
            else
              v[0] = v[0] * c + partner * s;
          }
        }
      }
      if (is_q) {
        float* dst = q_out + ((size_t)r * q_heads + head) * D;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = lane + 64 * j;
          if (j < per_lane && d < D) dst[d] = v[j];
        }
      } else {
        const int which = is_v ? 1 : 0;
        const int kvh = head - q_heads - (is_v ? kv_heads : 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int d = lane + 64 * j;
          if (j < per_lane && d < D) {
            const uint64_t at2 = kv_index(kv, layer, slot, which, kvh, d);
            if (kv.f32)
              static_cast<float*>(kv.pool)[at2] = v[j];
            else
              static_cast<_Float16*>(kv.pool)[at2] = to_half(v[j]);
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------ greedy argmax

__device__ inline Best wave_best(Best x) {
  for (int o = 32; o > 0; o >>= 1) {
    Best y{__shfl_xor(x.value, o, 64), __shfl_xor(x.index, o, 64)};
    x = better(x, y);
  }
  return x;
}

__global__ void __launch_bounds__(kBlock) argmax_partial_kernel(const float* logits,
                                                               const int32_t* device_rows, int cols,
                                                               int parts, float* part_val,
                                                               int32_t* part_idx, int32_t* flags) {
  __shared__ float sv[4];
  __shared__ int si[4];
  const int r = blockIdx.x, part = blockIdx.y;
  if (r >= *device_rows) return;
  // Parts of whole 4-column groups when the row allows 16-byte loads (the first maximum
  // does not depend on how the columns are dealt).
  const bool vec = (cols & 3) == 0 && ((uintptr_t)logits & 15) == 0;
  const int chunk = vec ? ((cols + parts - 1) / parts + 3) & ~3 : (cols + parts - 1) / parts;
  const int c0 = part * chunk, c1 = min(cols, c0 + chunk);
  const float* row = logits + (size_t)r * cols;
  Best best{-INFINITY, 0x7fffffff};
  bool bad = false;
  if (vec) {
    for (int c = c0 + 4 * (int)threadIdx.x; c < c1; c += 4 * (int)blockDim.x) {
      const floatx4 x = *reinterpret_cast<const floatx4*>(row + c);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        bad |= !isfinite(x[j]);
        best = better(best, Best{x[j], c + j});
      }
    }
  } else {
    for (int c = c0 + threadIdx.x; c < c1; c += blockDim.x) {
      const float x = row[c];
      bad |= !isfinite(x);
      best = better(best, Best{x, c});
    }
  }
  if (bad) atomicOr(flags, 2);
  best = wave_best(best);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    sv[wave] = best.value;
    si[wave] = best.index;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    Best b{sv[0], si[0]};
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) b = better(b, Best{sv[w], si[w]});
    part_val[(size_t)r * parts + part] = b.value;
    part_idx[(size_t)r * parts + part] = b.index;
  }
}

__global__ void argmax_final_kernel(const int32_t* device_rows, int parts, const float* part_val,
                                    const int32_t* part_idx, int32_t* tokens, const int32_t* sample_item,
                                    const ItemMeta* items, int32_t* last_token) {
  const int r = blockIdx.x;
  if (r >= *device_rows) return;
  Best best{-INFINITY, 0x7fffffff};
  for (int p = threadIdx.x; p < parts; p += 64) {
    best = better(best, Best{part_val[(size_t)r * parts + p], part_idx[(size_t)r * parts + p]});
  }
  best = wave_best(best);
  if (threadIdx.x == 0) {
    const int token = best.index == 0x7fffffff ? 0 : best.index;
    tokens[r] = token;
    if (last_token) last_token[items[sample_item[r]].sequence] = token;
  }
}

__global__ void record_tokens_kernel(const int32_t* tokens, const int32_t* sample_item,
                                     const int32_t* sample_count, const ItemMeta* items,
                                     int32_t* last_token) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j < *sample_count) last_token[items[sample_item[j]].sequence] = tokens[j];
}

// ------------------------------------------------------------------ checkpoint relayout

__device__ inline uint64_t splitmix64(uint64_t state) {
  uint64_t z = state + 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Irwin-Hall(12) approximation of N(0,1) from a counter-based SplitMix64 stream, then
// mean + n * sigma with one rounding per operation (no fused multiply-add).
__device__ inline float synth_value(uint64_t seed, uint64_t tensor_id, uint64_t index, float mean,
                                    float sigma) {
#pragma clang fp contract(off)
  const uint64_t base = (tensor_id << 40) + 3ull * index;
  int sum = 0;
#pragma unroll
  for (uint64_t j = 0; j < 3; ++j) {
    const uint64_t bits = splitmix64(seed + 0x9e3779b97f4a7c15ull * (base + j));
    sum += (int)(bits & 0xffffu) + (int)((bits >> 16) & 0xffffu) + (int)((bits >> 32) & 0xffffu) +
           (int)(bits >> 48);
  }
  const float n = (float)(sum + 6 - 6 * 65536) * (1.0f / 65536.0f);
  const float scaled = n * sigma;
  return mean + scaled;
}

__device__ inline float source_value(const RelayoutArgs& a, uint64_t r, uint64_t c) {
  const uint64_t i = r * a.cols + c;
  if (!a.src) {
    const float v = synth_value(a.seed, a.tensor_id, (a.row_base + r) * a.cols + c, a.mean, a.sigma);
    return a.src_dtype == HLLM_DTYPE_F16 ? (float)to_half(v) : v;
  }
  switch (a.src_dtype) {
    case HLLM_DTYPE_F32:
      return static_cast<const float*>(a.src)[i];
    case HLLM_DTYPE_F16:
      return from_half_bits(static_cast<const uint16_t*>(a.src)[i]);
    default: {
      const uint32_t w = (uint32_t) static_cast<const uint16_t*>(a.src)[i] << 16;
      return __builtin_bit_cast(float, w);
    }
  }
}

__global__ void __launch_bounds__(kBlock) relayout_kernel(RelayoutArgs a) {
  const uint64_t chunks_per_row = (a.cols + 7) / 8;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= a.rows * chunks_per_row) return;
  const uint64_t r = t / chunks_per_row;
  const uint64_t c0 = (t - r * chunks_per_row) * 8;
  int bad = 0;
  if (a.dst_f32) {  // vector weights keep F32 storage of the resident value
    for (uint64_t c = c0; c < c0 + 8 && c < a.cols; ++c) {
      float v = source_value(a, r, c);
      if (!isfinite(v)) bad |= 1;
      if (a.f16_resident) {
        const _Float16 h = to_half(v);
        if (!isfinite((float)h)) bad |= 4;
        v = (float)h;
      }
      a.dst_f32[(a.row_base + r) * a.cols + c] = v;
    }
  } else {
    const uint64_t tr = a.row_base + r;
    uint64_t dr = a.row_offset + tr;
    if (a.row_mode == 1) dr = a.row_offset + (tr / 32) * 64 + (tr % 32);
    if (a.row_mode == 2) dr = a.row_offset + (tr / 32) * 64 + 32 + (tr % 32);
    half8 vh = {}, vl = {};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (c0 + j < a.cols) {
        const float v = source_value(a, r, c0 + j);
        if (!isfinite(v)) bad |= 1;
        vh[j] = to_half(v);
        if (a.f16_resident && !isfinite((float)vh[j])) bad |= 4;
        vl[j] = to_half((v - (float)vh[j]) * kLoScale);
      }
    }
    const uint64_t at = flayout_index(dr, c0, a.dst_cols_padded);
    *reinterpret_cast<half8*>(a.dst_hi + at) = vh;
    if (a.dst_lo) *reinterpret_cast<half8*>(a.dst_lo + at) = vl;
  }
  if (bad) atomicOr(a.flags, bad);
}

// ------------------------------------------------------------------ read probe

// Streaming read of n 16-byte words, four loads in flight per thread per iteration; the
// sum is stored only if it equals a value it never takes, so that the loads stay.
__global__ void __launch_bounds__(256) read_probe_kernel(const floatx4* p, size_t n, float* out) {
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  for (; i + 3 * stride < n; i += 4 * stride) {
    const floatx4 a = p[i], b = p[i + stride], c = p[i + 2 * stride], d = p[i + 3 * stride];
    acc += a + b + c + d;
  }
  for (; i < n; i += stride) acc += p[i];
  if (acc[0] == -1234.5f) out[0] = acc[1];
}

// ------------------------------------------------------------------ MFMA rate probe

// Eight independent accumulation chains per wave of one F16 MFMA shape (16 = 16x16x32,
// 32 = 32x32x16), operands from registers: the issue rate of the matrix cores with no
// memory traffic. The sums are stored only if they equal a value they never take.
template <int SHAPE>
__global__ void __launch_bounds__(256) mfma_probe_kernel(int iters, float* out) {
  half8 a, b;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[j] = (_Float16)((threadIdx.x & 7) * 0.125f + j);
    b[j] = (_Float16)((threadIdx.x >> 3) * 0.0625f - j);
  }
  float total = 0.f;
  if constexpr (SHAPE == 16) {
    floatx4 acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) acc[k] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[k], 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) total += acc[k][0] + acc[k][3];
  } else {
    floatx16 acc[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[k][e] = 0.f;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
      for (int k = 0; k < 8; ++k) acc[k] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[k], 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) total += acc[k][0] + acc[k][15];
  }
  if (total == -1234.5f) out[0] = total;
}

}  // namespace

// ------------------------------------------------------------------ launchers

double launch_mfma_probe(hipStream_t stream, int shape, int blocks, int iters, float* out) {
  if (shape == 16) {
    observed("mfma_probe_kernel<16>", [&] { mfma_probe_kernel<16><<<blocks, 256, 0, stream>>>(iters, out); });
  } else {
    observed("mfma_probe_kernel<32>", [&] { mfma_probe_kernel<32><<<blocks, 256, 0, stream>>>(iters, out); });
  }
  // FLOPs: blocks x 4 waves x iters x 8 chains x (16 x 16 x 32 or 32 x 32 x 16) x 2.
  return (double)blocks * 4 * iters * 8 * (shape == 16 ? 16.0 * 16 * 32 : 32.0 * 32 * 16) * 2.0;
}

void launch_read_probe(hipStream_t stream, const void* p, size_t bytes, float* out) {
  observed("read_probe_kernel", [&] {
    read_probe_kernel<<<512, 256, 0, stream>>>(static_cast<const floatx4*>(p), bytes / 16, out);
  });
}

void launch_pack(hipStream_t stream, const ItemMeta* items, int n_items, const int32_t* host_tokens,
                 const int32_t* last_token, const int32_t* block_table, int table_width,
                 int block_tokens, PackOut out) {
  observed("pack_kernel", [&] { pack_kernel<<<n_items, kBlock, 0, stream>>>(items, n_items, host_tokens, last_token, block_table,
                                               table_width, block_tokens, out); });
}

void launch_embed(hipStream_t stream, const uint16_t* table_hi, const uint16_t* table_lo,
                  uint64_t cols_padded, const int32_t* row_token, int rows, int hidden, float* h) {
  observed("embed_kernel", [&] { embed_kernel<<<rows, kBlock, 0, stream>>>(table_hi, table_lo, cols_padded, row_token, hidden, h); });
}

void launch_boundary_decode(hipStream_t stream, const uint16_t* in, int rows, int hidden, float* h) {
  const uint64_t n = (uint64_t)rows * hidden;
  observed("boundary_decode_kernel", [&] { boundary_decode_kernel<<<(unsigned)((n + kBlock - 1) / kBlock), kBlock, 0, stream>>>(in, n, h); });
}

void launch_boundary_encode(hipStream_t stream, const float* h, int rows, int hidden, uint16_t* out,
                            int32_t* flags) {
  const uint64_t n = (uint64_t)rows * hidden;
  observed("boundary_encode_kernel", [&] { boundary_encode_kernel<<<(unsigned)((n + kBlock - 1) / kBlock), kBlock, 0, stream>>>(h, n, out,
                                                                                      flags); });
}

__global__ void __launch_bounds__(256) residual_sum_kernel(float* h, int64_t elements, Partials residual) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= elements) return;
  float y = 0.0f;
  for (int s = 0; s < residual.parts; ++s) y += residual.data[(size_t)s * residual.stride + e];
  h[e] += y;
}

void launch_residual_sum(hipStream_t stream, float* h, int rows, int hidden, Partials residual) {
  if (rows <= 0 || residual.parts <= 0) return;
  const int64_t elements = (int64_t)rows * hidden;
  observed("residual_sum_kernel", [&] {
    residual_sum_kernel<<<(unsigned)((elements + 255) / 256), 256, 0, stream>>>(h, elements, residual);
  });
}

void launch_rmsnorm_flayout(hipStream_t stream, float* h, int hidden, const int32_t* row_index,
                            int rows, const int32_t* device_rows, const float* weight, float eps,
                            uint16_t* out_hi, uint16_t* out_lo, uint64_t cols_padded,
                            Partials residual) {
  if (rows <= 0) return;
  // Chunks of 8 columns up to the padded width (the operand's zero padding is written too).
  const int chunks = (int)((std::max<uint64_t>(hidden, cols_padded) + 7) / 8);
  const int threads = std::min(1024, (chunks + 63) / 64 * 64);
  const auto go = [&](auto kernel, const char* name) {
    observed(name, [&] {
      kernel<<<rows, threads, 0, stream>>>(h, hidden, row_index, rows, device_rows, weight, eps, out_hi, out_lo,
                                           cols_padded, residual);
    });
  };
  if (chunks > 2 * 1024) fail(HLLM_INTERNAL, "hidden size exceeds the RMSNorm kernel");
  // Partial loads in flight per thread: the partial count rounded up to 4, 8, 12 or 16 (at
  // most sixteen, four when a thread holds two chunks; more partials take several rounds).
  const int parts = residual.parts;
  if (chunks > 1024)
    go(&rmsnorm_flayout_kernel<2, 4>, "rmsnorm_flayout_kernel<2, 4>");
  else if (parts <= 4)
    go(&rmsnorm_flayout_kernel<1, 4>, "rmsnorm_flayout_kernel<1, 4>");
  else if (parts <= 8)
    go(&rmsnorm_flayout_kernel<1, 8>, "rmsnorm_flayout_kernel<1, 8>");
  else if (parts <= 12)
    go(&rmsnorm_flayout_kernel<1, 12>, "rmsnorm_flayout_kernel<1, 12>");
  else
    go(&rmsnorm_flayout_kernel<1, 16>, "rmsnorm_flayout_kernel<1, 16>");
}

void launch_qkv_rope_append(hipStream_t stream, const float* qkv, int rows, int q_heads, int kv_heads,
                            int head_dim, const float* q_norm, const float* k_norm, float eps,
                            const float* rope_cos, const float* rope_sin, const int32_t* row_position,
                            const int32_t* row_slot, KvView kv, int layer, float* q_out,
                            Partials qkv_parts) {
  const int heads = q_heads + 2 * kv_heads;
  // Two partials per round when the projection has at most two (no clamped repeats), then
  // with three heads per wave (four waves per block: 16 waves per Qwen3 row of 48 heads;
  // 15.8 -> 14.1 us at 575 rows); four or eight partials per round (one round for up to
  // eight) and one head per wave otherwise (three heads per wave measured 10% slower there).
  const int parts = qkv_parts.parts;
  const bool two = parts <= 2;
  const int hb = two ? 3 : 1;
  const dim3 grid(rows, (heads + 4 * hb - 1) / (4 * hb));
  const auto go = [&](auto kernel) {
    observed("qkv_rope_append_kernel", [&] {
      kernel<<<grid, kBlock, 0, stream>>>(qkv, q_heads, kv_heads, head_dim, q_norm, k_norm, eps, rope_cos, rope_sin,
                                          row_position, row_slot, kv, layer, q_out, qkv_parts);
    });
  };
  if (head_dim <= 64)
    two ? go(&qkv_rope_append_kernel<1, 2, 3>) : parts <= 4 ? go(&qkv_rope_append_kernel<1, 4, 1>)
                                                              : go(&qkv_rope_append_kernel<1, 8, 1>);
  else if (head_dim <= 128)
    two ? go(&qkv_rope_append_kernel<2, 2, 3>) : parts <= 4 ? go(&qkv_rope_append_kernel<2, 4, 1>)
                                                              : go(&qkv_rope_append_kernel<2, 8, 1>);
  else if (head_dim <= 256)
    two ? go(&qkv_rope_append_kernel<4, 2, 3>) : parts <= 4 ? go(&qkv_rope_append_kernel<4, 4, 1>)
                                                              : go(&qkv_rope_append_kernel<4, 8, 1>);
  else
    fail(HLLM_INTERNAL, "head dimension exceeds the RoPE kernel");
}

void launch_argmax(hipStream_t stream, const float* logits, const int32_t* device_rows, int max_rows,
                   int cols, float* part_val, int32_t* part_idx, int parts, int32_t* tokens,
                   int32_t* flags, const int32_t* sample_item, const ItemMeta* items, int32_t* last_token) {
  if (max_rows <= 0) return;
  observed("argmax_partial_kernel", [&] { argmax_partial_kernel<<<dim3(max_rows, parts), kBlock, 0, stream>>>(logits, device_rows, cols,
                                                                      parts, part_val, part_idx,
                                                                      flags); });
  observed("argmax_final_kernel", [&] {
    argmax_final_kernel<<<max_rows, 64, 0, stream>>>(device_rows, parts, part_val, part_idx, tokens, sample_item, items,
                                                     last_token);
  });
}

void launch_argmax_final(hipStream_t stream, const int32_t* device_rows, int max_rows, int parts,
                         const float* part_val, const int32_t* part_idx, int32_t* tokens,
                         const int32_t* sample_item, const ItemMeta* items, int32_t* last_token) {
  if (max_rows <= 0) return;
  observed("argmax_final_kernel", [&] {
    argmax_final_kernel<<<max_rows, 64, 0, stream>>>(device_rows, parts, part_val, part_idx, tokens, sample_item, items,
                                                     last_token);
  });
}

void launch_record_tokens(hipStream_t stream, const int32_t* tokens, const int32_t* sample_item,
                          const int32_t* sample_count, const ItemMeta* items, int32_t* last_token) {
  observed("record_tokens_kernel", [&] { record_tokens_kernel<<<8, 128, 0, stream>>>(tokens, sample_item, sample_count, items, last_token); });
}

void launch_relayout(hipStream_t stream, const RelayoutArgs& a) {
  const uint64_t threads = a.rows * ((a.cols + 7) / 8);
  observed("relayout_kernel", [&] { relayout_kernel<<<(unsigned)((threads + kBlock - 1) / kBlock), kBlock, 0, stream>>>(a); });
}

}  // namespace hllm_rocm
