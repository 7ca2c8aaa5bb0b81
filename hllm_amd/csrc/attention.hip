// Ragged causal GQA attention over the paged KV cache.
//
// F16 KV, head_dim in {64, 128, 256}: MFMA flash attention. A work item is a block of up
// to 64 query vectors (query rows x the G query heads that share one KV head) against one
// split of its key range, for one KV head. Scores are computed transposed, S^T = K Q^T
// (v_mfma_f32_16x16x32_f16 with a cached key fragment as the A operand, loaded straight
// from the paged cache), so that each lane holds four positions of one query vector; the
// probabilities of 32 positions then form the B operand of O^T = V^T P directly in
// registers: both operands list the positions in the same k-slot order (keys are stored in
// operand order with their rows permuted so a lane's scores are 8 consecutive positions, and
// the values are stored transposed per block, so each V^T row segment is one 16-byte load). Online softmax runs in
// F32 per query vector. Blocks of at most 16 vectors (decode rows) let the four waves
// interleave 32-key tiles and merge through LDS; larger blocks give each wave 16 vectors.
//
// F32 KV (F32 execution) or other head dims: the F32 VALU kernel, one work item per
// (row, KV head, split), one thread per key for the scores and coalesced value reads.
//
// Splits of one query block are merged by the combine kernel. Scores, softmax and
// accumulation are F32 (cpp/src/cpu/llama.cpp:67-112; cpp/src/cuda/stage.cpp:291-300).
#include "kernels.hpp"

#include <algorithm>

namespace hllm_rocm {
namespace {


constexpr int kThreads = 256;
constexpr int kTile = 256;
constexpr int kMaxPairs = 8;  // (head, dim) pairs per thread: G * D <= 2048

__device__ inline floatx4 mfma(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ inline float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
// exp(m - reference) with the empty-softmax convention: a -inf maximum contributes nothing.
__device__ inline float rescale(float m, float reference) {
  return m == -INFINITY ? 0.0f : expf(m - reference);
}
// The MFMA kernel keeps scores in base 2 (log2 e folded into the query scale): 2^x is one
// v_exp_f32, which also maps -inf to 0.
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
__device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline float* partial_at(const AttentionArgs& a, int row, int qh, int split) {
  return a.partial + (((size_t)row * a.q_heads + qh) * a.max_splits + split) * (a.head_dim + 2);
}

template <int E, bool kCoherent>
__device__ inline void merge_splits(const AttentionArgs& a, int r, int qh, int splits, int lane);

// ---------------------------------------------------------------- MFMA flash attention

// LDS of the MFMA kernel: the split-key merge uses [128 + 4 * D * 16] floats; fused decode
// rows stage after it their query vectors [16][D] F32 and the row's own key and value
// [2][D] F16.
template <int D>
constexpr int kFusedBase = 128 + 4 * D * 16;

// Fused decode rows (AttentionRope), D = 128: lane l holds elements l and l + 64, the two
// halves of a rotate-half pair. Each of the item's G query heads (and, for the item holding
// the row's own position, its key and value) is computed in the order of
// qkv_rope_append_kernel: the projection's K-split partials summed in split order from
// zero, QK-norm v * (inv * w), then RoPE; the key and value are rounded to F16, appended to
// the cache at the row's slot and staged; the query vectors are staged in F32. A wave takes
// its jobs two at a time and issues every load of both (the first four partial splits, the
// norm weights, the RoPE factors and the slot) before any arithmetic: the phase is one memory
// round trip per pair instead of three per job. Called by every thread of the workgroup (it
// holds the workgroup's barrier).
template <int D>
__device__ void fused_projection(const AttentionArgs& a, const AttnWork& w, int kvh, int G, int wave, int lane,
                                 bool holds_self) {
  extern __shared__ float smem[];
  constexpr int kWaves = kThreads / 64;
  float* qs = smem + kFusedBase<D>;
  _Float16* self_kv = reinterpret_cast<_Float16*>(qs + 16 * D);
  const AttentionRope& rp = a.rope;
  const int heads = a.q_heads + 2 * a.kv_heads;
  const size_t row_at = (size_t)w.row0 * heads * D;
  const int jobs = G + (holds_self ? 2 : 0);
  const int parts = rp.parts.parts;
  const float c = rp.rope_cos[(size_t)w.position0 * (D / 2) + lane];
  const float sn = rp.rope_sin[(size_t)w.position0 * (D / 2) + lane];
  const int slot = holds_self ? uniform_load(rp.row_slot + w.row0) : 0;
  for (int job0 = wave; job0 < jobs; job0 += 2 * kWaves) {  // wave-uniform
    // Job k of the pair is job0 + k * kWaves; a second job past the last one repeats the
    // last one's loads and writes nothing.
    int job[2];
    bool is_q[2], is_v[2];
    size_t at[2];
    float p[2][4][2], nwv[2][2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      job[k] = min(job0 + k * kWaves, jobs - 1);
      is_q[k] = job[k] < G;
      is_v[k] = job[k] == G + 1;
      const int head = is_q[k] ? kvh * G + job[k] : a.q_heads + (is_v[k] ? a.kv_heads : 0) + kvh;
      at[k] = row_at + (size_t)head * D + lane;
      if (parts > 0) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int j = 0; j < 2; ++j) p[k][u][j] = rp.parts.data[(size_t)min(u, parts - 1) * rp.parts.stride + at[k] + 64 * j];
      } else {
#pragma unroll
        for (int j = 0; j < 2; ++j) p[k][0][j] = rp.qkv[at[k] + 64 * j];
      }
      const float* nw = is_q[k] ? rp.q_norm : rp.k_norm;
#pragma unroll
      for (int j = 0; j < 2; ++j) nwv[k][j] = nw && !is_v[k] ? nw[lane + 64 * j] : 1.0f;
    }
    float x[2][2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        if (parts > 0) {
          x[k][j] = 0.0f;
#pragma unroll
          for (int u = 0; u < 4; ++u) x[k][j] = u < parts ? x[k][j] + p[k][u][j] : x[k][j];
        } else {
          x[k][j] = p[k][0][j];
        }
      }
      for (int s0 = 4; s0 < parts; s0 += 4) {  // splits past the first four (none on most shapes)
        float q[4][2];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int j = 0; j < 2; ++j) q[u][j] = rp.parts.data[(size_t)min(s0 + u, parts - 1) * rp.parts.stride + at[k] + 64 * j];
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int j = 0; j < 2; ++j) x[k][j] = s0 + u < parts ? x[k][j] + q[u][j] : x[k][j];
      }
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if (!is_v[k]) {
        if (is_q[k] ? rp.q_norm : rp.k_norm) {
          float squares = 0.0f;
#pragma unroll
          for (int j = 0; j < 2; ++j) squares += x[k][j] * x[k][j];
          squares = wave_sum(squares);
          const float inverse = 1.0f / sqrtf(squares / (float)D + rp.eps);
#pragma unroll
          for (int j = 0; j < 2; ++j) x[k][j] = x[k][j] * (inverse * nwv[k][j]);
        }
        const float x0 = x[k][0], x1 = x[k][1];
        x[k][0] = x0 * c - x1 * sn;
        x[k][1] = x1 * c + x0 * sn;
      }
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if (job0 + k * kWaves >= jobs) continue;
      if (is_q[k]) {
        qs[job[k] * D + lane] = x[k][0];
        qs[job[k] * D + lane + 64] = x[k][1];
      } else {
        const int which = is_v[k] ? 1 : 0;
        const int block = slot / a.kv.block_tokens, offset = slot - block * a.kv.block_tokens;
        _Float16* pool = static_cast<_Float16*>(a.kv.pool);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int d = lane + 64 * j;
          const _Float16 h = to_half(x[k][j]);
          self_kv[which * D + d] = h;
          pool[which ? kv_value_index(a.kv, a.layer, (uint64_t)block, offset, kvh, d)
                     : kv_key_index(a.kv, a.layer, (uint64_t)block, offset, kvh, d)] = h;
        }
      }
    }
  }
  __syncthreads();
}

// The own-key score of vector g of a fused item (the F16 scaled query times the F16 key,
// summed in F32), from the vectors and key staged by fused_projection; called by a whole wave.
template <int D>
__device__ float own_key_score(int g, int lane, float qscale) {
  extern __shared__ float smem[];
  const float* qs = smem + kFusedBase<D>;
  const _Float16* self_kv = reinterpret_cast<const _Float16*>(qs + 16 * D);
  float part = 0.0f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int d = lane + 64 * j;
    part += (float)to_half(qs[g * D + d] * qscale) * (float)self_kv[d];
  }
  return wave_sum(part);
}

// Three workgroups per CU for D <= 128: decode-like blocks hold one K/V tile per wave at a
// time (registers for a second one would allow only two), so that more work items are in
// flight for about the same bytes in flight.
template <int D>
__global__ void __launch_bounds__(kThreads, D <= 128 ? 3 : 1) attention_mfma_kernel(AttentionArgs a) {
  constexpr int KK = D / 32;  // 32-wide chunks of the QK contraction
  constexpr int DF = D / 16;  // 16-row fragments of O^T
  extern __shared__ float smem[];
  // Workgroups loop over (work item, KV head) pairs, KV heads innermost so that the
  // dispatch follows the list's order (the list's size is written by the pack kernel); a
  // launch may have fewer workgroups than pairs.
  const int count = uniform_load(a.work_count) * a.kv_heads;
  for (int idx = blockIdx.x; idx < count; idx += gridDim.x) {
  [&] {
  const int wi = idx / a.kv_heads, kvh = idx - wi * a.kv_heads;
  AttnWork w;
  {
    const int32_t* wp = reinterpret_cast<const int32_t*>(a.work + wi);
    w = AttnWork{uniform_load(wp), uniform_load(wp + 1), uniform_load(wp + 2), uniform_load(wp + 3),
                 uniform_load(wp + 4), uniform_load(wp + 5), uniform_load(wp + 6), uniform_load(wp + 7)};
  }
  const int G = a.q_heads / a.kv_heads;
  const int nvec = w.rows * G;
  const bool split_keys = nvec <= 16;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int quad = lane >> 4, col = lane & 15;
  const int vf = split_keys ? 0 : wave;
  const int v = vf * 16 + col;
  const bool v_ok = v < nvec;
  const int vr = v / G, vg = v - vr * G;
  const int my_pos = w.position0 + vr;
  const int seq = uniform_load(&a.items[w.item].sequence);
  const int bt = a.kv.block_tokens, KVH = a.kv_heads;
  // Waves whose vectors lie past the block's end still stage K/V tiles and meet the
  // barriers of the prefill path; their results are never written.
  // A tile's physical block: a wave-uniform table entry, read through the scalar cache so
  // that waiting for it never drains the vector loads of the tile in flight. Tiles are
  // 32-key aligned and blocks a multiple of 32 keys, so a tile lies in one block.
  const int32_t* table = a.block_table + (size_t)seq * a.table_width;
  auto block_of = [&](int logical) -> uint64_t {
    return (uint64_t)(uint32_t)uniform_load(table + __builtin_amdgcn_readfirstlane(logical));
  };
  const _Float16* pool = static_cast<const _Float16*>(a.kv.pool) + (uint64_t)a.layer * a.kv.layer_stride;
  // Fused decode rows (AttentionRope): the item holding the row's own position takes that
  // key from registers, so its tiles end one position earlier.
  const bool fused = D == 128 && a.rope.qkv != nullptr;
  const bool holds_self = fused && w.key_end == w.position0 + 1;
  const int key_end = holds_self ? w.key_end - 1 : w.key_end;
  const _Float16* self_kv = reinterpret_cast<const _Float16*>(smem + kFusedBase<D> + 16 * D);  // fused: [2][D]

  // Q^T as the B operand (1/sqrt(D) and log2 e folded in): lane holds Q[v][32 kk + 8 quad + j].
  const float qscale = a.scale * kLog2e;
  half8 qf[KK];
  if constexpr (D == 128) {
    if (fused) fused_projection<D>(a, w, kvh, G, wave, lane, holds_self);
  }
  if (fused) {
    // The scaled vectors staged by fused_projection, read as 16-byte vectors whether or not
    // the lane's vector exists (a conditional read per element would be 32 dependent LDS
    // round trips).
    const float* qrow = smem + kFusedBase<D> + (v_ok ? vg : 0) * D;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const floatx4 x0 = *reinterpret_cast<const floatx4*>(qrow + 32 * kk + 8 * quad);
      const floatx4 x1 = *reinterpret_cast<const floatx4*>(qrow + 32 * kk + 8 * quad + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qf[kk][j] = v_ok ? to_half(x0[j] * qscale) : (_Float16)0.0f;
        qf[kk][4 + j] = v_ok ? to_half(x1[j] * qscale) : (_Float16)0.0f;
      }
    }
  } else {
    const float* qrow = a.q + ((size_t)(w.row0 + (v_ok ? vr : 0)) * a.q_heads + kvh * G + vg) * D;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const floatx4 x0 = *reinterpret_cast<const floatx4*>(qrow + 32 * kk + 8 * quad);
      const floatx4 x1 = *reinterpret_cast<const floatx4*>(qrow + 32 * kk + 8 * quad + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qf[kk][j] = v_ok ? to_half(x0[j] * qscale) : (_Float16)0.0f;
        qf[kk][4 + j] = v_ok ? to_half(x1[j] * qscale) : (_Float16)0.0f;
      }
    }
  }
  floatx4 o[DF];
#pragma unroll
  for (int df = 0; df < DF; ++df) o[df] = floatx4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;

  // K and V fragments of one 32-key tile.
  struct Tile {
    half8 k0[KK], k1[KK];
    half8 v[DF];
  };
  auto fetch = [&](int t, uint64_t blk, Tile& f) {
    const int off = t % bt;
    const _Float16* kb = pool + ((blk * 2 * KVH + kvh) * bt + off) * D;
    const _Float16* vb = pool + ((blk * 2 + 1) * KVH + kvh) * (uint64_t)bt * D + (uint64_t)(off >> 5) * D * 32;
    // The tile's keys are stored as the operands themselves (kv_key_index): score
    // fragment 0 row 4q+i is position 8q+i and fragment 1 row 4q+i is position 8q+4+i, so
    // lane (q, v) holds the scores of the 8 consecutive positions 8q..8q+7, which is also
    // the order of its 16-byte V^T load. Each operand is one contiguous 1 KiB load. The
    // cache is read once per pass and layer: non-temporal loads keep it from displacing
    // other lines (measured: 32 -> 29 us for a 64-row decode layer).
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      f.k0[kk] = __builtin_nontemporal_load(reinterpret_cast<const half8*>(kb + (size_t)((2 * kk) * 64 + lane) * 8));
      f.k1[kk] = __builtin_nontemporal_load(reinterpret_cast<const half8*>(kb + (size_t)((2 * kk + 1) * 64 + lane) * 8));
    }
#pragma unroll
    for (int df = 0; df < DF; ++df) {
      f.v[df] = __builtin_nontemporal_load(reinterpret_cast<const half8*>(vb + (size_t)(16 * df + col) * 32 + 8 * quad));
    }
  };
  // One tile's scores, online softmax update and value accumulation.
  auto consume = [&](int t, const Tile& f) {
  floatx4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    s0 = mfma(f.k0[kk], qf[kk], s0);
    s1 = mfma(f.k1[kk], qf[kk], s1);
  }
  // Scores (base 2) of the tile's positions, -inf past the key range or the vector's own
  // position. A tile wholly before the block's first position and inside the range needs
  // no mask (the usual case). Vectors past the block's end are not masked: their results
  // are never written.
  float sc[8];
  if (t + 32 <= key_end && t + 31 <= w.position0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = s0[i];
      sc[4 + i] = s1[i];
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p0 = t + 8 * quad + i, p1 = t + 8 * quad + 4 + i;
      sc[i] = (p0 <= my_pos && p0 < key_end) ? s0[i] : -INFINITY;
      sc[4 + i] = (p1 <= my_pos && p1 < key_end) ? s1[i] : -INFINITY;
    }
  }
  float tmax = sc[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) tmax = fmaxf(tmax, sc[i]);
  tmax = fmaxf(tmax, __shfl_xor(tmax, 16, 64));
  tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
  const float m_new = fmaxf(m, tmax);
  const float base = m_new == -INFINITY ? 0.0f : m_new;
  const float alpha = exp2_fast(m - base);
  half8 pf;
  float psum = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float p = exp2_fast(sc[i] - base);
    psum += p;
    pf[i] = to_half(p);
  }
  psum += __shfl_xor(psum, 16, 64);
  psum += __shfl_xor(psum, 32, 64);
  l = l * alpha + psum;
  m = m_new;
  // A tile that runs past the key range reads cache slots no pass has written: zero
  // them, since a zero probability does not cancel a non-finite value.
  const bool tail = t + 32 > key_end;
#pragma unroll
  for (int df = 0; df < DF; ++df) {
    o[df][0] *= alpha;
    o[df][1] *= alpha;
    o[df][2] *= alpha;
    o[df][3] *= alpha;
    half8 av = f.v[df];
    if (tail) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (t + 8 * quad + j >= key_end) av[j] = (_Float16)0.0f;
    }
    o[df] = mfma(av, pf, o[df]);
  }
  };

  if (split_keys) {
    // Decode-like blocks: the four waves take interleaved tiles, each loading its own
    // fragments from HBM straight into registers, one tile per wave at a time (the other
    // workgroups on the CU keep the memory busy meanwhile). The next tile's block is read
    // one iteration early; past the range it re-reads the range's last tile's block.
    if (key_end > w.key_begin) {  // a fused row's first position has no cached keys
      const int last_tile = w.key_begin + ((key_end - 1 - w.key_begin) & ~31);
      auto clamp_tile = [&](int x) { return x < key_end ? x : last_tile; };
      constexpr int stride = 4;
      int t = w.key_begin + 32 * wave;
      uint64_t blk = block_of(clamp_tile(t) / bt);
      for (; t < key_end; t += 32 * stride) {
        Tile cur;
        fetch(t, blk, cur);
        blk = block_of(clamp_tile(t + 32 * stride) / bt);
        consume(t, cur);
      }
    }
    float own = 0.0f;  // wave 0: the own-key score of this lane's vector (all vectors in turn)
    if constexpr (D == 128) {
      if (holds_self && wave == 0)
        for (int g = 0; g < G; ++g) {
          const float sg = own_key_score<D>(g, lane, qscale);
          if (g == vg) own = sg;
        }
    }
    if (holds_self && wave == 0 && v_ok) {
      // The row's own key and value (staged by fused_projection), one more softmax step:
      // the probability enters the sum in F32 and the value product in F16, as in a tile.
      const float sv = own;
      const float m_new = fmaxf(m, sv);
      const float alpha = exp2_fast(m - m_new);
      const float p = exp2_fast(sv - m_new);
      l = l * alpha + p;
      m = m_new;
      const float p16 = (float)to_half(p);
#pragma unroll
      for (int df = 0; df < DF; ++df)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[df][i] = o[df][i] * alpha + p16 * (float)self_kv[D + 16 * df + 4 * quad + i];
    }
  } else {
    // Prefill blocks: every wave needs every tile, so the workgroup copies each 32-key K/V
    // tile once into LDS, straight from the cache (global_load_lds), NSTAGE tiles deep: the
    // copies of tiles i + 1 and i + 2 are in flight while tile i is used. Keys are copied as
    // stored (operand order: each operand read is 1 KiB of consecutive LDS), values as the
    // tile's [D][32] sub-tile with the 16-byte chunks of row d permuted (chunk c at
    // c ^ ((d >> 2) & 3)) so that the fragment reads below hit distinct LDS banks.
    constexpr int KB = 32 * D * 2;              // key bytes per tile
    constexpr int SB = KB + D * 32 * 2;         // key and value bytes per tile
    constexpr int NSTAGE = 3;
    constexpr int CP = SB / (kThreads * 16);    // 16-byte copies per lane per tile
    static_assert(SB % (kThreads * 16) == 0 && KB % (kThreads * 16) == 0, "attention tile copies");
    const uint32_t lds_base = (uint32_t)(size_t)((__attribute__((address_space(3))) float*)smem);
    const int tiles = (w.key_end - w.key_begin + 31) / 32;
    // Block-table entries of the range, one per lane, 64 blocks at a time: a table read
    // inside the pipelined loop would be a vector load (the copies clobber memory as far as
    // the compiler knows), and waiting for it would drain the copies in flight.
    const int last_block = (w.key_end - 1) / bt;
    int held_base = 0, held = 0;
    // Copy-side state, advanced once per issued tile so that no division or modulo runs in
    // the loop (scalar instructions are shared by the CU's waves): the next tile's block
    // (relative to held_base), its offset in the block and its stage's LDS offset.
    int rel = 0, off = 0;
    uint32_t next_stage = 0;
    const _Float16* key_base = pool + (uint64_t)kvh * bt * D;
    const _Float16* value_base = pool + (uint64_t)(KVH + kvh) * bt * D;
    const uint64_t block_elems = (uint64_t)2 * KVH * bt * D;
    // This wave's copies of the next tile into its stage: wave-sized 1 KiB pieces of the
    // stage, interleaved over the waves, the first KB / 1024 of them keys. A tile's values
    // start off * D elements into the block's value region, as its keys do (off is a
    // multiple of 32).
    auto issue = [&]() {
      const uint64_t at = (uint64_t)(uint32_t)__builtin_amdgcn_readlane(held, rel) * block_elems + (uint64_t)off * D;
      const _Float16* kb = key_base + at;
      const _Float16* vb = value_base + at;
      const uint32_t stage = lds_base + next_stage;
#pragma unroll
      for (int q = 0; q < CP; ++q) {
        const int piece = q * (kThreads / 64) + wave;
        const int p = piece * 1024 + lane * 16;  // this lane's byte in the stage
        if (q * (kThreads / 64) * 1024 < KB) {
          lds_copy16(kb, (uint32_t)p, stage + piece * 1024);
        } else {
          const int d = (p - KB) / 64, c = ((p - KB) % 64) / 16;
          lds_copy16(vb, (uint32_t)(d * 64 + ((c ^ ((d >> 2) & 3)) * 16)), stage + piece * 1024);
        }
      }
      off += 32;
      if (off == bt) {
        off = 0;
        ++rel;
      }
      next_stage = next_stage == (NSTAGE - 1) * SB ? 0 : next_stage + SB;
    };
    auto read_tile = [&](uint32_t stage_offset, Tile& f) {
      const char* ks = reinterpret_cast<const char*>(smem) + stage_offset;
      const char* vs = ks + KB;
      const int lane16 = (threadIdx.x & 63) * 16;
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        f.k0[kk] = *reinterpret_cast<const half8*>(ks + (2 * kk) * 1024 + lane16);
        f.k1[kk] = *reinterpret_cast<const half8*>(ks + (2 * kk + 1) * 1024 + lane16);
      }
#pragma unroll
      for (int df = 0; df < DF; ++df) {
        const int d = 16 * df + col;
        f.v[df] = *reinterpret_cast<const half8*>(vs + d * 64 + ((quad ^ ((d >> 2) & 3)) * 16));
      }
    };
    uint32_t read_stage = 0;
    for (int i0 = 0; i0 < tiles;) {
      // Tiles [i0, i1) lie in the 64 blocks held from held_base; the pipeline restarts
      // after each such group (ranges of more than 64 blocks only).
      held_base = (w.key_begin + 32 * i0) / bt;
      held = table[min(held_base + lane, last_block)];
      rel = 0;
      off = (w.key_begin + 32 * i0) % bt;
      const int i1 = min(tiles, ((held_base + 64) * bt - w.key_begin) / 32);
      issue();
      if (i0 + 1 < i1) issue();
      for (int i = i0; i < i1; ++i) {
        // Tile i has landed once this wave's later copies (tile i + 1's) are all that is
        // outstanding and every wave has got here; that also means every wave is done
        // with tile i - 1, whose stage tile i + 2 overwrites.
        if (i + 1 < i1)
          stage_barrier<CP, 0>();
        else
          stage_barrier<0, 0>();
        if (i + 2 < i1) issue();  // tile i + 2; workgroup-uniform
        Tile f;
        read_tile(read_stage, f);
        read_stage = read_stage == (NSTAGE - 1) * SB ? 0 : read_stage + SB;
        consume(w.key_begin + 32 * i, f);
      }
      i0 = i1;
    }
  }

  // Decode-like blocks with split keys merge them here: the split workgroup that arrives
  // last (a device-scope count per block and KV head) merges every split in split order,
  // with the combine kernel's arithmetic. Workgroup-uniform.
  const bool fold = split_keys && w.splits > 1 && a.fold;
  float m_fin = m, l_fin = l;
  if (split_keys) {
    // Merge the four waves' partial softmax states (vectors 0..15) through LDS. A lane's
    // accumulators are stored lane-private, [wave][df][lane] x 4 floats, so that wave 0's
    // lane reads the other waves' values of its own (vector, dimensions) as 16-byte vectors.
    float* sm_m = smem;                                        // [4][16]
    float* sm_l = smem + 64;                                   // [4][16]
    floatx4* sm_o = reinterpret_cast<floatx4*>(smem + 128);    // [4][DF][64]
    if (quad == 0) {
      sm_m[wave * 16 + col] = m;
      sm_l[wave * 16 + col] = l;
    }
    if (wave != 0) {
#pragma unroll
      for (int df = 0; df < DF; ++df) sm_o[(wave * DF + df) * 64 + lane] = o[df];
    }
    __syncthreads();
    if (wave != 0 && !fold) return;
    if (wave == 0) {
      float mm = -INFINITY;
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) mm = fmaxf(mm, sm_m[ww * 16 + col]);
      float weights[4];
      l_fin = 0.0f;
#pragma unroll
      for (int ww = 0; ww < 4; ++ww) {
        weights[ww] = exp2_fast(sm_m[ww * 16 + col] - (mm == -INFINITY ? 0.0f : mm));
        l_fin += sm_l[ww * 16 + col] * weights[ww];
      }
      m_fin = mm;
#pragma unroll
      for (int df = 0; df < DF; ++df) {
        floatx4 others[3];
#pragma unroll
        for (int ww = 1; ww < 4; ++ww) others[ww - 1] = sm_o[(ww * DF + df) * 64 + lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float s = 0.0f + o[df][i] * weights[0];
#pragma unroll
          for (int ww = 1; ww < 4; ++ww) s += others[ww - 1][i] * weights[ww];
          o[df][i] = s;
        }
      }
    }
  }
  if (fold) {
    // Wave 0 publishes this split's partial with device-scope stores, waits for them to
    // complete and counts the arrival; the count's last arrival resets it for the next
    // launch and the four waves merge the block's vectors. No cache-wide fence is needed:
    // every access to the partials and the count is a relaxed agent-scope atomic, which
    // gfx950 performs at the device's coherence point (`sc1` stores write through the
    // XCD's L2, `sc1` loads do not hit a stale line of it). An agent-scope release fence
    // would add `buffer_wbl2` (write back the whole L2, for plain stores, of which the
    // merge reads none) to the `s_waitcnt vmcnt(0)` below, and an acquire fence
    // `buffer_inv` (for plain loads, of which it issues none); the wait alone orders the
    // partial's stores before the count, and the merge's loads follow the count's value.
    int32_t* arrivals = a.split_arrivals + (size_t)w.row0 * a.kv_heads + kvh;
    int* arrived = reinterpret_cast<int*>(smem);  // wave 0 has finished reading the merge area
    if (wave == 0) {
      if (v_ok) {
        float* out = partial_at(a, w.row0 + vr, kvh * G + vg, w.split);
#pragma unroll
        for (int df = 0; df < DF; ++df)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            __hip_atomic_store(out + 16 * df + 4 * quad + i, o[df][i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (quad == 0) {
          __hip_atomic_store(out + D, m_fin * kLn2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(out + D + 1, l_fin, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      int before = 0;
      if (lane == 0) before = __hip_atomic_fetch_add(arrivals, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      before = __shfl(before, 0, 64);
      if (lane == 0) *arrived = before;
      if (before == w.splits - 1 && lane == 0)
        __hip_atomic_store(arrivals, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (*arrived != w.splits - 1) return;
    asm volatile("" ::: "memory");
    for (int vv = wave; vv < nvec; vv += kThreads / 64)
      merge_splits<D / 64, true>(a, w.row0 + vv / G, kvh * G + vv % G, w.splits, lane);
    return;
  }
  if (!v_ok) return;
  const int row = w.row0 + vr, qh = kvh * G + vg;
  if (w.splits == 1) {
    const float inv = 1.0f / l_fin;
#pragma unroll
    for (int df = 0; df < DF; ++df) {
      half4 y;
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = to_half(o[df][i] * inv);
      const uint64_t at = flayout_index(row, (uint64_t)qh * D + 16 * df + 4 * quad, a.out_cols_padded);
      *reinterpret_cast<half4*>(a.out_hi + at) = y;
    }
  } else {
    float* out = partial_at(a, row, qh, w.split);
#pragma unroll
    for (int df = 0; df < DF; ++df)
#pragma unroll
      for (int i = 0; i < 4; ++i) out[16 * df + 4 * quad + i] = o[df][i];
    if (quad == 0) {
      out[D] = m_fin * kLn2;  // the combine kernel takes natural-log maxima
      out[D + 1] = l_fin;
    }
  }
  }();
  __syncthreads();  // the next work item reuses the LDS
  }
}

// ---------------------------------------------------------------- F32 VALU attention

__device__ inline int valu_split_length(int ctx, int max_splits, int unit) {
  int splits = (ctx + unit - 1) / unit;
  splits = splits < max_splits ? splits : max_splits;
  const int per = (ctx + splits - 1) / splits;
  return (per + 15) & ~15;
}

template <typename KV>
__global__ void __launch_bounds__(kThreads) attention_valu_kernel(AttentionArgs a) {
  const int r = blockIdx.x, kvh = blockIdx.y, s = blockIdx.z;
  const int ctx = a.row_position[r] + 1;
  const int per = valu_split_length(ctx, a.max_splits, a.split_unit);
  const int p0 = s * per;
  if (p0 >= ctx) return;
  const int p1 = min(ctx, p0 + per);
  const int D = a.head_dim, G = a.q_heads / a.kv_heads;
  const int seq = a.items[a.row_item[r]].sequence;
  const int32_t* table = a.block_table + (size_t)seq * a.table_width;
  const KV* pool = static_cast<const KV*>(a.kv.pool);
  const int bt = a.kv.block_tokens;

  extern __shared__ float smem[];
  float* qs = smem;                 // [G][D]
  float* sc = qs + G * D;           // [G][kTile]
  float* stat = sc + G * kTile;     // [G] tile max, [G] tile sum
  const int tid = threadIdx.x;
  for (int e = tid; e < G * D; e += kThreads) qs[e] = a.q[((size_t)r * a.q_heads + kvh * G) * D + e];
  const int my_d = tid % D;
  const int h_first = tid / D, h_step = kThreads / D > 0 ? kThreads / D : 1;
  float acc[kMaxPairs], run_max[kMaxPairs], run_sum[kMaxPairs];
#pragma unroll
  for (int k = 0; k < kMaxPairs; ++k) {
    acc[k] = 0.0f;
    run_max[k] = -INFINITY;
    run_sum[k] = 0.0f;
  }
  __syncthreads();
  for (int t0 = p0; t0 < p1; t0 += kTile) {
    const int n = min(kTile, p1 - t0);
    if (tid < n) {
      const int p = t0 + tid;
      const KV* k = pool + kv_key_index(a.kv, a.layer, (uint64_t)table[p / bt], p % bt, kvh, 0);
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
    const int wave = tid >> 6, lane = tid & 63;
    for (int g = wave; g < G; g += kThreads / 64) {
      float mx = -INFINITY;
      for (int i = lane; i < n; i += 64) mx = fmaxf(mx, sc[g * kTile + i]);
      mx = wave_max(mx);
      float sum = 0.0f;
      for (int i = lane; i < n; i += 64) {
        const float e = expf(sc[g * kTile + i] - mx);
        sc[g * kTile + i] = e;
        sum += e;
      }
      sum = wave_sum(sum);
      if (lane == 0) {
        stat[g] = mx;
        stat[G + g] = sum;
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kMaxPairs; ++k) {
      const int g = h_first + k * h_step;
      if (tid < G * D && g < G) {
        const float tile_max = stat[g];
        const float new_max = fmaxf(run_max[k], tile_max);
        const float old_scale = rescale(run_max[k], new_max);
        const float tile_scale = expf(tile_max - new_max);
        run_sum[k] = run_sum[k] * old_scale + stat[G + g] * tile_scale;
        run_max[k] = new_max;
        acc[k] *= old_scale;
        float part = 0.0f;
        for (int i = 0; i < n; ++i) {
          const int p = t0 + i;
          const KV* v = pool + kv_value_index(a.kv, a.layer, (uint64_t)table[p / bt], p % bt, kvh, my_d);
          part += sc[g * kTile + i] * (float)*v;
        }
        acc[k] += part * tile_scale;
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < kMaxPairs; ++k) {
    const int g = h_first + k * h_step;
    if (tid < G * D && g < G) {
      float* out = partial_at(a, r, kvh * G + g, s);
      out[my_d] = acc[k];
      if (my_d == 0) {
        out[D] = run_max[k];
        out[D + 1] = run_sum[k];
      }
    }
  }
}

// ---------------------------------------------------------------- split combine

// Merges the splits of one (row, query head) in split order, normalises and writes the
// operand; called by a whole wave. Lane s < splits holds split s's statistics; lane L owns
// head dimensions L*E .. L*E+E-1 (E = D / 64, at least 1). The statistics and the first
// four splits' vectors are loaded together (unconditionally, at clamped addresses): the
// merge is a short latency-bound chain. kCoherent: the partials were written by workgroups
// of this launch, possibly on other XCDs, and are read with device-scope loads (which do not
// hit a stale line of this XCD's L2); the arithmetic is the same either way.
template <int E, bool kCoherent>
__device__ inline void merge_splits(const AttentionArgs& a, int r, int qh, int splits, int lane) {
  auto ld = [](const float* p) -> float {
    if constexpr (kCoherent)
      return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      return *p;
  };
  const int D = a.head_dim;
  const int stride = D + 2;
  const float* part = partial_at(a, r, qh, 0);
  const int dl = min(lane * E, D - E);  // lanes past D re-read the last elements
  const float* stat = part + (size_t)min(lane, splits - 1) * stride + D;
  const float ms_raw = ld(stat), ls_raw = ld(stat + 1);
  float pv[4][E];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int e = 0; e < E; ++e) pv[u][e] = ld(part + (size_t)min(u, splits - 1) * stride + dl + e);
  const float ms = lane < splits ? ms_raw : -INFINITY;
  const float ls = lane < splits ? ls_raw : 0.0f;
  float m = ms;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  const float ref = m == -INFINITY ? 0.0f : m;
  const float ws = lane < splits ? rescale(ms, ref) : 0.0f;
  float total = ls * ws;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) total += __shfl_xor(total, o, 64);
  const float inv = 1.0f / total;
  float v[E];
#pragma unroll
  for (int e = 0; e < E; ++e) v[e] = 0.0f;
  for (int sp0 = 0; sp0 < splits; sp0 += 4) {
    if (sp0 > 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < E; ++e) pv[u][e] = ld(part + (size_t)min(sp0 + u, splits - 1) * stride + dl + e);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float w = __shfl(ws, min(sp0 + u, 63), 64);
#pragma unroll
      for (int e = 0; e < E; ++e) v[e] = sp0 + u < splits ? v[e] + pv[u][e] * w : v[e];
    }
  }
  if (lane * E < D) {
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const float y = v[e] * inv;
      const uint64_t at = flayout_index(r, (uint64_t)qh * D + lane * E + e, a.out_cols_padded);
      const _Float16 hi = to_half(y);
      a.out_hi[at] = __builtin_bit_cast(uint16_t, hi);
      if (a.out_lo) a.out_lo[at] = __builtin_bit_cast(uint16_t, to_half((y - (float)hi) * kLoScale));
    }
  }
  // Zero the operand's padded columns (their weights are zero; the values must be finite).
  if (qh == 0) {
    for (uint64_t c = (uint64_t)a.q_heads * D + lane; c < a.out_cols_padded; c += 64) {
      const uint64_t at = flayout_index(r, c, a.out_cols_padded);
      a.out_hi[at] = 0;
      if (a.out_lo) a.out_lo[at] = 0;
    }
  }
}

// One wave per (row, query head), four per block: merge_splits of the row's splits.
// MFMA-path rows with a single split (or merged by the attention kernel) are skipped.
template <int E>
__global__ void __launch_bounds__(256) attention_combine_kernel(AttentionArgs a, int mfma_path) {
  const int pair = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (pair >= a.rows * a.q_heads) return;
  const int r = pair / a.q_heads, qh = pair - r * a.q_heads;
  int splits;
  if (mfma_path) {
    splits = uniform_load(a.row_splits + r);
    if (splits == 1) return;
  } else {
    const int ctx = uniform_load(a.row_position + r) + 1;
    const int per = valu_split_length(ctx, a.max_splits, a.split_unit);
    splits = (ctx + per - 1) / per;
  }
  merge_splits<E, false>(a, r, qh, splits, lane);
}

template <int D>
void launch_mfma(hipStream_t stream, const AttentionArgs& a) {
  // The decode path's merge area and the prefill path's three K/V stages share the memory.
  const size_t lds = std::max((size_t)(128 + 4 * D * 16) * sizeof(float),
                              (size_t)3 * (32 * D + D * 32) * sizeof(_Float16));
  static const bool configured = [&] {
    HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_mfma_kernel<D>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    return true;
  }();
  (void)configured;
  observed(kernel_name<D>("attention_mfma_kernel"),
           [&] { attention_mfma_kernel<D><<<dim3(a.work_grid * a.kv_heads), kThreads, lds, stream>>>(a); });
}

}  // namespace

bool attention_uses_mfma(int head_dim, bool kv_f32) {
  return !kv_f32 && (head_dim == 64 || head_dim == 128 || head_dim == 256);
}

void launch_attention(hipStream_t stream, const AttentionArgs& a) {
  if (a.rows <= 0) return;
  const bool mfma_path = attention_uses_mfma(a.head_dim, a.kv.f32 != 0);
  if (mfma_path) {
    if (a.work_grid > 0) {
      if (a.head_dim == 64) launch_mfma<64>(stream, a);
      if (a.head_dim == 128) launch_mfma<128>(stream, a);
      if (a.head_dim == 256) launch_mfma<256>(stream, a);
    }
  } else {
    const int G = a.q_heads / a.kv_heads;
    const size_t lds = ((size_t)G * a.head_dim + (size_t)G * kTile + 2 * G) * sizeof(float);
    dim3 grid(a.rows, a.kv_heads, a.max_splits);
    if (a.kv.f32)
      observed("attention_valu_kernel<float>", [&] { attention_valu_kernel<float><<<grid, kThreads, lds, stream>>>(a); });
    else
      observed("attention_valu_kernel<_Float16>", [&] { attention_valu_kernel<_Float16><<<grid, kThreads, lds, stream>>>(a); });
  }
  // MFMA-path blocks with a single split write their rows directly.
  if (mfma_path && !a.any_split) return;
  const unsigned blocks = (unsigned)(a.rows * a.q_heads + 3) / 4;
  const int path = mfma_path ? 1 : 0;
  observed("attention_combine_kernel", [&] {
    if (a.head_dim <= 64)
      attention_combine_kernel<1><<<blocks, 256, 0, stream>>>(a, path);
    else if (a.head_dim <= 128)
      attention_combine_kernel<2><<<blocks, 256, 0, stream>>>(a, path);
    else
      attention_combine_kernel<4><<<blocks, 256, 0, stream>>>(a, path);
  });
}

}  // namespace hllm_rocm
