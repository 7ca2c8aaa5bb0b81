// Dense projections Y[M, N] = X[M, K] * W[N, K]^T on v_mfma_f32_16x16x32_f16.
//
// Both operands are in the F-layout (common.hpp), so every operand fragment is one
// coalesced 1 KiB load per wave straight from HBM/L2 into registers. The MFMA's A side is
// the weight fragment (16 output features x 32 k) and its B side the activation fragment
// (32 k x 16 tokens); lane L of the 16x16 result holds features 4*(L/16)+v of token L%16.
//
// A workgroup owns BN = 16*NF*WN output features x BM = 16*MF*WM rows for a K range. Its
// WK K-waves interleave the K fragments of that range; each wave keeps a ring of P
// fragment loads in flight (weights and activations) so that the weight stream is
// bandwidth- rather than latency-bound. Few-row (decode) passes split K across
// workgroups too, so that every CU streams weights: block IDs are ordered so that all
// K splits of a tile are dispatched to the same XCD (workgroups go round-robin over the
// 8 XCDs), and the last split of a tile to arrive (an atomic counter it resets) sums the
// partial tiles in split order, so results are deterministic.
//
// Split precision (F32 execution) adds a second accumulator for the lo parts of split
// operands: x*w ~= hi*hi + (lo*hi + hi*lo) / 2048.
#include "gemm.hpp"

#include <algorithm>
#include <atomic>
#include <cstdlib>

namespace hllm_rocm {
namespace {

constexpr int kXcds = 8;

// Block -> (K split, weight tile, row tile) of the many-row kernels. Block b runs on XCD
// b % 8, and a unit's (K split, weight tile) row tiles are consecutive blocks of one XCD, so
// they share that XCD's L2 copy of the weight tile. With K splits, units in split-major
// order are cut into eight contiguous ranges whose sizes differ by at most one, one per XCD:
// the units of an XCD mostly share K splits, so each XCD fetches the activation columns of
// few splits (dealt round-robin, every XCD fetched nearly all of them: 1-4% slower). Without
// K splits the weight tiles are dealt round-robin (0.9% faster for gate+up at 576 rows).
// Either way every XCD holds within one unit of the same work.
struct TileCoord {
  int split, tile_n, tile_m;
  bool valid;
};
__device__ inline TileCoord xcd_tile(int block, int n_tiles, int m_tiles, int units) {
  const int x = block % kXcds, j = block / kXcds;
  const int local = j / m_tiles, tile_m = j - local * m_tiles;
  if (units == n_tiles) {
    const int u = local * kXcds + x;
    return {0, u, tile_m, u < units};
  }
  const int first = x * units / kXcds, end = (x + 1) * units / kXcds;
  const int u = first + local;
  return {u / n_tiles, u % n_tiles, tile_m, u < end};
}
inline unsigned xcd_grid(int units, int m_tiles) { return (unsigned)((units + kXcds - 1) / kXcds * kXcds * m_tiles); }

__device__ inline floatx4 mfma(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

template <int MF, int NF, int WM, int WN, int WK, int P, int PREC>
__global__ void __launch_bounds__(64 * WM * WN * WK)
    gemm_kernel(GemmArgs a, int n_tiles, int tiles, int tiles_padded) {
  constexpr int BM = 16 * MF * WM, BN = 16 * NF * WN, NT = 64 * WM * WN * WK;
  constexpr int LDT = BN + 4;  // padded LDS row (floats)
  extern __shared__ float lds[];  // [WK][BM][LDT] + flag
  const int M = a.device_m ? *a.device_m : a.M;
  // Block order: id = split * tiles_padded + tile (tiles_padded % 8 == 0), so every split
  // of a tile has the same id modulo 8, i.e. runs on the same XCD.
  const int id = blockIdx.x;
  const int split = id / tiles_padded;
  const int tile = id - split * tiles_padded;
  if (tile >= tiles) return;
  const int tile_n = tile % n_tiles, tile_m = tile / n_tiles;
  if (tile_m * BM >= M) return;  // uniform over the whole tile (all of its splits)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wk = wave % WK, wn = (wave / WK) % WN, wm = wave / (WK * WN);
  const int KT = (int)(a.Kp >> 5);
  const int per = (KT + a.ksplit - 1) / a.ksplit;
  const int kt0 = split * per, kt1 = min(KT, kt0 + per);
  const int nfrag0 = tile_n * (BN / 16) + wn * NF;
  const int mfrag0 = tile_m * (BM / 16) + wm * MF;

  const half8* W = reinterpret_cast<const half8*>(a.w_hi) + (size_t)nfrag0 * KT * 64 + lane;
  const half8* WL = reinterpret_cast<const half8*>(a.w_lo) + (size_t)nfrag0 * KT * 64 + lane;
  const half8* X = reinterpret_cast<const half8*>(a.x_hi) + (size_t)mfrag0 * KT * 64 + lane;
  const half8* XL = reinterpret_cast<const half8*>(a.x_lo) + (size_t)mfrag0 * KT * 64 + lane;
  const size_t frag_stride = (size_t)KT * 64;  // half8s between consecutive fragment rows

  floatx4 acc[MF][NF];
  floatx4 acc2[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) {
      acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
      acc2[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

  // Ring of P in-flight k-steps for this wave: k-step s of the ring is kt = first + s*WK.
  constexpr bool kLoA = PREC >= kSplitA, kLoB = PREC == kSplitAB;
  half8 rb[P][NF], rx[P][MF];
  half8 rxl[kLoA ? P : 1][kLoA ? MF : 1];
  half8 rbl[kLoB ? P : 1][kLoB ? NF : 1];
  const int first = kt0 + wk;
  const int steps = first < kt1 ? (kt1 - first + WK - 1) / WK : 0;
  // Loads are unconditional so that the compiler can count them (a conditional load makes
  // every wait drain the whole ring); k-steps past the range re-read the range's last one.
  const int kt_last = max(0, min(kt1, KT) - 1);
  auto load = [&](int slot, int kt) {
    kt = min(kt, kt_last);
#pragma unroll
    for (int j = 0; j < NF; ++j) rb[slot][j] = W[j * frag_stride + (size_t)kt * 64];
#pragma unroll
    for (int i = 0; i < MF; ++i) rx[slot][i] = X[i * frag_stride + (size_t)kt * 64];
    if constexpr (kLoA) {
#pragma unroll
      for (int i = 0; i < MF; ++i) rxl[slot][i] = XL[i * frag_stride + (size_t)kt * 64];
    }
    if constexpr (kLoB) {
#pragma unroll
      for (int j = 0; j < NF; ++j) rbl[slot][j] = WL[j * frag_stride + (size_t)kt * 64];
    }
  };
  auto compute = [&](int s) {
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int j = 0; j < NF; ++j) acc[i][j] = mfma(rb[s][j], rx[s][i], acc[i][j]);
    if constexpr (kLoA) {
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) acc2[i][j] = mfma(rb[s][j], rxl[s][i], acc2[i][j]);
    }
    if constexpr (kLoB) {
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) acc2[i][j] = mfma(rbl[s][j], rx[s][i], acc2[i][j]);
    }
  };
#pragma unroll
  for (int s = 0; s < P; ++s) load(s, first + s * WK);
  // Whole groups of P k-steps run branch-free, so each slot waits only for its own loads
  // while the other P - 1 slots stay in flight; the last partial group follows.
  int base = 0;
  for (; base + P <= steps; base += P) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      compute(s);
      load(s, first + (base + s + P) * WK);
      // Keep the slot's reload right after its MFMAs (the scheduler would otherwise sink
      // every reload to the end of the group and leave nothing in flight).
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int s = 0; s < P; ++s)
    if (base + s < steps) compute(s);

  // Per-wave partial tiles -> one tile. Each K-wave stores its tile in an LDS area of its
  // own; each element is then summed over the areas in wave order (the order of a
  // sequential accumulation, so the sum is deterministic), by the thread that writes it.
  {
    float* mine = lds + (size_t)wk * BM * LDT;
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int j = 0; j < NF; ++j) {
        floatx4 v = acc[i][j];
        if constexpr (PREC >= kSplitA) {
          v[0] += acc2[i][j][0] * kLoUnscale;
          v[1] += acc2[i][j][1] * kLoUnscale;
          v[2] += acc2[i][j][2] * kLoUnscale;
          v[3] += acc2[i][j][3] * kLoUnscale;
        }
        const int m = (wm * MF + i) * 16 + (lane & 15);
        const int n = (wn * NF + j) * 16 + (lane >> 4) * 4;
        *reinterpret_cast<floatx4*>(mine + m * LDT + n) = v;
      }
    __syncthreads();
  }
  // Element (m, n .. n + 3) of the tile summed over the K-wave areas in wave order.
  auto tile_sum = [&](int m, int n) {
    floatx4 sum = *reinterpret_cast<const floatx4*>(lds + m * LDT + n);
#pragma unroll
    for (int t = 1; t < WK; ++t) {
      const floatx4 x = *reinterpret_cast<const floatx4*>(lds + (size_t)t * BM * LDT + m * LDT + n);
      sum[0] += x[0];
      sum[1] += x[1];
      sum[2] += x[2];
      sum[3] += x[3];
    }
    return sum;
  };

  if (a.ksplit > 1) {
    // The K split's partial goes straight from the summed areas to memory.
    if (a.defer_reduce) {
      // A row-major [M][N] matrix of its own; the consumer of the projection sums the
      // splits in order.
      float* ws = a.workspace + (size_t)split * a.M * a.N;
      const bool vec = (a.N & 3) == 0;
      for (int e = threadIdx.x; e < BM * BN / 4; e += NT) {
        const int m = e / (BN / 4), n = (e % (BN / 4)) * 4;
        const int row = tile_m * BM + m, col = tile_n * BN + n;
        if (row >= M || col >= a.N) continue;
        const floatx4 sum = tile_sum(m, n);
        float* dst = ws + (size_t)row * a.N + col;
        if (vec) {
          *reinterpret_cast<floatx4*>(dst) = sum;
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (col + t < a.N) dst[t] = sum[t];
        }
      }
    } else {
      // A partial tile; gemm_reduce_kernel sums the splits in order and applies the
      // epilogue after this kernel completes (no device-scope fences needed).
      float* ws = a.workspace + ((size_t)tile * a.ksplit + split) * BM * BN;
      for (int e = threadIdx.x; e < BM * BN / 4; e += NT) {
        const int m = e / (BN / 4), n = (e % (BN / 4)) * 4;
        *reinterpret_cast<floatx4*>(ws + m * BN + n) = tile_sum(m, n);
      }
    }
    return;
  }
  if constexpr (WK > 1) {
    for (int e = threadIdx.x; e < BM * BN / 4; e += NT) {
      const int m = e / (BN / 4), n = (e % (BN / 4)) * 4;
      *reinterpret_cast<floatx4*>(lds + m * LDT + n) = tile_sum(m, n);
    }
    __syncthreads();
  }

  // Epilogue from the LDS tile.
  const int m_base = tile_m * BM, n_base = tile_n * BN;
  if (a.epilogue == kEpiSwiglu) {
    // Columns come in 64-wide groups: 32 gate features then the 32 matching up features.
    constexpr int GROUPS = BN / 64;
    for (int e = threadIdx.x; e < BM * GROUPS * 4; e += NT) {
      const int m = e / (GROUPS * 4);
      const int g = (e / 4) % GROUPS;
      const int c8 = e % 4;
      const uint64_t col = (uint64_t)(n_base / 64 + g) * 32 + c8 * 8;
      // Tiles can reach past the last gate/up group when the padded width is not a
      // multiple of the tile; those columns do not exist in the operand.
      if (m_base + m >= M || col >= a.out_cols_padded) continue;
      half8 vh, vl;
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const float gate = lds[m * LDT + g * 64 + c8 * 8 + t];
        const float up = lds[m * LDT + g * 64 + 32 + c8 * 8 + t];
        const float y = silu_mul(gate, up);
        vh[t] = to_half(y);
        vl[t] = to_half((y - (float)vh[t]) * kLoScale);
      }
      const uint64_t at = flayout_index(m_base + m, col, a.out_cols_padded);
      *reinterpret_cast<half8*>(a.out_hi + at) = vh;
      if (a.out_lo) *reinterpret_cast<half8*>(a.out_lo + at) = vl;
    }
    return;
  }
  for (int e = threadIdx.x; e < BM * (BN / 4); e += NT) {
    const int m = e / (BN / 4);
    const int n = (e % (BN / 4)) * 4;
    const int gm = m_base + m;
    if (gm >= M) continue;
    float* out = a.out + (size_t)gm * a.ldo + n_base + n;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (n_base + n + t < a.N) {
        const float v = lds[m * LDT + n + t];
        if (a.epilogue == kEpiResidual)
          out[t] += v;
        else
          out[t] = v;
      }
    }
  }
}

// Activation-staged variant for passes of many rows: the workgroup's four waves split N
// (each owns NFW weight fragment rows, streamed from HBM through a ring of P k-steps), and
// the activation fragments of the tile (BM = 16*MF rows) are staged once per workgroup in
// LDS (chunks of KC k-steps, double-buffered) and read by all four waves, so activation
// traffic per weight byte is BM / BN. Epilogues are applied straight from the accumulators.
//
// Block order is XCD-aware (xcd_tile): the row tiles of one weight tile and K split run
// together on one XCD, so the weight tile is read from HBM once.
template <int MF, int NFW, int KC, int P, int PREC>
__global__ void __launch_bounds__(256, PREC == kF16 && MF <= 8 ? 2 : 1)
    gemm_xlds_kernel(GemmArgs a, int n_tiles, int m_tiles, int units) {
  constexpr int BM = 16 * MF, BN = 64 * NFW, NT = 256;
  constexpr bool kLoA = PREC >= kSplitA, kLoB = PREC == kSplitAB;
  constexpr int XP = kLoA ? 2 : 1;                  // activation parts (hi, lo)
  constexpr int CHUNK = MF * KC * 64 * XP;          // half8s per staged chunk
  static_assert(KC % P == 0, "the ring slot of a k-step must be a compile-time index");
  extern __shared__ float lds[];
  half8* xs = reinterpret_cast<half8*>(lds);        // [2][XP][MF][KC][64]
  const int M = a.device_m ? *a.device_m : a.M;
  const TileCoord at = xcd_tile(blockIdx.x, n_tiles, m_tiles, units);
  const int split = at.split, tile_n = at.tile_n, tile_m = at.tile_m;
  if (!at.valid || tile_m * BM >= M) return;  // uniform over the workgroup
  const int tile = tile_m * n_tiles + tile_n;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int KT = (int)(a.Kp >> 5);
  const int per = ((KT + a.ksplit - 1) / a.ksplit + KC - 1) / KC * KC;
  const int kt0 = split * per, kt1 = min(KT, kt0 + per);
  const int nfrag0 = tile_n * (BN / 16) + wave * NFW;
  const int mfrag0 = tile_m * MF;
  const size_t frag_stride = (size_t)KT * 64;
  const half8* W = reinterpret_cast<const half8*>(a.w_hi) + (size_t)nfrag0 * frag_stride + lane;
  const half8* WL = reinterpret_cast<const half8*>(a.w_lo) + (size_t)nfrag0 * frag_stride + lane;
  const half8* X = reinterpret_cast<const half8*>(a.x_hi) + (size_t)mfrag0 * frag_stride;
  const half8* XL = reinterpret_cast<const half8*>(a.x_lo) + (size_t)mfrag0 * frag_stride;

  floatx4 acc[MF][NFW], acc2[kLoA ? MF : 1][kLoA ? NFW : 1];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < NFW; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  if constexpr (kLoA) {
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int j = 0; j < NFW; ++j) acc2[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  const int steps = kt1 > kt0 ? kt1 - kt0 : 0;
  const int chunks = (steps + KC - 1) / KC;

  // Staging of chunk c (k-steps kt0 + c*KC ...) into buffer c % 2: thread-strided pieces.
  // Activation rows past the operand's padding are not read: the operand is padded to the
  // tile height by the caller (gemm_padded_rows).
  constexpr int PIECES = (CHUNK + NT - 1) / NT;
  half8 stage[PIECES];
  auto fetch_x = [&](int c) {
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      const int e = threadIdx.x + q * NT;  // (part, i, j, lane) flattened
      if (e < CHUNK) {
        const int ln = e & 63, j = (e >> 6) % KC, i = (e / (64 * KC)) % MF, part = e / (64 * KC * MF);
        const int kt = kt0 + c * KC + j;
        const half8* src = part ? XL : X;
        stage[q] = kt < kt1 ? src[(size_t)i * frag_stride + (size_t)kt * 64 + ln] : half8{};
      }
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      const int e = threadIdx.x + q * NT;
      if (e < CHUNK) xs[buf * CHUNK + e] = stage[q];
    }
  };

  half8 rb[P][NFW];
  half8 rbl[kLoB ? P : 1][kLoB ? NFW : 1];
  // Unconditional weight loads (see gemm_kernel); past the range they re-read the last k-step.
  const int kt_last = max(0, min(kt1, KT) - 1);
  auto load_w = [&](int slot, int kt) {
    kt = min(kt, kt_last);
#pragma unroll
    for (int j = 0; j < NFW; ++j) rb[slot][j] = W[j * frag_stride + (size_t)kt * 64];
    if constexpr (kLoB) {
#pragma unroll
      for (int j = 0; j < NFW; ++j) rbl[slot][j] = WL[j * frag_stride + (size_t)kt * 64];
    }
  };
#pragma unroll
  for (int sl = 0; sl < P; ++sl) load_w(sl, kt0 + sl);
  if (chunks > 0) {
    fetch_x(0);
    store_x(0);
  }
  __syncthreads();
  for (int c = 0; c < chunks; ++c) {
    if (c + 1 < chunks) fetch_x(c + 1);
    const half8* xb = xs + (c & 1) * CHUNK;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int step = c * KC + j;
      const int slot = j % P;  // P divides KC, so step % P == j % P
      if (step < steps) {
#pragma unroll
        for (int i = 0; i < MF; ++i) {
          const half8 x = xb[(i * KC + j) * 64 + lane];
#pragma unroll
          for (int n = 0; n < NFW; ++n) acc[i][n] = mfma(rb[slot][n], x, acc[i][n]);
          if constexpr (kLoA) {
            const half8 xl = xb[MF * KC * 64 + (i * KC + j) * 64 + lane];
#pragma unroll
            for (int n = 0; n < NFW; ++n) acc2[i][n] = mfma(rb[slot][n], xl, acc2[i][n]);
          }
          if constexpr (kLoB) {
#pragma unroll
            for (int n = 0; n < NFW; ++n) acc2[i][n] = mfma(rbl[slot][n], x, acc2[i][n]);
          }
        }
      }
      load_w(slot, kt0 + step + P);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (c + 1 < chunks) store_x((c + 1) & 1);
    __syncthreads();
  }

  // Lane (q = lane / 16, t = lane % 16) of accumulator (i, n) holds row 16 i + t, features
  // 16 n + 4 q .. + 3 of the wave's NFW * 16.
  auto value = [&](int i, int n) {
    floatx4 v = acc[i][n];
    if constexpr (kLoA) {
      v[0] += acc2[i][n][0] * kLoUnscale;
      v[1] += acc2[i][n][1] * kLoUnscale;
      v[2] += acc2[i][n][2] * kLoUnscale;
      v[3] += acc2[i][n][3] * kLoUnscale;
    }
    return v;
  };
  const int q4 = (lane >> 4) * 4, t16 = lane & 15;
  const bool vec = (a.N & 3) == 0 && (a.ldo & 3) == 0;
  if (a.ksplit > 1 && a.defer_reduce) {
    // Partial output of this K split as a row-major [M][N] matrix (see gemm_kernel).
    float* ws = a.workspace + (size_t)split * a.M * a.N;
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      const int row = tile_m * BM + i * 16 + t16;
      if (row >= M) continue;
#pragma unroll
      for (int n = 0; n < NFW; ++n) {
        const int col = tile_n * BN + (wave * NFW + n) * 16 + q4;
        const floatx4 v = value(i, n);
        float* dst = ws + (size_t)row * a.N + col;
        if (vec && col + 3 < a.N) {
          *reinterpret_cast<floatx4*>(dst) = v;
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (col + t < a.N) dst[t] = v[t];
        }
      }
    }
    return;
  }
  if (a.ksplit > 1) {
    // Partial tile of this K split, summed in split order by gemm_reduce_kernel.
    float* ws = a.workspace + ((size_t)tile * a.ksplit + split) * BM * BN;
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int n = 0; n < NFW; ++n)
        *reinterpret_cast<floatx4*>(ws + (i * 16 + t16) * BN + (wave * NFW + n) * 16 + q4) = value(i, n);
    return;
  }
  const int m_base = tile_m * BM;
  if (a.epilogue == kEpiSwiglu) {
    // A wave's features are whole 64-wide groups: 32 gate features (fragments 4g, 4g+1),
    // then the 32 matching up features (fragments 4g+2, 4g+3).
    static_assert(NFW % 4 == 0, "SwiGLU needs whole gate/up groups per wave");
#pragma unroll
    for (int gq = 0; gq < NFW / 4; ++gq) {
      const uint64_t g = (uint64_t)(tile_n * BN + wave * NFW * 16) / 64 + gq;
#pragma unroll
      for (int i = 0; i < MF; ++i) {
        const int row = m_base + i * 16 + t16;
        if (row >= M) continue;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint64_t col = g * 32 + h * 16 + q4;
          if (col >= a.out_cols_padded) continue;
          const floatx4 gate = value(i, 4 * gq + h), up = value(i, 4 * gq + 2 + h);
          half4 vh, vl;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float y = silu_mul(gate[t], up[t]);
            vh[t] = to_half(y);
            vl[t] = to_half((y - (float)vh[t]) * kLoScale);
          }
          const uint64_t at = flayout_index(row, col, a.out_cols_padded);
          *reinterpret_cast<half4*>(a.out_hi + at) = vh;
          if (a.out_lo) *reinterpret_cast<half4*>(a.out_lo + at) = vl;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < MF; ++i) {
    const int row = m_base + i * 16 + t16;
    if (row >= M) continue;
#pragma unroll
    for (int n = 0; n < NFW; ++n) {
      const int col = tile_n * BN + (wave * NFW + n) * 16 + q4;
      if (col >= a.N) continue;
      float* out = a.out + (size_t)row * a.ldo + col;
      const floatx4 v = value(i, n);
      if (vec && col + 3 < a.N) {
        floatx4* o4 = reinterpret_cast<floatx4*>(out);
        if (a.epilogue == kEpiResidual) {
          floatx4 s = *o4;
          s[0] += v[0];
          s[1] += v[1];
          s[2] += v[2];
          s[3] += v[3];
          *o4 = s;
        } else {
          *o4 = v;
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (col + t < a.N) {
            if (a.epilogue == kEpiResidual)
              out[t] += v[t];
            else
              out[t] = v[t];
          }
        }
      }
    }
  }
}

// Sum of a tile's K-split partials (in split order) plus the epilogue. One thread per 8
// consecutive outputs of one row (8 activations for SwiGLU).
template <int BM, int BN>
__global__ void __launch_bounds__(256) gemm_reduce_kernel(GemmArgs a, int n_tiles, int tiles) {
  const int M = a.device_m ? *a.device_m : a.M;
  const int per_tile = BM * BN / 8;
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)tiles * per_tile) return;
  const int tile = (int)(e / per_tile);
  const int rem = (int)(e - (int64_t)tile * per_tile);
  const int tile_n = tile % n_tiles, tile_m = tile / n_tiles;
  const float* ws = a.workspace + (size_t)tile * a.ksplit * BM * BN;
  if (a.epilogue == kEpiSwiglu) {
    // rem -> (row m, 64-column group g, 8-wide chunk c8 of the 32 activations of the group)
    constexpr int GROUPS = BN / 64;
    const int m = rem / (GROUPS * 4), g = (rem / 4) % GROUPS, c8 = rem % 4;
    if (rem >= BM * GROUPS * 4) return;
    const uint64_t col = (uint64_t)(tile_n * (BN / 64) + g) * 32 + c8 * 8;
    if (tile_m * BM + m >= M || col >= a.out_cols_padded) return;
    float gate[8], up[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) gate[t] = up[t] = 0.0f;
    // Four splits' loads in flight at a time (clamped, unconditional), summed in split order.
    const float* base = ws + m * BN + g * 64 + c8 * 8;
    for (int p0 = 0; p0 < a.ksplit; p0 += 4) {
      floatx4 q[4][4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float* src = base + (size_t)min(p0 + u, a.ksplit - 1) * BM * BN;
        q[u][0] = *reinterpret_cast<const floatx4*>(src);
        q[u][1] = *reinterpret_cast<const floatx4*>(src + 4);
        q[u][2] = *reinterpret_cast<const floatx4*>(src + 32);
        q[u][3] = *reinterpret_cast<const floatx4*>(src + 36);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const bool live = p0 + u < a.ksplit;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          gate[t] = live ? gate[t] + q[u][0][t] : gate[t];
          gate[4 + t] = live ? gate[4 + t] + q[u][1][t] : gate[4 + t];
          up[t] = live ? up[t] + q[u][2][t] : up[t];
          up[4 + t] = live ? up[4 + t] + q[u][3][t] : up[4 + t];
        }
      }
    }
    half8 vh, vl;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float y = silu_mul(gate[t], up[t]);
      vh[t] = to_half(y);
      vl[t] = to_half((y - (float)vh[t]) * kLoScale);
    }
    const uint64_t at = flayout_index(tile_m * BM + m, col, a.out_cols_padded);
    *reinterpret_cast<half8*>(a.out_hi + at) = vh;
    if (a.out_lo) *reinterpret_cast<half8*>(a.out_lo + at) = vl;
    return;
  }
  const int m = rem / (BN / 8), n = (rem % (BN / 8)) * 8;
  const int gm = tile_m * BM + m, gn = tile_n * BN + n;
  if (gm >= M) return;
  float v[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) v[t] = 0.0f;
  for (int p0 = 0; p0 < a.ksplit; p0 += 4) {
    floatx4 q[4][2];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float* src = ws + (size_t)min(p0 + u, a.ksplit - 1) * BM * BN + m * BN + n;
      q[u][0] = *reinterpret_cast<const floatx4*>(src);
      q[u][1] = *reinterpret_cast<const floatx4*>(src + 4);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const bool live = p0 + u < a.ksplit;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        v[t] = live ? v[t] + q[u][0][t] : v[t];
        v[4 + t] = live ? v[4 + t] + q[u][1][t] : v[4 + t];
      }
    }
  }
  float* out = a.out + (size_t)gm * a.ldo + gn;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    if (gn + t < a.N) {
      if (a.epilogue == kEpiResidual)
        out[t] += v[t];
      else
        out[t] = v[t];
    }
  }
}

// Pipelined variant for passes of many rows (F16 execution): both operands go from HBM/L2
// straight into LDS with direct-to-LDS loads (no register staging) through a ring of
// one-k-step buffers. Tile BM (128 or 256) x 256 features; WM x WN waves, each computing
// BM / WM rows x 256 / WN features from LDS fragments. Every wave copies its share of a
// k-step's fragments (1 KiB each: one 16-byte load per lane). The waves meet at a barrier
// every two k-steps; a wave then reads the next k-step into one register set while its
// MFMAs consume the other. The copies are issued from inline assembly so that the compiler,
// which cannot tell the buffers apart, does not drain every copy in flight before each LDS
// read; the waits on them are written out by hand.
namespace dma {
constexpr int BN = 256;
constexpr int kLdsMax = 160 * 1024;
template <int BM>
struct Ring {
  static constexpr int kFrags = BM / 16 + BN / 16;  // fragments per k-step
  static constexpr int kBytes = kFrags * 1024;      // one buffer
  static constexpr int kBuffers = kLdsMax / kBytes > 6 ? 6 : kLdsMax / kBytes;
  static constexpr int kLds = kBuffers * kBytes;
};
}  // namespace dma

template <int BM, int WM, int WN>
__global__ void __launch_bounds__(64 * WM * WN, 8 / (WM * WN))
    gemm_dma_kernel(GemmArgs a, int n_tiles, int m_tiles, int units) {
  using namespace dma;
  using R = Ring<BM>;
  constexpr int NS = R::kBuffers;
  constexpr int MF = BM / 16 / WM;                    // activation fragments per wave
  constexpr int NF = BN / 16 / WN;                    // weight fragments per wave
  // Copies per wave per k-step; when the waves do not divide the fragments, the extra copies
  // repeat the last fragment (same source, same LDS bytes), so every wave issues the same
  // number of copies per k-step and the in-flight counts below hold for all of them.
  constexpr int kPer = (R::kFrags + WM * WN - 1) / (WM * WN);
  constexpr int kReads = MF + NF;                     // LDS reads per wave per k-step
  static_assert(NS >= 5 && kReads <= 15, "DMA GEMM shape");
  extern __shared__ float lds[];
  const uint32_t lds_base = (uint32_t)(size_t)((__attribute__((address_space(3))) float*)lds);
  const int M = a.device_m ? *a.device_m : a.M;
  const TileCoord at = xcd_tile(blockIdx.x, n_tiles, m_tiles, units);
  const int split = at.split, tile_n = at.tile_n, tile_m = at.tile_m;
  if (!at.valid || tile_m * BM >= M) return;  // uniform over the workgroup
  const int tile = tile_m * n_tiles + tile_n;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int wm = wave / WN, wn = wave % WN;
  const int KT = (int)(a.Kp >> 5);
  const int per = (KT + a.ksplit - 1) / a.ksplit;
  const int kt0 = split * per, kt1 = min(KT, kt0 + per);
  const int steps = kt1 > kt0 ? kt1 - kt0 : 0;
  const size_t frag_stride = (size_t)KT * 64;  // half8s between fragment rows
  const char* X = reinterpret_cast<const char*>(a.x_hi) + (size_t)tile_m * (BM / 16) * frag_stride * 16;
  const char* W = reinterpret_cast<const char*>(a.w_hi) + (size_t)tile_n * (BN / 16) * frag_stride * 16;
  const uint32_t lane_bytes = (uint32_t)lane * 16;
  // K-steps come in pairs: an odd count gets one more, a copy of the last k-step whose
  // MFMAs are skipped.
  const int stages = (steps + 1) & ~1;
  const int kt_last = max(kt0, kt1 - 1);
  // This wave's copies of k-step st into buffer st % NS (the caller keeps st < stages).
  auto issue = [&](int st) {
    const uint32_t buf = lds_base + (uint32_t)(st % NS) * R::kBytes;
    const size_t k = (size_t)min(kt0 + st, kt_last) * 1024;
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      const int f = min(wave * kPer + c, R::kFrags - 1);
      const char* src = f < BM / 16 ? X + (size_t)f * frag_stride * 16 : W + (size_t)(f - BM / 16) * frag_stride * 16;
      lds_copy16(src + k, lane_bytes, __builtin_amdgcn_readfirstlane(buf + (uint32_t)f * 1024));
    }
  };
  const half8* ldsh = reinterpret_cast<const half8*>(lds);
  auto read = [&](int st, half8 (&x)[MF], half8 (&w)[NF]) {
    const half8* stage = ldsh + (size_t)(st % NS) * (R::kBytes / 16) + lane;
#pragma unroll
    for (int i = 0; i < MF; ++i) x[i] = stage[(wm * MF + i) * 64];
#pragma unroll
    for (int n = 0; n < NF; ++n) w[n] = stage[(BM / 16 + wn * NF + n) * 64];
  };

  floatx4 acc[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int n = 0; n < NF; ++n) acc[i][n] = floatx4{0.f, 0.f, 0.f, 0.f};
  auto multiply = [&](const half8 (&x)[MF], const half8 (&w)[NF]) {
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int n = 0; n < NF; ++n) acc[i][n] = mfma(w[n], x[i], acc[i][n]);
  };

  // Copies are issued in k-step order and only for k-steps < stages: 0 .. NS - 2 before
  // the loop, then st + NS - 1 and st + NS after the barrier at pair st (even), into the
  // buffers of st - 1 and st, whose k-steps were read into registers during pair st - 2
  // (st's before the loop for st = 0). At that barrier k-steps st + 1 and st + 2 must have
  // landed; when all of st + 3 .. st + NS - 2 were issued, NS - 4 k-steps may stay in
  // flight, otherwise none. A copy issued at barrier st is needed at barrier st + 4: two
  // pairs of MFMAs cover its latency. Every LDS read a wave issued has returned before it
  // reaches the barrier (the last group was issued a half-iteration of MFMAs earlier), so
  // the refilled buffers are free, and the register sets are complete when their MFMAs start.
  for (int st = 0; st < NS - 1; ++st)
    if (st < stages) issue(st);
  if (stages >= NS - 1)
    stage_barrier<(NS - 2) * kPer, 0>();
  else
    stage_barrier<0, 0>();
  half8 xa[MF], wa[NF], xb[MF], wb[NF];
  read(0, xa, wa);
  for (int st = 0; st < stages; st += 2) {
    wait_counts<63, 0>();  // on both paths below; stated once for the compiler's benefit
    if (st + NS - 2 < stages)
      stage_barrier<(NS - 4) * kPer, 0>();
    else
      stage_barrier<0, 0>();
    if (st + NS - 1 < stages) issue(st + NS - 1);
    if (st + NS < stages) issue(st + NS);
    // Each register set is read a whole half-iteration of MFMAs before it is used; the
    // scheduling barriers keep the compiler from sinking the reads next to their uses, and
    // the explicit waits (on reads issued that long ago) keep it from waiting on the
    // reads just issued.
    read(st + 1, xb, wb);
    __builtin_amdgcn_sched_barrier(0);
    multiply(xa, wa);
    __builtin_amdgcn_sched_barrier(0);
    wait_counts<63, 0>();
    read(st + 2, xa, wa);  // past the last k-step this reads a buffer that is never used
    __builtin_amdgcn_sched_barrier(0);
    // An odd step count ends on a copy of the last k-step, whose MFMAs are skipped (a
    // workgroup-uniform branch: zeroing the operand instead costs a select per register
    // in every pair).
    if (st + 1 < steps) multiply(xb, wb);
  }
  // Drain the copies still in flight before the workgroup's LDS can be reused.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Lane (q, t) of accumulator (i, n) holds row 16 (MF wm + i) + t, features 16 (NF wn + n)
  // + 4 q .. + 3 of the tile.
  const int q4 = (lane >> 4) * 4, t16 = lane & 15;
  const int row0 = tile_m * BM + wm * MF * 16, col0 = tile_n * BN + wn * NF * 16;
  if (a.ksplit > 1 && a.defer_reduce) {
    float* ws = a.workspace + (size_t)split * a.M * a.N;
    const bool vec = (a.N & 3) == 0;
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      const int row = row0 + i * 16 + t16;
      if (row >= M) continue;
#pragma unroll
      for (int n = 0; n < NF; ++n) {
        const int col = col0 + n * 16 + q4;
        float* dst = ws + (size_t)row * a.N + col;
        if (vec && col + 3 < a.N) {
          *reinterpret_cast<floatx4*>(dst) = acc[i][n];
        } else {
#pragma unroll
          for (int t = 0; t < 4; ++t)
            if (col + t < a.N) dst[t] = acc[i][n][t];
        }
      }
    }
    return;
  }
  if (a.ksplit > 1) {
    // Partial tile of this K split (row-major BM x BN), summed by gemm_reduce_kernel.
    float* ws = a.workspace + ((size_t)tile * a.ksplit + split) * BM * BN;
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int n = 0; n < NF; ++n)
        *reinterpret_cast<floatx4*>(ws + (wm * MF * 16 + i * 16 + t16) * BN + wn * NF * 16 + n * 16 + q4) = acc[i][n];
    return;
  }
  if (a.epilogue == kEpiSwiglu) {
    // The wave's features are 64-wide groups: 32 gate features (fragments 4g, 4g + 1),
    // then the 32 matching up features (fragments 4g + 2, 4g + 3).
#pragma unroll
    for (int gq = 0; gq < NF / 4; ++gq) {
      const uint64_t g = (uint64_t)col0 / 64 + gq;
#pragma unroll
      for (int i = 0; i < MF; ++i) {
        const int row = row0 + i * 16 + t16;
        if (row >= M) continue;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint64_t col = g * 32 + h * 16 + q4;
          if (col >= a.out_cols_padded) continue;
          const floatx4 gate = acc[i][4 * gq + h], up = acc[i][4 * gq + 2 + h];
          half4 vh, vl;
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float y = silu_mul(gate[t], up[t]);
            vh[t] = to_half(y);
            vl[t] = to_half((y - (float)vh[t]) * kLoScale);
          }
          const uint64_t at = flayout_index(row, col, a.out_cols_padded);
          *reinterpret_cast<half4*>(a.out_hi + at) = vh;
          if (a.out_lo) *reinterpret_cast<half4*>(a.out_lo + at) = vl;
        }
      }
    }
    return;
  }
  const bool vec = (a.N & 3) == 0 && (a.ldo & 3) == 0;
#pragma unroll
  for (int i = 0; i < MF; ++i) {
    const int row = row0 + i * 16 + t16;
    if (row >= M) continue;
#pragma unroll
    for (int n = 0; n < NF; ++n) {
      const int col = col0 + n * 16 + q4;
      if (col >= a.N) continue;
      float* out = a.out + (size_t)row * a.ldo + col;
      const floatx4 v = acc[i][n];
      if (vec && col + 3 < a.N) {
        floatx4* o4 = reinterpret_cast<floatx4*>(out);
        if (a.epilogue == kEpiResidual) {
          floatx4 s4 = *o4;
          s4[0] += v[0];
          s4[1] += v[1];
          s4[2] += v[2];
          s4[3] += v[3];
          *o4 = s4;
        } else {
          *o4 = v;
        }
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (col + t >= a.N) continue;
          if (a.epilogue == kEpiResidual)
            out[t] += v[t];
          else
            out[t] = v[t];
        }
      }
    }
  }
}

template <int MF, int NF, int WM, int WN, int WK, int P, int PREC>
void run(dim3 grid, int threads, size_t lds, hipStream_t stream, const GemmArgs& a, int n_tiles,
         int tiles, int tiles_padded) {
  static const bool configured = [lds] {
    // Tiles above 64 KiB of LDS need the kernel's dynamic-LDS limit raised (160 KiB on gfx950).
    HIP_CHECK(hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_kernel<MF, NF, WM, WN, WK, P, PREC>),
        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    return true;
  }();
  (void)configured;
  observed(kernel_name<MF, NF, WM, WN, WK, P, PREC>("gemm_kernel"), [&] { gemm_kernel<MF, NF, WM, WN, WK, P, PREC><<<grid, threads, lds, stream>>>(a, n_tiles, tiles,
                                                                           tiles_padded); });
}

// Fits the K split to the workspace: tile partials for the reduce kernel, or whole partial
// output matrices when the consumer sums them.
int fit_ksplit(const GemmArgs& a, int ksplit, size_t tiles, size_t tile_floats) {
  const size_t need = a.defer_reduce ? (size_t)a.M * a.N : tiles * tile_floats;
  return (size_t)ksplit * need > a.workspace_floats ? 1 : ksplit;
}

template <int MF, int NF, int WM, int WN, int WK, int P>
int launch_config(hipStream_t stream, GemmArgs a, int prec, int rows_bound, int target_ctas,
                  int min_k_per_wave, int forced_ksplit) {
  constexpr int BM = 16 * MF * WM, BN = 16 * NF * WN, NT = 64 * WM * WN * WK;
  const int n_tiles = (a.N + BN - 1) / BN;
  const int m_tiles = (rows_bound + BM - 1) / BM;
  const int KT = (int)(a.Kp >> 5);
  if ((uint64_t)n_tiles * BN > a.w_rows_padded) fail(HLLM_INTERNAL, "GEMM tile exceeds the weight padding");
  if ((uint64_t)m_tiles * BM > a.x_rows_padded) fail(HLLM_INTERNAL, "GEMM tile exceeds the activation padding");
  const int tiles = n_tiles * m_tiles;
  int ksplit = 1;
  if (forced_ksplit > 0) {
    ksplit = forced_ksplit;
  } else if (tiles < target_ctas) {
    ksplit = (target_ctas + tiles - 1) / tiles;
  }
  ksplit = std::min(ksplit, std::max(1, KT / (WK * min_k_per_wave)));
  const int tiles_padded = (tiles + kXcds - 1) / kXcds * kXcds;
  ksplit = fit_ksplit(a, ksplit, tiles, (size_t)BM * BN);
  a.ksplit = ksplit;
  const size_t lds = ((size_t)WK * BM * (BN + 4) + 4) * sizeof(float);
  dim3 grid(tiles_padded * ksplit, 1, 1);
  switch (prec) {
    case kF16:
      run<MF, NF, WM, WN, WK, P, kF16>(grid, NT, lds, stream, a, n_tiles, tiles, tiles_padded);
      break;
    case kSplitA:
      run<MF, NF, WM, WN, WK, P, kSplitA>(grid, NT, lds, stream, a, n_tiles, tiles, tiles_padded);
      break;
    default:
      run<MF, NF, WM, WN, WK, P, kSplitAB>(grid, NT, lds, stream, a, n_tiles, tiles, tiles_padded);
      break;
  }
  if (ksplit > 1 && a.defer_reduce) return ksplit;
  if (ksplit > 1) {
    const int64_t threads = (int64_t)tiles * BM * BN / 8;
    observed(kernel_name<BM, BN>("gemm_reduce_kernel"), [&] { gemm_reduce_kernel<BM, BN><<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(a, n_tiles, tiles); });
  }
  return 0;
}

template <int MF, int NFW, int KC, int P>
int launch_xlds(hipStream_t stream, GemmArgs a, int prec, int rows_bound, int target_ctas,
                 int forced_ksplit) {
  if constexpr (MF > 8) {
    // Tiles above 128 rows hold their accumulators in AGPRs; the split-precision variants
    // would need twice as many, so they run on 128-row tiles.
    if (prec != kF16) return launch_xlds<8, NFW, KC, P>(stream, a, prec, rows_bound, target_ctas, forced_ksplit);
  }
  constexpr int BM = 16 * MF, BN = 64 * NFW;
  const int n_tiles = (a.N + BN - 1) / BN;
  const int m_tiles = (rows_bound + BM - 1) / BM;
  const int tiles = n_tiles * m_tiles;
  const int KT = (int)(a.Kp >> 5);
  if ((uint64_t)n_tiles * BN > a.w_rows_padded) fail(HLLM_INTERNAL, "GEMM tile exceeds the weight padding");
  if ((uint64_t)m_tiles * BM > a.x_rows_padded) fail(HLLM_INTERNAL, "GEMM tile exceeds the activation padding");
  int ksplit = forced_ksplit > 0 ? forced_ksplit : (tiles < target_ctas ? (target_ctas + tiles - 1) / tiles : 1);
  ksplit = std::min(ksplit, std::max(1, KT / (2 * KC)));
  ksplit = fit_ksplit(a, ksplit, tiles, (size_t)BM * BN);
  a.ksplit = ksplit;
  const int xp = prec >= kSplitA ? 2 : 1;
  const size_t lds = (size_t)2 * MF * KC * 64 * xp * 16;
  const int units = ksplit * n_tiles;
  dim3 grid(xcd_grid(units, m_tiles));
  auto go = [&](auto kernel, const char* name) {
    static const bool configured = [kernel] {
      HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
      return true;
    }();
    (void)configured;
    observed(name, [&] { kernel<<<grid, 256, lds, stream>>>(a, n_tiles, m_tiles, units); });
  };
  if constexpr (MF > 8) {
    go(&gemm_xlds_kernel<MF, NFW, KC, P, kF16>, kernel_name<MF, NFW, KC, P, kF16>("gemm_xlds_kernel"));
  } else {
    switch (prec) {
      case kF16:
        go(&gemm_xlds_kernel<MF, NFW, KC, P, kF16>, kernel_name<MF, NFW, KC, P, kF16>("gemm_xlds_kernel"));
        break;
      case kSplitA:
        go(&gemm_xlds_kernel<MF, NFW, KC, P, kSplitA>, kernel_name<MF, NFW, KC, P, kSplitA>("gemm_xlds_kernel"));
        break;
      default:
        go(&gemm_xlds_kernel<MF, NFW, KC, P, kSplitAB>, kernel_name<MF, NFW, KC, P, kSplitAB>("gemm_xlds_kernel"));
        break;
    }
  }
  if (ksplit > 1 && a.defer_reduce) return ksplit;
  if (ksplit > 1) {
    const int64_t threads = (int64_t)tiles * BM * BN / 8;
    observed(kernel_name<BM, BN>("gemm_reduce_kernel"), [&] { gemm_reduce_kernel<BM, BN><<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(a, n_tiles, tiles); });
  }
  return 0;
}

template <int BM, int WM, int WN>
int launch_dma(hipStream_t stream, GemmArgs a, int prec, int rows_bound, int target_ctas, int forced_ksplit) {
  using namespace dma;
  using R = Ring<BM>;
  if (prec != kF16) return launch_xlds<8, 4, 4, 2>(stream, a, prec, rows_bound, target_ctas, forced_ksplit);
  const int n_tiles = (a.N + BN - 1) / BN;
  const int m_tiles = (rows_bound + BM - 1) / BM;
  const int tiles = n_tiles * m_tiles;
  const int KT = (int)(a.Kp >> 5);
  if ((uint64_t)n_tiles * BN > a.w_rows_padded) fail(HLLM_INTERNAL, "GEMM tile exceeds the weight padding");
  if ((uint64_t)m_tiles * BM > a.x_rows_padded) fail(HLLM_INTERNAL, "GEMM tile exceeds the activation padding");
  int ksplit = forced_ksplit > 0 ? forced_ksplit : (tiles < target_ctas ? (target_ctas + tiles - 1) / tiles : 1);
  ksplit = std::min(ksplit, std::max(1, KT / (2 * R::kBuffers)));  // at least two rings of k-steps per split
  ksplit = fit_ksplit(a, ksplit, tiles, (size_t)BM * BN);
  a.ksplit = ksplit;
  static const bool configured = [] {
    HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_dma_kernel<BM, WM, WN>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, R::kLds));
    return true;
  }();
  (void)configured;
  const int units = ksplit * n_tiles;
  const dim3 grid(xcd_grid(units, m_tiles));
  observed(kernel_name<BM, WM, WN>("gemm_dma_kernel"), [&] {
    gemm_dma_kernel<BM, WM, WN><<<grid, 64 * WM * WN, R::kLds, stream>>>(a, n_tiles, m_tiles, units);
  });
  if (ksplit > 1 && a.defer_reduce) return ksplit;
  if (ksplit > 1) {
    const int64_t threads = (int64_t)tiles * BM * BN / 8;
    observed(kernel_name<BM, BN>("gemm_reduce_kernel"), [&] { gemm_reduce_kernel<BM, BN><<<(unsigned)((threads + 255) / 256), 256, 0, stream>>>(a, n_tiles, tiles); });
  }
  return 0;
}

}  // namespace


// Decode projections (F16, at most 16 * MF rows): every wave streams the weights of its own
// NFW fragment rows (16 features each) over the workgroup's K range through a P-deep register
// ring, so weights are read exactly once and no K-wave reduction is needed. The rows'
// activations are staged in LDS in double-buffered chunks of KC k-steps, once per workgroup
// of WAVES waves. With PAIR, a wave's two fragment rows are a gate fragment and its up
// fragment (rows 4g + h and 4g + 2 + h of the interleaved gate/up matrix), so SwiGLU is
// applied from the accumulators and no split-K reduction is ever needed for it. K is split
// across workgroups only for deferred consumers (the K-split partials are summed in split
// order by the kernel that reads the projection). With `whole` (deferred projections whose
// split's activations fit in LDS), the split's activation fragments are copied into LDS once,
// straight from memory (global_load_lds), before the loop: the activations of a decode pass
// were just written by the previous kernel and miss in this XCD's L2, so one wait for all
// of them replaces one per chunk, and the waves then run without per-chunk barriers.
template <int MF, int WAVES, int NFW, int KC, int P, bool PAIR, int PW>
__global__ void __launch_bounds__(64 * WAVES) gemm_decode_kernel(GemmArgs a, int n_tiles, int whole) {
  constexpr int NT = 64 * WAVES, FR = WAVES * NFW;
  constexpr int CHUNK = MF * KC * 64;  // half8s per staged chunk
  constexpr int PIECES = (CHUNK + NT - 1) / NT;
  static_assert(KC % P == 0, "the ring slot of a k-step must be a compile-time index");
  static_assert(PW * NFW < 64, "the whole path's weight loads in flight fit the wait count");
  static_assert(!PAIR || (NFW == 2 && WAVES % 2 == 0), "gate/up pairs: two fragment rows per wave");
  extern __shared__ float lds[];
  half8* xs = reinterpret_cast<half8*>(lds);  // [2][MF][KC][64]
  const int M = a.device_m ? *a.device_m : a.M;
  const int tile_n = blockIdx.x % n_tiles, split = blockIdx.x / n_tiles;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int KT = (int)(a.Kp >> 5);
  const int per = ((KT + a.ksplit - 1) / a.ksplit + KC - 1) / KC * KC;
  const int kt0 = split * per, kt1 = min(KT, kt0 + per);
  const int steps = kt1 > kt0 ? kt1 - kt0 : 0;
  const int chunks = (steps + KC - 1) / KC;
  const size_t frag_stride = (size_t)KT * 64;
  // This wave's fragment rows.
  int frag[NFW];
  if constexpr (PAIR) {
    const int group = tile_n * (FR / 4) + (wave >> 1), h = wave & 1;
    frag[0] = 4 * group + h;
    frag[1] = 4 * group + 2 + h;
  } else {
#pragma unroll
    for (int j = 0; j < NFW; ++j) frag[j] = tile_n * FR + wave * NFW + j;
  }
  const half8* W[NFW];
#pragma unroll
  for (int j = 0; j < NFW; ++j) W[j] = reinterpret_cast<const half8*>(a.w_hi) + (size_t)frag[j] * frag_stride + lane;
  const half8* X = reinterpret_cast<const half8*>(a.x_hi);

  floatx4 acc[MF][NFW];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < NFW; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  half8 stage[PIECES];
  auto fetch_x = [&](int c) {
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      const int e = threadIdx.x + q * NT;  // (i, j, lane) flattened
      if (e < CHUNK) {
        const int ln = e & 63, j = (e >> 6) % KC, i = e / (64 * KC);
        const int kt = kt0 + c * KC + j;
        stage[q] = kt < kt1 ? X[(size_t)i * frag_stride + (size_t)kt * 64 + ln] : half8{};
      }
    }
  };
  auto store_x = [&](int buf) {
#pragma unroll
    for (int q = 0; q < PIECES; ++q) {
      const int e = threadIdx.x + q * NT;
      if (e < CHUNK) xs[buf * CHUNK + e] = stage[q];
    }
  };
  half8 rb[P][NFW];
  // Unconditional weight loads (see gemm_kernel); past the range they re-read the last k-step.
  const int kt_last = max(0, min(kt1, KT) - 1);
  auto load_w = [&](int slot, int kt) {
    kt = min(kt, kt_last);
#pragma unroll
    for (int j = 0; j < NFW; ++j) rb[slot][j] = __builtin_nontemporal_load(W[j] + (size_t)kt * 64);
  };
  if (!PAIR && whole) {
    // LDS holds fragment (i, s) of the split at (i * per + s) * 64 half8s. The copies are
    // issued before the first PW k-steps of weights and waited for alone (loads complete in
    // issue order), so the weight ring stays in flight across the barrier.
    half8 rw[PW][NFW];
    auto load_ww = [&](int slot, int kt) {
      kt = min(kt, kt_last);
#pragma unroll
      for (int j = 0; j < NFW; ++j) rw[slot][j] = __builtin_nontemporal_load(W[j] + (size_t)kt * 64);
    };
    const uint32_t lds_base = (uint32_t)(size_t)((__attribute__((address_space(3))) float*)lds);
#pragma unroll
    for (int i = 0; i < MF; ++i)
      for (int s = wave; s < steps; s += WAVES)  // wave-uniform
        lds_copy16(X + (size_t)i * frag_stride + (size_t)(kt0 + s) * 64, (uint32_t)lane * 16,
                   lds_base + (uint32_t)(i * per + s) * 1024);
#pragma unroll
    for (int sl = 0; sl < PW; ++sl) load_ww(sl, kt0 + sl);
    wait_counts<PW * NFW, 15>();
    __syncthreads();
    for (int s0 = 0; s0 < steps; s0 += PW) {
#pragma unroll
      for (int j = 0; j < PW; ++j) {
        const int step = s0 + j;
        if (step < steps) {
#pragma unroll
          for (int i = 0; i < MF; ++i) {
            const half8 x = xs[(i * per + step) * 64 + lane];
#pragma unroll
            for (int n = 0; n < NFW; ++n) acc[i][n] = mfma(rw[j][n], x, acc[i][n]);
          }
        }
        load_ww(j, kt0 + step + PW);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  } else {
  // The first chunk's activation loads go out before the weight ring's, so that staging
  // them waits for them alone.
  if (chunks > 0) fetch_x(0);
#pragma unroll
  for (int sl = 0; sl < P; ++sl) load_w(sl, kt0 + sl);
  if (chunks > 0) store_x(0);
  __syncthreads();
  for (int c = 0; c < chunks; ++c) {
    if (c + 1 < chunks) fetch_x(c + 1);
    const half8* xb = xs + (c & 1) * CHUNK;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int step = c * KC + j;
      const int slot = j % P;
      if (step < steps) {
#pragma unroll
        for (int i = 0; i < MF; ++i) {
          const half8 x = xb[(i * KC + j) * 64 + lane];
#pragma unroll
          for (int n = 0; n < NFW; ++n) acc[i][n] = mfma(rb[slot][n], x, acc[i][n]);
        }
      }
      load_w(slot, kt0 + step + P);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (c + 1 < chunks) store_x((c + 1) & 1);
    __syncthreads();
  }
  }

  // Lane (q = lane / 16, t = lane % 16) of accumulator (i, n) holds row 16 i + t, features
  // 16 frag[n] + 4 q .. + 3.
  const int q4 = (lane >> 4) * 4, t16 = lane & 15;
  if constexpr (PAIR) {
    const int group = tile_n * (FR / 4) + (wave >> 1), h = wave & 1;
    const uint64_t col = (uint64_t)group * 32 + h * 16 + q4;
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      const int row = i * 16 + t16;
      if (row >= M || col >= a.out_cols_padded) continue;
      half4 vh;
#pragma unroll
      for (int t = 0; t < 4; ++t) vh[t] = to_half(silu_mul(acc[i][0][t], acc[i][1][t]));
      *reinterpret_cast<half4*>(a.out_hi + flayout_index(row, col, a.out_cols_padded)) = vh;
    }
    return;
  }
  if (a.epilogue == kEpiArgmax) {
    // No output: this workgroup's first maximum of every row over its features. The four
    // lanes of a row combine through shuffles, then the waves in wave order through LDS
    // (the staged operand is no longer read); the order does not change the result.
    Best* cand = reinterpret_cast<Best*>(lds);  // [WAVES][16 * MF]
    __syncthreads();
    bool bad = false;
#pragma unroll
    for (int i = 0; i < MF; ++i) {
      const int row = i * 16 + t16;
      Best b{-INFINITY, 0x7fffffff};
#pragma unroll
      for (int n = 0; n < NFW; ++n)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int col = frag[n] * 16 + q4 + t;
          if (row < M && col < a.N) {
            const float v = acc[i][n][t];
            bad |= !isfinite(v);
            b = better(b, Best{v, col});
          }
        }
      for (int o = 16; o < 64; o <<= 1) b = better(b, Best{__shfl_xor(b.value, o, 64), __shfl_xor(b.index, o, 64)});
      if (lane < 16) cand[wave * 16 * MF + row] = b;
    }
    if (bad) atomicOr(a.argmax_flags, 2);
    __syncthreads();
    for (int row = threadIdx.x; row < 16 * MF; row += NT) {
      if (row >= M) continue;
      Best b = cand[row];
      for (int w = 1; w < WAVES; ++w) b = better(b, cand[w * 16 * MF + row]);
      a.argmax_val[(size_t)row * a.argmax_parts + tile_n] = b.value;
      a.argmax_idx[(size_t)row * a.argmax_parts + tile_n] = b.index;
    }
    return;
  }
  const bool partial = a.ksplit > 1;  // deferred: a row-major [M][N] matrix per K split
  float* base = partial ? a.workspace + (size_t)split * a.M * a.N : a.out;
  const int ld = partial ? a.N : a.ldo;
  const bool vec = (a.N & 3) == 0 && (ld & 3) == 0;
#pragma unroll
  for (int i = 0; i < MF; ++i) {
    const int row = i * 16 + t16;
    if (row >= M) continue;
#pragma unroll
    for (int n = 0; n < NFW; ++n) {
      const int col = frag[n] * 16 + q4;
      if (col >= a.N) continue;
      const floatx4 v = acc[i][n];
      float* dst = base + (size_t)row * ld + col;
      if (!partial && a.epilogue == kEpiResidual) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (col + t < a.N) dst[t] += v[t];
      } else if (vec && col + 3 < a.N) {
        *reinterpret_cast<floatx4*>(dst) = v;
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (col + t < a.N) dst[t] = v[t];
      }
    }
  }
}

// LDS a decode workgroup may give to its split's whole activation range.
constexpr size_t kDecodeWholeLds = 144 * 1024;
namespace {
int env_int(const char* name, int fallback);
}  // namespace

// Launches the decode kernel with `waves` waves per workgroup (4, 8 or 16) and the given
// K split; returns the number of deferred partials (0: the epilogue has been applied).
template <int MF, int NFW, int KC, int P, bool PAIR, int PW>
int launch_decode_waves(hipStream_t stream, GemmArgs a, int waves, int ksplit) {
  const int fr = waves * NFW;
  const int n_tiles = (a.N + 16 * fr - 1) / (16 * fr);
  if ((uint64_t)n_tiles * fr * 16 > a.w_rows_padded) fail(HLLM_INTERNAL, "GEMM tile exceeds the weight padding");
  if ((uint64_t)MF * 16 > a.x_rows_padded) fail(HLLM_INTERNAL, "GEMM tile exceeds the activation padding");
  if (ksplit > 1 && (!a.defer_reduce || PAIR)) fail(HLLM_INTERNAL, "decode GEMM splits K only for deferred consumers");
  if (ksplit > 1 && (size_t)ksplit * a.M * a.N > a.workspace_floats) ksplit = 1;
  a.ksplit = ksplit;
  // A deferred projection stages its split's activations whole when they fit in LDS
  // (HLLM_ROCM_DECODE_WHOLE=0, read at every launch: chunk by chunk, the path of K ranges
  // that do not fit; for tests).
  const int KT = (int)(a.Kp >> 5);
  const int per = ((KT + ksplit - 1) / ksplit + KC - 1) / KC * KC;
  const size_t whole_lds = (size_t)MF * per * 1024;
  const int whole = !PAIR && whole_lds <= kDecodeWholeLds && env_int("HLLM_ROCM_DECODE_WHOLE", 1) != 0;
  const size_t lds = whole ? whole_lds : 2 * (size_t)MF * KC * 64 * 16;
  const dim3 grid((unsigned)(n_tiles * ksplit));
  auto go = [&](auto kernel, const char* name) {
    static const bool configured = [kernel] {
      HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
      return true;
    }();
    (void)configured;
    observed(name, [&] { kernel<<<grid, 64 * waves, lds, stream>>>(a, n_tiles, whole); });
  };
  if (waves >= 8)
    go(&gemm_decode_kernel<MF, 8, NFW, KC, P, PAIR, PW>,
       kernel_name<MF, 8, NFW, KC, P, PAIR ? 1 : 0, PW>("gemm_decode_kernel"));
  else
    go(&gemm_decode_kernel<MF, 4, NFW, KC, P, PAIR, PW>,
       kernel_name<MF, 4, NFW, KC, P, PAIR ? 1 : 0, PW>("gemm_decode_kernel"));
  return ksplit > 1 ? ksplit : 0;
}

// Configuration table (ids are stable for the tuning harness):
//   0..2: decode, BM = 16/32/64, BN = 64, four K-waves, ring of 4 k-steps
//   3:    prefill, 128 x 128, 2 x 2 waves, ring of 2 k-steps
//   4..6: decode, BM = 16/32/64, BN = 128 (NF = 8), two K-waves, ring of 4
int launch_gemm_config(hipStream_t stream, const GemmArgs& args, int prec, int rows_bound, int cus,
                        int config, int forced_ksplit) {
  switch (config) {
    case 0:
      return launch_config<1, 4, 1, 1, 4, 4>(stream, args, prec, rows_bound, cus * 5 / 8, 2, forced_ksplit);
      break;
    case 1:
      return launch_config<2, 4, 1, 1, 4, 4>(stream, args, prec, rows_bound, cus * 5 / 8, 2, forced_ksplit);
      break;
    case 2:
      return launch_config<4, 4, 1, 1, 4, 4>(stream, args, prec, rows_bound, cus * 5 / 8, 2, forced_ksplit);
      break;
    case 4:
      return launch_config<1, 8, 1, 1, 2, 4>(stream, args, prec, rows_bound, 2 * cus, 2, forced_ksplit);
      break;
    case 5:
      return launch_config<2, 8, 1, 1, 2, 4>(stream, args, prec, rows_bound, 2 * cus, 2, forced_ksplit);
      break;
    case 6:
      return launch_config<4, 8, 1, 1, 2, 4>(stream, args, prec, rows_bound, 2 * cus, 2, forced_ksplit);
      break;
    case 7:  // activation-staged: BM 64 x BN 256
      return launch_xlds<4, 4, 4, 4>(stream, args, prec, rows_bound, 2 * cus, forced_ksplit);
      break;
    case 8:  // BM 128 x BN 256, chunks of 2 k-steps, ring of 2
      return launch_xlds<8, 4, 2, 2>(stream, args, prec, rows_bound, 2 * cus, forced_ksplit);
      break;
    case 9:  // BM 128 x BN 256, chunks of 4, ring of 2
      return launch_xlds<8, 4, 4, 2>(stream, args, prec, rows_bound, 2 * cus, forced_ksplit);
      break;
    case 10:  // BM 128 x BN 256, chunks of 4, ring of 4
      return launch_xlds<8, 4, 4, 4>(stream, args, prec, rows_bound, 2 * cus, forced_ksplit);
      break;
    case 11:  // BM 32 x BN 256
      return launch_xlds<2, 4, 4, 4>(stream, args, prec, rows_bound, 2 * cus, forced_ksplit);
      break;
    case 12:  // BM 64 x BN 256, chunks of 8, ring of 4
      return launch_xlds<4, 4, 8, 4>(stream, args, prec, rows_bound, 2 * cus, forced_ksplit);
      break;
    case 13:  // BM 192 x BN 256, chunks of 2, ring of 2 (accumulators in AGPRs, one wave per SIMD)
      return launch_xlds<12, 4, 2, 2>(stream, args, prec, rows_bound, 2 * cus, forced_ksplit);
    case 14:  // BM 128 x BN 256, both operands copied to LDS (F16 execution), 2 x 2 waves
      return launch_dma<128, 2, 2>(stream, args, prec, rows_bound, cus, forced_ksplit);
    case 15:  // as 14 with 2 x 4 waves (two per SIMD), each 64 rows x 64 features
      return launch_dma<128, 2, 4>(stream, args, prec, rows_bound, cus, forced_ksplit);
    case 16:  // BM 256 x BN 256, 2 x 4 waves, each 128 rows x 64 features
      return launch_dma<256, 2, 4>(stream, args, prec, rows_bound, cus, forced_ksplit);
    case 18:  // BM 192 x BN 256, 2 x 4 waves, each 96 rows x 64 features (28 copies, 4 per wave)
      return launch_dma<192, 2, 4>(stream, args, prec, rows_bound, cus, forced_ksplit);
    default:
      return launch_config<4, 4, 2, 2, 1, 2>(stream, args, prec, rows_bound, cus, 8, forced_ksplit);
      break;
  }
}

namespace {

struct Choice {
  int config;
  int ksplit;  // 0: the configuration's own rule
};

// Projection configuration by pass rows and shape, from sweeps of the Qwen3 projection
// shapes on MI355X with weights streamed from HBM:
//  - up to 64 rows: the register-streaming decode kernels (BM 16/32/64), except for very
//    wide outputs (gate+up, LM head) with more than 32 rows, where staging the activations
//    in LDS once per 256-feature tile wins;
//  - more rows: the activation-staged kernel, BM 64, or BM 128 from 384 rows; wide outputs
//    from 192 to 768 rows use the kernels that copy both operands to LDS (BM 128 below
//    448 rows, BM 256 from there), and BM 128 activation-staged tiles beyond; so do the
//    deferred projections of chunk-sized F16 passes (BM 128, fewer K splits than the
//    activation-staged kernel needs, so their consumers also read fewer partials).
// K is split while there are few output tiles. When the consumer sums the partials
// (`deferred`) a split costs one partial write, so about 220-280 workgroups are targeted;
// otherwise a reduce kernel reads every partial back, so splits stop at about 200
// workgroups, in powers of two.
Choice gemm_choice(int rows, int n, uint64_t kp, bool deferred, bool f16, int cus) {
  const bool wide = n >= 16384;
  const auto rounded = [](double x) { return std::max(1, (int)(x + 0.5)); };
  if (f16 && deferred && rows > 64 && rows <= 768) {
    // Deferred projections of chunk-sized F16 passes, with the most K splits whose
    // workgroups fit every XCD's CUs at once (xcd_tile; one workgroup per CU: a second round
    // costs up to a third more, q/k/v at 160 rows 18.4 -> 24.1 us).
    const int n_tiles = (n + 255) / 256, per_xcd = std::max(1, cus / kXcds);
    const auto splits = [&](int bm, int least, int most) {
      const int m_tiles = (rows + bm - 1) / bm;
      int ks = most;
      while (ks > least && (n_tiles * ks + kXcds - 1) / kXcds * m_tiles > per_xcd) --ks;
      return ks;
    };
    if (rows >= 224) {
      // From 224 rows both operands are copied to LDS in 128 x 256 tiles (2 to 8 splits).
      // Measured on the Qwen3-4B projections against the activation-staged kernel: down 28
      // against 34-42 us from 288 to 384 rows, q/k/v 20 / 23 against 24 / 27 us at 224 /
      // 352 rows, o within 1 us. 192 x 256 tiles instead when they allow at least twice the
      // K splits (a quarter less work per workgroup) and those splits still hold 32 k-steps
      // or more: down of 513-576-row passes (three row tiles against five), 43.7 -> 37.2 us.
      // Where 192-row tiles gain less they measured slower (q/k/v at 320-384 rows), and o
      // (16 k-steps per split) gains 0.6 us while its consumer reads twice the partials.
      const int ks128 = splits(128, 2, 8), ks192 = splits(192, 2, 8);
      const bool long_splits = (int)(kp >> 5) / ks192 >= 32;
      return ks192 >= 2 * ks128 && long_splits ? Choice{18, ks192} : Choice{15, ks128};
    }
    // 65-223 rows: 64-row activation-staged tiles (at least two chunks per split), or the
    // 128-row LDS-copy tiles where they allow more than twice the K splits (less work per
    // workgroup). Measured at 96-208 rows: o 12.0-15.3 us, down 21.5-26.7, q/k/v 13.8-18.3
    // (q/k/v at 160-208 rows 24-28 us with the earlier rule of ~280 workgroups, which took
    // a second round of workgroups on some XCDs).
    const int ks64 = splits(64, 1, std::min(8, std::max(1, (int)(kp >> 5) / 16)));
    const int ks128 = splits(128, 2, 8);
    return 2 * ks64 < ks128 ? Choice{15, ks128} : Choice{12, ks64};
  }
  if (rows <= 64 && (!wide || rows <= 32)) {
    const int config = rows <= 16 ? 0 : rows <= 32 ? 1 : 2;
    const int tiles = (n + 63) / 64;
    const int cap = std::max(1, (int)(kp >> 5) / 8);  // at least two k-steps per K-wave
    return {config, deferred ? std::min(rounded(220.0 / tiles), cap) : 0};
  }
  if (wide && !deferred && rows > 192 && rows <= 768) {
    // Both operands copied to LDS, with the tile height that fits the rows in the fewest
    // rounds of workgroups over the CUs (gate+up of Qwen3-4B, 76 weight tiles: 128-row tiles
    // up to 384 rows, 192-row tiles (three row tiles, 228 workgroups) up to 576, 256-row
    // tiles above). Up to 192 rows the activation-staged 64-row tiles fit in one round
    // (228 workgroups): 35.8 against 45.3 us at 192 rows.
    return {rows <= 384 ? 15 : rows <= 576 ? 18 : 16, 1};
  }
  const int bm = rows >= 384 || (wide && rows > 192) ? 128 : 64;
  const int config = bm == 128 ? 9 : 12;
  const int kc = bm == 128 ? 4 : 8;
  const long tiles = (long)((n + 255) / 256) * ((rows + bm - 1) / bm);
  const int cap = std::max(1, (int)(kp >> 5) / (2 * kc));
  int ks = 1;
  if (deferred) {
    ks = std::min(rounded(280.0 / (double)tiles), 8);
  } else if (tiles < 150) {
    const double want = 200.0 / (double)tiles;
    while (ks * 2 <= want * 1.5 && ks < 16) ks *= 2;  // nearest power of two
  }
  return {config, std::min(ks, cap)};
}

}  // namespace

namespace {

int env_int(const char* name, int fallback) {
  const char* v = std::getenv(name);
  return v ? std::atoi(v) : fallback;
}

// The decode kernel's launch shapes, from sweeps of the Qwen3-4B decode projections at 64
// rows (weights streamed from HBM, launches back to back): waves per workgroup, the waves per
// CU the K split aims at, the weight ring depth, the staged chunk (k-steps) and the fragment
// rows per wave. Deferred projections: eight waves of one fragment row, chunks of four;
// gate/up pairs: four waves, chunks of sixteen through a ring of eight (chunks of eight:
// 25.9 against 24.9 us for Qwen3-4B at 64 rows; a ring of sixteen 26.0).
// HLLM_ROCM_DECODE_WAVES / _TARGET / _RING / _CHUNK / _FRAGS override the deferred shape,
// HLLM_ROCM_DECODE_PAIR_WAVES / _PAIR_CHUNK the paired one, for sweeps.
struct DecodeShape {
  int waves, target_waves_per_cu, ring, chunk, frags, whole_ring;
};
const DecodeShape& decode_shape(bool pair) {
  static const DecodeShape deferred{env_int("HLLM_ROCM_DECODE_WAVES", 8), env_int("HLLM_ROCM_DECODE_TARGET", 6),
                                    env_int("HLLM_ROCM_DECODE_RING", 4), env_int("HLLM_ROCM_DECODE_CHUNK", 4),
                                    env_int("HLLM_ROCM_DECODE_FRAGS", 1),
                                    env_int("HLLM_ROCM_DECODE_WHOLE_RING", 4)};
  static const DecodeShape paired{env_int("HLLM_ROCM_DECODE_PAIR_WAVES", 4), 0, 8,
                                  env_int("HLLM_ROCM_DECODE_PAIR_CHUNK", 16), 2, 8};
  return pair ? paired : deferred;
}

// Whether the decode kernel runs this projection: F16, at most 64 rows, and either a consumer
// that sums K splits, SwiGLU (never split), or enough output features to fill the GPU unsplit.
bool decode_applies(const GemmArgs& a, int prec, int rows, int cus) {
  if (prec != kF16 || rows > 64 || rows <= 0) return false;
  if (a.defer_reduce || a.epilogue == kEpiSwiglu) return true;
  const int waves = decode_shape(false).waves >= 8 ? 8 : 4;
  const int n_tiles = (a.N + 16 * waves - 1) / (16 * waves);
  return n_tiles * waves >= 4 * cus;
}

// Fragment rows per wave of the unpaired decode variant: the configured count, halved while
// the workgroups' tiles would read past the weight rows (padded to 256).
int decode_frags(const GemmArgs& a, int waves) {
  const DecodeShape& d = decode_shape(false);
  int nfw = d.frags >= 4 ? 4 : d.frags >= 2 ? 2 : 1;
  while (nfw > 1 && (uint64_t)((a.N + 16 * waves * nfw - 1) / (16 * waves * nfw)) * waves * nfw * 16 > a.w_rows_padded)
    nfw /= 2;
  return nfw;
}

template <int MF, int KC, int P, int PW>
int launch_decode_variant(hipStream_t stream, const GemmArgs& a, int cus) {
  const bool pair = a.epilogue == kEpiSwiglu;
  const DecodeShape& d = decode_shape(pair);
  const int chunks = (int)((a.Kp >> 5) + KC - 1) / KC;
  const int waves = d.waves >= 8 ? 8 : 4;
  const int nfw = pair ? 2 : decode_frags(a, waves);
  const int fr = waves * nfw;
  const int n_tiles = (a.N + 16 * fr - 1) / (16 * fr);
  int ksplit = 1;
  if (a.defer_reduce) {
    // Splits of whole chunks, none of them empty.
    const double want = (double)d.target_waves_per_cu * cus / ((double)n_tiles * waves);
    ksplit = std::max(1, std::min((int)(want + 0.5), chunks / 2 > 0 ? chunks / 2 : 1));
    const int per = (chunks + ksplit - 1) / ksplit;
    ksplit = (chunks + per - 1) / per;
  }
  if (pair) return launch_decode_waves<MF, 2, KC, P, true, P>(stream, a, waves, 1);
  if (nfw == 4) return launch_decode_waves<MF, 4, KC, P, false, (PW > 8 ? 8 : PW)>(stream, a, waves, ksplit);
  if (nfw == 2) return launch_decode_waves<MF, 2, KC, P, false, PW>(stream, a, waves, ksplit);
  return launch_decode_waves<MF, 1, KC, P, false, PW>(stream, a, waves, ksplit);
}

template <int MF>
int launch_decode_rows(hipStream_t stream, const GemmArgs& a, int cus) {
  const DecodeShape& d = decode_shape(a.epilogue == kEpiSwiglu);
  if (d.chunk <= 4) {
    if (d.whole_ring >= 16) return launch_decode_variant<MF, 4, 4, 16>(stream, a, cus);
    if (d.whole_ring >= 8) return launch_decode_variant<MF, 4, 4, 8>(stream, a, cus);
    return launch_decode_variant<MF, 4, 4, 4>(stream, a, cus);
  }
  if (d.chunk <= 8) return launch_decode_variant<MF, 8, 8, 8>(stream, a, cus);
  return launch_decode_variant<MF, 16, 8, 8>(stream, a, cus);
}

int launch_decode(hipStream_t stream, const GemmArgs& a, int rows, int cus) {
  if (rows <= 16) return launch_decode_rows<1>(stream, a, cus);
  if (rows <= 32) return launch_decode_rows<2>(stream, a, cus);
  return launch_decode_rows<4>(stream, a, cus);
}

std::atomic<int>& forced_config() {
  static std::atomic<int> forced{[] {
    const char* v = std::getenv("HLLM_ROCM_GEMM_CONFIG");
    return v ? std::atoi(v) : -1;
  }()};
  return forced;
}
}  // namespace

int set_forced_gemm_config(int config) { return forced_config().exchange(config); }

int forced_gemm_config() { return forced_config().load(std::memory_order_relaxed); }

int gemm_argmax_parts(const GemmArgs& a, int prec, int rows_bound, int cus) {
  if (env_int("HLLM_ROCM_FUSED_ARGMAX", 1) == 0 || a.defer_reduce || a.epilogue == kEpiSwiglu) return 0;
  const int forced = forced_config().load(std::memory_order_relaxed);
  if (forced >= 0 || env_int("HLLM_ROCM_DECODE_OFF", 0) != 0 || !decode_applies(a, prec, rows_bound, cus)) return 0;
  const int waves = decode_shape(false).waves >= 8 ? 8 : 4;
  const int cols = 16 * waves * decode_frags(a, waves);  // features per workgroup
  return (a.N + cols - 1) / cols;
}

int launch_gemm(hipStream_t stream, const GemmArgs& args, int prec, int rows_bound, int cus) {
  if (rows_bound <= 0) return 0;
  const int forced = forced_config().load(std::memory_order_relaxed);
  if (args.epilogue == kEpiArgmax) {
    // Only the decode kernel has the argmax epilogue (gemm_argmax_parts says when it runs).
    if (gemm_argmax_parts(args, prec, rows_bound, cus) != args.argmax_parts || args.argmax_parts <= 0)
      fail(HLLM_INTERNAL, "the argmax epilogue needs the decode kernel");
    return launch_decode(stream, args, rows_bound, cus);
  }
  if (forced < 0 && env_int("HLLM_ROCM_DECODE_OFF", 0) == 0 && decode_applies(args, prec, rows_bound, cus))
    return launch_decode(stream, args, rows_bound, cus);
  if (forced == kDecodeConfig && prec == kF16 && rows_bound <= 64 && (args.defer_reduce || args.epilogue == kEpiSwiglu))
    return launch_decode(stream, args, rows_bound, cus);
  Choice c = gemm_choice(rows_bound, args.N, args.Kp, args.defer_reduce != 0, prec == kF16, cus);
  if (forced >= 0 && forced != kDecodeConfig) c = {forced, 0};
  return launch_gemm_config(stream, args, prec, rows_bound, cus, c.config, c.ksplit);
}

}  // namespace hllm_rocm
