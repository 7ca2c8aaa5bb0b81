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
#include <cstdlib>

namespace hllm_rocm {
namespace {

constexpr int kXcds = 8;

__device__ inline floatx4 mfma(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

template <int MF, int NF, int WM, int WN, int WK, int P, int PREC>
__global__ void __launch_bounds__(64 * WM * WN * WK)
    gemm_kernel(GemmArgs a, int n_tiles, int tiles, int tiles_padded) {
  constexpr int BM = 16 * MF * WM, BN = 16 * NF * WN, NT = 64 * WM * WN * WK;
  constexpr int LDT = BN + 4;  // padded LDS row (floats)
  extern __shared__ float lds[];  // [BM][LDT] + flag
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
  auto load = [&](int slot, int kt) {
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
#pragma unroll
  for (int s = 0; s < P; ++s)
    if (s < steps) load(s, first + s * WK);
  for (int base = 0; base < steps; base += P) {
#pragma unroll
    for (int s = 0; s < P; ++s) {
      const int step = base + s;
      if (step < steps) {
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
        if (step + P < steps) load(s, first + (step + P) * WK);
      }
    }
  }

  // Per-wave partial tiles -> one LDS tile, the K-interleaved waves adding in turn
  // (fixed order, so the sum is deterministic).
#pragma unroll
  for (int turn = 0; turn < WK; ++turn) {
    if (wk == turn) {
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
          floatx4* dst = reinterpret_cast<floatx4*>(lds + m * LDT + n);
          if (turn == 0) {
            *dst = v;
          } else {
            floatx4 s = *dst;
            s[0] += v[0];
            s[1] += v[1];
            s[2] += v[2];
            s[3] += v[3];
            *dst = s;
          }
        }
    }
    __syncthreads();
  }

  if (a.ksplit > 1) {
    float* ws = a.workspace + (size_t)tile * a.ksplit * BM * BN;
    for (int e = threadIdx.x; e < BM * BN / 4; e += NT) {
      const int m = e / (BN / 4), n = (e % (BN / 4)) * 4;
      *reinterpret_cast<floatx4*>(ws + (size_t)split * BM * BN + m * BN + n) =
          *reinterpret_cast<const floatx4*>(lds + m * LDT + n);
    }
    __threadfence();
    __syncthreads();
    int* last = reinterpret_cast<int*>(lds + (size_t)BM * LDT);
    if (threadIdx.x == 0) *last = atomicAdd(a.counters + tile, 1) == a.ksplit - 1;
    __syncthreads();
    if (!*last) return;
    __threadfence();
    for (int e = threadIdx.x; e < BM * BN / 4; e += NT) {
      const int m = e / (BN / 4), n = (e % (BN / 4)) * 4;
      floatx4 s = *reinterpret_cast<const floatx4*>(ws + m * BN + n);
      for (int p = 1; p < a.ksplit; ++p) {
        const floatx4 t = *reinterpret_cast<const floatx4*>(ws + (size_t)p * BM * BN + m * BN + n);
        s[0] += t[0];
        s[1] += t[1];
        s[2] += t[2];
        s[3] += t[3];
      }
      *reinterpret_cast<floatx4*>(lds + m * LDT + n) = s;
    }
    if (threadIdx.x == 0) a.counters[tile] = 0;
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
  gemm_kernel<MF, NF, WM, WN, WK, P, PREC><<<grid, threads, lds, stream>>>(a, n_tiles, tiles,
                                                                           tiles_padded);
}

template <int MF, int NF, int WM, int WN, int WK, int P>
void launch_config(hipStream_t stream, GemmArgs a, int prec, int rows_bound, int target_ctas,
                   int min_k_per_wave, int forced_ksplit) {
  constexpr int BM = 16 * MF * WM, BN = 16 * NF * WN, NT = 64 * WM * WN * WK;
  const int n_tiles = (a.N + BN - 1) / BN;
  const int m_tiles = (rows_bound + BM - 1) / BM;
  const int KT = (int)(a.Kp >> 5);
  const int tiles = n_tiles * m_tiles;
  int ksplit = 1;
  if (forced_ksplit > 0) {
    ksplit = forced_ksplit;
  } else if (tiles < target_ctas) {
    ksplit = (target_ctas + tiles - 1) / tiles;
  }
  ksplit = std::min(ksplit, std::max(1, KT / (WK * min_k_per_wave)));
  const int tiles_padded = (tiles + kXcds - 1) / kXcds * kXcds;
  if ((size_t)tiles_padded * ksplit * BM * BN > a.workspace_floats || tiles_padded > a.counter_count)
    ksplit = 1;
  a.ksplit = ksplit;
  const size_t lds = ((size_t)BM * (BN + 4) + 4) * sizeof(float);
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
}

}  // namespace

int gemm_tile_rows(int rows_bound) { return rows_bound <= 64 ? 64 : 128; }

// Configuration table (ids are stable for the tuning harness):
//   0..2: decode, BM = 16/32/64, BN = 64, four K-waves, ring of 4 k-steps
//   3:    prefill, 128 x 128, 2 x 2 waves, ring of 2 k-steps
//   4..6: decode, BM = 16/32/64, BN = 128 (NF = 8), two K-waves, ring of 4
void launch_gemm_config(hipStream_t stream, const GemmArgs& args, int prec, int rows_bound, int cus,
                        int config, int forced_ksplit) {
  switch (config) {
    case 0:
      launch_config<1, 4, 1, 1, 4, 4>(stream, args, prec, rows_bound, 2 * cus, 2, forced_ksplit);
      break;
    case 1:
      launch_config<2, 4, 1, 1, 4, 4>(stream, args, prec, rows_bound, 2 * cus, 2, forced_ksplit);
      break;
    case 2:
      launch_config<4, 4, 1, 1, 4, 4>(stream, args, prec, rows_bound, 2 * cus, 2, forced_ksplit);
      break;
    case 4:
      launch_config<1, 8, 1, 1, 2, 4>(stream, args, prec, rows_bound, 2 * cus, 2, forced_ksplit);
      break;
    case 5:
      launch_config<2, 8, 1, 1, 2, 4>(stream, args, prec, rows_bound, 2 * cus, 2, forced_ksplit);
      break;
    case 6:
      launch_config<4, 8, 1, 1, 2, 4>(stream, args, prec, rows_bound, 2 * cus, 2, forced_ksplit);
      break;
    default:
      launch_config<4, 4, 2, 2, 1, 2>(stream, args, prec, rows_bound, cus, 8, forced_ksplit);
      break;
  }
}

int gemm_default_config(int rows_bound) {
  if (rows_bound <= 16) return 0;
  if (rows_bound <= 32) return 1;
  if (rows_bound <= 64) return 2;
  return 3;
}

void launch_gemm(hipStream_t stream, const GemmArgs& args, int prec, int rows_bound, int cus) {
  if (rows_bound <= 0) return;
  static const int forced = [] {
    const char* v = std::getenv("HLLM_ROCM_GEMM_CONFIG");
    return v ? std::atoi(v) : -1;
  }();
  int config = gemm_default_config(rows_bound);
  if (forced >= 0 && (rows_bound <= 64) == (forced != 3)) config = forced;
  // Splitting K across workgroups needs device-scope fences around the partial tiles, which
  // cost more than the parallelism gains (measured); one workgroup per tile by default.
  launch_gemm_config(stream, args, prec, rows_bound, cus, config, 1);
}

}  // namespace hllm_rocm
