// Dense projections Y[M, N] = X[M, K] * W[N, K]^T on v_mfma_f32_16x16x32_f16.
//
// Both operands are in the F-layout (common.hpp), so every operand fragment is one
// coalesced 1 KiB load per wave straight from HBM/L2 into registers. The MFMA's A side
// is the weight fragment (16 output features x 32 k) and its B side the activation
// fragment (32 k x 16 tokens); lane L of the 16x16 result holds features 4*(L/16)+v of
// token L%16.
//
// Decode passes have few rows: a workgroup owns BN = 64 output features for a K range,
// its four waves interleave the K fragments of that range, and the K range itself may be
// split across workgroups so that every CU streams weights. Partial tiles are summed in a
// fixed order by the last workgroup of a tile to arrive (an atomic counter it resets), so
// results are deterministic. Prefill passes use 128x128 tiles of four waves.
//
// Split precision (F32 execution) adds a second accumulator for the lo parts of split
// operands: x*w ~= hi*hi + (lo*hi + hi*lo) / 2048.
#include "gemm.hpp"

namespace hllm_rocm {
namespace {

__device__ inline floatx4 mfma(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ inline float silu_mul(float g, float u) { return (g / (1.0f + expf(-g))) * u; }

template <int MF, int NF, int WM, int WN, int WK, int PREC>
__global__ void __launch_bounds__(64 * WM * WN * WK)
    gemm_kernel(GemmArgs a) {
  constexpr int BM = 16 * MF * WM, BN = 16 * NF * WN, NT = 64 * WM * WN * WK;
  constexpr int LDT = BN + 4;  // padded LDS row (floats)
  extern __shared__ float lds[];  // [BM][LDT] + flag
  const int M = a.device_m ? *a.device_m : a.M;
  const int tile_n = blockIdx.x, tile_m = blockIdx.y, split = blockIdx.z;
  if (tile_m * BM >= M) return;  // uniform over the whole tile (all of its splits)
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wk = wave % WK, wn = (wave / WK) % WN, wm = wave / (WK * WN);
  const int KT = (int)(a.Kp >> 5);
  const int per = (KT + a.ksplit - 1) / a.ksplit;
  const int kt0 = split * per, kt1 = min(KT, kt0 + per);
  const int nfrag0 = tile_n * (BN / 16) + wn * NF;
  const int mfrag0 = tile_m * (BM / 16) + wm * MF;

  const half8* W = reinterpret_cast<const half8*>(a.w_hi);
  const half8* WL = reinterpret_cast<const half8*>(a.w_lo);
  const half8* X = reinterpret_cast<const half8*>(a.x_hi);
  const half8* XL = reinterpret_cast<const half8*>(a.x_lo);

  floatx4 acc[MF][NF];
  floatx4 acc2[MF][NF];
#pragma unroll
  for (int i = 0; i < MF; ++i)
#pragma unroll
    for (int j = 0; j < NF; ++j) {
      acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
      acc2[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

  for (int kt = kt0 + wk; kt < kt1; kt += WK) {
    half8 b[NF], x[MF];
#pragma unroll
    for (int j = 0; j < NF; ++j) b[j] = W[((size_t)(nfrag0 + j) * KT + kt) * 64 + lane];
#pragma unroll
    for (int i = 0; i < MF; ++i) x[i] = X[((size_t)(mfrag0 + i) * KT + kt) * 64 + lane];
    if constexpr (PREC >= kSplitA) {
      half8 xl[MF];
#pragma unroll
      for (int i = 0; i < MF; ++i) xl[i] = XL[((size_t)(mfrag0 + i) * KT + kt) * 64 + lane];
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) acc2[i][j] = mfma(b[j], xl[i], acc2[i][j]);
    }
    if constexpr (PREC == kSplitAB) {
      half8 bl[NF];
#pragma unroll
      for (int j = 0; j < NF; ++j) bl[j] = WL[((size_t)(nfrag0 + j) * KT + kt) * 64 + lane];
#pragma unroll
      for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) acc2[i][j] = mfma(bl[j], x[i], acc2[i][j]);
    }
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
      for (int j = 0; j < NF; ++j) acc[i][j] = mfma(b[j], x[i], acc[i][j]);
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
    const int tile = tile_m * gridDim.x + tile_n;
    float* ws = a.workspace + (size_t)tile * a.ksplit * BM * BN;
    for (int e = threadIdx.x; e < BM * BN; e += NT) {
      ws[(size_t)split * BM * BN + e] = lds[(e / BN) * LDT + e % BN];
    }
    __threadfence();
    __syncthreads();
    int* last = reinterpret_cast<int*>(lds + (size_t)BM * LDT);
    if (threadIdx.x == 0) *last = atomicAdd(a.counters + tile, 1) == a.ksplit - 1;
    __syncthreads();
    if (!*last) return;
    __threadfence();
    for (int e = threadIdx.x; e < BM * BN; e += NT) {
      float s = ws[e];
      for (int p = 1; p < a.ksplit; ++p) s += ws[(size_t)p * BM * BN + e];
      lds[(e / BN) * LDT + e % BN] = s;
    }
    if (threadIdx.x == 0) a.counters[tile] = 0;
    __syncthreads();
  }

  // Epilogue from slab 0.
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

template <int MF, int NF, int WM, int WN, int WK, int PREC>
void run(dim3 grid, int threads, size_t lds, hipStream_t stream, const GemmArgs& a) {
  static const bool configured = [lds] {
    // Tiles above 64 KiB of LDS need the kernel's dynamic-LDS limit raised (160 KiB on gfx950).
    HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_kernel<MF, NF, WM, WN, WK, PREC>),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    return true;
  }();
  (void)configured;
  gemm_kernel<MF, NF, WM, WN, WK, PREC><<<grid, threads, lds, stream>>>(a);
}

template <int MF, int NF, int WM, int WN, int WK>
void launch_config(hipStream_t stream, GemmArgs a, int prec, int rows_bound, int max_ctas) {
  constexpr int BM = 16 * MF * WM, BN = 16 * NF * WN, NT = 64 * WM * WN * WK;
  const int n_tiles = (a.N + BN - 1) / BN;
  const int m_tiles = (rows_bound + BM - 1) / BM;
  const int KT = (int)(a.Kp >> 5);
  const int tiles = n_tiles * m_tiles;
  int ksplit = 1;
  const int min_frags = WK == 1 ? 16 : 2 * WK;
  if (tiles < max_ctas) {
    ksplit = (max_ctas + tiles - 1) / tiles;
    ksplit = min(ksplit, max(1, KT / min_frags));
  }
  if ((size_t)tiles * ksplit * BM * BN > a.workspace_floats || tiles > a.counter_count) ksplit = 1;
  a.ksplit = ksplit;
  const size_t lds = ((size_t)BM * (BN + 4) + 4) * sizeof(float);
  dim3 grid(n_tiles, m_tiles, ksplit);
  switch (prec) {
    case kF16:
      run<MF, NF, WM, WN, WK, kF16>(grid, NT, lds, stream, a);
      break;
    case kSplitA:
      run<MF, NF, WM, WN, WK, kSplitA>(grid, NT, lds, stream, a);
      break;
    default:
      run<MF, NF, WM, WN, WK, kSplitAB>(grid, NT, lds, stream, a);
      break;
  }
}

}  // namespace

int gemm_tile_rows(int rows_bound) { return rows_bound <= 64 ? 64 : 128; }

void launch_gemm(hipStream_t stream, const GemmArgs& args, int prec, int rows_bound, int cus) {
  if (rows_bound <= 0) return;
  if (rows_bound <= 16)
    launch_config<1, 4, 1, 1, 4>(stream, args, prec, rows_bound, 2 * cus);
  else if (rows_bound <= 32)
    launch_config<2, 4, 1, 1, 4>(stream, args, prec, rows_bound, 2 * cus);
  else if (rows_bound <= 64)
    launch_config<4, 4, 1, 1, 4>(stream, args, prec, rows_bound, 2 * cus);
  else
    launch_config<4, 4, 2, 2, 1>(stream, args, prec, rows_bound, cus);
}

}  // namespace hllm_rocm
