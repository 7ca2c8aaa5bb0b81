// MFMA projections over F-layout operands (see gemm.hip).
#pragma once

#include "common.hpp"

namespace hllm_rocm {

enum Epilogue : int {
  kEpiStore = 0,     // out[m][n] = y            (F32 row-major, leading dimension ldo)
  kEpiResidual = 1,  // out[m][n] += y           (the F32 residual stream)
  kEpiSwiglu = 2,    // F-layout act[m][i] = silu(gate) * up, gate/up in 32-wide interleaved groups
  kEpiArgmax = 3,    // no output: each workgroup's first maximum of every row over its features
                     // (argmax_val / argmax_idx [m][parts], parts = gemm_argmax_parts)
};

struct GemmArgs {
  const uint16_t* w_hi;        // F-layout weights [N rows][Kp]
  const uint16_t* w_lo;        // lo parts (F32 residency) or nullptr
  const uint16_t* x_hi;        // F-layout activations [rows][Kp]
  const uint16_t* x_lo;        // lo parts (F32 execution) or nullptr
  int M;                       // rows, unless device_m is set
  const int32_t* device_m;     // rows read on the device (sampled rows), <= the launch bound
  int N;                       // output features
  uint64_t w_rows_padded;      // weight rows allocated (tiles never read past them)
  uint64_t x_rows_padded;      // activation rows allocated (row tiles never read past them)
  uint64_t Kp;                 // K padded to 32 (same for both operands)
  int ksplit;                  // set by the launcher
  float* workspace;            // split-K partial tiles
  size_t workspace_floats;
  int32_t* counters;           // per-tile arrival counters, zero between launches
  int counter_count;
  int defer_reduce;            // leave K-split partials as [split][M][N] for the consumer
  int epilogue;
  float* out;                  // kEpiStore / kEpiResidual
  int ldo;
  uint16_t* out_hi;            // kEpiSwiglu
  uint16_t* out_lo;
  uint64_t out_cols_padded;
  float* argmax_val;           // kEpiArgmax: [M][argmax_parts] candidates
  int32_t* argmax_idx;
  int32_t* argmax_flags;       // bit 1 set when an output is not finite
  int argmax_parts;
};

// Activation rows a buffer needs so that every row tile of a launch over up to `rows`
// rows lies inside it (row tiles are at most 256 rows).
inline uint64_t gemm_padded_rows(uint64_t rows) { return (rows + 256 + 127) / 128 * 128; }
// Returns 0 when the epilogue has been applied, or (defer_reduce only) the number of K-split
// partial output matrices left in the workspace for the consumer to sum in order.
int launch_gemm(hipStream_t stream, const GemmArgs& args, int prec, int rows_bound, int cus);
// An explicit configuration of the table in gemm.hip (tuning), optionally forcing the K split.
int launch_gemm_config(hipStream_t stream, const GemmArgs& args, int prec, int rows_bound, int cus,
                        int config, int forced_ksplit);
// Highest configuration id of the table (17 is not a table entry: see kDecodeConfig).
constexpr int kGemmConfigs = 18;
// Forced configuration meaning "the decode kernel wherever it applies" (F16, at most 64 rows,
// deferred K splits or SwiGLU); other projections keep the choice by shape.
constexpr int kDecodeConfig = 17;
// Process-wide override of the configuration choice for every later launch_gemm (-1: the
// choice by shape; initially HLLM_ROCM_GEMM_CONFIG when set). Returns the previous value.
int set_forced_gemm_config(int config);
// The configuration every projection is forced onto (-1: the choice by shape).
int forced_gemm_config();
// The number of per-workgroup argmax candidates per row when launch_gemm can run this
// projection with the kEpiArgmax epilogue (the decode kernel, one pass over N), else 0;
// HLLM_ROCM_FUSED_ARGMAX=0, read at every call, says 0 (for tests).
int gemm_argmax_parts(const GemmArgs& args, int prec, int rows_bound, int cus);

}  // namespace hllm_rocm
