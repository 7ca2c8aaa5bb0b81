// Shared definitions for the gfx950 decoder stage worker.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "hllm_rocm.h"

namespace hllm_rocm {

// ------------------------------------------------------------------ errors

// Mirrors runtime::Error (cpp/include/hllm/runtime/error.hpp:20-40): a category plus a
// message; translated to hllm_status at the C ABI.
struct Failure : std::runtime_error {
  hllm_status status;
  Failure(hllm_status s, const std::string& message) : std::runtime_error(message), status(s) {}
};

[[noreturn]] inline void fail(hllm_status s, const std::string& message) { throw Failure(s, message); }

inline void check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return;
  if (e == hipErrorOutOfMemory) fail(HLLM_RESOURCE_EXHAUSTED, std::string(what) + ": out of device memory");
  fail(HLLM_INTERNAL, std::string(what) + ": " + hipGetErrorString(e));
}
#define HIP_CHECK(expr) ::hllm_rocm::check_hip((expr), #expr)

// ------------------------------------------------------------------ launch observation
//
// Per-kernel timing: a stage that profiles installs an observer for the launches it issues
// from its thread; every launcher brackets each kernel launch with `observed`, naming the
// kernel as the profiler names it (template arguments included).
struct LaunchObserver {
  virtual void before(const char* kernel) = 0;
  virtual void after(const char* kernel) = 0;

 protected:
  ~LaunchObserver() = default;
};
extern thread_local LaunchObserver* launch_observer;

template <typename F>
inline void observed(const char* kernel, F&& launch) {
  LaunchObserver* o = launch_observer;
  if (o) o->before(kernel);
  launch();
  if (o) o->after(kernel);
}

// "base<a, b, ...>" for integer template arguments, built once per instantiation.
template <int... I>
inline const char* kernel_name(const char* base) {
  static const std::string name = [base] {
    std::string s = std::string(base) + "<";
    const int v[] = {I...};
    for (size_t i = 0; i < sizeof...(I); ++i) s += (i ? ", " : "") + std::to_string(v[i]);
    return s + ">";
  }();
  return name.c_str();
}

// ------------------------------------------------------------------ vectors

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// ------------------------------------------------------------------ F-layout
//
// Matrix operands of every GEMM live in a fragment-tiled layout sized for the
// v_mfma_f32_16x16x32_f16 operand fragment: rows are padded to 16, columns to 32; each
// 16x32 fragment is 1 KiB contiguous (fragments row-block-major), and inside a fragment
// lane L = (r % 16) + 16 * ((c % 32) / 8) holds the 8 consecutive columns c..c+7 of row r.
// A wave therefore loads one whole fragment with one coalesced 16-byte load per lane.
__host__ __device__ inline uint64_t pad16(uint64_t x) { return (x + 15) & ~uint64_t(15); }
__host__ __device__ inline uint64_t pad32(uint64_t x) { return (x + 31) & ~uint64_t(31); }
__host__ __device__ inline uint64_t flayout_index(uint64_t r, uint64_t c, uint64_t cols_padded) {
  return (((((r >> 4) * (cols_padded >> 5) + (c >> 5)) << 6) + (r & 15) + ((c & 31) >> 3) * 16) << 3) +
         (c & 7);
}

// Split F32 operands: x ~= hi + lo / 2048 with hi = f16(x), lo = f16((x - hi) * 2048).
constexpr float kLoScale = 2048.0f;
constexpr float kLoUnscale = 1.0f / 2048.0f;

// ------------------------------------------------------------------ F16 (device)

// Round-to-nearest-even F32 -> F16 with the reference codec's results for all finite and
// infinite inputs (cpp/src/half.cpp:36-88); the hardware conversion rounds to nearest even.
__device__ inline _Float16 to_half(float x) { return static_cast<_Float16>(x); }
__device__ inline uint16_t half_bits(float x) {
  _Float16 h = static_cast<_Float16>(x);
  return __builtin_bit_cast(uint16_t, h);
}
__device__ inline float from_half_bits(uint16_t b) {
  return static_cast<float>(__builtin_bit_cast(_Float16, b));
}

// ------------------------------------------------------------------ greedy argmax

// A candidate of the first-maximum search: larger values win, equal values keep the lower
// index, NaN never wins (so the result does not depend on the order of the comparisons).
struct Best {
  float value;
  int index;
};
__device__ inline Best better(Best a, Best b) {
  if (b.value > a.value || (b.value == a.value && b.index < a.index)) return b;
  return a;
}

// ------------------------------------------------------------------ precision

// How GEMM operands are represented:
//   1: f16 activations x f16 weights (F16 execution)
//   2: split activations (hi + lo) x f16 weights (F32 execution over F16-resident weights)
//   3: split activations x split weights (F32 execution over F32-resident weights)
enum Precision : int { kF16 = 1, kSplitA = 2, kSplitAB = 3 };

// ------------------------------------------------------------ uniform loads

// A load of a wave-uniform address from memory no kernel of the launch writes (work lists,
// item tables, block tables, row maps, counts written by earlier launches): through the
// constant address space, so that the compiler issues it as a scalar load instead of a vector
// load it would have to wait for with the vector loads in flight.
template <typename T>
__device__ inline T uniform_load(const T* p) {
  return *(const __attribute__((address_space(4))) T*)(p);
}

// ------------------------------------------------------------ direct copies to LDS

// One 16-byte copy per lane from sbase + voffset to LDS byte m0 + 16 * lane; sbase and
// the LDS offset are uniform over the wave.
__device__ inline void lds_copy16(const void* sbase, uint32_t voffset, uint32_t lds_byte_offset) {
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voffset), "s"(sbase),
               "s"(lds_byte_offset)
               : "memory", "m0");
#pragma clang diagnostic pop
}

// s_waitcnt with the given vector-memory and LDS counts (expcnt left open). Issued through
// the builtin so that the compiler knows which of its own LDS reads have completed.
template <int vm, int lgkm>
__device__ inline void wait_counts() {
  static_assert(vm >= 0 && vm < 64 && lgkm >= 0 && lgkm < 16, "s_waitcnt field range");
  __builtin_amdgcn_s_waitcnt((vm & 0xF) | ((vm >> 4) << 14) | (0x7 << 4) | (lgkm << 8));
}

// Wait until at most `in_flight` of this wave's copies are outstanding and all but its
// last `reads` LDS reads have returned, then meet the other waves.
template <int in_flight, int reads>
__device__ inline void stage_barrier() {
  wait_counts<in_flight, reads>();
  asm volatile("s_barrier" ::: "memory");
}

}  // namespace hllm_rocm
