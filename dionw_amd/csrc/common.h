// Shared helpers of the dionw HIP library: error reporting, vector types,
// wavefront reductions and the pointer tables kernels receive by value.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>

#include "dionw_hip.h"

#include <cstdint>
#include <cstdio>
#include <string>

namespace dionw {

// ---- error convention -------------------------------------------------------
// Every C entry point returns 0 on success, DIONW_EINVAL for a rejected
// argument and DIONW_EHIP for a failed launch; the message is kept per thread.
enum : int { kOk = 0, kInvalid = 1, kHipError = 2 };

void set_error(const char* fmt, ...);
int check_launch(const char* what);

#define DIONW_REQUIRE(cond, ...)          \
  do {                                    \
    if (!(cond)) {                        \
      ::dionw::set_error(__VA_ARGS__);    \
      return ::dionw::kInvalid;           \
    }                                     \
  } while (0)

#define DIONW_TRY(expr)                   \
  do {                                    \
    int _rc = (expr);                     \
    if (_rc != 0) return _rc;             \
  } while (0)

// ---- vector types -----------------------------------------------------------
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kWave = 64;

// Element codes shared with the Python side.
enum ElemType : int { kF16 = 0, kBF16 = 1, kF32 = 2 };

// Butterfly sum over the 64 lanes of a wavefront. Every lane ends with the
// same value: at each level lane i adds lane i^off, a fixed tree that a CPU
// restatement can reproduce exactly (pairs (i, i+32), then (i, i+16), ...).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// torch's lerp, as the EMA uses it (ATen Lerp.h: |w| < 0.5 ? self + w (end -
// self) : end - (end - self)(1 - w)), with the multiply-adds fused the way
// hipcc fuses them under its default contraction; spelled out so every kernel
// that updates a shadow rounds identically whatever its file's contraction mode.
__device__ __forceinline__ float ema_lerp(float self, float end, float weight) {
  const float diff = end - self;
  return fabsf(weight) < 0.5f ? __builtin_fmaf(weight, diff, self)
                              : __builtin_fmaf(-diff, 1.f - weight, end);
}

// Rounding to the 16-bit storage types (round to nearest even).
__device__ __forceinline__ _Float16 to_f16(float x) { return (_Float16)x; }
__device__ __forceinline__ __bf16 to_bf16(float x) { return (__bf16)x; }

// Pointer tables travel in kernel arguments (no device-side table, no host
// sync): one launch covers up to kMaxTensors tensors; longer lists are split.
constexpr int kMaxTensors = 48;

struct RowTable {            // same-shape tensors of a bucket run
  const float* grad[kMaxTensors];
  float* param[kMaxTensors];
  int count;
};

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }
inline int64_t round_up(int64_t a, int64_t b) { return ceil_div(a, b) * b; }

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

}  // namespace dionw
