// Multi-tensor AdamW (the route of _adamw.py:25-61 through torch._fused_adamw_)
// and the GPU weight EMA (ema/_update.py:32-70, _foreach_lerp_ / _foreach_copy_).
//
// The arithmetic follows ATen's fused AdamW element for element so that the
// results are bit-identical: moments and weight decay in double, rounded to
// float on store; bias corrections in double, handed to the element math as
// float; step size and denominator float. Lerp takes the two-branch form
// s + w (p - s) for |w| < 0.5, else p - (p - s)(1 - w), in float. This file is
// compiled with the same (default) contraction as torch's kernels.
#include "common.h"

#include <cmath>

namespace dionw {
namespace {

// Elements per workgroup: four float4 per lane and array. Each workgroup issues
// every load of its chunk before its first store and exits; on MI355X this
// split streams AdamW's 4-read/3-write mix at ~5.8 TB/s, against ~5.1-5.3 TB/s
// for 16384-element chunks walked two float4 per array at a time.
constexpr int kChunk = 4096;
constexpr int kVec = kChunk / (4 * 256);  // float4 per lane and array
constexpr int kMaxAdam = 48;

struct AdamTable {
  float* p[kMaxAdam];
  const float* g[kMaxAdam];
  float* m[kMaxAdam];
  float* v[kMaxAdam];
  const float* step[kMaxAdam];
  float* shadow[kMaxAdam];  // EMA shadows updated from the new parameters (fused EMA)
  int64_t numel[kMaxAdam];
  int32_t chunk0[kMaxAdam + 1];  // first chunk of each tensor
  int count;
};

__device__ __forceinline__ int find_tensor(const int32_t* chunk0, int count, int chunk) {
  int lo = 0, hi = count - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (chunk0[mid] <= chunk) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

struct AdamScalars {
  double lr, beta1, beta2, weight_decay, eps;
};

__device__ __forceinline__ void adamw_element(float& param_io, float grad, float& exp_avg_io,
                                              float& exp_avg_sq_io, const AdamScalars& s,
                                              float bias_correction1, float bias_correction2_sqrt) {
  // The fused multiply-adds are spelled out (and contraction is off) so that
  // the rounding does not depend on how the compiler schedules the caller's
  // loop: this is the form that reproduces torch's fused AdamW bit for bit.
#pragma clang fp contract(off)
  float param = param_io;
  float exp_avg = exp_avg_io;
  float exp_avg_sq = exp_avg_sq_io;
  const double g = grad;
  if (s.weight_decay != 0)
    param = (float)__builtin_fma(-(s.lr * s.weight_decay), (double)param, (double)param);
  exp_avg = (float)__builtin_fma(s.beta1, (double)exp_avg, (1 - s.beta1) * g);
  exp_avg_sq = (float)__builtin_fma(s.beta2, (double)exp_avg_sq, ((1 - s.beta2) * g) * g);
  const float step_size = s.lr / bias_correction1;
  const float denom = (std::sqrt(exp_avg_sq) / bias_correction2_sqrt) + s.eps;
  param -= step_size * exp_avg / denom;
  param_io = param;
  exp_avg_io = exp_avg;
  exp_avg_sq_io = exp_avg_sq;
}

template <bool EMA>
__global__ __launch_bounds__(256) void adamw_kernel(AdamTable t, AdamScalars s, float ema_weight) {
  const int tensor = find_tensor(t.chunk0, t.count, blockIdx.x);
  const int64_t local = (int64_t)(blockIdx.x - t.chunk0[tensor]) * kChunk;
  const int64_t n = t.numel[tensor] - local;
  const int64_t end = n < kChunk ? n : kChunk;
  const double stepd = (double)*t.step[tensor];
  const float bc1 = (float)(1 - ::pow(s.beta1, stepd));
  const float bc2s = (float)std::sqrt(1 - ::pow(s.beta2, stepd));
  float* p = t.p[tensor] + local;
  const float* g = t.g[tensor] + local;
  float* m = t.m[tensor] + local;
  float* v = t.v[tensor] + local;
  float* sh = EMA ? t.shadow[tensor] + local : nullptr;
  const bool vec = ((reinterpret_cast<uintptr_t>(p) | reinterpret_cast<uintptr_t>(g) |
                     reinterpret_cast<uintptr_t>(m) | reinterpret_cast<uintptr_t>(v) |
                     reinterpret_cast<uintptr_t>(sh)) & 15) == 0;
  int64_t i = 0;
  if (vec) {
    f32x4* p4 = reinterpret_cast<f32x4*>(p);
    const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
    f32x4* m4 = reinterpret_cast<f32x4*>(m);
    f32x4* v4 = reinterpret_cast<f32x4*>(v);
    f32x4* s4 = reinterpret_cast<f32x4*>(sh);
    // Every element is read once and written once: streaming (non-temporal)
    // loads and stores, all loads of the chunk in flight before the first store.
    auto ld = [](const f32x4* x) { return __builtin_nontemporal_load(x); };
    const int64_t n4 = end >> 2;
    f32x4 pv[kVec], gv[kVec], mv[kVec], vv[kVec], sv[kVec];
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const int64_t q = threadIdx.x + u * 256;
      if (q < n4) {
        pv[u] = ld(p4 + q);
        gv[u] = ld(g4 + q);
        mv[u] = ld(m4 + q);
        vv[u] = ld(v4 + q);
        if (EMA) sv[u] = ld(s4 + q);
      }
    }
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const int64_t q = threadIdx.x + u * 256;
      if (q >= n4) continue;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float pe = pv[u][e], me = mv[u][e], ve = vv[u][e];
        adamw_element(pe, gv[u][e], me, ve, s, bc1, bc2s);
        pv[u][e] = pe;
        mv[u][e] = me;
        vv[u][e] = ve;
      }
      __builtin_nontemporal_store(pv[u], p4 + q);
      __builtin_nontemporal_store(mv[u], m4 + q);
      __builtin_nontemporal_store(vv[u], v4 + q);
      if (EMA) {
#pragma unroll
        for (int e = 0; e < 4; ++e) sv[u][e] = ema_lerp(sv[u][e], pv[u][e], ema_weight);
        __builtin_nontemporal_store(sv[u], s4 + q);
      }
    }
    i = end & ~(int64_t)3;
  }
  for (int64_t e = i + threadIdx.x; e < end; e += 256) {
    float pe = p[e], me = m[e], ve = v[e];
    adamw_element(pe, g[e], me, ve, s, bc1, bc2s);
    p[e] = pe;
    m[e] = me;
    v[e] = ve;
    if (EMA) sh[e] = ema_lerp(sh[e], pe, ema_weight);
  }
}

struct StepTable {
  float* step[256];
  int count;
};

__global__ void increment_steps_kernel(StepTable t) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < t.count) *t.step[i] = *t.step[i] + 1.f;
}

// ---- EMA ----------------------------------------------------------------------

struct EmaTable {
  float* shadow[kMaxAdam];
  const float* src[kMaxAdam];
  int64_t numel[kMaxAdam];
  int32_t chunk0[kMaxAdam + 1];
  int count;
};

template <bool COPY>
__global__ __launch_bounds__(256) void ema_kernel(EmaTable t, float weight) {
  const int tensor = find_tensor(t.chunk0, t.count, blockIdx.x);
  const int64_t local = (int64_t)(blockIdx.x - t.chunk0[tensor]) * kChunk;
  const int64_t n = t.numel[tensor] - local;
  const int64_t end = n < kChunk ? n : kChunk;
  float* s = t.shadow[tensor] + local;
  const float* p = t.src[tensor] + local;
  const bool vec = ((reinterpret_cast<uintptr_t>(s) | reinterpret_cast<uintptr_t>(p)) & 15) == 0;
  int64_t i = 0;
  if (vec) {
    // Streaming (non-temporal) accesses, each element touched once; all loads
    // of the chunk in flight before the first store.
    f32x4* s4 = reinterpret_cast<f32x4*>(s);
    const f32x4* p4 = reinterpret_cast<const f32x4*>(p);
    const int64_t n4 = end >> 2;
    f32x4 pv[kVec], sv[kVec];
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const int64_t q = threadIdx.x + u * 256;
      if (q < n4) {
        pv[u] = __builtin_nontemporal_load(p4 + q);
        if (!COPY) sv[u] = __builtin_nontemporal_load(s4 + q);
      }
    }
#pragma unroll
    for (int u = 0; u < kVec; ++u) {
      const int64_t q = threadIdx.x + u * 256;
      if (q >= n4) continue;
      if (!COPY) {
#pragma unroll
        for (int e = 0; e < 4; ++e) pv[u][e] = ema_lerp(sv[u][e], pv[u][e], weight);
      }
      __builtin_nontemporal_store(pv[u], s4 + q);
    }
    i = end & ~(int64_t)3;
  }
  for (int64_t e = i + threadIdx.x; e < end; e += 256)
    s[e] = COPY ? p[e] : ema_lerp(s[e], p[e], weight);
}

// One launch per kMaxAdam tensors; shadows (may be null) get the fused EMA lerp.
int adamw_launch(float* const* params, const float* const* grads, float* const* exp_avgs,
                 float* const* exp_avg_sqs, const float* const* steps, float* const* shadows,
                 const int64_t* numels, int32_t count, const AdamScalars& s, float ema_weight,
                 hipStream_t stream) {
  for (int32_t start = 0; start < count;) {
    AdamTable t{};
    int32_t chunks = 0;
    while (start < count && t.count < kMaxAdam) {
      const int i = start;
      DIONW_REQUIRE(params[i] && grads[i] && exp_avgs[i] && exp_avg_sqs[i] && steps[i],
                    "adamw: null pointer in tensor %d", i);
      DIONW_REQUIRE(!shadows || shadows[i], "adamw: null EMA shadow in tensor %d", i);
      DIONW_REQUIRE(numels[i] >= 0, "adamw: negative numel");
      const int64_t c = ceil_div(numels[i], kChunk);
      if ((int64_t)chunks + c > INT32_MAX / 2) break;
      ++start;
      if (c == 0) continue;
      t.p[t.count] = params[i];
      t.g[t.count] = grads[i];
      t.m[t.count] = exp_avgs[i];
      t.v[t.count] = exp_avg_sqs[i];
      t.step[t.count] = steps[i];
      t.shadow[t.count] = shadows ? shadows[i] : nullptr;
      t.numel[t.count] = numels[i];
      t.chunk0[t.count] = chunks;
      chunks += (int32_t)c;
      ++t.count;
    }
    if (t.count == 0) continue;
    t.chunk0[t.count] = chunks;
    if (shadows)
      hipLaunchKernelGGL(adamw_kernel<true>, dim3((unsigned)chunks), dim3(256), 0, stream, t, s,
                         ema_weight);
    else
      hipLaunchKernelGGL(adamw_kernel<false>, dim3((unsigned)chunks), dim3(256), 0, stream, t, s,
                         0.f);
    DIONW_TRY(check_launch("adamw"));
  }
  return kOk;
}

}  // namespace
}  // namespace dionw

using namespace dionw;

extern "C" {

int dionw_increment_steps(float* const* steps, int32_t count, hipStream_t stream) {
  for (int32_t start = 0; start < count; start += 256) {
    StepTable t{};
    t.count = (count - start) < 256 ? (count - start) : 256;
    for (int i = 0; i < t.count; ++i) {
      DIONW_REQUIRE(steps[start + i], "increment_steps: null step %d", start + i);
      t.step[i] = steps[start + i];
    }
    hipLaunchKernelGGL(increment_steps_kernel, dim3(1), dim3(256), 0, stream, t);
    DIONW_TRY(check_launch("increment_steps"));
  }
  return kOk;
}

int dionw_adamw(float* const* params, const float* const* grads, float* const* exp_avgs,
                float* const* exp_avg_sqs, const float* const* steps, const int64_t* numels,
                int32_t count, double lr, double beta1, double beta2, double weight_decay,
                double eps, hipStream_t stream) {
  return adamw_launch(params, grads, exp_avgs, exp_avg_sqs, steps, nullptr, numels, count,
                      AdamScalars{lr, beta1, beta2, weight_decay, eps}, 0.f, stream);
}

int dionw_adamw_ema(float* const* params, const float* const* grads, float* const* exp_avgs,
                    float* const* exp_avg_sqs, const float* const* steps, float* const* shadows,
                    const int64_t* numels, int32_t count, double lr, double beta1, double beta2,
                    double weight_decay, double eps, float ema_weight, hipStream_t stream) {
  DIONW_REQUIRE(shadows, "adamw_ema: null shadow table");
  return adamw_launch(params, grads, exp_avgs, exp_avg_sqs, steps, shadows, numels, count,
                      AdamScalars{lr, beta1, beta2, weight_decay, eps}, ema_weight, stream);
}

int dionw_ema_update(float* const* shadows, const float* const* sources, const int64_t* numels,
                     int32_t count, float weight, int32_t copy, hipStream_t stream) {
  for (int32_t start = 0; start < count;) {
    EmaTable t{};
    int32_t chunks = 0;
    while (start < count && t.count < kMaxAdam) {
      const int i = start;
      DIONW_REQUIRE(shadows[i] && sources[i], "ema_update: null pointer in tensor %d", i);
      const int64_t c = ceil_div(numels[i], kChunk);
      if ((int64_t)chunks + c > INT32_MAX / 2) break;
      ++start;
      if (c == 0) continue;
      t.shadow[t.count] = shadows[i];
      t.src[t.count] = sources[i];
      t.numel[t.count] = numels[i];
      t.chunk0[t.count] = chunks;
      chunks += (int32_t)c;
      ++t.count;
    }
    if (t.count == 0) continue;
    t.chunk0[t.count] = chunks;
    if (copy)
      hipLaunchKernelGGL(ema_kernel<true>, dim3((unsigned)chunks), dim3(256), 0, stream, t, weight);
    else
      hipLaunchKernelGGL(ema_kernel<false>, dim3((unsigned)chunks), dim3(256), 0, stream, t,
                         weight);
    DIONW_TRY(check_launch("ema_update"));
  }
  return kOk;
}

}  // extern "C"
