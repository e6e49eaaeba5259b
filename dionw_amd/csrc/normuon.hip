// Steps 4 and 5 of a Dion block update: NorMuon row normalization
// (_row_normalization.py:41-60) and the weight update (_matrix_step.py:274-311).
//
//  row stats   per selected row: s = sum of O^2 (O the bf16 orthogonalized
//              rows), v' = lerp(v, s / cols, 1 - beta2) written back into the
//              bucket variance, d = sqrt(v') + 1e-8.
//  block scale per block: ||O||_F / max(||O / d||_F, 1e-8) * step, with
//              ||O / d||_F^2 taken as sum_rows s / d^2.
//  apply       W = W * decay on every row (when weight decay is on), then on
//              the selected rows W += (O / d) * scale, so that the update is
//              never materialized in HBM.
//
// Contraction is off in this file: every product and sum rounds on its own,
// as the reference's separate torch ops do.
#pragma clang fp contract(off)

#include "common.h"

#include <mutex>

namespace dionw {
namespace {

// Device scratch of dionw_normuon_stats_noalloc: the per-row sums s and
// s / d^2 (two floats per selected row) that block_scale_kernel reduces.
// Every element it reads is written first by row_stats_kernel in the same
// call, so nothing needs clearing between calls. One copy per GPU, held until
// the process ends; calls that overlap on one GPU race on it.
constexpr int64_t kNoAllocRows = int64_t(1) << 19;  // 524288 selected rows, 4 MiB
static __device__ __align__(256) float scratch[2 * kNoAllocRows];

struct StatArgs {
  const __bf16* o;      // [B, k, cols]
  float* variance;      // [B, rows] run variance (updated at the selected rows)
  const int32_t* idx;   // [B, k] or nullptr (every row)
  float* rowd;          // [B, k]
  float* rows_s;        // [B, k]
  float* rows_t;        // [B, k]
  int64_t blocks, k, rows, cols;
  float weight;         // 1 - beta2
  int vec;
};

__global__ __launch_bounds__(256) void row_stats_kernel(StatArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= a.blocks * a.k) return;
  const __bf16* o = a.o + r * a.cols;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  if (a.vec) {
    const int64_t n8 = a.cols >> 3;
    const bf16x8* o8 = reinterpret_cast<const bf16x8*>(o);
    for (int64_t c = lane; c < n8; c += kWave) {
      bf16x8 v = o8[c];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float x = (float)v[e], y = (float)v[e + 1];
        acc[e >> 1] += x * x + y * y;
      }
    }
  } else {
    for (int64_t c = lane; c < a.cols; c += kWave) {
      float x = (float)o[c];
      acc.x += x * x;
    }
  }
  const float s = wave_sum((acc.x + acc.y) + (acc.z + acc.w));
  if (lane == 0) {
    const int64_t b = r / a.k, p = r - b * a.k;
    const int64_t vrow = b * a.rows + (a.idx ? (int64_t)a.idx[r] : p);
    const float v = a.variance[vrow];
    const float ms = s / (float)a.cols;
    const float w = a.weight;
    const float nv = w < 0.5f ? v + w * (ms - v) : ms - (ms - v) * (1.f - w);
    a.variance[vrow] = nv;
    const float d = sqrtf(nv) + 1e-8f;
    a.rowd[r] = d;
    a.rows_s[r] = s;
    a.rows_t[r] = s / (d * d);
  }
}

__global__ __launch_bounds__(64) void block_scale_kernel(const float* rows_s, const float* rows_t,
                                                         float* scale, int64_t k, float step) {
  const int64_t b = blockIdx.x;
  float s = 0.f, t = 0.f;
  for (int64_t i = threadIdx.x; i < k; i += kWave) {
    s += rows_s[b * k + i];
    t += rows_t[b * k + i];
  }
  s = wave_sum(s);
  t = wave_sum(t);
  if (threadIdx.x == 0) {
    const float restore = sqrtf(s) / fmaxf(sqrtf(t), 1e-8f);
    scale[b] = restore * step;
  }
}

struct ApplyArgs {
  RowTable t;             // parameters, rows_per_tensor rows of cols each
  const __bf16* o;        // [B, k, cols]
  const int32_t* slot;    // [B, rows] slot of each row or -1; nullptr: slot = row
  const int32_t* idx;     // [B, k] (only_selected)
  const float* rowd;      // [B, k] or nullptr (no row normalization)
  const float* scale;     // [B] or nullptr (use step)
  float step, decay;
  int apply_decay, only_selected, vec;
  int64_t rows_per_tensor, rows, cols, k;
  // Per parameter, laid out like it: the EMA shadow (kApplyEma) or the pinned
  // host staging buffer the new weights are also written to (kApplyStage).
  float* side[kMaxTensors];
  float ema_weight;
};

// What the apply pass does besides W's update.
enum ApplyMode : int {
  kApplyPlain = 0,  // nothing
  kApplyEma = 1,    // S = lerp(S, W_new) on every row (GPU EMA fused in)
  kApplyStage = 2,  // every row's W_new also stored to host memory (CPU EMA snapshot)
};

__device__ __forceinline__ float update_one(float w, float o, float d, float s,
                                            bool normalized, float decay, bool apply_decay) {
  if (apply_decay) w = w * decay;
  const float n = normalized ? o / d : o;
  return w + n * s;
}

// One 256-thread workgroup per row (a row sweep of 4 KiB per step streams
// faster than a wavefront per row).
constexpr int kApplyThreads = 256;

// kApplyEma: every row's shadow also moves to the row's new weights (lerp with
// ema_weight), also on rows that are only decayed or not changed at all.
// kApplyStage: every row's new weights are also stored to the row's place in a
// pinned host buffer (over the host link; the device copy is not read again).
template <int Mode>
__global__ __launch_bounds__(kApplyThreads) void apply_kernel(ApplyArgs a) {
  constexpr bool EMA = Mode == kApplyEma;
  constexpr bool STAGE = Mode == kApplyStage;
  const int tid = threadIdx.x;
  const int64_t r = blockIdx.x;  // the grid has exactly one workgroup per row
  int64_t gr, slot, b;
  if (a.only_selected) {
    b = r / a.k;
    slot = r - b * a.k;
    gr = b * a.rows + a.idx[r];
  } else {
    gr = r;
    b = gr / a.rows;
    const int64_t in_block = gr - b * a.rows;
    slot = a.slot ? (int64_t)a.slot[b * a.rows + in_block] : in_block;
  }
  const int tensor = (int)(gr / a.rows_per_tensor);
  const int64_t offset = (gr - (int64_t)tensor * a.rows_per_tensor) * a.cols;
  float* w = a.t.param[tensor] + offset;
  float* sh = (EMA || STAGE) ? a.side[tensor] + offset : nullptr;
  const bool apply_decay = a.apply_decay != 0;
  constexpr int U = 4;  // chunks whose loads are issued together
  constexpr int T = kApplyThreads;
  // The new weights' other destination: the EMA shadow's lerp or the host copy.
  auto side4 = [&](f32x4 wv, int64_t c) {
    f32x4* s4 = reinterpret_cast<f32x4*>(sh);
    if (EMA) {
      f32x4 sv = __builtin_nontemporal_load(s4 + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) sv[e] = ema_lerp(sv[e], wv[e], a.ema_weight);
      __builtin_nontemporal_store(sv, s4 + c);
    }
    if (STAGE) s4[c] = wv;
  };
  auto side1 = [&](float wv, int64_t c) {
    if (EMA) sh[c] = ema_lerp(sh[c], wv, a.ema_weight);
    if (STAGE) sh[c] = wv;
  };
  // Every element is read once and written once: the vector paths stream
  // (non-temporal loads and stores), which moves this traffic faster.
  if (slot < 0) {
    if (!apply_decay && !EMA && !STAGE) return;
    // Rows outside the selection: W = W d (weight decay), and the side copy.
    auto row_end = [&](f32x4 wv, int64_t c) {
      if (apply_decay) {
        wv = wv * a.decay;
        __builtin_nontemporal_store(wv, reinterpret_cast<f32x4*>(w) + c);
      }
      side4(wv, c);
    };
    if (a.vec) {
      const f32x4* w4 = reinterpret_cast<const f32x4*>(w);
      const int64_t n4 = a.cols >> 2;
      int64_t c = tid;
      for (; c + (U - 1) * T < n4; c += U * T) {
        f32x4 wv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) wv[u] = __builtin_nontemporal_load(w4 + c + u * T);
#pragma unroll
        for (int u = 0; u < U; ++u) row_end(wv[u], c + u * T);
      }
      for (; c < n4; c += T) row_end(__builtin_nontemporal_load(w4 + c), c);
    } else {
      for (int64_t c = tid; c < a.cols; c += T) {
        float wv = w[c];
        if (apply_decay) w[c] = wv = wv * a.decay;
        side1(wv, c);
      }
    }
    return;
  }
  const int64_t orow = b * a.k + slot;
  const __bf16* o = a.o + orow * a.cols;
  const bool normalized = a.rowd != nullptr;
  const float d = normalized ? a.rowd[orow] : 1.f;
  const float s = a.scale ? a.scale[b] : a.step;
  if (a.vec) {
    f32x4* w4 = reinterpret_cast<f32x4*>(w);
    const bf16x4* o4 = reinterpret_cast<const bf16x4*>(o);
    auto upd = [&](f32x4 wv, bf16x4 ov) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        wv[e] = update_one(wv[e], (float)ov[e], d, s, normalized, a.decay, apply_decay);
      return wv;
    };
    auto store = [&](int64_t c, f32x4 wv) {
      __builtin_nontemporal_store(wv, w4 + c);
      side4(wv, c);
    };
    const int64_t n4 = a.cols >> 2;
    int64_t c = tid;
    for (; c + (U - 1) * T < n4; c += U * T) {
      f32x4 wv[U];
      bf16x4 ov[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        wv[u] = __builtin_nontemporal_load(w4 + c + u * T);
        ov[u] = __builtin_nontemporal_load(o4 + c + u * T);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) store(c + u * T, upd(wv[u], ov[u]));
    }
    for (; c < n4; c += T)
      store(c, upd(__builtin_nontemporal_load(w4 + c), __builtin_nontemporal_load(o4 + c)));
  } else {
    for (int64_t c = tid; c < a.cols; c += T) {
      const float wv = update_one(w[c], (float)o[c], d, s, normalized, a.decay, apply_decay);
      w[c] = wv;
      side1(wv, c);
    }
  }
}

// The device-side address of a host buffer the apply pass writes to: it must be
// pinned host memory mapped into the device's address space (hipHostMalloc, or
// torch's pin_memory=True); anything else is rejected before a launch.
int host_staging_address(float* host, int index, float** device) {
  DIONW_REQUIRE(host, "apply_update_stage: null host staging buffer %d", index);
  hipPointerAttribute_t attr{};
  const hipError_t rc = hipPointerGetAttributes(&attr, host);
  if (rc != hipSuccess) {
    (void)hipGetLastError();  // an unknown pointer leaves the error set: clear it
    set_error("apply_update_stage: host staging buffer %d is not pinned host memory (%s)", index,
              hipGetErrorString(rc));
    return kInvalid;
  }
  DIONW_REQUIRE(attr.type == hipMemoryTypeHost && attr.devicePointer,
                "apply_update_stage: host staging buffer %d is not pinned host memory mapped "
                "for the device (memory type %d)", index, (int)attr.type);
  *device = static_cast<float*>(attr.devicePointer);
  return kOk;
}

// One launch per kMaxTensors parameters. `side` (null for kApplyPlain) holds one
// buffer per parameter: EMA shadows (kApplyEma) or host staging (kApplyStage).
int apply_launch(int mode, float* const* params, float* const* side, int32_t count,
                 int64_t blocks_per_tensor, int64_t rows, int64_t cols, int64_t k,
                 const void* orthogonal, const int32_t* idx, const int32_t* slot,
                 const float* rowd, const float* scale, float step, float decay,
                 int32_t apply_decay, float ema_weight, hipStream_t stream) {
  DIONW_REQUIRE(orthogonal && count >= 0 && blocks_per_tensor > 0 && rows > 0 && cols > 0 &&
                    k > 0 && k <= rows,
                "apply_update: bad arguments");
  DIONW_REQUIRE(k == rows || (idx && slot), "apply_update: row selection needs idx and slot");
  DIONW_REQUIRE((mode == kApplyPlain) == (side == nullptr), "apply_update: bad side table");
  for (int32_t start = 0; start < count; start += kMaxTensors) {
    ApplyArgs a{};
    a.t.count = (count - start) < kMaxTensors ? (count - start) : kMaxTensors;
    bool aligned = cols % 4 == 0;
    for (int i = 0; i < a.t.count; ++i) {
      DIONW_REQUIRE(params[start + i], "apply_update: null parameter %d", start + i);
      a.t.param[i] = params[start + i];
      aligned = aligned && aligned16(params[start + i]);
      if (mode == kApplyEma) {
        DIONW_REQUIRE(side[start + i], "apply_update: null EMA shadow %d", start + i);
        a.side[i] = side[start + i];
      } else if (mode == kApplyStage) {
        DIONW_TRY(host_staging_address(side[start + i], start + i, &a.side[i]));
      }
      if (side) aligned = aligned && aligned16(a.side[i]);
    }
    const int64_t b0 = (int64_t)start * blocks_per_tensor;
    a.o = reinterpret_cast<const __bf16*>(orthogonal) + b0 * k * cols;
    a.idx = idx ? idx + b0 * k : nullptr;
    a.slot = (slot && k < rows) ? slot + b0 * rows : nullptr;
    a.rowd = rowd ? rowd + b0 * k : nullptr;
    a.scale = scale ? scale + b0 : nullptr;
    a.step = step;
    a.decay = decay;
    a.apply_decay = apply_decay;
    a.rows_per_tensor = blocks_per_tensor * rows;
    a.rows = rows;
    a.cols = cols;
    a.k = k;
    a.vec = aligned && (reinterpret_cast<uintptr_t>(a.o) & 7) == 0;
    a.ema_weight = ema_weight;
    // The EMA and the host copy cover every row, so every row is visited.
    a.only_selected = !apply_decay && mode == kApplyPlain && k < rows;
    const int64_t n = a.only_selected ? (int64_t)a.t.count * blocks_per_tensor * k
                                      : (int64_t)a.t.count * a.rows_per_tensor;
    if (n == 0) continue;
    DIONW_REQUIRE(n * kApplyThreads <= (int64_t)UINT32_MAX,
                  "apply_update: %lld rows exceed one launch", (long long)n);
    const dim3 grid((unsigned)n), block(kApplyThreads);
    switch (mode) {
      case kApplyEma:
        hipLaunchKernelGGL(apply_kernel<kApplyEma>, grid, block, 0, stream, a);
        break;
      case kApplyStage:
        hipLaunchKernelGGL(apply_kernel<kApplyStage>, grid, block, 0, stream, a);
        break;
      default:
        hipLaunchKernelGGL(apply_kernel<kApplyPlain>, grid, block, 0, stream, a);
    }
    DIONW_TRY(check_launch("apply_update"));
  }
  return kOk;
}

int stats_launch(const void* orthogonal, int64_t blocks, int64_t k, int64_t rows, int64_t cols,
                 const int32_t* idx, float* variance, float beta2, float step, float* rowd,
                 float* partials, float* scale, hipStream_t stream) {
  DIONW_REQUIRE(orthogonal && variance && rowd && partials && scale,
                "normuon_stats: null pointer");
  DIONW_REQUIRE(blocks >= 0 && k > 0 && k <= rows && cols > 0, "normuon_stats: bad sizes");
  DIONW_REQUIRE(blocks < (int64_t{1} << 31) && ceil_div(blocks * k, 4) <= INT32_MAX,
                "normuon_stats: %lld blocks x %lld selected rows exceed one launch",
                (long long)blocks, (long long)k);
  DIONW_REQUIRE(idx || k == rows, "normuon_stats: every-row mode needs k == rows");
  if (blocks == 0) return kOk;
  StatArgs a{};
  a.o = reinterpret_cast<const __bf16*>(orthogonal);
  a.variance = variance;
  a.idx = idx;
  a.rowd = rowd;
  a.rows_s = partials;
  a.rows_t = partials + blocks * k;
  a.blocks = blocks;
  a.k = k;
  a.rows = rows;
  a.cols = cols;
  a.weight = 1.f - beta2;
  a.vec = cols % 8 == 0 && aligned16(orthogonal);
  hipLaunchKernelGGL(row_stats_kernel, dim3((unsigned)ceil_div(blocks * k, 4)), dim3(256), 0,
                     stream, a);
  DIONW_TRY(check_launch("normuon_stats"));
  hipLaunchKernelGGL(block_scale_kernel, dim3((unsigned)blocks), dim3(64), 0, stream, a.rows_s,
                     a.rows_t, scale, k, step);
  return check_launch("normuon_scale");
}

// The device address of `scratch` on the stream's GPU, looked up once per
// device with that device current (each GPU holds its own copy at its own
// address; the array's name in host code is only a stand-in for it).
constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
float* g_scratch[kMaxDevices] = {};

int device_scratch(hipStream_t stream, float** out) {
  int current = -1;
  hipError_t rc = hipGetDevice(&current);
  if (rc != hipSuccess) {
    set_error("normuon_stats_noalloc: hipGetDevice failed: %s", hipGetErrorString(rc));
    return kHipError;
  }
  int device = current;
  if (stream) {
    rc = hipStreamGetDevice(stream, &device);
    if (rc != hipSuccess) {
      set_error("normuon_stats_noalloc: hipStreamGetDevice failed: %s", hipGetErrorString(rc));
      return kHipError;
    }
  }
  DIONW_REQUIRE(device == current,
                "normuon_stats_noalloc: the stream is on device %d but device %d is current",
                device, current);
  DIONW_REQUIRE(device >= 0 && device < kMaxDevices, "normuon_stats_noalloc: device %d", device);
  std::lock_guard<std::mutex> hold(g_scratch_lock);
  if (!g_scratch[device]) {
    void* ptr = nullptr;
    rc = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (rc != hipSuccess || !ptr) {
      set_error("normuon_stats_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(rc));
      return kHipError;
    }
    g_scratch[device] = static_cast<float*>(ptr);
  }
  *out = g_scratch[device];
  return kOk;
}

}  // namespace
}  // namespace dionw

using namespace dionw;

extern "C" {

int dionw_normuon_stats(const void* orthogonal, int64_t blocks, int64_t k, int64_t rows,
                        int64_t cols, const int32_t* idx, float* variance, float beta2,
                        float step, float* rowd, float* partials, float* scale,
                        hipStream_t stream) {
  return stats_launch(orthogonal, blocks, k, rows, cols, idx, variance, beta2, step, rowd,
                      partials, scale, stream);
}

int dionw_normuon_stats_noalloc(const void* orthogonal, int64_t blocks, int64_t k, int64_t rows,
                                int64_t cols, const int32_t* idx, float* variance, float beta2,
                                float step, float* rowd, float* scale, hipStream_t stream) {
  DIONW_REQUIRE(blocks >= 0, "normuon_stats: bad sizes");
  DIONW_REQUIRE(blocks == 0 || k <= 0 || (k <= kNoAllocRows && blocks <= kNoAllocRows / k),
                "normuon_stats_noalloc: %lld blocks x %lld selected rows exceed the %lld rows "
                "of its device scratch (use dionw_normuon_stats with a caller workspace)",
                (long long)blocks, (long long)k, (long long)kNoAllocRows);
  float* partials = nullptr;
  DIONW_TRY(device_scratch(stream, &partials));
  return stats_launch(orthogonal, blocks, k, rows, cols, idx, variance, beta2, step, rowd,
                      partials, scale, stream);
}

int dionw_apply_update(float* const* params, int32_t count, int64_t blocks_per_tensor,
                       int64_t rows, int64_t cols, int64_t k, const void* orthogonal,
                       const int32_t* idx, const int32_t* slot, const float* rowd,
                       const float* scale, float step, float decay, int32_t apply_decay,
                       hipStream_t stream) {
  return apply_launch(kApplyPlain, params, nullptr, count, blocks_per_tensor, rows, cols, k,
                      orthogonal, idx, slot, rowd, scale, step, decay, apply_decay, 0.f, stream);
}

int dionw_apply_update_ema(float* const* params, float* const* shadows, int32_t count,
                           int64_t blocks_per_tensor, int64_t rows, int64_t cols, int64_t k,
                           const void* orthogonal, const int32_t* idx, const int32_t* slot,
                           const float* rowd, const float* scale, float step, float decay,
                           int32_t apply_decay, float ema_weight, hipStream_t stream) {
  DIONW_REQUIRE(shadows, "apply_update_ema: null shadow table");
  return apply_launch(kApplyEma, params, shadows, count, blocks_per_tensor, rows, cols, k,
                      orthogonal, idx, slot, rowd, scale, step, decay, apply_decay, ema_weight,
                      stream);
}

int dionw_apply_update_stage(float* const* params, float* const* staged, int32_t count,
                             int64_t blocks_per_tensor, int64_t rows, int64_t cols, int64_t k,
                             const void* orthogonal, const int32_t* idx, const int32_t* slot,
                             const float* rowd, const float* scale, float step, float decay,
                             int32_t apply_decay, hipStream_t stream) {
  DIONW_REQUIRE(staged, "apply_update_stage: null host staging table");
  return apply_launch(kApplyStage, params, staged, count, blocks_per_tensor, rows, cols, k,
                      orthogonal, idx, slot, rowd, scale, step, decay, apply_decay, 0.f, stream);
}

}  // extern "C"
