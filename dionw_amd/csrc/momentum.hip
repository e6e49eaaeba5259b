// Momentum passes of a Dion bucket run and the Newton-Schulz input cast.
//
//  accumulate   M += G per row, with the row's l1 score and sum of squares
//               (the selected path; replaces _momentum_kernels.py:40-55).
//  full sumsq   sum of squares of the Newton-Schulz input U of every row, no
//               writes (first pass of the every-row path, _momentum_kernels.py:58-77).
//  block denom  per block: sqrt(sum of the rows' sums of squares) * safety + eps.
//
// The sums of squares feed the Frobenius normalization of the Newton-Schulz
// input. For the float16 Gram iteration they are sums of the float32 values
// (_gram.py:85-86, the norm of x.float()). The bfloat16 quintics normalize the
// input rounded to bfloat16 by its norm, itself a bfloat16 tensor
// (_polar_express.py:57-58, 89-92: x.bfloat16(), then x.norm()): with elem
// kBF16 the sums take the bf16-rounded values and the norm is rounded to
// bfloat16 before the safety factor and eps are applied in float32, as the
// compiled reference evaluates x / (norm * safety + eps).
//  prepare      the single pass that writes the decayed momentum and the
//               normalized 16-bit Newton-Schulz input in the orientations the
//               iteration reads (_matrix_step.py:172-178 and _gram.py:83-87
//               fused), in 64 x 64 tiles (through LDS for the transpose).
//
// Row reductions use one 256-thread workgroup per row (its four waves sweep
// 4 KiB of each stream per step: 8% more HBM throughput than a wave per row at
// 4096 columns). Thread t accumulates four partial sums (one per float4
// component) over its float4 chunks t, t + 256, ... in column order, combines
// them as (x + y) + (z + w); each wave combines its lanes by the xor butterfly
// of wave_sum and the four wave sums combine as (w0 + w1) + (w2 + w3): the l1
// score is a fixed-order fp32 sum that the CPU oracle restates bit for bit.
#pragma clang fp contract(off)

#include "common.h"

#include <algorithm>
#include <type_traits>

namespace dionw {
namespace {

constexpr int kRowThreads = 256;  // one workgroup of four waves per row

enum AccMode : int { kScores = 0, kFullSumsq = 1 };

struct AccArgs {
  RowTable t;
  float* momentum;        // [count * rows_per_tensor, cols], run-contiguous
  float* scores;          // [rows] l1 of M + G (kScores)
  float* rowsq;           // [rows] sum of squares of M + G, or of U (kFullSumsq)
  int64_t rows_per_tensor;
  int64_t cols;
  float mu;               // kFullSumsq: momentum decay
  int nesterov;           // kFullSumsq: U = G + mu (M + G) instead of M + G
  int vec;                // float4 path: cols % 4 == 0 and 16-byte aligned rows
  int round_bf16;         // sums of squares of the bf16-rounded values
};

__device__ __forceinline__ float bf16_round(float x) { return (float)(__bf16)x; }

__device__ __forceinline__ f32x4 bf16_round4(f32x4 v) {
  return f32x4{bf16_round(v.x), bf16_round(v.y), bf16_round(v.z), bf16_round(v.w)};
}

// The normalization denominator of a block from its sum of squares s.
__device__ __forceinline__ float norm_denom(float s, float safety, float eps, bool round_bf16) {
  const float norm = round_bf16 ? bf16_round(sqrtf(s)) : sqrtf(s);
  return norm * safety + eps;
}

// Four consecutive input elements (float4 index c of a row of IN) as floats,
// streamed. IN is float, or the 16-bit type of an Orthogonalize input
// (dionw_normalize_input), whose conversion to float is exact.
template <typename IN>
__device__ __forceinline__ f32x4 load4_nt(const IN* row, int64_t c) {
  if constexpr (std::is_same<IN, float>::value) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(row) + c);
  } else {
    typedef IN in4 __attribute__((ext_vector_type(4)));
    const in4 v = __builtin_nontemporal_load(reinterpret_cast<const in4*>(row) + c);
    return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
  }
}

// (s0 + s1) + (s2 + s3) of the four wave sums of a row's workgroup.
__device__ __forceinline__ float row_sum(float v, float* part) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = v;
  __syncthreads();
  return (part[0] + part[1]) + (part[2] + part[3]);
}

template <int MODE, typename IN = float>
__global__ __launch_bounds__(kRowThreads) void accumulate_kernel(AccArgs a) {
  static_assert(MODE == kFullSumsq || std::is_same<IN, float>::value,
                "only the sums of squares read 16-bit inputs");
  __shared__ float part[2][4];
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.x;  // the grid has exactly one workgroup per row
  const int tensor = (int)(row / a.rows_per_tensor);
  const int64_t local = row - (int64_t)tensor * a.rows_per_tensor;
  const IN* g = reinterpret_cast<const IN*>(a.t.grad[tensor]) + local * a.cols;
  float* m = a.momentum ? a.momentum + row * a.cols : nullptr;

  f32x4 l1 = {0.f, 0.f, 0.f, 0.f};
  f32x4 sq = {0.f, 0.f, 0.f, 0.f};
  if (a.vec) {
    const int64_t n4 = a.cols >> 2;
    f32x4* m4 = reinterpret_cast<f32x4*>(m);
    const bool has_m = MODE == kScores || a.momentum;
    // M is read once and written once: streaming (non-temporal) loads and
    // stores of it, as of G, move this mix ~7% faster than cached ones.
    auto load_m = [&](int64_t c) {
      if (!has_m) return f32x4{0.f, 0.f, 0.f, 0.f};
      return MODE == kScores ? __builtin_nontemporal_load(m4 + c) : m4[c];
    };
    auto step = [&](int64_t c, f32x4 gv, f32x4 mv) {
      f32x4 s = mv + gv;
      if (MODE == kScores) {
        __builtin_nontemporal_store(s, m4 + c);
        l1 += __builtin_elementwise_abs(s);
        const f32x4 r = a.round_bf16 ? bf16_round4(s) : s;
        sq += r * r;
      } else {
        f32x4 u = s;
        if (a.nesterov) u = gv + s * a.mu;
        if (a.round_bf16) u = bf16_round4(u);
        sq += u * u;
      }
    };
    // Loads of kUnroll chunks are issued together (more bytes in flight per
    // thread); the sums still take the chunks in column order.
    constexpr int kUnroll = 4;
    int64_t c = tid;
    for (; c + (kUnroll - 1) * kRowThreads < n4; c += kUnroll * kRowThreads) {
      f32x4 gv[kUnroll], mv[kUnroll];
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) {
        gv[u] = load4_nt(g, c + u * kRowThreads);
        mv[u] = load_m(c + u * kRowThreads);
      }
#pragma unroll
      for (int u = 0; u < kUnroll; ++u) step(c + u * kRowThreads, gv[u], mv[u]);
    }
    for (; c < n4; c += kRowThreads)
      step(c, load4_nt(g, c), load_m(c));
  } else {
    // Scalar path (any cols, any alignment): component 0 carries the sums.
    for (int64_t c = tid; c < a.cols; c += kRowThreads) {
      float gv = (float)g[c];
      float s = ((MODE == kScores || a.momentum) ? m[c] : 0.f) + gv;
      if (MODE == kScores) {
        m[c] = s;
        l1.x += fabsf(s);
        const float r = a.round_bf16 ? bf16_round(s) : s;
        sq.x += r * r;
      } else {
        float u = a.nesterov ? gv + s * a.mu : s;
        if (a.round_bf16) u = bf16_round(u);
        sq.x += u * u;
      }
    }
  }
  const float sqs = row_sum((sq.x + sq.y) + (sq.z + sq.w), part[0]);
  if (MODE == kScores) {
    const float l = row_sum((l1.x + l1.y) + (l1.z + l1.w), part[1]);
    if (tid == 0) {
      a.scores[row] = l;
      a.rowsq[row] = sqs;
    }
  } else if (tid == 0) {
    a.rowsq[row] = sqs;
  }
}

// den[b] = norm_denom(sum of rowsq over the block's rows); one wave per block.
__global__ __launch_bounds__(64) void block_denom_kernel(const float* rowsq, float* den,
                                                         int64_t rows, float safety, float eps,
                                                         int round_bf16) {
  const int64_t b = blockIdx.x;
  const float* r = rowsq + b * rows;
  float s = 0.f;
  for (int64_t i = threadIdx.x; i < rows; i += kWave) s += r[i];
  s = wave_sum(s);
  if (threadIdx.x == 0) den[b] = norm_denom(s, safety, eps, round_bf16 != 0);
}

// ---- prepare: decayed momentum + normalized 16-bit Newton-Schulz input ------

struct PrepArgs {
  RowTable t;             // gradients (full mode only)
  float* momentum;        // run momentum [B, rows, cols]
  const int32_t* idx;     // [B, k] selected rows (ascending), nullptr in full mode
  const float* den;       // [B] Frobenius norm + eps of the block's input
  void* out_r;            // [B, P_pad, J_pad]: row p of the input, W orientation (may be nullptr)
  void* out_t;            // [B, J_pad, P_pad]: its transpose (may be nullptr)
  int64_t rows, cols, k;  // block rows, cols, selected rows
  int64_t p_pad, j_pad;   // padded extents (zeros written in the padding)
  int64_t blocks_per_tensor;
  float mu;
  int full;               // every row: M = mu (M + G), U = M + G or Nesterov
  int nesterov;
  int write_m;            // write the decayed momentum
  int elem;               // kF16, kBF16 (quintic: bf16 input rounded first), kF32 (raw)
  int vec;                // float4 loads are legal (cols % 4 == 0, aligned)
};

constexpr int kTile = 64;

template <int ELEM, typename IN = float>
__global__ __launch_bounds__(256) void prepare_kernel(PrepArgs a) {
  using T = typename std::conditional<ELEM == kF16, _Float16, __bf16>::type;
  __shared__ T tile[kTile][kTile + 8];
  const int tx = threadIdx.x & 15;   // 4 columns each
  const int ty = threadIdx.x >> 4;   // rows ty + 16 i
  const int64_t b = blockIdx.z;
  const int64_t j0 = (int64_t)blockIdx.x * kTile + 4 * tx;
  const int64_t p_base = (int64_t)blockIdx.y * kTile;
  const float den = a.den[b];

  T vals[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t p = p_base + ty + 16 * i;
    float u[4] = {0.f, 0.f, 0.f, 0.f};
    if (p < a.k) {
      const int64_t src_row = a.full ? p : (int64_t)a.idx[b * a.k + p];
      float* m = a.momentum ? a.momentum + (b * a.rows + src_row) * a.cols : nullptr;
      const IN* g = nullptr;
      if (a.full) {
        const int64_t tensor = b / a.blocks_per_tensor;
        const int64_t local_row = (b - tensor * a.blocks_per_tensor) * a.rows + p;
        g = reinterpret_cast<const IN*>(a.t.grad[tensor]) + local_row * a.cols;
      }
      if (a.vec && j0 + 3 < a.cols) {
        f32x4 mv = m ? *reinterpret_cast<const f32x4*>(m + j0) : f32x4{0.f, 0.f, 0.f, 0.f};
        f32x4 uv, nm;
        if (a.full) {
          f32x4 gv = load4_nt(g + j0, 0);
          f32x4 s = mv + gv;
          nm = s * a.mu;
          uv = a.nesterov ? gv + nm : s;
        } else {
          uv = mv;
          nm = mv * a.mu;
        }
        if (a.write_m) *reinterpret_cast<f32x4*>(m + j0) = nm;
        u[0] = uv.x; u[1] = uv.y; u[2] = uv.z; u[3] = uv.w;
      } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const int64_t j = j0 + c;
          if (j < a.cols) {
            float mv = m ? m[j] : 0.f, uv, nm;
            if (a.full) {
              float gv = (float)g[j];
              float s = mv + gv;
              nm = s * a.mu;
              uv = a.nesterov ? gv + nm : s;
            } else {
              uv = mv;
              nm = mv * a.mu;
            }
            if (a.write_m) m[j] = nm;
            u[c] = uv;
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      float x;
      if (ELEM == kBF16) {
        // Keller / Polar Express: the input is rounded to bf16 before the division.
        x = (float)(__bf16)u[c] / den;
      } else {
        x = u[c] / den;
      }
      vals[i][c] = (T)x;  // padding rows/cols hold u = 0 -> 0
    }
  }
  // Row-major output [P_pad, J_pad] (may be skipped).
  T* out_r = a.out_r ? reinterpret_cast<T*>(a.out_r) + b * a.p_pad * a.j_pad : nullptr;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t p = p_base + ty + 16 * i;
    if (out_r && p < a.p_pad) {
      if (j0 + 3 < a.j_pad) {
        typedef T t4 __attribute__((ext_vector_type(4)));
        t4 v = {vals[i][0], vals[i][1], vals[i][2], vals[i][3]};
        *reinterpret_cast<t4*>(out_r + p * a.j_pad + j0) = v;
      } else {
        for (int c = 0; c < 4; ++c)
          if (j0 + c < a.j_pad) out_r[p * a.j_pad + j0 + c] = vals[i][c];
      }
    }
  }
  if (a.out_t == nullptr) return;
  // Transposed output [J_pad, P_pad] through LDS.
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int c = 0; c < 4; ++c) tile[4 * tx + c][ty + 16 * i] = vals[i][c];
  __syncthreads();
  T* out_t = reinterpret_cast<T*>(a.out_t) + b * a.j_pad * a.p_pad;
  const int jj = threadIdx.x >> 2;          // tile column -> output row
  const int pp = (threadIdx.x & 3) * 16;    // 16 consecutive p
  const int64_t j = (int64_t)blockIdx.x * kTile + jj;
  if (j < a.j_pad) {
    T* dst = out_t + j * a.p_pad + p_base + pp;
    if (p_base + pp + 15 < a.p_pad) {
      typedef T t8 __attribute__((ext_vector_type(8)));
      t8 v0, v1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v0[e] = tile[jj][pp + e];
        v1[e] = tile[jj][pp + 8 + e];
      }
      reinterpret_cast<t8*>(dst)[0] = v0;
      reinterpret_cast<t8*>(dst)[1] = v1;
    } else {
      for (int e = 0; e < 16; ++e)
        if (p_base + pp + e < a.p_pad) dst[e] = tile[jj][pp + e];
    }
  }
}

// X = 16-bit(x / den) of a 16-bit input x (dionw_normalize_input): the
// every-row prepare pass without momentum, with 8 columns per thread so that
// loads and stores are 16 bytes per lane (a.vec: 8-element rows from a 16-byte
// aligned address). The same arithmetic, padding and outputs as prepare_kernel.
template <int ELEM, typename IN>
__global__ __launch_bounds__(256) void prepare_input16_kernel(PrepArgs a) {
  using T = typename std::conditional<ELEM == kF16, _Float16, __bf16>::type;
  typedef IN in8 __attribute__((ext_vector_type(8)));
  typedef T t8 __attribute__((ext_vector_type(8)));
  __shared__ T tile[kTile][kTile + 8];
  const int tx = threadIdx.x & 7;   // 8 columns each
  const int ty = threadIdx.x >> 3;  // rows ty + 32 i
  const int64_t b = blockIdx.z;
  const int64_t j0 = (int64_t)blockIdx.x * kTile + 8 * tx;
  const int64_t p_base = (int64_t)blockIdx.y * kTile;
  const float den = a.den[b];
  const IN* x = reinterpret_cast<const IN*>(a.t.grad[0]) + b * a.rows * a.cols;

  T vals[2][8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t p = p_base + ty + 32 * i;
    float u[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (p < a.k) {
      const IN* row = x + p * a.cols;
      if (a.vec && j0 + 7 < a.cols) {
        const in8 v = __builtin_nontemporal_load(reinterpret_cast<const in8*>(row + j0));
#pragma unroll
        for (int c = 0; c < 8; ++c) u[c] = (float)v[c];
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c)
          if (j0 + c < a.cols) u[c] = (float)row[j0 + c];
      }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float q;
      if (ELEM == kBF16) {
        q = (float)(__bf16)u[c] / den;
      } else {
        q = u[c] / den;
      }
      vals[i][c] = (T)q;  // padding rows/cols hold u = 0 -> 0
    }
  }
  T* out_r = a.out_r ? reinterpret_cast<T*>(a.out_r) + b * a.p_pad * a.j_pad : nullptr;
  const bool store8 = (reinterpret_cast<uintptr_t>(a.out_r) & 15) == 0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int64_t p = p_base + ty + 32 * i;
    if (out_r && p < a.p_pad) {
      if (j0 + 7 < a.j_pad && store8) {
        t8 v;
#pragma unroll
        for (int c = 0; c < 8; ++c) v[c] = vals[i][c];
        *reinterpret_cast<t8*>(out_r + p * a.j_pad + j0) = v;
      } else {
        for (int c = 0; c < 8; ++c)
          if (j0 + c < a.j_pad) out_r[p * a.j_pad + j0 + c] = vals[i][c];
      }
    }
  }
  if (a.out_t == nullptr) return;
  // Transposed output [J_pad, P_pad] through LDS, read out as in prepare_kernel.
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int c = 0; c < 8; ++c) tile[8 * tx + c][ty + 32 * i] = vals[i][c];
  __syncthreads();
  T* out_t = reinterpret_cast<T*>(a.out_t) + b * a.j_pad * a.p_pad;
  const int jj = threadIdx.x >> 2;          // tile column -> output row
  const int pp = (threadIdx.x & 3) * 16;    // 16 consecutive p
  const int64_t j = (int64_t)blockIdx.x * kTile + jj;
  if (j < a.j_pad) {
    T* dst = out_t + j * a.p_pad + p_base + pp;
    if (p_base + pp + 15 < a.p_pad) {
      t8 v0, v1;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        v0[e] = tile[jj][pp + e];
        v1[e] = tile[jj][pp + 8 + e];
      }
      reinterpret_cast<t8*>(dst)[0] = v0;
      reinterpret_cast<t8*>(dst)[1] = v1;
    } else {
      for (int e = 0; e < 16; ++e)
        if (p_base + pp + e < a.p_pad) dst[e] = tile[jj][pp + e];
    }
  }
}

// Raw fp32 copy of the input rows for a user-supplied orthogonalization
// ([B, k, cols], no normalization), with the same momentum writes.
__global__ __launch_bounds__(256) void prepare_raw_kernel(PrepArgs a) {
  const int64_t b = blockIdx.z;
  const int64_t p = (int64_t)blockIdx.y;
  float* out = reinterpret_cast<float*>(a.out_r) + (b * a.k + p) * a.cols;
  const int64_t src_row = a.full ? p : (int64_t)a.idx[b * a.k + p];
  float* m = a.momentum ? a.momentum + (b * a.rows + src_row) * a.cols : nullptr;
  const float* g = nullptr;
  if (a.full) {
    const int64_t tensor = b / a.blocks_per_tensor;
    const int64_t local_row = (b - tensor * a.blocks_per_tensor) * a.rows + p;
    g = a.t.grad[tensor] + local_row * a.cols;
  }
  for (int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x; j < a.cols;
       j += (int64_t)gridDim.x * 256) {
    float mv = m ? m[j] : 0.f, uv, nm;
    if (a.full) {
      float gv = g[j];
      float s = mv + gv;
      nm = s * a.mu;
      uv = a.nesterov ? gv + nm : s;
    } else {
      uv = mv;
      nm = mv * a.mu;
    }
    if (a.write_m) m[j] = nm;
    out[j] = uv;
  }
}

bool table_aligned(const RowTable& t, int64_t cols) {
  if (cols % 4) return false;
  for (int i = 0; i < t.count; ++i)
    if (!aligned16(t.grad[i])) return false;
  return true;
}

}  // namespace
}  // namespace dionw

using namespace dionw;

extern "C" {

int dionw_accumulate_scores(const float* const* grads, int32_t count, int64_t rows_per_tensor,
                            int64_t cols, float* momentum, float* scores, float* row_sumsq,
                            int32_t elem, hipStream_t stream) {
  DIONW_REQUIRE(count >= 0 && rows_per_tensor > 0 && cols > 0,
                "accumulate_scores: bad sizes (count=%d rows=%lld cols=%lld)", count,
                (long long)rows_per_tensor, (long long)cols);
  DIONW_REQUIRE(momentum && scores && row_sumsq, "accumulate_scores: null output");
  DIONW_REQUIRE(elem == kF16 || elem == kBF16 || elem == kF32, "accumulate_scores: bad elem %d",
                elem);
  for (int32_t start = 0; start < count; start += kMaxTensors) {
    AccArgs a{};
    a.t.count = (count - start) < kMaxTensors ? (count - start) : kMaxTensors;
    for (int i = 0; i < a.t.count; ++i) {
      DIONW_REQUIRE(grads[start + i], "accumulate_scores: null gradient %d", start + i);
      a.t.grad[i] = grads[start + i];
    }
    const int64_t row0 = (int64_t)start * rows_per_tensor;
    a.momentum = momentum + row0 * cols;
    a.scores = scores + row0;
    a.rowsq = row_sumsq + row0;
    a.rows_per_tensor = rows_per_tensor;
    a.cols = cols;
    a.vec = table_aligned(a.t, cols) && aligned16(a.momentum);
    a.round_bf16 = elem == kBF16;
    const int64_t rows = (int64_t)a.t.count * rows_per_tensor;
    DIONW_REQUIRE(rows * kRowThreads <= (int64_t)UINT32_MAX,
                  "accumulate_scores: %lld rows exceed one launch", (long long)rows);
    hipLaunchKernelGGL(accumulate_kernel<kScores>, dim3((unsigned)rows), dim3(kRowThreads), 0,
                       stream, a);
    DIONW_TRY(check_launch("accumulate_scores"));
  }
  return kOk;
}

int dionw_full_sumsq(const float* const* grads, int32_t count, int64_t rows_per_tensor,
                     int64_t cols, const float* momentum, float mu, int32_t nesterov,
                     float* row_sumsq, int32_t elem, hipStream_t stream) {
  DIONW_REQUIRE(count >= 0 && rows_per_tensor > 0 && cols > 0, "full_sumsq: bad sizes");
  DIONW_REQUIRE(row_sumsq, "full_sumsq: null pointer");
  DIONW_REQUIRE(elem == kF16 || elem == kBF16 || elem == kF32, "full_sumsq: bad elem %d", elem);
  for (int32_t start = 0; start < count; start += kMaxTensors) {
    AccArgs a{};
    a.t.count = (count - start) < kMaxTensors ? (count - start) : kMaxTensors;
    for (int i = 0; i < a.t.count; ++i) {
      DIONW_REQUIRE(grads[start + i], "full_sumsq: null gradient %d", start + i);
      a.t.grad[i] = grads[start + i];
    }
    const int64_t row0 = (int64_t)start * rows_per_tensor;
    a.momentum = momentum ? const_cast<float*>(momentum) + row0 * cols : nullptr;
    a.rowsq = row_sumsq + row0;
    a.rows_per_tensor = rows_per_tensor;
    a.cols = cols;
    a.mu = mu;
    a.nesterov = nesterov;
    a.vec = table_aligned(a.t, cols) && (!a.momentum || aligned16(a.momentum));
    a.round_bf16 = elem == kBF16;
    const int64_t rows = (int64_t)a.t.count * rows_per_tensor;
    DIONW_REQUIRE(rows * kRowThreads <= (int64_t)UINT32_MAX,
                  "full_sumsq: %lld rows exceed one launch", (long long)rows);
    hipLaunchKernelGGL(accumulate_kernel<kFullSumsq>, dim3((unsigned)rows), dim3(kRowThreads), 0,
                       stream, a);
    DIONW_TRY(check_launch("full_sumsq"));
  }
  return kOk;
}

int dionw_block_denom(const float* row_sumsq, int64_t blocks, int64_t rows, float safety,
                      float eps, float* den, int32_t elem, hipStream_t stream) {
  DIONW_REQUIRE(row_sumsq && den && blocks >= 0 && rows > 0, "block_denom: bad arguments");
  DIONW_REQUIRE(elem == kF16 || elem == kBF16 || elem == kF32, "block_denom: bad elem %d", elem);
  if (blocks == 0) return kOk;
  hipLaunchKernelGGL(block_denom_kernel, dim3((unsigned)blocks), dim3(64), 0, stream, row_sumsq,
                     den, rows, safety, eps, (int)(elem == kBF16));
  return check_launch("block_denom");
}

// See include/dionw_hip.h for the argument contract.
int dionw_normalize_input(const void* x, int32_t x_elem, int64_t blocks, int64_t rows,
                          int64_t cols, float safety, float eps, float* row_sumsq, float* den,
                          int64_t p_pad, int64_t j_pad, int32_t elem, void* out_rowmajor,
                          void* out_transposed, hipStream_t stream) {
  DIONW_REQUIRE(x && row_sumsq && den && (out_rowmajor || out_transposed),
                "normalize_input: null pointer");
  DIONW_REQUIRE(x_elem == kF16 || x_elem == kBF16 || x_elem == kF32,
                "normalize_input: bad input type %d", x_elem);
  DIONW_REQUIRE(elem == kF16 || elem == kBF16, "normalize_input: bad output type %d", elem);
  DIONW_REQUIRE(blocks >= 0 && rows > 0 && cols > 0, "normalize_input: bad sizes");
  DIONW_REQUIRE(p_pad >= rows && j_pad >= cols && p_pad % 8 == 0 && j_pad % 8 == 0,
                "normalize_input: padded extents must cover the block and be multiples of 8");
  if (blocks == 0) return kOk;
  DIONW_REQUIRE(blocks <= 65535 && ceil_div(p_pad, kTile) <= 65535 &&
                    blocks * rows * kRowThreads <= (int64_t)UINT32_MAX,
                "normalize_input: grid too large");
  // float4 loads of any input type: rows of a multiple of 4 elements from an
  // address aligned to 4 elements.
  const size_t in_size = x_elem == kF32 ? 4 : 2;
  const bool vec = cols % 4 == 0 && reinterpret_cast<uintptr_t>(x) % (4 * in_size) == 0;
  // Row sums of squares: the every-row pass without momentum (U = x).
  AccArgs acc{};
  acc.t.count = 1;
  acc.t.grad[0] = static_cast<const float*>(x);  // reinterpreted as the input type
  acc.rowsq = row_sumsq;
  acc.rows_per_tensor = blocks * rows;
  acc.cols = cols;
  acc.vec = vec;
  acc.round_bf16 = elem == kBF16;
  const dim3 row_grid((unsigned)(blocks * rows));
  if (x_elem == kF32)
    hipLaunchKernelGGL((accumulate_kernel<kFullSumsq, float>), row_grid, dim3(kRowThreads), 0,
                       stream, acc);
  else if (x_elem == kF16)
    hipLaunchKernelGGL((accumulate_kernel<kFullSumsq, _Float16>), row_grid, dim3(kRowThreads), 0,
                       stream, acc);
  else
    hipLaunchKernelGGL((accumulate_kernel<kFullSumsq, __bf16>), row_grid, dim3(kRowThreads), 0,
                       stream, acc);
  DIONW_TRY(check_launch("normalize_input"));
  hipLaunchKernelGGL(block_denom_kernel, dim3((unsigned)blocks), dim3(64), 0, stream, row_sumsq,
                     den, rows, safety, eps, (int)(elem == kBF16));
  DIONW_TRY(check_launch("normalize_input"));
  // X = 16-bit(x / den): the every-row prepare pass without momentum writes.
  PrepArgs a{};
  a.t.count = 1;
  a.t.grad[0] = static_cast<const float*>(x);
  a.den = den;
  a.out_r = out_rowmajor;
  a.out_t = out_transposed;
  a.rows = rows;
  a.cols = cols;
  a.k = rows;
  a.p_pad = p_pad;
  a.j_pad = j_pad;
  a.blocks_per_tensor = blocks;
  a.full = 1;
  a.elem = elem;
  a.vec = vec;
  const dim3 grid((unsigned)ceil_div(j_pad, kTile), (unsigned)ceil_div(p_pad, kTile),
                  (unsigned)blocks);
  if (x_elem == kF32) {
    if (elem == kF16) hipLaunchKernelGGL((prepare_kernel<kF16, float>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((prepare_kernel<kBF16, float>), grid, dim3(256), 0, stream, a);
    return check_launch("normalize_input");
  }
  // 16-bit input: 8 columns per thread, 16-byte accesses where rows allow them.
  a.vec = cols % 8 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
  if (elem == kF16) {
    if (x_elem == kF16) hipLaunchKernelGGL((prepare_input16_kernel<kF16, _Float16>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((prepare_input16_kernel<kF16, __bf16>), grid, dim3(256), 0, stream, a);
  } else {
    if (x_elem == kF16) hipLaunchKernelGGL((prepare_input16_kernel<kBF16, _Float16>), grid, dim3(256), 0, stream, a);
    else hipLaunchKernelGGL((prepare_input16_kernel<kBF16, __bf16>), grid, dim3(256), 0, stream, a);
  }
  return check_launch("normalize_input");
}

// See include/dionw_hip.h for the argument contract.
int dionw_prepare_ns_input(const float* const* grads, int32_t count, float* momentum,
                           const int32_t* idx, const float* den, int64_t blocks, int64_t rows,
                           int64_t cols, int64_t k, int64_t p_pad, int64_t j_pad, float mu,
                           int32_t nesterov, int32_t write_m, int32_t elem, void* out_rowmajor,
                           void* out_transposed, hipStream_t stream) {
  const bool full = idx == nullptr;
  DIONW_REQUIRE(den && (out_rowmajor || out_transposed), "prepare_ns_input: null pointer");
  DIONW_REQUIRE(out_rowmajor || elem != kF32, "prepare_ns_input: fp32 output needs out_rowmajor");
  DIONW_REQUIRE(momentum || (idx == nullptr && !write_m),
                "prepare_ns_input: only every-row mode without momentum writes may omit momentum");
  DIONW_REQUIRE(blocks >= 0 && rows > 0 && cols > 0 && k > 0 && k <= rows,
                "prepare_ns_input: bad sizes");
  DIONW_REQUIRE(!full || k == rows, "prepare_ns_input: every-row mode needs k == rows");
  DIONW_REQUIRE(elem == kF16 || elem == kBF16 || elem == kF32, "prepare_ns_input: bad elem %d",
                elem);
  if (elem != kF32)
    DIONW_REQUIRE(p_pad >= k && j_pad >= cols && p_pad % 8 == 0 && j_pad % 8 == 0,
                  "prepare_ns_input: padded extents must cover the block and be multiples of 8");
  else
    DIONW_REQUIRE(out_transposed == nullptr, "prepare_ns_input: fp32 output has no transpose");
  if (blocks == 0) return kOk;
  if (full) DIONW_REQUIRE(count > 0 && blocks % count == 0,
                          "prepare_ns_input: every-row mode needs gradients dividing the blocks");
  const int64_t bpt = full ? blocks / count : blocks;
  const int64_t out_elems = elem == kF32 ? k * cols : p_pad * j_pad;  // per block
  const size_t out_size = elem == kF32 ? 4 : 2;
  // Every-row mode walks the gradient list kMaxTensors at a time; selected mode
  // needs no table and runs in one launch.
  const int32_t chunks = full ? (int32_t)ceil_div(count, kMaxTensors) : 1;
  for (int32_t chunk = 0; chunk < chunks; ++chunk) {
    PrepArgs a{};
    int64_t b0 = 0, nb = blocks;
    if (full) {
      const int32_t t0 = chunk * kMaxTensors;
      a.t.count = std::min<int32_t>(kMaxTensors, count - t0);
      for (int i = 0; i < a.t.count; ++i) {
        DIONW_REQUIRE(grads[t0 + i], "prepare_ns_input: null gradient %d", t0 + i);
        a.t.grad[i] = grads[t0 + i];
      }
      b0 = (int64_t)t0 * bpt;
      nb = (int64_t)a.t.count * bpt;
    }
    a.momentum = momentum ? momentum + b0 * rows * cols : nullptr;
    a.idx = idx;
    a.den = den + b0;
    a.out_r = out_rowmajor ? static_cast<char*>(out_rowmajor) + b0 * out_elems * out_size
                           : nullptr;
    a.out_t = out_transposed ? static_cast<char*>(out_transposed) + b0 * out_elems * out_size
                             : nullptr;
    a.rows = rows;
    a.cols = cols;
    a.k = k;
    a.mu = mu;
    a.full = full;
    a.nesterov = nesterov;
    a.write_m = write_m;
    a.elem = elem;
    a.blocks_per_tensor = bpt;
    a.vec = (cols % 4 == 0) && (!a.momentum || aligned16(a.momentum)) &&
            (!full || table_aligned(a.t, cols));
    if (elem == kF32) {
      a.p_pad = k;
      a.j_pad = cols;
      dim3 grid((unsigned)std::min<int64_t>(ceil_div(cols, 256), 64), (unsigned)k, (unsigned)nb);
      DIONW_REQUIRE(nb <= 65535 && k <= 65535, "prepare_ns_input: grid too large");
      hipLaunchKernelGGL(prepare_raw_kernel, grid, dim3(256), 0, stream, a);
    } else {
      a.p_pad = p_pad;
      a.j_pad = j_pad;
      dim3 grid((unsigned)ceil_div(j_pad, kTile), (unsigned)ceil_div(p_pad, kTile), (unsigned)nb);
      DIONW_REQUIRE(nb <= 65535 && grid.y <= 65535, "prepare_ns_input: grid too large");
      if (elem == kF16)
        hipLaunchKernelGGL(prepare_kernel<kF16>, grid, dim3(256), 0, stream, a);
      else
        hipLaunchKernelGGL(prepare_kernel<kBF16>, grid, dim3(256), 0, stream, a);
    }
    DIONW_TRY(check_launch("prepare_ns_input"));
  }
  return kOk;
}

}  // extern "C"
