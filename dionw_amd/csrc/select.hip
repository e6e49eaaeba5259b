// Top-k row selection of each block by its momentum l1 score
// (replaces torch.topk(sorted=False) + gather of _matrix_step.py:172-180).
//
// One workgroup per block. Scores are non-negative fp32, so their bit
// patterns order like the values: a 4-pass 8-bit radix select finds the k-th
// largest key exactly; rows above it are taken, and of the rows equal to it
// the lowest indices. The index set is therefore a pure function of the
// scores. Outputs come in ascending row order, with the inverse map (slot of
// each row or -1) that the apply pass reads, and the block's input
// denominator: sqrt(sum of the selected rows' sums of squares) * safety + eps,
// the square root rounded to bfloat16 first when the iteration runs in bfloat16
// (the reference's quintics take the norm of their bf16 input as a bf16 tensor,
// _polar_express.py:57-58, 89-92).
#include "common.h"

namespace dionw {
namespace {

constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / kWave;

struct SelArgs {
  const float* scores;   // [B, rows]
  const float* rowsq;    // [B, rows]
  int32_t* idx;          // [B, k]
  int32_t* slot;         // [B, rows]
  float* den;            // [B]
  int64_t rows, k;
  float safety, eps;
  int round_bf16;
};

__global__ __launch_bounds__(kSelThreads) void select_kernel(SelArgs a) {
  __shared__ uint32_t hist[256];
  __shared__ uint32_t s_prefix, s_remaining;
  __shared__ uint32_t wave_gt[kSelWaves], wave_eq[kSelWaves];
  __shared__ float wave_part[kSelWaves];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int64_t b = blockIdx.x;
  const uint32_t* keys = reinterpret_cast<const uint32_t*>(a.scores + b * a.rows);

  uint32_t prefix = 0, mask = 0, remaining = (uint32_t)a.k;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < 256; i += kSelThreads) hist[i] = 0;
    __syncthreads();
    for (int64_t i = tid; i < a.rows; i += kSelThreads) {
      const uint32_t key = keys[i];
      if ((key & mask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t above = 0;
      int digit = 255;
      for (; digit > 0; --digit) {
        if (above + hist[digit] >= remaining) break;
        above += hist[digit];
      }
      s_prefix = prefix | ((uint32_t)digit << shift);
      s_remaining = remaining - above;
    }
    __syncthreads();
    prefix = s_prefix;
    remaining = s_remaining;
    mask |= 255u << shift;
    __syncthreads();
  }
  const uint32_t kth = prefix;       // the k-th largest key
  const uint32_t need_eq = remaining;  // how many rows equal to it are taken

  // Index-ordered compaction.
  uint32_t gt_before = 0, eq_before = 0;
  float part = 0.f;
  const float* rowsq = a.rowsq + b * a.rows;
  for (int64_t base = 0; base < a.rows; base += kSelThreads) {
    const int64_t i = base + tid;
    const bool valid = i < a.rows;
    const uint32_t key = valid ? keys[i] : 0u;
    const bool gt = valid && key > kth;
    const bool eq = valid && key == kth;
    const uint64_t mgt = __ballot(gt), meq = __ballot(eq);
    const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    const uint32_t lgt = __popcll(mgt & below), leq = __popcll(meq & below);
    if (lane == 0) {
      wave_gt[wave] = __popcll(mgt);
      wave_eq[wave] = __popcll(meq);
    }
    __syncthreads();
    uint32_t wgt = 0, weq = 0, tgt = 0, teq = 0;
    for (int w = 0; w < kSelWaves; ++w) {
      if (w < wave) {
        wgt += wave_gt[w];
        weq += wave_eq[w];
      }
      tgt += wave_gt[w];
      teq += wave_eq[w];
    }
    const uint32_t my_gt = gt_before + wgt + lgt;
    const uint32_t my_eq = eq_before + weq + leq;
    const bool take = gt || (eq && my_eq < need_eq);
    if (valid) {
      const uint32_t pos = my_gt + (my_eq < need_eq ? my_eq : need_eq);
      if (take) {
        a.idx[b * a.k + pos] = (int32_t)i;
        part += rowsq[i];
      }
      a.slot[b * a.rows + i] = take ? (int32_t)pos : -1;
    }
    gt_before += tgt;
    eq_before += teq;
    __syncthreads();
  }
  part = wave_sum(part);
  if (lane == 0) wave_part[wave] = part;
  __syncthreads();
  if (tid == 0) {
    float s = 0.f;
    for (int w = 0; w < kSelWaves; ++w) s += wave_part[w];
    const float norm = a.round_bf16 ? (float)(__bf16)sqrtf(s) : sqrtf(s);
    a.den[b] = norm * a.safety + a.eps;
  }
}

}  // namespace
}  // namespace dionw

using namespace dionw;

extern "C" int dionw_select_rows(const float* scores, const float* row_sumsq, int64_t blocks,
                                 int64_t rows, int64_t k, float safety, float eps, int32_t* idx,
                                 int32_t* slot, float* den, int32_t elem, hipStream_t stream) {
  DIONW_REQUIRE(scores && row_sumsq && idx && slot && den, "select_rows: null pointer");
  DIONW_REQUIRE(elem == kF16 || elem == kBF16 || elem == kF32, "select_rows: bad elem %d", elem);
  DIONW_REQUIRE(rows > 0 && k > 0 && k <= rows && rows < (int64_t)1 << 31,
                "select_rows: need 0 < k <= rows < 2^31 (k=%lld rows=%lld)", (long long)k,
                (long long)rows);
  if (blocks == 0) return kOk;
  SelArgs a{scores, row_sumsq, idx, slot, den, rows, k, safety, eps, (int)(elem == kBF16)};
  hipLaunchKernelGGL(select_kernel, dim3((unsigned)blocks), dim3(kSelThreads), 0, stream, a);
  return check_launch("select_rows");
}
