// MFMA products of the Newton-Schulz iterations and their drivers.
//
// Every product is one "NT" form, C[i,j] = sum_k A[i,k] B[j,k] with both
// operands row-major along k, computed with v_mfma_f32_32x32x16_{f16,bf16}
// (fp32 accumulation) from LDS-staged k tiles (64 deep; 32 deep where k is an
// odd multiple of 32). The epilogue forms
// alpha * acc + beta * D[i,j] and rounds once to the storage type; in mode
// kOutRoundAcc it rounds the product to the storage type first, then forms
// alpha * bf16(acc) + beta * D and rounds again (a product stored by one
// matmul and combined by a separate elementwise op, as the reference's cuBLAS
// quintic does, _polar_express.py:61-70). Float32 operands run on
// v_mfma_f32_32x32x2_f32 (gemm_f32_kernel).
//
//  symmetric mode  only tiles on and above the diagonal are computed and each
//                  is stored twice (itself and its mirror): X X^T (syrk,
//                  _symmetric_kernels.py:81-144), c A A + b A of a symmetric A
//                  (:147-218), and the products of the commuting symmetric
//                  polynomials in X X^T that Gram Newton-Schulz updates
//                  (_gram.py:58-69).
//  transposed out  a second store of C^T, so that the next product can read
//                  the result as its B operand (B must be k-contiguous).
//
// Drivers: dionw_newton_schulz sequences the Gram iteration (_gram.py:50-69,
// restart at iteration 2), the standard Polar Express iteration for square
// blocks (_gram.py:41-47) and the bf16 quintic of Keller / Polar Express
// (_polar_express.py:74-104) over a caller-provided workspace.
#include "common.h"

#include <cmath>
#include <mutex>
#include <vector>
#include <algorithm>

namespace dionw {
namespace {

constexpr int BK = 64;  // k depth of one LDS stage (4 MFMA k-steps of 16)

// kOutSame: output in the operand type. kOutBf16ViaF16: float16 operands, output
// rounded to float16 and then to bfloat16 (the Gram iteration's last product,
// _gram.py:89). kOutRoundAcc: output in the operand type, the product rounded to
// it before alpha and beta D are applied.
enum OutMode : int { kOutSame = 0, kOutBf16ViaF16 = 1, kOutRoundAcc = 2 };

struct GemmArgs {
  const void* a;
  const void* b;
  const void* d;
  void* c;
  void* ct;
  void* c_diag;
  int64_t lda, ldb, ldd, ldc, ldct;
  int64_t sa, sb, sd, sc, sct;
  int m, n, k;          // compute extents
  int m_lim, n_lim;     // store extents (<= m, n)
  float alpha, beta, diag_shift;
  int sym;
  int ct_vec;           // transposed store may use 8-byte vectors
  int tiles_m, tiles_n;
  int b_kn;             // B given as [k, n] (row-major along n) instead of [n, k]
  int xcd_group;        // 0: each XCD takes one contiguous range of tiles; G > 0:
                        // XCD x takes every 8th run of G consecutive tiles
};

struct Problem {
  int elem;  // kF16 / kBF16
  int out_mode;
  int64_t batch;
  GemmArgs g;
  int with_next;  // independent of the program's next product: they may share a launch
};

template <typename T>
struct Mfma;
template <>
struct Mfma<_Float16> {
  typedef f16x8 vec;
  __device__ static f32x16 run(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<__bf16> {
  typedef bf16x8 vec;
  __device__ static f32x16 run(vec a, vec b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// LDS layout of a [rows][64] k tile: 16-byte chunk q of row r sits at chunk
// q ^ ((r >> 1) & 7), so the 16 lanes of a read phase (rows r..r+15, same
// chunk) land on 16 distinct 16-byte bank groups.
__device__ __forceinline__ int lds_off(int row, int chunk) {
  return row * BK + ((chunk ^ ((row >> 1) & 7)) << 3);
}

// The float32 result is rounded once more to the 16-bit output. The empty asm
// keeps that float32 value: without it the compiler may fold the conversion
// into the preceding multiply-add (v_fma_mixlo_f16, a single rounding) in some
// epilogues and not in others, so that the same product could round apart.
template <typename OUT_T, int MODE>
__device__ __forceinline__ OUT_T round_out(float v) {
  asm volatile("" : "+v"(v));
  if (MODE == kOutBf16ViaF16) return (OUT_T)(float)(_Float16)v;
  return (OUT_T)v;
}

// alpha * acc + beta * d with one fixed rounding sequence (beta * d rounded,
// then one fused multiply-add), so that every epilogue gives the same bits.
__device__ __forceinline__ float axpby(float alpha, float acc, float beta, float d) {
  return __builtin_fmaf(alpha, acc, beta * d);
}

// The product as the epilogue combines it: the float32 accumulator, or in mode
// kOutRoundAcc the accumulator rounded to the output type.
template <typename OUT_T, int MODE>
__device__ __forceinline__ float product_value(float acc) {
  if constexpr (MODE == kOutRoundAcc) return (float)round_out<OUT_T, kOutSame>(acc);
  return acc;
}

// Decodes the upper-triangle tile t (0 .. T(T+1)/2 - 1) into (tm, tn), tm <= tn.
__device__ __forceinline__ void tri_tile(int t, int& tm, int& tn) {
  int n = (int)((sqrtf(8.f * (float)t + 1.f) - 1.f) * 0.5f);
  while ((n + 1) * (n + 2) / 2 <= t) ++n;
  while (n * (n + 1) / 2 > t) --n;
  tn = n;
  tm = t - n * (n + 1) / 2;
}

template <typename T, typename OUT_T, int BM, int BN, int WM, int WN, int MODE>
__global__ __launch_bounds__(WM* WN * 64) void gemm_nt_kernel(GemmArgs g) {
  constexpr int NT = WM * WN * 64;
  constexpr int WTM = BM / WM, WTN = BN / WN;  // wave tile
  constexpr int FM = WTM / 32, FN = WTN / 32;  // 32x32 fragments per wave
  constexpr int A_CH = BM * BK / 8 / NT;        // 16-byte chunks per thread
  constexpr int B_CH = BN * BK / 8 / NT;
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small for the thread count");
  using V = typename Mfma<T>::vec;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T* lds = reinterpret_cast<T*>(smem);
  constexpr int STAGE = (BM + BN) * BK;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  const int64_t batch = blockIdx.y;

  int tm, tn;
  if (g.sym) {
    tri_tile(blockIdx.x, tm, tn);
  } else {
    // Groups of 8 tile rows sweep the columns together (operand reuse in L2).
    const int t = blockIdx.x;
    const int group = 8 * g.tiles_n;
    const int first = (t / group) * 8;
    const int gm = min(g.tiles_m - first, 8);
    tm = first + (t % group) % gm;
    tn = (t % group) / gm;
  }
  const int m0 = tm * BM, n0 = tn * BN;
  const T* A = reinterpret_cast<const T*>(g.a) + batch * g.sa;
  const T* B = reinterpret_cast<const T*>(g.b) + batch * g.sb;

  u32x4 ra[A_CH], rb[B_CH];
  auto load = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int c = 0; c < A_CH; ++c) {
      const int q = tid + c * NT;
      const int row = q >> 3, ch = q & 7;
      const int gr = m0 + row, gk = k0 + ch * 8;
      ra[c] = (gr < g.m && gk < g.k)
                  ? *reinterpret_cast<const u32x4*>(A + (int64_t)gr * g.lda + gk)
                  : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int c = 0; c < B_CH; ++c) {
      const int q = tid + c * NT;
      const int row = q >> 3, ch = q & 7;
      const int gr = n0 + row, gk = k0 + ch * 8;
      rb[c] = (gr < g.n && gk < g.k)
                  ? *reinterpret_cast<const u32x4*>(B + (int64_t)gr * g.ldb + gk)
                  : u32x4{0u, 0u, 0u, 0u};
    }
  };
  auto store = [&](int buf) {
    T* As = lds + buf * STAGE;
    T* Bs = As + BM * BK;
#pragma unroll
    for (int c = 0; c < A_CH; ++c) {
      const int q = tid + c * NT;
      *reinterpret_cast<u32x4*>(As + lds_off(q >> 3, q & 7)) = ra[c];
    }
#pragma unroll
    for (int c = 0; c < B_CH; ++c) {
      const int q = tid + c * NT;
      *reinterpret_cast<u32x4*>(Bs + lds_off(q >> 3, q & 7)) = rb[c];
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int kt_count = (g.k + BK - 1) / BK;
  load(0);
  store(0);
  __syncthreads();
  const int lrow = lane & 31, lk = lane >> 5;
  for (int kt = 0; kt < kt_count; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < kt_count) load(kt + 1);
    const T* As = lds + buf * STAGE;
    const T* Bs = As + BM * BK;
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      V af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const V*>(As + lds_off(wm * WTM + i * 32 + lrow, 2 * ks + lk));
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const V*>(Bs + lds_off(wn * WTN + j * 32 + lrow, 2 * ks + lk));
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = Mfma<T>::run(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < kt_count) store(buf ^ 1);
    __syncthreads();
  }

  // Epilogue. Fragment element e of lane l holds row 8(e/4) + 4(l/32) + e%4,
  // column l%32 of its 32x32 block.
  const T* D = g.d ? reinterpret_cast<const T*>(g.d) + batch * g.sd : nullptr;
  OUT_T* C = g.c ? reinterpret_cast<OUT_T*>(g.c) + batch * g.sc : nullptr;
  OUT_T* CT = g.ct ? reinterpret_cast<OUT_T*>(g.ct) + batch * g.sct : nullptr;
  OUT_T* CD = g.c_diag ? reinterpret_cast<OUT_T*>(g.c_diag) + batch * g.sc : nullptr;
  const bool diag_tile = g.sym && tm == tn;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int col = n0 + wn * WTN + j * 32 + lrow;
#pragma unroll
      for (int e4 = 0; e4 < 4; ++e4) {
        const int row0 = m0 + wm * WTM + i * 32 + 8 * e4 + 4 * lk;
        OUT_T v[4], vd[4];
        bool in[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = row0 + e;
          in[e] = row < g.m_lim && col < g.n_lim;
          const float pv = product_value<OUT_T, MODE>(acc[i][j][4 * e4 + e]);
          const float x = D && in[e] ? axpby(g.alpha, pv, g.beta,
                                             (float)D[(int64_t)row * g.ldd + col])
                                     : g.alpha * pv;
          v[e] = round_out<OUT_T, MODE>(x);
          if (CD) {
            float y = (float)v[e] + (row == col ? g.diag_shift : 0.f);
            vd[e] = (OUT_T)y;
          }
        }
        // Straight store: on the diagonal tile only the upper half (i <= j).
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int row = row0 + e;
          if (!in[e] || (diag_tile && row > col)) continue;
          if (C) C[(int64_t)row * g.ldc + col] = v[e];
          if (CD) CD[(int64_t)row * g.ldc + col] = vd[e];
        }
        // Transposed / mirrored store: 4 consecutive rows -> one 8-byte store.
        if (CT || (g.sym && CD)) {
          const bool full4 = g.ct_vec && in[0] && in[3] && !(diag_tile && row0 + 3 >= col);
          if (full4 && CT) {
            typedef OUT_T o4 __attribute__((ext_vector_type(4)));
            o4 w = {v[0], v[1], v[2], v[3]};
            *reinterpret_cast<o4*>(CT + (int64_t)col * g.ldct + row0) = w;
            if (g.sym && CD) {
              o4 wd = {vd[0], vd[1], vd[2], vd[3]};
              *reinterpret_cast<o4*>(CD + (int64_t)col * g.ldc + row0) = wd;
            }
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int row = row0 + e;
              if (!in[e] || (diag_tile && row >= col)) continue;
              if (CT) CT[(int64_t)col * g.ldct + row] = v[e];
              if (g.sym && CD) CD[(int64_t)col * g.ldc + row] = vd[e];
            }
          }
        }
      }
    }
  }
}

// ---- pipelined tile kernels ----------------------------------------------------
//
// Two tile shapes (PipeCfg): 256x256 per workgroup of 16 waves (4x4, 64x64 per
// wave: 4 accumulators of 32x32) and 128x128 per workgroup of 4 waves (2x2,
// 64x64 per wave, two workgroups per CU). k advances through an LDS ring filled
// by direct-to-LDS loads (global_load_lds_dwordx4): two 64-deep stages when k
// is a multiple of 64, four 32-deep stages when it is an odd multiple of 32; a
// stage is requested one stage (64-deep) or three stages (32-deep) before it is
// consumed. Waits are explicit: before a stage is read every wave waits for its
// own loads of it (vmcnt) and for its reads of the stage about to be refilled
// (lgkmcnt), then the workgroup meets at one barrier. Rows beyond m / n load a
// clamped valid row (only outputs that are never stored see them), so every
// wave issues the same number of loads per stage and the vmcnt arithmetic is
// exact; k must be a multiple of 32.

// Tile configuration: BM x BN output tile, WM x WN waves, STAGES-deep LDS ring of
// BK-deep stages.
template <int BM_, int BN_, int WM_, int WN_, int STAGES_, int BK_>
struct PipeCfg {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, STAGES = STAGES_, BK = BK_;
  static constexpr int threads = WM * WN * 64;
  static constexpr int stage_elems = (BM + BN) * BK;          // A then B
  static constexpr int loads_a = BM * BK / 8 / threads;       // 16-byte loads per thread
  static constexpr int loads_b = BN * BK / 8 / threads;
  static constexpr size_t lds_bytes = (size_t)STAGES * stage_elems * 2;
  static_assert(loads_a >= 1 && loads_b >= 1, "tile too small for the thread count");
  static_assert(BK == 32 || BK == 64, "stage depth 32 or 64");
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// A stage row holds BK/8 chunks of 16 bytes. Chunk q of row r sits at
// q ^ ((r >> 2) & 3) (BK 32) or q ^ ((r >> 1) & 7) (BK 64): the 16 lanes of a
// read phase (rows r..r+15, same chunk) cover all 64 banks once.
template <int BK>
__device__ __forceinline__ int swz(int row, int chunk) {
  return BK == 32 ? chunk ^ ((row >> 2) & 3) : chunk ^ ((row >> 1) & 7);
}
template <int BK>
__device__ __forceinline__ int plds_off(int row, int chunk) {
  return row * BK + (swz<BK>(row, chunk) << 3);
}

// ---- LDS-staged epilogue of the large-tile kernels ------------------------------
//
// The output tile (BM x BN, 16-bit) is assembled in LDS, so that every global
// access is a 16-byte vector per lane: the addend D is loaded row by row,
// each lane forms alpha * acc + beta * D for its fragment elements and rounds
// once, then rows are stored straight (C, and C + shift I) and columns are
// gathered for the transposed / mirrored store (CT). The tile row stride
// ELD = BN + 8 keeps rows 16-byte aligned.

template <int BN>
constexpr int epi_ld() { return BN + 8; }

template <int BM, int BN>
constexpr size_t epi_lds_bytes() { return (size_t)BM * epi_ld<BN>() * 2; }

template <typename T, typename OUT_T, int MODE, int NT, int BM, int BN, int FM, int FN>
__device__ __forceinline__ void staged_epilogue(const GemmArgs& g, f32x16 (&acc)[FM][FN],
                                                int64_t bidx, int m0, int n0, int wrow0,
                                                int wcol0, bool diag_tile, unsigned char* smem) {
  constexpr int ELD = epi_ld<BN>();
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  const int tid = threadIdx.x, lane = tid & 63, lrow = lane & 31, lk = lane >> 5;
  OUT_T* tile = reinterpret_cast<OUT_T*>(smem);
  const T* D = g.d ? reinterpret_cast<const T*>(g.d) + bidx * g.sd : nullptr;
  OUT_T* C = g.c ? reinterpret_cast<OUT_T*>(g.c) + bidx * g.sc : nullptr;
  OUT_T* CT = g.ct ? reinterpret_cast<OUT_T*>(g.ct) + bidx * g.sct : nullptr;
  OUT_T* CD = g.c_diag ? reinterpret_cast<OUT_T*>(g.c_diag) + bidx * g.sc : nullptr;
  const bool vec_rows = (g.ldd % 8 == 0) && (g.ldc % 8 == 0) && (g.sc % 8 == 0) &&
                        (g.sd % 8 == 0);
  // Interior tiles: every thread issues all its 16-byte loads of D at once (one
  // memory latency per tile instead of one per chunk), before the pipeline's
  // LDS is released.
  constexpr int DQ = BM * BN / 8 / NT;
  static_assert(DQ * NT * 8 == BM * BN, "D chunks must divide evenly over the threads");
  const bool d_whole = D && vec_rows && m0 + BM <= g.m_lim && n0 + BN <= g.n_lim;
  u4 dv[DQ];
  if (d_whole) {
#pragma unroll
    for (int i = 0; i < DQ; ++i) {
      const int q = tid + i * NT, r = q / (BN / 8), c8 = (q % (BN / 8)) * 8;
      dv[i] = *reinterpret_cast<const u4*>(D + (int64_t)(m0 + r) * g.ldd + n0 + c8);
    }
  }
  // Every wave is done with the pipeline's LDS before the tile overwrites it.
  __builtin_amdgcn_s_waitcnt(7 << 4);  // vmcnt(0) lgkmcnt(0)
  __syncthreads();
  if (d_whole) {
#pragma unroll
    for (int i = 0; i < DQ; ++i) {
      const int q = tid + i * NT, r = q / (BN / 8), c8 = (q % (BN / 8)) * 8;
      *reinterpret_cast<u4*>(reinterpret_cast<T*>(tile) + r * ELD + c8) = dv[i];
    }
    __syncthreads();
  } else if (D) {
    for (int q = tid; q < BM * BN / 8; q += NT) {
      const int r = q / (BN / 8), c8 = (q % (BN / 8)) * 8;
      const int gr = m0 + r, gc = n0 + c8;
      T* dst = reinterpret_cast<T*>(tile) + r * ELD + c8;
      if (gr < g.m_lim && gc + 8 <= g.n_lim && vec_rows) {
        *reinterpret_cast<u4*>(dst) = *reinterpret_cast<const u4*>(D + (int64_t)gr * g.ldd + gc);
      } else {
        for (int e = 0; e < 8; ++e)
          dst[e] = (gr < g.m_lim && gc + e < g.n_lim) ? D[(int64_t)gr * g.ldd + gc + e] : (T)0.f;
      }
    }
    __syncthreads();
  }
  // Each lane replaces its fragment elements of D with the result; a fragment's
  // 16 reads of D are issued before its 16 writes (one LDS wait per fragment).
  if (D) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = wcol0 + j * 32 + lrow;
        float dval[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = wrow0 + i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
          dval[e] = (float)reinterpret_cast<const T*>(tile)[row * ELD + col];
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = wrow0 + i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
          tile[row * ELD + col] = round_out<OUT_T, MODE>(
              axpby(g.alpha, product_value<OUT_T, MODE>(acc[i][j][e]), g.beta, dval[e]));
        }
      }
  } else {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int col = wcol0 + j * 32 + lrow;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int row = wrow0 + i * 32 + 8 * (e >> 2) + 4 * lk + (e & 3);
          tile[row * ELD + col] =
              round_out<OUT_T, MODE>(g.alpha * product_value<OUT_T, MODE>(acc[i][j][e]));
        }
      }
  }
  __syncthreads();
  // A diagonal tile of a symmetric product takes its lower triangle from its
  // upper one inside LDS (reads stay above the diagonal, writes below it), then
  // leaves whole through the straight stores: its mirror is itself.
  if (diag_tile) {
    // Consecutive lanes take consecutive rows r of one chunk column: the gathers
    // (column r of rows c8 .. c8 + 7) read adjacent elements and the 16-byte
    // writes fall 4 banks apart.
    for (int q = tid; q < BM * BN / 8; q += NT) {
      const int r = q % BM, c8 = (q / BM) * 8;
      if (c8 >= r) continue;  // no element of this chunk lies below the diagonal
      OUT_T v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e)
        v[e] = c8 + e < r ? tile[(c8 + e) * ELD + r] : (OUT_T)0.f;
      OUT_T* dst = tile + r * ELD + c8;
      if (c8 + 8 <= r) {
        u4 w;
        __builtin_memcpy(&w, v, 16);
        *reinterpret_cast<u4*>(dst) = w;
      } else {
        for (int e = 0; e < r - c8; ++e) dst[e] = v[e];
      }
    }
    __syncthreads();
  }
  // Straight stores: rows of the tile.
  if (C || CD) {
    for (int q = tid; q < BM * BN / 8; q += NT) {
      const int r = q / (BN / 8), c8 = (q % (BN / 8)) * 8;
      const int gr = m0 + r, gc = n0 + c8;
      if (gr >= g.m_lim || gc >= g.n_lim) continue;
      const OUT_T* src = tile + r * ELD + c8;
      const bool whole = gc + 8 <= g.n_lim && vec_rows;
      if (whole && !(CD && gr >= gc && gr < gc + 8)) {
        const u4 v = *reinterpret_cast<const u4*>(src);
        if (C) *reinterpret_cast<u4*>(C + (int64_t)gr * g.ldc + gc) = v;
        if (CD) *reinterpret_cast<u4*>(CD + (int64_t)gr * g.ldc + gc) = v;
      } else {
        for (int e = 0; e < 8; ++e) {
          const int c = gc + e;
          if (c >= g.n_lim) continue;
          if (C) C[(int64_t)gr * g.ldc + c] = src[e];
          if (CD) CD[(int64_t)gr * g.ldc + c] = (OUT_T)((float)src[e] + (gr == c ? g.diag_shift : 0.f));
        }
      }
    }
  }
  // Transposed / mirrored stores: column c of the tile becomes row n0 + c (off-diagonal
  // tiles only). Lane -> (8 columns, 8 row blocks of 8) so that 8 lanes write 128
  // contiguous bytes.
  OUT_T* TT = CT && !diag_tile ? CT : nullptr;
  if (TT) {
    const int64_t ldt = g.ct ? g.ldct : g.ldc;
    for (int q = tid; q < BM * BN / 8; q += NT) {
      const int c = (q / 64) % (BN / 8) * 8 + (q & 7);
      const int r8 = ((q & 63) >> 3) * 8 + (q / (64 * (BN / 8))) * 64;
      if (r8 >= BM) continue;
      const int gr = m0 + r8, gc = n0 + c;
      if (gc >= g.n_lim || gr >= g.m_lim) continue;
      OUT_T v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = tile[(r8 + e) * ELD + c];
      if (gr + 8 <= g.m_lim && ldt % 8 == 0 && g.sct % 8 == 0 &&
          (reinterpret_cast<uintptr_t>(TT) & 15) == 0) {
        u4 w;
        __builtin_memcpy(&w, v, 16);
        *reinterpret_cast<u4*>(TT + (int64_t)gc * ldt + gr) = w;
        if (g.sym && CD) *reinterpret_cast<u4*>(CD + (int64_t)gc * g.ldc + gr) = w;  // no shift
      } else {
        for (int e = 0; e < 8; ++e) {
          const int r = r8 + e;
          if (m0 + r >= g.m_lim) continue;
          TT[(int64_t)gc * ldt + m0 + r] = v[e];
          if (g.sym && CD) CD[(int64_t)gc * g.ldc + m0 + r] = v[e];
        }
      }
    }
  }
}

template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  // s_waitcnt vmcnt(N) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((N >> 4) << 14));
}

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16* lds_v4i16_t;

// One output tile: logical tile w of the problem (batch index w / tiles).
// BKN: B is [k, n] (row-major along n, such as the iterate X of Q X) instead
// of [n, k]. Its stages are then k-major in LDS, [k][n], with 16-byte chunk ch
// of row k at ch ^ (4 * (k % 4)), and each B fragment is two transpose reads
// (ds_read_b64_tr_b16): a lane of a 16-lane group addressing row base + i / 4,
// columns 4 (i % 4) .. + 3 hands lane i column i, rows base .. base + 3. With the
// swizzle, a half-wave's 32 reads hit 16 distinct 16-byte bank groups.
template <typename T, typename OUT_T, int MODE, typename CFG, bool BKN>
__device__ __forceinline__ void pipe_tile(const GemmArgs& g, int w) {
  constexpr int PBM = CFG::BM, PBN = CFG::BN, PWN = CFG::WN, PSTAGES = CFG::STAGES;
  constexpr int PSTAGE_ELEMS = CFG::stage_elems, LA = CFG::loads_a, LB = CFG::loads_b;
  constexpr int SBK = CFG::BK, CPR = SBK / 8;  // stage depth, 16-byte chunks per row
  constexpr int WTM = PBM / CFG::WM, WTN = PBN / PWN;  // wave tile
  constexpr int FM = WTM / 32, FN = WTN / 32;      // 32x32 fragments
  using V = typename Mfma<T>::vec;
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  T* lds = reinterpret_cast<T*>(smem);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / PWN, wn = wave % PWN;

  const int tiles = g.sym ? g.tiles_m * (g.tiles_m + 1) / 2 : g.tiles_m * g.tiles_n;
  const int64_t bidx = w / tiles;
  const int t = w - (int)bidx * tiles;
  int tm, tn;
  if (g.sym) {
    tri_tile(t, tm, tn);
  } else {
    const int group = 8 * g.tiles_n;
    const int first = (t / group) * 8;
    const int gm = min(g.tiles_m - first, 8);
    tm = first + (t % group) % gm;
    tn = (t % group) / gm;
  }
  const int m0 = tm * PBM, n0 = tn * PBN;
  const T* A = reinterpret_cast<const T*>(g.a) + bidx * g.sa;
  const T* B = reinterpret_cast<const T*>(g.b) + bidx * g.sb;

  // Per-thread load slots: slot j of wave w covers LDS chunks
  // [(w * L + j) * 64, +64) of the operand's stage area (L loads per thread).
  const T* a_src[LA];
  const T* b_src[LB];
#pragma unroll
  for (int j = 0; j < LA; ++j) {
    const int pos = (wave * LA + j) * 64 + lane;  // 16-byte chunk index
    const int row = pos / CPR, logical = swz<SBK>(row, pos % CPR);
    a_src[j] = A + (int64_t)min(m0 + row, g.m - 1) * g.lda + logical * 8;
  }
  constexpr int NCH = PBN / 8;  // 16-byte chunks per k-row of a k-major B stage
#pragma unroll
  for (int j = 0; j < LB; ++j) {
    const int pos = (wave * LB + j) * 64 + lane;
    if (BKN) {
      // Columns past n load a clamped valid chunk (n is a multiple of 8).
      const int krow = pos / NCH, ch = (pos % NCH) ^ (4 * (krow % 4));
      b_src[j] = B + (int64_t)krow * g.ldb + min(n0 + ch * 8, g.n - 8);
    } else {
      const int row = pos / CPR, logical = swz<SBK>(row, pos % CPR);
      b_src[j] = B + (int64_t)min(n0 + row, g.n - 1) * g.ldb + logical * 8;
    }
  }
  const int64_t b_step = BKN ? (int64_t)SBK * g.ldb : SBK;  // B elements per stage
  auto issue = [&](int kt) {
    T* stage = lds + (kt % PSTAGES) * PSTAGE_ELEMS;
    const int k0 = kt * SBK;
#pragma unroll
    for (int j = 0; j < LA; ++j)  // wave-uniform LDS destination: lane i lands at +16 i bytes
      __builtin_amdgcn_global_load_lds((const void*)(a_src[j] + k0),
                                       (lds_ptr_t)(stage + (wave * LA + j) * 512), 16, 0, 0);
#pragma unroll
    for (int j = 0; j < LB; ++j)
      __builtin_amdgcn_global_load_lds((const void*)(b_src[j] + kt * b_step),
                                       (lds_ptr_t)(stage + PBM * SBK + (wave * LB + j) * 512), 16,
                                       0, 0);
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  const int kt_count = g.k / SBK;
#pragma unroll
  for (int s = 0; s < PSTAGES - 1; ++s)
    if (s < kt_count) issue(s);
  const int lrow = lane & 31, lk = lane >> 5;
  // A wave computes nothing when no element of its block is ever stored: in a
  // diagonal tile of a symmetric product, a block wholly below the diagonal
  // (its first row past its last column; the epilogue overwrites that part with
  // the mirror of the upper one), and a block wholly past the stored rows or
  // columns (the padding of a ragged side). Under the board's power limit the
  // MFMAs saved buy clock for the rest. The wave still issues its share of the
  // stage loads and takes every barrier, in a loop of its own (a branch inside
  // the main loop costs the 4-wave 128x128 kernel registers and time).
  const bool diag_tile = g.sym && tm == tn;
  const bool idle = (diag_tile && wm * WTM >= (wn + 1) * WTN) || m0 + wm * WTM >= g.m_lim ||
                    n0 + wn * WTN >= g.n_lim;
  // Stage kt has landed for every wave; the stage PSTAGES - 1 ahead is issued.
  auto advance = [&](int kt) {
    const int ahead = min(PSTAGES - 2, kt_count - 1 - kt);  // stages issued after kt
    static_assert(PSTAGES >= 2 && PSTAGES <= 4, "waits cover 0..2 stages ahead");
    static_assert(2 * (LA + LB) <= 63, "vmcnt counts to 63");
    if (ahead >= 2) wait_vm_lgkm0<2 * (LA + LB)>();
    else if (ahead == 1) wait_vm_lgkm0<LA + LB>();
    else wait_vm_lgkm0<0>();
    __builtin_amdgcn_s_barrier();
    if (kt + PSTAGES - 1 < kt_count) issue(kt + PSTAGES - 1);
  };
  if (idle) {
    for (int kt = 0; kt < kt_count; ++kt) advance(kt);
  } else for (int kt = 0; kt < kt_count; ++kt) {
    advance(kt);
    const T* As = lds + (kt % PSTAGES) * PSTAGE_ELEMS;
    const T* Bs = As + PBM * SBK;
    // Fragments of k-step ks + 1 are read while the MFMAs of k-step ks run.
    V af[2][FM], bfr[2][FN];
    auto frag = [&](int ks, int set) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[set][i] = *reinterpret_cast<const V*>(As + plds_off<SBK>(wm * WTM + i * 32 + lrow, 2 * ks + lk));
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        if (BKN) {
          const int G = lane >> 4, i16 = lane & 15;
          const int col = wn * WTN + j * 32 + 16 * (G & 1) + 4 * (i16 & 3);
          v4i16 half[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int krow = ks * 16 + 8 * (G >> 1) + 4 * h + (i16 >> 2);
            const int ch = (col >> 3) ^ (4 * (krow & 3));
            half[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_v4i16_t)(Bs + krow * PBN + ch * 8 + (col & 7)));
          }
          bfr[set][j] = __builtin_bit_cast(
              V, __builtin_shufflevector(half[0], half[1], 0, 1, 2, 3, 4, 5, 6, 7));
        } else {
          bfr[set][j] = *reinterpret_cast<const V*>(Bs + plds_off<SBK>(wn * WTN + j * 32 + lrow, 2 * ks + lk));
        }
      }
    };
    frag(0, 0);
#pragma unroll
    for (int ks = 0; ks < SBK / 16; ++ks) {
      if (ks + 1 < SBK / 16) frag(ks + 1, (ks + 1) & 1);
      // Without this fence the scheduler sinks the reads below the MFMAs and the
      // two fragment sets share registers again.
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
          acc[i][j] = Mfma<T>::run(af[ks & 1][i], bfr[ks & 1][j], acc[i][j]);
    }
  }

  staged_epilogue<T, OUT_T, MODE, CFG::threads, PBM, PBN, FM, FN>(
      g, acc, bidx, m0, n0, wm * WTM, wn * WTN, diag_tile, smem);
}

// XCD-aware order: the hardware deals workgroup b to XCD b % 8, and an XCD's
// workgroups start in the order of b. With group G == 0 each XCD gets one
// contiguous range of the problem's logical tiles, so that its L2 sees reuse
// from one round of tiles to the next. With G > 0 (G = the tiles an XCD runs
// at once) XCD x takes runs x, x + 8, ... of G consecutive tiles: each round of
// the 8 XCDs covers 8 G consecutive tiles, so the blocks in flight (and the
// operand bytes the Infinity Cache must hold) are a few instead of eight; the
// tiles past the last full 8 G are dealt contiguously. Returns -1 for the b
// that only pad the grid to a multiple of 8.
__device__ __forceinline__ int xcd_tile(int b, int total, int group) {
  const int x = b % 8, i = b / 8;
  int full = 0;
  if (group > 0) {
    full = total / (8 * group) * (8 * group);
    if (i < full / 8) return ((i / group) * 8 + x) * group + i % group;
  }
  const int rest = total - full, i2 = i - full / 8;
  const int per = rest / 8, extra = rest % 8;
  if (i2 >= per + (x < extra ? 1 : 0)) return -1;
  return full + x * per + min(x, extra) + i2;
}

__device__ __forceinline__ int tile_count(const GemmArgs& g) {
  return g.sym ? g.tiles_m * (g.tiles_m + 1) / 2 : g.tiles_m * g.tiles_n;
}

template <typename T, typename OUT_T, int MODE, typename CFG, bool BKN>
__global__ __launch_bounds__(CFG::threads, 1) void gemm_nt_pipe_kernel(GemmArgs g, int batch) {
  pipe_tile<T, OUT_T, MODE, CFG, BKN>(g, xcd_tile((int)blockIdx.x, tile_count(g) * batch,
                                                  g.xcd_group));
}

// Several independent products in one launch (the same product of several
// Newton-Schulz runs): problem q owns workgroups [start[q], start[q + 1]), each
// range a multiple of 8 long so that every problem keeps its XCD-aware order.
constexpr int kMaxGroup = 8;

struct GemmGroup {
  GemmArgs g[kMaxGroup];
  int batch[kMaxGroup];
  int start[kMaxGroup];
  int count;
};

template <typename T, typename OUT_T, int MODE, typename CFG, bool BKN>
__global__ __launch_bounds__(CFG::threads, 1) void gemm_nt_pipe_group_kernel(GemmGroup grp) {
  int q = 0;
  for (int j = 1; j < grp.count; ++j)
    if ((int)blockIdx.x >= grp.start[j]) q = j;
  const GemmArgs& g = grp.g[q];
  const int w = xcd_tile((int)blockIdx.x - grp.start[q], tile_count(g) * grp.batch[q],
                        g.xcd_group);
  if (w < 0) return;  // the whole workgroup: w depends on blockIdx only
  pipe_tile<T, OUT_T, MODE, CFG, BKN>(g, w);
}

// ---- float32 products -----------------------------------------------------------
//
// alpha A B^T + beta D with float32 operands and output on v_mfma_f32_32x32x2_f32:
// products and sums in float32, as the reference's symmetric kernels compute
// float32 inputs (tl.dot with "ieee" precision, _symmetric_kernels.py:275, 311).
// 64x64 output tile per workgroup of 4 waves (one 32x32 fragment each); k moves
// through 32-deep LDS stages, the next stage held in registers while the current
// one is multiplied. Any sizes and strides: rows and k past the edge load zeros.
// Symmetric mode computes the tiles on and above the diagonal and stores each
// also mirrored (the diagonal tiles' lower halves from their upper ones).
constexpr int kF32Tile = 64, kF32Depth = 32, kF32Ld = kF32Depth + 1;

__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs g, int64_t tiles, int vec) {
  __shared__ float as[2][kF32Tile * kF32Ld];
  __shared__ float bs[2][kF32Tile * kF32Ld];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t bidx = (int64_t)blockIdx.x / tiles;
  const int t = (int)((int64_t)blockIdx.x - bidx * tiles);
  int tm, tn;
  if (g.sym) {
    tri_tile(t, tm, tn);
  } else {
    tm = t / g.tiles_n;
    tn = t - tm * g.tiles_n;
  }
  const int m0 = tm * kF32Tile, n0 = tn * kF32Tile;
  const float* A = reinterpret_cast<const float*>(g.a) + bidx * g.sa;
  const float* B = reinterpret_cast<const float*>(g.b) + bidx * g.sb;
  // Thread tid stages k columns 4 (tid % 8) .. + 3 of tile rows tid / 8 and
  // tid / 8 + 32 of each operand.
  const int lrow = tid >> 3, lk = 4 * (tid & 7);
  float ra[2][4], rb[2][4];
  auto fetch = [&](const float* M, int64_t ld, int r0, int lim, int k0, float (&r)[2][4]) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = r0 + lrow + 32 * h, kk = k0 + lk;
      const float* src = M + (int64_t)row * ld + kk;
      if (row < lim && vec && kk + 3 < g.k) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(src);
        r[h][0] = v.x; r[h][1] = v.y; r[h][2] = v.z; r[h][3] = v.w;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) r[h][e] = (row < lim && kk + e < g.k) ? src[e] : 0.f;
      }
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        as[buf][(lrow + 32 * h) * kF32Ld + lk + e] = ra[h][e];
        bs[buf][(lrow + 32 * h) * kF32Ld + lk + e] = rb[h][e];
      }
  };
  f32x16 acc;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc[e] = 0.f;
  const int stages = (g.k + kF32Depth - 1) / kF32Depth;
  fetch(A, g.lda, m0, g.m, 0, ra);
  fetch(B, g.ldb, n0, g.n, 0, rb);
  stash(0);
  __syncthreads();
  const int frow = lane & 31, fk = lane >> 5;
  for (int st = 0; st < stages; ++st) {
    const int buf = st & 1;
    if (st + 1 < stages) {
      fetch(A, g.lda, m0, g.m, (st + 1) * kF32Depth, ra);
      fetch(B, g.ldb, n0, g.n, (st + 1) * kF32Depth, rb);
    }
    const float* a_t = as[buf] + (wm * 32 + frow) * kF32Ld + fk;
    const float* b_t = bs[buf] + (wn * 32 + frow) * kF32Ld + fk;
#pragma unroll
    for (int ks = 0; ks < kF32Depth / 2; ++ks)
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a_t[2 * ks], b_t[2 * ks], acc, 0, 0, 0);
    if (st + 1 < stages) stash(buf ^ 1);
    __syncthreads();
  }
  // Element e of lane l: row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32.
  const float* D = g.d ? reinterpret_cast<const float*>(g.d) + bidx * g.sd : nullptr;
  float* C = g.c ? reinterpret_cast<float*>(g.c) + bidx * g.sc : nullptr;
  float* CT = g.ct ? reinterpret_cast<float*>(g.ct) + bidx * g.sct : nullptr;
  const bool diag_tile = g.sym && tm == tn;
  const int col = n0 + wn * 32 + frow;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const int row = m0 + wm * 32 + 8 * (e >> 2) + 4 * fk + (e & 3);
    if (row >= g.m_lim || col >= g.n_lim) continue;
    const float v = D ? axpby(g.alpha, acc[e], g.beta, D[(int64_t)row * g.ldd + col])
                      : g.alpha * acc[e];
    if (C && !(diag_tile && row > col)) C[(int64_t)row * g.ldc + col] = v;
    if (CT && !(g.sym && row >= col)) CT[(int64_t)col * g.ldct + row] = v;
  }
}

int launch_f32(const Problem& p, hipStream_t stream) {
  GemmArgs g = p.g;
  g.tiles_m = (g.m + kF32Tile - 1) / kF32Tile;
  g.tiles_n = (g.n + kF32Tile - 1) / kF32Tile;
  const int64_t tiles = g.sym ? (int64_t)g.tiles_m * (g.tiles_m + 1) / 2
                              : (int64_t)g.tiles_m * g.tiles_n;
  if (tiles * p.batch > INT32_MAX) {
    set_error("gemm: grid too large");
    return kInvalid;
  }
  const bool vec = g.lda % 4 == 0 && g.ldb % 4 == 0 && g.sa % 4 == 0 && g.sb % 4 == 0 &&
                   aligned16(g.a) && aligned16(g.b);
  hipLaunchKernelGGL(gemm_f32_kernel, dim3((unsigned)(tiles * p.batch)), dim3(256), 0, stream, g,
                     tiles, (int)vec);
  return check_launch("gemm_f32");
}

// ---- launch configuration ----------------------------------------------------


template <typename T, typename OUT_T, int BM, int BN, int WM, int WN, int MODE>
int launch_cfg(const Problem& p, hipStream_t stream) {
  GemmArgs g = p.g;
  g.ct_vec = !g.ct || (g.ldct % 4 == 0 && g.sct % 4 == 0 &&
                       (reinterpret_cast<uintptr_t>(g.ct) & 7) == 0);
  if (g.c_diag && g.sym) g.ct_vec = g.ct_vec && g.ldc % 4 == 0 && g.sc % 4 == 0;
  constexpr size_t lds_bytes = 2 * (size_t)(BM + BN) * BK * sizeof(T);
  auto kern = gemm_nt_kernel<T, OUT_T, BM, BN, WM, WN, MODE>;
  static std::once_flag once;
  static hipError_t attr_rc = hipSuccess;
  std::call_once(once, [&] {
    attr_rc = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
  });
  if (attr_rc != hipSuccess) {
    set_error("gemm: hipFuncSetAttribute failed: %s", hipGetErrorString(attr_rc));
    return kHipError;
  }
  g.tiles_m = (g.m + BM - 1) / BM;
  g.tiles_n = (g.n + BN - 1) / BN;
  int64_t tiles;
  if (g.sym) {
    if (BM != BN || g.m != g.n) {
      set_error("gemm: symmetric mode needs a square output and square tiles");
      return kInvalid;
    }
    tiles = (int64_t)g.tiles_m * (g.tiles_m + 1) / 2;
  } else {
    tiles = (int64_t)g.tiles_m * g.tiles_n;
  }
  if (tiles > INT32_MAX || p.batch > 65535) {
    set_error("gemm: grid too large");
    return kInvalid;
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)tiles, (unsigned)p.batch), dim3(WM * WN * 64),
                     lds_bytes, stream, g);
  return check_launch("gemm_nt");
}

template <typename CFG>
constexpr size_t pipe_lds_bytes() {
  return CFG::lds_bytes > epi_lds_bytes<CFG::BM, CFG::BN>() ? CFG::lds_bytes
                                                            : epi_lds_bytes<CFG::BM, CFG::BN>();
}

// The kernel-side fields of a pipelined product; returns its workgroup count
// (tiles x batch) or -1 with the error set.
template <typename CFG>
int64_t pipe_args(const Problem& p, GemmArgs& g) {
  g = p.g;
  g.ct_vec = !g.ct || (g.ldct % 4 == 0 && g.sct % 4 == 0 &&
                       (reinterpret_cast<uintptr_t>(g.ct) & 7) == 0);
  if (g.c_diag && g.sym) g.ct_vec = g.ct_vec && g.ldc % 4 == 0 && g.sc % 4 == 0;
  g.tiles_m = (g.m + CFG::BM - 1) / CFG::BM;
  g.tiles_n = (g.n + CFG::BN - 1) / CFG::BN;
  if (g.sym && (g.m != g.n || CFG::BM != CFG::BN)) {
    set_error("gemm: symmetric mode needs a square output and square tiles");
    return -1;
  }
  const int64_t tiles = g.sym ? (int64_t)g.tiles_m * (g.tiles_m + 1) / 2
                              : (int64_t)g.tiles_m * g.tiles_n;
  if (tiles * p.batch > INT32_MAX) {
    set_error("gemm: grid too large");
    return -1;
  }
  // Blocks of many 256x256 tiles are dealt in runs of 32 (one tile per CU of
  // an XCD): measured on Llama-3-8B, -2.6% of product time against contiguous
  // ranges; blocks of fewer tiles (whose operands stay in cache across an
  // XCD's rounds) and the 128x128 kernel keep contiguous ranges, where the
  // runs of 32 or 64 measured 1-1.5% slower (MoE runs).
  g.xcd_group = CFG::BM == 256 && tiles >= 64 ? 32 : 0;
  return tiles * p.batch;
}

// Raises a kernel's dynamic LDS limit once per process (one flag per kernel).
template <auto kern>
int allow_lds(size_t lds_bytes) {
  static std::once_flag once;
  static hipError_t rc = hipSuccess;
  std::call_once(once, [&] {
    rc = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes);
  });
  if (rc != hipSuccess) {
    set_error("gemm: hipFuncSetAttribute failed: %s", hipGetErrorString(rc));
    return kHipError;
  }
  return kOk;
}

template <typename T, typename OUT_T, int MODE, typename CFG, bool BKN>
int launch_pipe_kn(const Problem& p, hipStream_t stream) {
  constexpr size_t lds_bytes = pipe_lds_bytes<CFG>();
  constexpr auto kern = gemm_nt_pipe_kernel<T, OUT_T, MODE, CFG, BKN>;
  DIONW_TRY(allow_lds<kern>(lds_bytes));
  GemmArgs g;
  const int64_t wgs = pipe_args<CFG>(p, g);
  if (wgs < 0) return kInvalid;
  hipLaunchKernelGGL(kern, dim3((unsigned)wgs), dim3(CFG::threads), lds_bytes, stream, g,
                     (int)p.batch);
  return check_launch("gemm_nt_pipe");
}

template <typename T, typename OUT_T, int MODE, typename CFG>
int launch_pipe(const Problem& p, hipStream_t stream) {
  if (p.g.b_kn) return launch_pipe_kn<T, OUT_T, MODE, CFG, true>(p, stream);
  return launch_pipe_kn<T, OUT_T, MODE, CFG, false>(p, stream);
}

// One launch of up to kMaxGroup products on one tile configuration with
// 64-deep stages, longest k first (its tiles take longest, so they start first).
template <typename T, typename OUT_T, int MODE, typename CFG, bool BKN>
int launch_pipe_group_kn(const std::vector<const Problem*>& ps, hipStream_t stream) {
  constexpr size_t lds_bytes = pipe_lds_bytes<CFG>();
  constexpr auto kern = gemm_nt_pipe_group_kernel<T, OUT_T, MODE, CFG, BKN>;
  DIONW_TRY(allow_lds<kern>(lds_bytes));
  std::vector<const Problem*> order(ps);
  std::stable_sort(order.begin(), order.end(),
                   [](const Problem* a, const Problem* b) { return a->g.k > b->g.k; });
  GemmGroup grp{};
  grp.count = (int)order.size();
  int64_t start = 0;
  for (int q = 0; q < grp.count; ++q) {
    const int64_t wgs = pipe_args<CFG>(*order[q], grp.g[q]);
    if (wgs < 0) return kInvalid;
    grp.batch[q] = (int)order[q]->batch;
    grp.start[q] = (int)start;
    start += (wgs + 7) / 8 * 8;
    if (start > INT32_MAX) {
      set_error("gemm: grid too large");
      return kInvalid;
    }
  }
  hipLaunchKernelGGL(kern, dim3((unsigned)start), dim3(CFG::threads), lds_bytes, stream, grp);
  return check_launch("gemm_nt_pipe_group");
}

// Tile of a grouped launch: 256x256 (16 waves, one workgroup per CU) or
// 128x128 (4 waves, two per CU).
enum GroupTile : int { kNoGroup = 0, kGroupBig = 1, kGroupMid = 2 };

template <typename T, typename OUT_T, int MODE>
int launch_pipe_group(const std::vector<const Problem*>& ps, GroupTile tile, hipStream_t stream) {
  using Big64 = PipeCfg<256, 256, 4, 4, 2, 64>;
  using Mid64 = PipeCfg<128, 128, 2, 2, 2, 64>;
  const bool kn = ps[0]->g.b_kn;
  if (tile == kGroupMid)
    return kn ? launch_pipe_group_kn<T, OUT_T, MODE, Mid64, true>(ps, stream)
              : launch_pipe_group_kn<T, OUT_T, MODE, Mid64, false>(ps, stream);
  return kn ? launch_pipe_group_kn<T, OUT_T, MODE, Big64, true>(ps, stream)
            : launch_pipe_group_kn<T, OUT_T, MODE, Big64, false>(ps, stream);
}

// Workgroups a tile size yields (symmetric products: upper-triangle tiles).
int64_t wgs_of(const Problem& p, int tile) {
  const int64_t tm = (p.g.m + tile - 1) / tile, tn = (p.g.n + tile - 1) / tile;
  return p.batch * (p.g.sym ? tm * (tm + 1) / 2 : tm * tn);
}

// Rounds of workgroups over the 256 CUs (one 256x256 or two 128x128 per CU),
// in units of one 256x256 round: a 128x128 round counts 2 * 128^2 / 256^2 *
// 1.3 (the smaller tile's rate is about 1/1.3 of the 256x256 tile's: with 1.2,
// MoE-Muon's 1408-row symmetric products took the smaller tile and ran 2.4%
// slower than on 256x256 tiles, while the MoE products that keep it are faster
// there).
// Both in twentieths of a 256x256 round (a 128x128 round is 0.65).
constexpr int kBigRound = 20, kMidRound = 13;
int64_t big_cost(const Problem& p) { return kBigRound * ((wgs_of(p, 256) + 255) / 256); }
int64_t mid_cost(const Problem& p) { return kMidRound * ((wgs_of(p, 128) + 511) / 512); }

template <typename T, typename OUT_T, int MODE>
int launch_typed(const Problem& p, hipStream_t stream) {
  auto wgs = [&](int tile) { return wgs_of(p, tile); };
  // 256x256 tiles run 16 waves of 64x64, 128x128 tiles 4 waves of 64x64. A k
  // depth that is a multiple of 64 takes 64-deep stages in a two-stage ring (half
  // the barriers per MFMA of 32-deep stages); other multiples of 32, four
  // 32-deep stages.
  using Big64 = PipeCfg<256, 256, 4, 4, 2, 64>;
  using Mid64 = PipeCfg<128, 128, 2, 2, 2, 64>;
  using Big32 = PipeCfg<256, 256, 4, 4, 4, 32>;
  using Mid32 = PipeCfg<128, 128, 2, 2, 4, 32>;
  const bool k64 = p.g.k % 64 == 0, k32 = p.g.k % 32 == 0;
  if (p.g.b_kn && !k32) {
    set_error("gemm: a [k, n] B operand needs k to be a multiple of 32");
    return kInvalid;
  }
#ifdef DIONW_FORCE_KERNEL
  // Tuning builds only: one tile shape for every product it can run.
  if (DIONW_FORCE_KERNEL == 1 && k32) {
    if (k64) return launch_pipe<T, OUT_T, MODE, Big64>(p, stream);
    return launch_pipe<T, OUT_T, MODE, Big32>(p, stream);
  }
  if (DIONW_FORCE_KERNEL == 2 && k32) {
    if (k64) return launch_pipe<T, OUT_T, MODE, Mid64>(p, stream);
    return launch_pipe<T, OUT_T, MODE, Mid32>(p, stream);
  }
  if (DIONW_FORCE_KERNEL == 3 && !p.g.b_kn) return launch_cfg<T, OUT_T, 128, 128, 2, 2, MODE>(p, stream);
  if (DIONW_FORCE_KERNEL == 4 && !p.g.b_kn) return launch_cfg<T, OUT_T, 64, 64, 2, 2, MODE>(p, stream);
#endif
  if (k32) {
    // The smaller tile wins when the big one leaves CUs idle or pads a ragged side.
    if (big_cost(p) <= mid_cost(p)) {
      if (k64) return launch_pipe<T, OUT_T, MODE, Big64>(p, stream);
      return launch_pipe<T, OUT_T, MODE, Big32>(p, stream);
    }
    if (k64) return launch_pipe<T, OUT_T, MODE, Mid64>(p, stream);
    return launch_pipe<T, OUT_T, MODE, Mid32>(p, stream);
  }
  if (wgs(128) >= 512) return launch_cfg<T, OUT_T, 128, 128, 2, 2, MODE>(p, stream);
  return launch_cfg<T, OUT_T, 64, 64, 2, 2, MODE>(p, stream);
}

bool operands_ok(const GemmArgs& g) {
  return !(g.k % 8 || g.lda % 8 || g.ldb % 8 || g.sa % 8 || g.sb % 8 || !aligned16(g.a) ||
           !aligned16(g.b));
}

int launch(const Problem& p, hipStream_t stream) {
  const GemmArgs& g = p.g;
  if (g.m <= 0 || g.n <= 0 || g.k <= 0 || p.batch <= 0) return kOk;
  if (p.elem == kF32) {
    if (g.b_kn) {
      set_error("gemm: float32 products take B as [n, k]");
      return kInvalid;
    }
    return launch_f32(p, stream);
  }
  if (!operands_ok(g)) {
    set_error("gemm: k, operand row strides and batch strides must be multiples of 8 "
              "elements and operands 16-byte aligned");
    return kInvalid;
  }
  if (g.b_kn && (g.n % 8 || g.sym)) {
    set_error("gemm: a [k, n] B operand needs n to be a multiple of 8 (and no symmetric mode)");
    return kInvalid;
  }
  if (p.elem == kF16) {
    if (p.out_mode == kOutBf16ViaF16) return launch_typed<_Float16, __bf16, kOutBf16ViaF16>(p, stream);
    return launch_typed<_Float16, _Float16, kOutSame>(p, stream);
  }
  if (p.elem == kBF16) {
    if (p.out_mode == kOutRoundAcc) return launch_typed<__bf16, __bf16, kOutRoundAcc>(p, stream);
    return launch_typed<__bf16, __bf16, kOutSame>(p, stream);
  }
  set_error("gemm: unsupported element type %d", p.elem);
  return kInvalid;
}

// Whether one grouped launch beats one launch per product, and on which tile.
// Time in 256x256 rounds times k (a round of 256x256 tiles over depth k costs
// k, a round of two 128x128 tiles per CU kGroupMidRate k: the rate the grouping
// choices were measured with, e.g. gram-ns's lone-run pair on 128x128 tiles,
// 1.35 -> 1.32 ms; the launcher's own tile rule counts kMidRound / kBigRound).
// Alone, each product takes its better tile (the launcher's rule); grouped, the
// tiles of all of them fill the
// CUs longest first, which costs their total work over the CUs plus about half
// a round of the shortest tiles, and no less than the longest tile.
//
// The same product of several runs (walk_groups' positions) groups on 256x256
// tiles on that estimate alone. Two independent products of one run, each one
// round of workgroups or less, also count the ramp and drain of a launch
// (kRamp, about 11 us: a third of a 256x256 round at k = 1024) and may group on
// either tile: two launches of one round each cost two ramps; one launch of
// both, one ramp and the rounds their tiles fill together. (Counting the ramp
// for the runs' positions too measured slower on GPT-2-small's runs, whose
// products then group on 128x128 tiles.)
constexpr double kRamp = 340.0;
constexpr double kGroupMidRate = 0.6;

GroupTile group_plan(const std::vector<const Problem*>& ps, bool pair) {
  const double ramp = pair ? kRamp : 0.0;
  double separate = 0.0, big = 0.0, mid = 0.0, kmax = 0.0, kmin = 1e300;
  for (const Problem* p : ps) {
    const double k = (double)p->g.k;
    separate += ramp + k * (double)std::min(big_cost(*p), mid_cost(*p)) / kBigRound;
    big += k * (double)wgs_of(*p, 256) / 256.0;
    mid += kGroupMidRate * k * (double)wgs_of(*p, 128) / 512.0;
    kmax = std::max(kmax, k);
    kmin = std::min(kmin, k);
  }
  const double big_total = ramp + std::max(big + 0.5 * kmin, kmax);
  const double mid_total =
      pair ? ramp + std::max(mid + 0.5 * kGroupMidRate * kmin, kGroupMidRate * kmax) : 1e300;
  if (std::min(big_total, mid_total) >= separate) return kNoGroup;
  return mid_total < big_total ? kGroupMid : kGroupBig;
}

// Independent products in as few launches as possible: one grouped launch when
// every product has the same types and a k depth that is a multiple of 64 (the
// tiles with 64-deep stages serve them all) and grouping pays, else one launch
// each.
std::vector<const Problem*> live_products(const std::vector<const Problem*>& ps) {
  std::vector<const Problem*> live;
  for (const Problem* p : ps)
    if (p->g.m > 0 && p->g.n > 0 && p->g.k > 0 && p->batch > 0) live.push_back(p);
  return live;
}

GroupTile groups(const std::vector<const Problem*>& live, bool pair = false) {
  bool together = live.size() >= 2 && live.size() <= (size_t)kMaxGroup;
  for (const Problem* p : live)
    together = together && p->elem == live[0]->elem && p->out_mode == live[0]->out_mode &&
               p->g.b_kn == live[0]->g.b_kn && p->g.k % 64 == 0 && p->batch <= INT32_MAX &&
               operands_ok(p->g) && !(p->g.b_kn && (p->g.n % 8 || p->g.sym));
  return together ? group_plan(live, pair) : kNoGroup;
}

int launch_group(const std::vector<const Problem*>& ps, hipStream_t stream, bool pair = false) {
  const std::vector<const Problem*> live = live_products(ps);
  const GroupTile tile = groups(live, pair);
  if (tile == kNoGroup) {
    for (const Problem* p : live) DIONW_TRY(launch(*p, stream));
    return kOk;
  }
  if (live[0]->elem == kF16) {
    if (live[0]->out_mode == kOutBf16ViaF16)
      return launch_pipe_group<_Float16, __bf16, kOutBf16ViaF16>(live, tile, stream);
    return launch_pipe_group<_Float16, _Float16, kOutSame>(live, tile, stream);
  }
  if (live[0]->out_mode == kOutRoundAcc)
    return launch_pipe_group<__bf16, __bf16, kOutRoundAcc>(live, tile, stream);
  return launch_pipe_group<__bf16, __bf16, kOutSame>(live, tile, stream);
}

// ---- Newton-Schulz drivers ---------------------------------------------------

struct Mat {  // a batch of row-major matrices
  void* p;
  int64_t ld, stride;
};

Problem product(int elem, int64_t batch, int m, int n, int k, Mat a, Mat b) {
  Problem p{};
  p.elem = elem;
  p.out_mode = kOutSame;
  p.batch = batch;
  p.g.a = a.p;
  p.g.lda = a.ld;
  p.g.sa = a.stride;
  p.g.b = b.p;
  p.g.ldb = b.ld;
  p.g.sb = b.stride;
  p.g.m = p.g.m_lim = m;
  p.g.n = p.g.n_lim = n;
  p.g.k = k;
  p.g.alpha = 1.f;
  p.g.beta = 0.f;
  return p;
}

void set_out(Problem& p, Mat c) {
  p.g.c = c.p;
  p.g.ldc = c.ld;
  p.g.sc = c.stride;
}
void set_out_t(Problem& p, Mat ct) {
  p.g.ct = ct.p;
  p.g.ldct = ct.ld;
  p.g.sct = ct.stride;
}
void set_addend(Problem& p, Mat d, float alpha, float beta) {
  p.g.d = d.p;
  p.g.ldd = d.ld;
  p.g.sd = d.stride;
  p.g.alpha = alpha;
  p.g.beta = beta;
}
void make_symmetric(Problem& p) {
  p.g.sym = 1;
  p.g.ct = p.g.c;
  p.g.ldct = p.g.ldc;
  p.g.sct = p.g.sc;
}

// Polar Express coefficients of the Gram iteration: the 5 published rows with
// the 1.05 safety factor folded in as (a / s, b / s^3, c / s^5).
void gram_coefficients(double out[5][3]) {
  static const double raw[5][3] = {
      {8.28721201814563, -23.595886519098837, 17.300387312530933},
      {4.107059111542203, -2.9478499167379106, 0.5448431082926601},
      {3.9486908534822946, -2.908902115962949, 0.5518191394370137},
      {3.3184196573706015, -2.488488024314874, 0.51004894012372},
      {2.300652019954817, -1.6689039845747493, 0.4188073119525673},
  };
  const double s = 1.05;
  for (int i = 0; i < 5; ++i) {
    out[i][0] = raw[i][0] / s;
    out[i][1] = raw[i][1] / (s * s * s);
    out[i][2] = raw[i][2] / (s * s * s * s * s);
  }
}

void polar_express_coefficients(double out[5][3]) {
  static const double pe[5][3] = {
      {8.156554524902461, -22.48329292557795, 15.878769915207462},
      {4.042929935166739, -2.808917465908714, 0.5000178451051316},
      {3.8916678022926607, -2.772484153217685, 0.5060648178503393},
      {3.285753657755655, -2.3681294933425376, 0.46449024233003106},
      {2.3465413258596377, -1.7097828382687081, 0.42323551169305323},
  };
  for (int i = 0; i < 5; ++i)
    for (int j = 0; j < 3; ++j) out[i][j] = pe[i][j];
}

void keller_coefficients(double out[5][3]) {
  for (int i = 0; i < 5; ++i) {
    out[i][0] = 3.4445;
    out[i][1] = -4.7750;
    out[i][2] = 2.0315;
  }
}

// Library kinds: the Gram iteration, the two bf16 quintics with each line's
// product and elementwise terms rounded once (the symmetric-kernel variants,
// _polar_express.py:74-104), and the same quintics with the products rounded
// to bf16 before the elementwise terms (the cuBLAS variants, :43-71).
enum Kind : int {
  kGram = 0,
  kPolarExpress = 1,
  kKeller = 2,
  kPolarExpressCublas = 3,
  kKellerCublas = 4,
};

size_t elems_needed(int kind, int64_t batch, int64_t r, int64_t c) {
  const bool gram = kind == kGram;  // the Gram iteration needs the most
  const int64_t sq = r * r, rc = r * c;
  return (size_t)batch * (gram ? (6 * sq + rc) : (2 * sq + rc));
}

// Final store of the real region into the bf16 output (W orientation).
void set_final_out(Problem& p, void* out, int transposed, int64_t out_ld, int64_t out_stride,
                   int64_t m_real, int64_t n_real) {
  p.g.m_lim = (int)m_real;
  p.g.n_lim = (int)n_real;
  if (transposed)
    set_out_t(p, Mat{out, out_ld, out_stride});
  else
    set_out(p, Mat{out, out_ld, out_stride});
}

}  // namespace
}  // namespace dionw

using namespace dionw;

extern "C" {

int dionw_gemm_nt(int32_t elem, int64_t batch, int64_t m, int64_t n, int64_t k, const void* a,
                  int64_t lda, int64_t stride_a, const void* b, int64_t ldb, int64_t stride_b,
                  const void* d, int64_t ldd, int64_t stride_d, float alpha, float beta, void* c,
                  int64_t ldc, int64_t stride_c, void* ct, int64_t ldct, int64_t stride_ct,
                  int32_t symmetric, hipStream_t stream) {
  DIONW_REQUIRE(a && b && (c || ct), "gemm_nt: null operand");
  DIONW_REQUIRE(m > 0 && n > 0 && k > 0 && m < INT32_MAX && n < INT32_MAX && k < INT32_MAX,
                "gemm_nt: bad sizes");
  DIONW_REQUIRE(!symmetric || (m == n && c && !ct), "gemm_nt: symmetric output needs m == n "
                "and a single output");
  Problem p = product(elem, batch, (int)m, (int)n, (int)k, Mat{(void*)a, lda, stride_a},
                      Mat{(void*)b, ldb, stride_b});
  if (d) set_addend(p, Mat{(void*)d, ldd, stride_d}, alpha, beta);
  else p.g.alpha = alpha;
  if (c) set_out(p, Mat{c, ldc, stride_c});
  if (ct) set_out_t(p, Mat{ct, ldct, stride_ct});
  if (symmetric) make_symmetric(p);
  return launch(p, stream);
}

size_t dionw_newton_schulz_workspace(int32_t kind, int64_t batch, int64_t r, int64_t c) {
  return elems_needed(kind, batch, r, c) * 2;
}

int dionw_ns_coefficients(int32_t kind, double* out) {
  DIONW_REQUIRE(out, "ns_coefficients: null output");
  DIONW_REQUIRE(kind >= kGram && kind <= kKellerCublas, "ns_coefficients: unknown kind %d", kind);
  double coef[5][3];
  if (kind == kGram) gram_coefficients(coef);
  else if (kind == kPolarExpress || kind == kPolarExpressCublas) polar_express_coefficients(coef);
  else keller_coefficients(coef);
  for (int i = 0; i < 5; ++i)
    for (int j = 0; j < 3; ++j) out[3 * i + j] = coef[i][j];
  return kOk;
}

}  // extern "C"

namespace dionw {
namespace {

// The products of one Newton-Schulz call, in order (validated; nothing launched).
int ns_program(int32_t kind, int64_t batch, int64_t r, int64_t c, void* x, void* xt,
               int64_t r_real, int64_t c_real, void* out, int32_t out_transposed, int64_t out_ld,
               int64_t out_stride, void* workspace, size_t workspace_bytes,
               std::vector<Problem>& prog) {
  DIONW_REQUIRE(kind >= kGram && kind <= kKellerCublas, "newton_schulz: unknown kind %d", kind);
  // With r a multiple of 32 the products that multiply X from the left read
  // it directly as a [k, n] operand, so xt is neither read nor written.
  const bool direct = r % 32 == 0;
  DIONW_REQUIRE(x && (xt || direct) && out && workspace, "newton_schulz: null pointer");
  DIONW_REQUIRE(r > 0 && c >= r && r % 8 == 0 && c % 8 == 0 && r < 65536 && c < INT32_MAX,
                "newton_schulz: need 0 < r <= c, both multiples of 8 (r=%lld c=%lld)",
                (long long)r, (long long)c);
  DIONW_REQUIRE(r_real <= r && c_real <= c && r_real > 0 && c_real > 0,
                "newton_schulz: real extents exceed the padded ones");
  DIONW_REQUIRE(workspace_bytes >= dionw_newton_schulz_workspace(kind, batch, r, c),
                "newton_schulz: workspace too small");
  if (batch == 0) return kOk;
  const int R = (int)r, C = (int)c;
  const int64_t sq = r * r, rc = r * c;
  const int elem = kind == kGram ? kF16 : kBF16;
  auto* ws = reinterpret_cast<uint16_t*>(workspace);
  auto mat_sq = [&](int slot) { return Mat{ws + (size_t)slot * batch * sq, r, sq}; };
  Mat X{x, c, rc}, XT{xt, r, rc};
  double coef[5][3];
  // Left multiplication by an r x r matrix L of the current iterate: reads X
  // itself ([k, n] operand) or its transpose.
  auto left_times = [&](Mat L, Mat x_cur, Mat xt_cur) {
    Problem p = product(elem, batch, R, C, R, L, direct ? x_cur : xt_cur);
    p.g.b_kn = direct;
    return p;
  };

  if (kind == kGram && c_real > r_real) {
    gram_coefficients(coef);
    Mat G = mat_sq(0), G2 = mat_sq(1), Z = mat_sq(2), Q = mat_sq(3), Q2 = mat_sq(4),
        RZ = mat_sq(5);
    // The last workspace slot holds the restarted iterate's transpose, or the
    // restarted iterate itself when the products read X directly.
    Mat XT2{ws + (size_t)6 * batch * sq, r, rc}, X2{ws + (size_t)6 * batch * sq, c, rc};
    // G = X X^T
    Problem p = product(elem, batch, R, R, C, X, X);
    set_out(p, G);
    make_symmetric(p);
    prog.push_back(p);
    Mat x_cur = X, xt_cur = XT;
    for (int i = 0; i < 5; ++i) {
      const float a = (float)coef[i][0], bb = (float)coef[i][1], cc = (float)coef[i][2];
      if (i == 2) {
        // Restart: X = Q X, G = X X^T. Read directly, X may not be overwritten
        // while other tiles still read it: the result goes to X2. Otherwise it
        // goes in place to X (the product reads X^T) and its transpose to XT2.
        p = left_times(Q, x_cur, xt_cur);
        if (direct) {
          set_out(p, X2);
          x_cur = X2;
        } else {
          set_out(p, X);
          set_out_t(p, XT2);
          xt_cur = XT2;
        }
        prog.push_back(p);
        p = product(elem, batch, R, R, C, x_cur, x_cur);
        set_out(p, G);
        make_symmetric(p);
        prog.push_back(p);
      }
      // Z = c G G + b G; at iterations 0 and 2 also Q = Z + a I.
      p = product(elem, batch, R, R, R, G, G);
      set_addend(p, G, cc, bb);
      set_out(p, Z);
      make_symmetric(p);
      if (i == 0 || i == 2) {
        p.g.c_diag = Q.p;
        p.g.diag_shift = a;
      }
      prog.push_back(p);
      if (i != 0 && i != 2) {
        // Q = a Q + Q Z (independent of the RZ product that follows it at
        // iteration 3: both read Z, neither writes what the other reads).
        p = product(elem, batch, R, R, R, Q, Z);
        set_addend(p, Q, 1.f, a);
        set_out(p, Q2);
        make_symmetric(p);
        p.with_next = i < 4 && i + 1 != 2;
        prog.push_back(p);
        std::swap(Q, Q2);
      }
      if (i < 4 && i + 1 != 2) {
        // RZ = a G + G Z; G = a RZ + Z RZ
        p = product(elem, batch, R, R, R, G, Z);
        set_addend(p, G, 1.f, a);
        set_out(p, RZ);
        make_symmetric(p);
        prog.push_back(p);
        p = product(elem, batch, R, R, R, Z, RZ);
        set_addend(p, RZ, 1.f, a);
        set_out(p, G2);
        make_symmetric(p);
        prog.push_back(p);
        std::swap(G, G2);
      }
    }
    // out = Q X, rounded to fp16 then bf16.
    p = left_times(Q, x_cur, xt_cur);
    p.out_mode = kOutBf16ViaF16;
    set_final_out(p, out, out_transposed, out_ld, out_stride, r_real, c_real);
    prog.push_back(p);
    return kOk;
  }

  // Standard iteration (square Gram blocks, fp16) or the bf16 quintic:
  // X = a X + (c A A + b A) X with A = X X^T, five times. The cuBLAS variants
  // round A A and P X to bf16 before the elementwise terms: P = b A + c bf16(A A),
  // X = a X + bf16(P X). A tall block is iterated in its wide orientation: the
  // reference's right products x^T x and x P of the tall x are the transposes of
  // X X^T and P X, with the same roundings.
  const bool cublas = kind == kPolarExpressCublas || kind == kKellerCublas;
  if (kind == kGram) gram_coefficients(coef);
  else if (kind == kPolarExpress || kind == kPolarExpressCublas) polar_express_coefficients(coef);
  else keller_coefficients(coef);
  Mat G = mat_sq(0), P = mat_sq(1);
  // The last workspace slot: the iterate's other transpose buffer, or its
  // other buffer when the products read X directly (X and X2 alternate).
  Mat XT2{ws + (size_t)2 * batch * sq, r, rc}, X2{ws + (size_t)2 * batch * sq, c, rc};
  Mat x_cur = X, x_next = X2, xt_cur = XT, xt_next = XT2;
  for (int i = 0; i < 5; ++i) {
    const float a = (float)coef[i][0], bb = (float)coef[i][1], cc = (float)coef[i][2];
    Problem p = product(elem, batch, R, R, C, x_cur, x_cur);
    set_out(p, G);
    make_symmetric(p);
    prog.push_back(p);
    p = product(elem, batch, R, R, R, G, G);
    set_addend(p, G, cc, bb);
    if (cublas) p.out_mode = kOutRoundAcc;
    set_out(p, P);
    make_symmetric(p);
    prog.push_back(p);
    p = left_times(P, x_cur, xt_cur);
    set_addend(p, x_cur, 1.f, a);
    if (cublas) p.out_mode = kOutRoundAcc;
    if (i < 4) {
      if (direct) {
        set_out(p, x_next);
        prog.push_back(p);
        std::swap(x_cur, x_next);
      } else {
        set_out(p, X);  // X is only read as the addend, element by element
        set_out_t(p, xt_next);
        prog.push_back(p);
        std::swap(xt_cur, xt_next);
      }
    } else {
      if (kind == kGram) p.out_mode = kOutBf16ViaF16;
      set_final_out(p, out, out_transposed, out_ld, out_stride, r_real, c_real);
      prog.push_back(p);
    }
  }
  return kOk;
}

bool same_structure(const std::vector<Problem>& a, const std::vector<Problem>& b) {
  if (a.size() != b.size()) return false;
  for (size_t i = 0; i < a.size(); ++i)
    if (a[i].elem != b[i].elem || a[i].out_mode != b[i].out_mode ||
        a[i].g.b_kn != b[i].g.b_kn || a[i].with_next != b[i].with_next)
      return false;
  return true;
}

// Runs whose sequences match product by product (length, types and
// independence) go together, kMaxGroup at a time: one launch per position of
// the sequence when grouping pays; a run on its own also shares one launch
// between two independent products when that pays. Counts the launches in *launches and, if issue,
// launches them.
int walk_groups(const std::vector<std::vector<Problem>>& progs, bool issue, hipStream_t stream,
                int64_t* launches) {
  const int count = (int)progs.size();
  std::vector<char> done(count, 0);
  for (int i = 0; i < count; ++i) {
    if (done[i]) continue;
    std::vector<int> runs{i};
    done[i] = 1;
    for (int j = i + 1; j < count && runs.size() < (size_t)kMaxGroup; ++j)
      if (!done[j] && same_structure(progs[i], progs[j])) {
        runs.push_back(j);
        done[j] = 1;
      }
    const std::vector<Problem>& prog = progs[i];
    for (size_t pos = 0; pos < prog.size(); ++pos) {
      if (prog[pos].with_next && pos + 1 < prog.size() && runs.size() == 1) {
        const std::vector<const Problem*> pair{&prog[pos], &prog[pos + 1]};
        if (groups(live_products(pair), true) != kNoGroup) {
          *launches += 1;
          if (issue) DIONW_TRY(launch_group(pair, stream, true));
          ++pos;
          continue;
        }
      }
      std::vector<const Problem*> ps;
      for (int j : runs) ps.push_back(&progs[j][pos]);
      const std::vector<const Problem*> live = live_products(ps);
      *launches += groups(live) != kNoGroup ? 1 : (int64_t)live.size();
      if (issue) DIONW_TRY(launch_group(ps, stream));
    }
  }
  return kOk;
}

}  // namespace
}  // namespace dionw

extern "C" {

int dionw_newton_schulz(int32_t kind, int64_t batch, int64_t r, int64_t c, void* x, void* xt,
                        int64_t r_real, int64_t c_real, void* out, int32_t out_transposed,
                        int64_t out_ld, int64_t out_stride, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  std::vector<std::vector<Problem>> progs(1);
  DIONW_TRY(ns_program(kind, batch, r, c, x, xt, r_real, c_real, out, out_transposed, out_ld,
                       out_stride, workspace, workspace_bytes, progs[0]));
  int64_t launches = 0;
  return walk_groups(progs, true, stream, &launches);
}

int dionw_newton_schulz_group(int32_t count, const int32_t* kind, const int64_t* batch,
                              const int64_t* r, const int64_t* c, void* const* x,
                              void* const* xt, const int64_t* r_real, const int64_t* c_real,
                              void* const* out, const int32_t* out_transposed,
                              const int64_t* out_ld, const int64_t* out_stride,
                              void* const* workspace, const size_t* workspace_bytes,
                              hipStream_t stream) {
  DIONW_REQUIRE(count >= 0 && count <= 4096, "newton_schulz_group: bad count %d", count);
  if (count == 0) return kOk;
  DIONW_REQUIRE(kind && batch && r && c && x && xt && r_real && c_real && out &&
                    out_transposed && out_ld && out_stride && workspace && workspace_bytes,
                "newton_schulz_group: null argument array");
  // Products of different runs execute together: their workspaces must not overlap.
  for (int i = 0; i < count; ++i)
    for (int j = i + 1; j < count; ++j) {
      const auto* a = static_cast<const char*>(workspace[i]);
      const auto* b = static_cast<const char*>(workspace[j]);
      DIONW_REQUIRE(a + workspace_bytes[i] <= b || b + workspace_bytes[j] <= a,
                    "newton_schulz_group: workspaces of runs %d and %d overlap", i, j);
    }
  std::vector<std::vector<Problem>> progs(count);
  for (int i = 0; i < count; ++i)
    DIONW_TRY(ns_program(kind[i], batch[i], r[i], c[i], x[i], xt[i], r_real[i], c_real[i],
                         out[i], out_transposed[i], out_ld[i], out_stride[i], workspace[i],
                         workspace_bytes[i], progs[i]));
  int64_t launches = 0;
  return walk_groups(progs, true, stream, &launches);
}

int64_t dionw_newton_schulz_group_launches(int32_t count, const int32_t* kind,
                                           const int64_t* batch, const int64_t* r,
                                           const int64_t* c, const int64_t* r_real,
                                           const int64_t* c_real) {
  if (count < 0 || count > 4096 || (count > 0 && !(kind && batch && r && c && r_real && c_real)))
    return -1;
  // The programs from shapes alone: placeholder addresses, never dereferenced.
  void* const fake = reinterpret_cast<void*>(uintptr_t{1} << 40);
  std::vector<std::vector<Problem>> progs(count);
  for (int i = 0; i < count; ++i) {
    const size_t need = dionw_newton_schulz_workspace(kind[i], batch[i], r[i], c[i]);
    if (ns_program(kind[i], batch[i], r[i], c[i], fake, fake, r_real[i], c_real[i], fake, 0,
                   c[i], r[i] * c[i], fake, need, progs[i]) != kOk)
      return -1;
  }
  int64_t launches = 0;
  if (walk_groups(progs, false, nullptr, &launches) != kOk) return -1;
  return launches;
}

}  // extern "C"
