/*
 * dionw_hip.h — C ABI of libdionw_hip.so, the MI355X (gfx950) kernels of the
 * Dion optimizer step.
 *
 * Conventions
 *  - Every function returns 0 on success, 1 for a rejected argument and 2 for
 *    a failed launch; dionw_last_error() holds the message (per thread).
 *  - Pointers are device pointers unless named otherwise; pointer *arrays*
 *    (grads, params, ...) are host arrays of device pointers, copied into the
 *    kernel arguments (no device table, no host synchronization).
 *  - Every launch is asynchronous on `stream`. The library never allocates,
 *    frees or synchronizes: buffers and workspaces come from the caller.
 *  - Matrices are row-major. A bucket run's momentum is [blocks, rows, cols]
 *    float32 and contiguous; every tensor of a run holds blocks_per_tensor
 *    blocks (rows_per_tensor = blocks_per_tensor * rows rows).
 *  - Element codes: 0 = float16, 1 = bfloat16, 2 = float32.
 *
 * Citations are to the reference implementation (JTriggerFish/dionw, src/dionw).
 */
#ifndef DIONW_HIP_H
#define DIONW_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* dionw_stream_t; /* hipStream_t */

/* Last error message of the calling thread ("" when none). */
const char* dionw_last_error(void);

/* ABI revision of this header (2). */
int dionw_abi_version(void);

/*
 * Norm element type (the `elem` argument of the functions that form the
 * Newton-Schulz normalization): the element code of the iteration the sums
 * normalize. 0 (float16 Gram) and 2: sums of squares of the float32 values and
 * den = sqrt(sum) * safety + eps (the norm of x.float(), _gram.py:85-86).
 * 1 (bfloat16 quintics): sums of squares of the values rounded to bfloat16 and
 * den = float(bf16(sqrt(sum))) * safety + eps, the norm of the bf16 input taken
 * as a bf16 tensor (_polar_express.py:57-58, 89-92).
 */

/*
 * M += G for every row of a run, with each row's l1 norm (the top-k score) and
 * sum of squares. Replaces accumulate_row_l1 (_momentum_kernels.py:89-103)
 * and the per-parameter loop of _accumulate_with_scores (_matrix_step.py:188-199).
 * The score is an fp32 sum in a fixed order (per-lane float4 partials in
 * column order, then an xor butterfly over the 64 lanes).
 *   grads[count]: float32 gradients, rows_per_tensor x cols each, contiguous.
 *   momentum: [count * rows_per_tensor, cols]; scores, row_sumsq: one per row.
 *   elem: the norm element type (row_sumsq of the bf16-rounded sums when 1).
 */
int dionw_accumulate_scores(const float* const* grads, int32_t count, int64_t rows_per_tensor,
                            int64_t cols, float* momentum, float* scores, float* row_sumsq,
                            int32_t elem, dionw_stream_t stream);

/*
 * Per-row sum of squares of the every-row Newton-Schulz input U = M + G
 * (heavy ball) or G + mu (M + G) (Nesterov), without writing anything: the
 * first of the two passes that replace accumulate_copy_decay
 * (_momentum_kernels.py:106-133; _matrix_step.py:217-237). momentum may be
 * NULL (U = G: the standalone orthogonalization of a given matrix).
 */
int dionw_full_sumsq(const float* const* grads, int32_t count, int64_t rows_per_tensor,
                     int64_t cols, const float* momentum, float mu, int32_t nesterov,
                     float* row_sumsq, int32_t elem, dionw_stream_t stream);

/* den[b] = sqrt(sum of row_sumsq over block b's rows) * safety + eps (the
 * square root rounded to bf16 first for elem 1): the Frobenius normalization
 * of _gram.py:86 (safety 1) and _polar_express.py:92 (safety 1.02 for Polar
 * Express, 1 for Keller). */
int dionw_block_denom(const float* row_sumsq, int64_t blocks, int64_t rows, float safety,
                      float eps, float* den, int32_t elem, dionw_stream_t stream);

/*
 * The normalization prologue of the Orthogonalize plugin on a contiguous
 * [blocks, rows, cols] input x of elem x_elem (0 fp16, 1 bf16, 2 fp32), read
 * as it is: row sums of squares as dionw_full_sumsq forms them (into
 * row_sumsq, blocks * rows floats), den as dionw_block_denom (both with the
 * norm element type elem), then
 * X = 16-bit(x / den) of type elem (0 or 1) written as dionw_prepare_ns_input
 * writes it in every-row mode without momentum (out_rowmajor and/or
 * out_transposed, padded to p_pad x j_pad). Bit-identical to those three calls
 * on a float32 copy of x, without the copy. Replaces x.float() and the
 * division by the norm of _gram.py:85-86 and _polar_express.py:89-92.
 */
int dionw_normalize_input(const void* x, int32_t x_elem, int64_t blocks, int64_t rows,
                          int64_t cols, float safety, float eps, float* row_sumsq, float* den,
                          int64_t p_pad, int64_t j_pad, int32_t elem, void* out_rowmajor,
                          void* out_transposed, dionw_stream_t stream);

/*
 * Top-k rows of each block by score: replaces torch.topk(sorted=False) and the
 * index bookkeeping of _selected_update (_matrix_step.py:172-180).
 * Exact: ties at the k-th score take the lowest row indices.
 *   idx [blocks, k]: selected rows, ascending; slot [blocks, rows]: position
 *   of each row in idx or -1; den [blocks]: sqrt(sum of the selected rows'
 *   row_sumsq) * safety + eps, as dionw_block_denom forms it for elem.
 */
int dionw_select_rows(const float* scores, const float* row_sumsq, int64_t blocks, int64_t rows,
                      int64_t k, float safety, float eps, int32_t* idx, int32_t* slot,
                      float* den, int32_t elem, dionw_stream_t stream);

/*
 * One pass writing the decayed momentum and the Newton-Schulz input.
 * Selected mode (idx != NULL): U = M[idx] (pre-decay) and M[idx] *= mu
 * (_matrix_step.py:176-179). Every-row mode (idx == NULL, grads given):
 * M = mu (M + G), U = M + G or, with nesterov, G + mu (M + G).
 * Then X = U / den[b] rounded to float16 (elem 0), or bf16(bf16(U) / den)
 * (elem 1, the Keller / Polar Express input), written, if out_rowmajor !=
 * NULL, as [blocks, p_pad, j_pad] (row p = selected row p) and, if
 * out_transposed != NULL, as its transpose [blocks, j_pad, p_pad], zeros in
 * the padding; at least one must be given. In every-row mode momentum may be
 * NULL with write_m == 0 (U = G). elem 2 writes the raw float32 U as
 * [blocks, k, cols] (out_rowmajor required) for a user-supplied
 * orthogonalization.
 * Replaces the prologue of gram_polar_express (_gram.py:83-87) and the
 * normalization of quintic_triton (_polar_express.py:89-92).
 */
int dionw_prepare_ns_input(const float* const* grads, int32_t count, float* momentum,
                           const int32_t* idx, const float* den, int64_t blocks, int64_t rows,
                           int64_t cols, int64_t k, int64_t p_pad, int64_t j_pad, float mu,
                           int32_t nesterov, int32_t write_m, int32_t elem, void* out_rowmajor,
                           void* out_transposed, dionw_stream_t stream);

/*
 * Batched C = alpha * A B^T + beta * D on MFMA (fp32 accumulation, one
 * rounding). A [m, k], B [n, k], D and C [m, n], all row-major with the given
 * leading dimensions and batch strides (elements); ct (optional) receives C^T
 * [n, m]. symmetric: only the tiles on and above the diagonal are computed and
 * mirrored (m == n, output c only). elem 0 or 1: k, lda, ldb and the operand
 * batch strides must be multiples of 8 and the operands 16-byte aligned.
 * elem 2: float32 operands and output, products and sums in float32 on the
 * fp32 MFMA (the reference's "ieee" dot for float32 inputs), any sizes and
 * strides.
 * Replaces ns_line_1 (alpha A A^T, _symmetric_kernels.py:252-277), ns_line_2
 * (c A A^T + b A, :280-312) and the baddbmm/bmm products of _gram.py:46-69
 * and _polar_express.py:98-103.
 */
int dionw_gemm_nt(int32_t elem, int64_t batch, int64_t m, int64_t n, int64_t k, const void* a,
                  int64_t lda, int64_t stride_a, const void* b, int64_t ldb, int64_t stride_b,
                  const void* d, int64_t ldd, int64_t stride_d, float alpha, float beta, void* c,
                  int64_t ldc, int64_t stride_c, void* ct, int64_t ldct, int64_t stride_ct,
                  int32_t symmetric, dionw_stream_t stream);

/*
 * The five (a, b, c) rows dionw_newton_schulz uses for kind (out: 15 doubles,
 * row-major; the kernels take them rounded to float): the Gram table of
 * _gram.py:24-35 with the 1.05 safety folded in as (a/s, b/s^3, c/s^5), the
 * Polar Express table of _polar_express.py:28-34, Keller's row of
 * _keller.py:20. Host only: no device work.
 */
int dionw_ns_coefficients(int32_t kind, double* out);

/* Workspace bytes dionw_newton_schulz needs. */
size_t dionw_newton_schulz_workspace(int32_t kind, int64_t batch, int64_t r, int64_t c);

/*
 * Newton-Schulz orthogonalization of a batch of wide, normalized matrices:
 * the Orthogonalize plugin (newton_schulz.py:30, 43-68) after its prologue.
 *   kind 0 (GRAM): fp16 Gram Newton-Schulz with restart at iteration 2 when
 *     c > r (_gram.py:50-69), the standard Polar Express iteration when
 *     c == r (_gram.py:41-47); output bf16(fp16(.)).
 *   kind 1 (POLAR_EXPRESS_TRITON) / 2 (KELLER_TRITON): the bf16 quintic with
 *     each line rounded once (_polar_express.py:74-104; _keller.py:20-34).
 *   kind 3 (POLAR_EXPRESS) / 4 (KELLER): the bf16 quintic with the products
 *     A A and P X rounded to bf16 before the elementwise terms, as the
 *     reference's cuBLAS variant computes it (_polar_express.py:43-71).
 *   x [batch, r, c] and xt [batch, c, r] (the input and its transpose, both
 *   overwritten), r <= c multiples of 8. With r a multiple of 32 the products
 *   read x itself where they multiply it from the left: xt is then neither
 *   read nor written and may be NULL. The real r_real x c_real region of
 *   the result goes to out (bf16) with leading dimension out_ld and batch
 *   stride out_stride, transposed when out_transposed (tall blocks).
 */
int dionw_newton_schulz(int32_t kind, int64_t batch, int64_t r, int64_t c, void* x, void* xt,
                        int64_t r_real, int64_t c_real, void* out, int32_t out_transposed,
                        int64_t out_ld, int64_t out_stride, void* workspace,
                        size_t workspace_bytes, dionw_stream_t stream);

/*
 * dionw_newton_schulz for count independent bucket runs at once: element i of
 * every array is run i's argument. Runs whose product sequences match (same
 * kind and shape class) execute together, up to 8 at a time, one launch per
 * product of the sequence, so that small runs fill the CUs a large run's
 * launches leave idle. Results are bit-identical to count separate calls.
 * The runs' workspaces must not overlap (checked); all arguments are checked
 * before anything is launched. Replaces the per-run orthogonalize calls of a
 * step (_matrix_step.py:254-265, one per run of optimizer.py:351-369).
 */
int dionw_newton_schulz_group(int32_t count, const int32_t* kind, const int64_t* batch,
                              const int64_t* r, const int64_t* c, void* const* x,
                              void* const* xt, const int64_t* r_real, const int64_t* c_real,
                              void* const* out, const int32_t* out_transposed,
                              const int64_t* out_ld, const int64_t* out_stride,
                              void* const* workspace, const size_t* workspace_bytes,
                              dionw_stream_t stream);

/*
 * Product launches dionw_newton_schulz_group would issue for runs of these
 * shapes (which of their products it groups), or -1 for invalid arguments;
 * nothing is launched and no memory is touched. For one run it is the length
 * of that run's product sequence. Callers use it to keep runs apart when
 * grouping would save nothing (each run's passes then follow its own
 * iteration while its output is still in cache).
 */
int64_t dionw_newton_schulz_group_launches(int32_t count, const int32_t* kind,
                                           const int64_t* batch, const int64_t* r,
                                           const int64_t* c, const int64_t* r_real,
                                           const int64_t* c_real);

/*
 * NorMuon statistics of the orthogonalized rows O (bf16 [blocks, k, cols]):
 * v = lerp(v, mean(O^2), 1 - beta2) written back into variance [blocks, rows]
 * at the selected rows (idx [blocks, k], or every row when idx == NULL),
 * rowd [blocks, k] = sqrt(v) + 1e-8, and scale [blocks] =
 * ||O||_F / max(||O / rowd||_F, 1e-8) * step. scratch: 2 * blocks * k floats.
 * Replaces normalize_rows (_row_normalization.py:41-60).
 */
int dionw_normuon_stats(const void* orthogonal, int64_t blocks, int64_t k, int64_t rows,
                        int64_t cols, const int32_t* idx, float* variance, float beta2,
                        float step, float* rowd, float* scratch, float* scale,
                        dionw_stream_t stream);

/*
 * dionw_normuon_stats without the scratch argument: the per-row partial sums
 * go to a device array inside the library (4 MiB per GPU, held until the
 * process ends), so the call allocates nothing. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Limit: blocks * k <= 524288 selected rows; larger calls are rejected.
 * The stream must belong to the current device. Calls that overlap on one GPU
 * (two streams, two threads) race on the shared array.
 */
int dionw_normuon_stats_noalloc(const void* orthogonal, int64_t blocks, int64_t k, int64_t rows,
                                int64_t cols, const int32_t* idx, float* variance, float beta2,
                                float step, float* rowd, float* scale, dionw_stream_t stream);

/*
 * The weight update of a run: W *= decay on every row when apply_decay, then
 * W[row] += O[slot] / rowd[slot] * scale[b] on the selected rows (rowd == NULL:
 * W[row] += O[slot] * (scale ? scale[b] : step)). Replaces _apply and
 * _add_blocks_ (_matrix_step.py:274-311) and finish()'s product with the step
 * (_row_normalization.py:18-38).
 */
int dionw_apply_update(float* const* params, int32_t count, int64_t blocks_per_tensor,
                       int64_t rows, int64_t cols, int64_t k, const void* orthogonal,
                       const int32_t* idx, const int32_t* slot, const float* rowd,
                       const float* scale, float step, float decay, int32_t apply_decay,
                       dionw_stream_t stream);

/*
 * dionw_apply_update with the GPU EMA fused in: after a row's new weights are
 * formed, its float32 shadow (same layout as the parameter, shadows[i] for
 * params[i]) becomes lerp(shadow, W_new, ema_weight), on every row (also those
 * only decayed or unchanged). Replaces the apply pass followed by
 * foreach_ema_update_ over the same parameters (_matrix_step.py:274-311, then
 * ema/_update.py:32-70 from ema/tracker.py:217-227) with one pass: 4 bytes per
 * element less than the two.
 */
int dionw_apply_update_ema(float* const* params, float* const* shadows, int32_t count,
                           int64_t blocks_per_tensor, int64_t rows, int64_t cols, int64_t k,
                           const void* orthogonal, const int32_t* idx, const int32_t* slot,
                           const float* rowd, const float* scale, float step, float decay,
                           int32_t apply_decay, float ema_weight, dionw_stream_t stream);

/*
 * dionw_apply_update that also writes every row's new weights (also the rows
 * only decayed or unchanged) into staged[i], a pinned host buffer laid out like
 * params[i] (hipHostMalloc or torch pin_memory=True; other memory is rejected
 * before any launch): the CPU EMA's snapshot of the parameters taken by the pass
 * that forms them. Replaces the apply pass followed by the side-stream
 * tmp_cpu.copy_(param, non_blocking=True) of every parameter
 * (_matrix_step.py:274-311, then ema/tracker.py:229-248). The snapshot is
 * complete once the work enqueued on `stream` up to this call has finished.
 */
int dionw_apply_update_stage(float* const* params, float* const* staged, int32_t count,
                             int64_t blocks_per_tensor, int64_t rows, int64_t cols, int64_t k,
                             const void* orthogonal, const int32_t* idx, const int32_t* slot,
                             const float* rowd, const float* scale, float step, float decay,
                             int32_t apply_decay, dionw_stream_t stream);

/* steps[i] += 1 (float32 device scalars): the _foreach_add_ of _adamw.py:47. */
int dionw_increment_steps(float* const* steps, int32_t count, dionw_stream_t stream);

/*
 * Multi-tensor AdamW with decoupled weight decay, bit-compatible with
 * torch._fused_adamw_ (called by adamw_step, _adamw.py:25-61): reads each
 * tensor's (already incremented) float32 step.
 */
int dionw_adamw(float* const* params, const float* const* grads, float* const* exp_avgs,
                float* const* exp_avg_sqs, const float* const* steps, const int64_t* numels,
                int32_t count, double lr, double beta1, double beta2, double weight_decay,
                double eps, dionw_stream_t stream);

/*
 * dionw_adamw with the GPU EMA fused in: shadows[i] = lerp(shadows[i], new
 * params[i], ema_weight). Replaces _fused_adamw_ followed by
 * foreach_ema_update_ over the same tensors (_adamw.py:45-61, then
 * ema/_update.py:32-70 from ema/tracker.py:217-227) with one pass.
 */
int dionw_adamw_ema(float* const* params, const float* const* grads, float* const* exp_avgs,
                    float* const* exp_avg_sqs, const float* const* steps, float* const* shadows,
                    const int64_t* numels, int32_t count, double lr, double beta1, double beta2,
                    double weight_decay, double eps, float ema_weight, dionw_stream_t stream);

/*
 * GPU EMA of float32 sources: shadow = lerp(shadow, source, weight), or a
 * copy when copy != 0. Replaces foreach_ema_update_ (ema/_update.py:32-70)
 * and the first-update _foreach_copy_ (ema/tracker.py:142-145).
 */
int dionw_ema_update(float* const* shadows, const float* const* sources, const int64_t* numels,
                     int32_t count, float weight, int32_t copy, dionw_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* DIONW_HIP_H */
