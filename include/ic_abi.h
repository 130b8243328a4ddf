/*
 * ic_abi.h - C ABI of the MI355X (gfx950) per-layer quantization library
 * (libicq.so).
 *
 * Conventions
 *  - All pointers are DEVICE pointers owned by the caller; matrices are
 *    row-major with an explicit leading dimension in elements.
 *  - Every call is asynchronous on `stream` (a hipStream_t passed as void*,
 *    NULL = default stream) and returns IC_OK (0) or a negative IC_ERR_*;
 *    ic_last_error() returns the message of the last failure in this thread.
 *  - Scratch memory is passed in by the caller; its size comes from the
 *    matching *_workspace_bytes() query.  No entry point allocates device
 *    memory unless its comment says so.
 *  - fp16 values travel as uint16_t bit patterns.
 *
 * Each entry point names the reference function whose arithmetic it
 * replaces (paths relative to the reference repository root).
 */
#ifndef IC_ABI_H
#define IC_ABI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IC_OK 0
#define IC_ERR_ARG (-1)
#define IC_ERR_HIP (-2)
#define IC_ERR_RANGE (-3)
#define IC_LOWRANK_REFUSED 1   /* ic_lowrank_eigs: rank certified too high */

#define IC_DTYPE_F32 0
#define IC_DTYPE_BF16 1
#define IC_DTYPE_F16 2

#define IC_ABI_VERSION 1

int ic_abi_version(void);
const char* ic_last_error(void);

/* ---------------------------------------------------------------- rotation */

/* Group-wise Hadamard rotation of rows: dst[r, :] = pad(src[r, :]) @ Hr^T for
 * every group of `rot` columns, where Hr is the regular Hadamard (H4/2)^kron
 * for powers of 4 and the normalised Sylvester matrix for other powers of 2.
 * src is f32/bf16/f16 [rows, cols] (ld_src), dst is f32 [rows, cols_pad]
 * (ld_dst) with cols_pad = cols rounded up to a multiple of rot; the padding
 * is zero before rotation.  src may alias dst when dtype is f32 and
 * ld_src == ld_dst.  rot: power of 2 in [1, 4096] (1 = convert/pad only).
 * When zero_above > 0, inputs with |w| > zero_above are replaced by 0 before
 * rotating and their number is added to *n_zeroed (device uint64, may be
 * NULL) - the outlier sanitising of converter/pipeline.py:527-537.
 * Replaces converter/rotation.py:95-125 (rotate_weights) and :128-153
 * (rotate_activations, same operation on a [-1, in] view). */
int ic_rotate_rows(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld_src,
                   float* dst, int64_t cols_pad, int64_t ld_dst, int rot, float zero_above,
                   unsigned long long* n_zeroed, void* stream);

/* Two-sided rotation H <- R^T src R of `batch` square fp32 matrices [n, n]
 * stored back to back with leading dimension ld (n multiple of rot); src has
 * the same layout and may be H itself (in place).
 * Replaces converter/rotation.py:156-248 (rotate_hessian, after padding). */
int ic_rotate_hessian(const float* src, float* H, int64_t batch, int64_t n, int64_t ld, int rot,
                      void* stream);

/* ic_rotate_rows with the reference's own fp32 rounding: every output is one
 * fused multiply-add chain over the group's inputs in increasing order from
 * zero, which is how the reference's `x @ H.T` (converter/rotation.py:82-92,
 * a CPU sgemm with K = rot) rounds; rot 512 adds the chains of its two halves,
 * as that sgemm does.  Runs on the matrix cores (K = 1 fp32 MFMA chains).
 * Same arguments as ic_rotate_rows; rot: power of 2 in [1, 512]; in place
 * needs f32, equal ld and rot <= 256.
 * Replaces converter/rotation.py:95-125 (rotate_weights) and :128-153
 * (rotate_activations). */
int ic_rotate_rows_exact(const void* src, int src_dtype, int64_t rows, int64_t cols, int64_t ld_src,
                         float* dst, int64_t cols_pad, int64_t ld_dst, int rot, float zero_above,
                         unsigned long long* n_zeroed, void* stream);

/* ic_rotate_hessian with the reference's rounding: per rot x rot block,
 * T = R^T B (chains over the block's rows in increasing order), then T R
 * (chains over T's columns), as einsum("kp,nkl,le->npe") contracts it
 * (converter/rotation.py:237-248).  rot: 1, 4, 16, 64 or 256 (the regular
 * matrices that rotate_hessian accepts).  lower_only (batch 1 only): write
 * only the rot x rot blocks on or below the block diagonal - all that a lower
 * Cholesky factorisation and the damping read; the rest of H is unspecified
 * (in place: src's values or partial results; out of place: unwritten).
 * Replaces converter/rotation.py:156-248 (rotate_hessian, after padding). */
int ic_rotate_hessian_exact(const float* src, float* H, int64_t batch, int64_t n, int64_t ld, int rot,
                            int lower_only, void* stream);

/* Per-row min / max / max-abs of an fp32 matrix; NaN propagates like
 * torch.amin/amax.  Any output pointer may be NULL.
 * Replaces the amin/amax/abs().amax reductions of converter/scales.py:85,
 * 144, 258-259, 338-339 and converter/gptq.py:257-258, 316. */
int ic_row_stats(const float* x, int64_t rows, int64_t cols, int64_t ld,
                 float* row_min, float* row_max, float* row_absmax, void* stream);

/* ---------------------------------------------------------------- RTN */

/* Per-row (= per group, with groups laid out as rows) RTN scales and
 * zero-points, with the optional clipping-ratio MSE search.
 *   bits 4 or 8; asym 0/1; ratios: HOST array of n_ratios (<= 16) floats.
 *   out scale16[rows] fp16 bits; zp[rows] int8 (asym only, else may be NULL).
 * Replaces converter/scales.py:25-99 (calculate_scales), 126-160
 * (calculate_scales_int8), 184-229 (_fix_asymmetric_scale), 232-282
 * (calculate_scales_asymmetric), 316-361 (calculate_scales_int8_asymmetric). */
int ic_rtn_scales(const float* W, int64_t rows, int64_t cols, int64_t ld, int bits, int asym,
                  const float* ratios, int n_ratios, uint16_t* scale16, int8_t* zp, void* stream);

/* RTN codes q = clamp(rhaz(W / scale [+ zp])) per row, scale[rows] read as
 * fp16 bits (scale_kind 0) or fp32 (1), zp[rows] fp32 (integral) or NULL.
 * Writes int8 codes [rows, cols] (ld_q) when `codes` is not NULL and packed
 * INT4 bytes [rows, ceil(cols/2)] (ld_p) when `packed` is not NULL (bits 4).
 * Replaces converter/scales.py:102-123, 163-178, 285-313, 364-384
 * (quantize_weights*), fused with converter/packing.py:30-46. */
int ic_rtn_quantize(const float* W, int64_t rows, int64_t cols, int64_t ld, int bits,
                    const void* scale, int scale_kind, const float* zp,
                    int8_t* codes, int64_t ld_q, uint8_t* packed, int64_t ld_p, void* stream);

/* ---------------------------------------------------------------- packing */

/* Validate and pack INT4 values.  src: int8 (src_kind 0) or f32 (1)
 * [rows, cols] (ld_src); dst uint8 [rows, ceil(cols/2)] (ld_dst), low nibble =
 * even column, odd tail padded with 0; dst NULL validates only.  flags
 * (device int32[3]) receives {any non-finite, any value < -8, any value > 7}
 * so the caller can raise INT4PackingError exactly like
 * converter/packing.py:17-27; the bytes are only meaningful when all three
 * flags are 0.  f32 values are truncated toward zero like .to(torch.int8).
 * Replaces converter/packing.py:17-46 (validate_int4_range, pack_int4). */
int ic_pack_int4(const void* src, int src_kind, int64_t rows, int64_t cols, int64_t ld_src,
                 uint8_t* dst, int64_t ld_dst, int32_t* flags, void* stream);

/* Unpack INT4 bytes to int8 [rows, k].  Replaces converter/packing.py:49-66. */
int ic_unpack_int4(const uint8_t* src, int64_t rows, int64_t k, int64_t ld_src,
                   int8_t* dst, int64_t ld_dst, void* stream);

/* ---------------------------------------------------------------- verification */

/* Quantisation error of codes against W: dequant = (q - zp) * scale with
 * scale read as fp16 bits (scale_kind 0) or fp32 (1) and zp NULL or int8.
 * Writes the fp64 sum of squared errors and the max |error| into
 * out_sumsq[0] / out_maxabs[0] (device).  mse = sumsq / (rows*cols).  The
 * reduction order is fixed, so repeated calls give identical bits.
 * workspace: ic_quant_error_workspace_bytes() bytes of device memory.
 * Replaces converter/pipeline.py:919-937 and the metric lines of
 * converter/gptq.py:398-405, ldlq.py:262-269. */
int64_t ic_quant_error_workspace_bytes(void);
int ic_quant_error(const float* W, int64_t rows, int64_t cols, int64_t ld,
                   const int8_t* codes, int64_t ld_q, const void* scale, int scale_kind,
                   const int8_t* zp, double* out_sumsq, float* out_maxabs, void* workspace,
                   void* stream);

/* flag[0] = 1 when any of the n scales (fp16 bits for scale_kind 0, fp32 for
 * 1) is +-Inf, NaN or 0, else 0 (device).  Replaces the bad-scale test of
 * converter/pipeline.py:938-940 (scales.isinf() | isnan() | == 0). */
int ic_scale_status(const void* scale, int scale_kind, int64_t n, int32_t* flag, void* stream);

/* ---------------------------------------------------------------- fp32 GEMM */

/* C = alpha * op(A) op(B) + beta * C on the fp32 matrix cores, row-major.
 * cmask 0 full / 1 lower (i >= j) / 2 upper (i <= j) output; krange 0 full /
 * 1 k >= max(tile i0, j0) / 2 k >= tile j0 / 3 k < tile i0 + 128 /
 * 4 k >= tile i0 (skips the zero half of a triangular operand).  beta == 0 never reads C.
 * alpha = -1, beta = 1 with op(A) = A subtracts one 128-wide chunk of K at a
 * time, C <- (..((C - P_0) - P_1)..) - P_last: the roundings of consecutive
 * rank-128 updates; otherwise the chunk sums are added and alpha, beta
 * applied once.  * Replaces the torch matmuls of converter/rounding.py:103 and
 * converter/gptq_triton.py:178-180 (lazy trailing update) and the LAPACK
 * level-3 kernels behind torch.linalg.cholesky / cholesky_inverse. */
int ic_sgemm(int transA, int transB, int64_t M, int64_t N, int64_t K, float alpha,
             const float* A, int64_t lda, const float* B, int64_t ldb, float beta,
             float* C, int64_t ldc, int cmask, int krange, void* stream);

/* ---------------------------------------------------------------- Hessian inverse */

/* In place on `batch` dense fp32 matrices [n, n] (back to back):
 *   H <- H + fp32(damping) * max(mean(diag H), 1e-6) * I;  L = chol(H);
 *   method 0 ("hinv"):     H <- H^-1 = L^-T L^-1 (full symmetric);
 *   method 1 ("cholesky"): H <- chol(H^-1)^T (upper; lower part zero);
 *   method 2 ("hinv", upper triangle): as method 0 on and above the
 *            diagonal, the strictly lower part left holding finite scratch
 *            values (for callers that read only rows j, columns >= j, as
 *            the GPTQ / LDLQ sweeps and lazy updates do).
 * info: device int32[2*batch]; info[b] > 0 is the 1-based column of the
 * first non-positive pivot of chol(H_b) (then H_b is not a valid result and
 * the caller falls back like converter/rounding.py:19-34); info[batch+b]
 * likewise for chol(H_b^-1) in method 1.
 * workspace: ic_hessian_inverse_workspace_bytes(batch, n) bytes.
 * Replaces converter/gptq.py:91-121 (_prepare_hessian, _prepare_hinv),
 * converter/rounding.py:19-34 (_invert_hessian, Cholesky branch),
 * converter/ldlq.py:64-92, 169-171, 207-209. */
int64_t ic_hessian_inverse_workspace_bytes(int64_t batch, int64_t n);
int ic_hessian_inverse(float* H, int64_t batch, int64_t n, float damping, int method,
                       int* info, void* workspace, void* stream);

/* Damping alone, in place on `batch` dense fp32 matrices [n, n] (back to
 * back): H <- H + fp32(damping) * max(mean(diag H), 1e-6) * I, the mean
 * summed in torch's CPU order (its scalar reduction of the strided
 * diagonal; one-thread order from n = 32768 on) and divided by n, as the
 * reference's H.diagonal().mean() (converter/gptq.py:104, 118;
 * converter/ldlq.py:83, 169, 207-209, where the damped H also feeds the
 * greedy search).  ic_hessian_inverse applies the same damping first. */
int ic_damp_hessian(float* H, int64_t batch, int64_t n, float damping, void* stream);

/* C [N, N] = alpha * W^T W (full symmetric; W [M, N] at row pitch ldw):
 * the upper triangle on the matrix cores, with ic_sgemm's accumulation
 * order, mirrored onto the lower one (each pair of entries is the same sum
 * of the same products).  Replaces converter/ldlq.py:186 (the weight-only
 * Hessian H = W.T @ W / M). */
int ic_gram_tn(const float* W, int64_t M, int64_t N, int64_t ldw, float alpha, float* C, void* stream);

/* Lower Cholesky factor in place (upper part of the diagonal 128-blocks set
 * to 0, the rest of the upper triangle untouched); info as above; workspace
 * as for ic_hessian_inverse.  Replaces torch.linalg.cholesky. */
int ic_cholesky(float* H, int64_t batch, int64_t n, int* info, void* workspace, void* stream);

/* ---------------------------------------------------------------- GPTQ / LDLQ */

/* Per-row GPTQ parameters from row statistics (converter/gptq.py:254-317):
 * INT4, or INT8 asymmetric: s = clamp((max-min)/spread, 1e-5, 65500) with the
 * zero-point clamp fix, zp = clamp(qmin - rhaz(min/s)), zero rows zp = 0;
 * INT8 symmetric: s = clamp(absmax/127, 1e-5, 65500).  Outputs (any but s32
 * may be NULL): s32 fp32, z32 fp32, s16 fp16 bits, z8 int8. */
int ic_gptq_row_params(const float* row_min, const float* row_max, const float* row_absmax,
                       int64_t rows, int bits, int asym, float* s32, float* z32, uint16_t* s16,
                       int8_t* z8, void* stream);

/* GPTQ sweep of a whole layer: W [rows, groups*gw] fp32 working weights
 * (modified), Hinv [groups, gw, gw] (groups == 1: the full inverse; > 1: the
 * block-diagonal inverses of a 3-D Hessian, each group of gw columns
 * independent), per-row s32 / z32 (z32 NULL = symmetric), block <= 128
 * columns of eager updates; the lazy updates are fp32-MFMA GEMMs, rank-block
 * inside super-blocks of 1024 columns (groups == 1) and one update with the
 * whole super-block's errors for the columns after it.
 * Q: int8 codes [rows, groups*gw].  workspace:
 * ic_gptq_workspace_bytes(rows, groups, block).
 * Replaces converter/rounding.py:37-103 (_gptq_block), converter/gptq.py:27-88
 * and 323-393 (_gptq_block_triton and the 2-D / 3-D dispatch),
 * converter/gptq_triton.py:18-184 (gptq_loop_triton). */
int64_t ic_gptq_workspace_bytes(int64_t rows, int64_t groups, int block);
int ic_gptq_quantize(float* W, int64_t rows, int64_t gw, int64_t groups, const float* Hinv,
                     const float* s32, const float* z32, int bits, int block, int8_t* Q,
                     void* workspace, void* stream);

/* ic_gptq_quantize with the weights read from W_in, which is left unchanged,
 * and the working residual kept in W [rows, groups*gw] (same layout), whose
 * initial contents are never read: the first block is swept from W_in and the
 * first lazy update of every other column reads W_in and writes W.  W == W_in
 * is ic_gptq_quantize.  Same codes as ic_gptq_quantize on a copy of W_in.
 * Replaces the working copy W_work = W.clone() of converter/gptq.py:320
 * together with the sweep of ic_gptq_quantize, without copying the layer. */
int ic_gptq_quantize_from(const float* W_in, float* W, int64_t rows, int64_t gw, int64_t groups,
                          const float* Hinv, const float* s32, const float* z32, int bits, int block,
                          int8_t* Q, void* workspace, void* stream);

/* Allocation-free variant of ic_gptq_quantize.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as ic_gptq_quantize without the
 * workspace: the lazy update's error matrix lives in a static device array
 * of ic_gptq_noalloc_scratch_bytes() = 128 MiB per GPU (held until the
 * process ends), which must hold groups x rows x S fp32 errors, S the
 * super-block width (1024 at block 128 for one matrix, the block for 3-D
 * groups), else IC_ERR_ARG: rows <= 32768 for one matrix, rows x groups
 * <= 262144 for 3-D groups at block 128.  The call allocates nothing and
 * records no profiler events.  Every call on a GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other host threads)
 * race. */
int64_t ic_gptq_noalloc_scratch_bytes(void);
int ic_gptq_quantize_noalloc(float* W, int64_t rows, int64_t gw, int64_t groups, const float* Hinv,
                             const float* s32, const float* z32, int bits, int block, int8_t* Q,
                             void* stream);

/* LDLQ sweep (converter/ldlq.py:369-417, converter/ldlq_triton.py:23-162,
 * converter/rounding.py:115-155): per-element scales [rows, N] (floored at
 * 1e-8), error times 1/max(Hinv_jj, 1e-8), no clamp, sign-flip rule.
 * Hinv [N, N]; W modified; Q int8 [rows, N]; workspace as for GPTQ. */
int ic_ldlq_quantize(float* W, int64_t rows, int64_t N, const float* Hinv, const float* scales,
                     int bits, int block, int8_t* Q, void* workspace, void* stream);

/* LDLQ initial per-element scales S[r, c] = max(absmax_r / (7 or 127), 1e-5)
 * (no upper clamp) and the row vector srow (may be NULL).
 * Replaces converter/ldlq.py:211-215. */
int ic_ldlq_init_scales(const float* row_absmax, int64_t rows, int64_t cols, int bits, float* srow,
                        float* S, void* stream);

/* Non-finite scales -> 1e-8 (NaN, -inf) / 1e30 (+inf), then floor 1e-8
 * (converter/ldlq.py:327-330, 499-502). */
int ic_sanitize_scales(float* S, int64_t n, void* stream);

/* sum((W - Q*S)^2) in fp64 into out_sumsq[0]; workspace 8192 bytes
 * (converter/ldlq.py:518). */
int ic_ldlq_mse(const float* W, const int8_t* Q, const float* S, int64_t n, double* out_sumsq,
                void* workspace, void* stream);

/* Iterative LDLQ scale update (converter/ldlq.py:553-599): where q != 0 and
 * sign(w) == sign(q) with |w| > 1e-8: out = momentum*cur + (1-momentum) *
 * clamp(|w|/|q|, lo, hi); where q != 0 otherwise: clamp(flat, lo, hi);
 * else cur. */
int ic_ldlq_update_scales(const float* W, const int8_t* Q, const float* cur, const float* flat,
                          int64_t n, float momentum, float lo, float hi, float* out, void* stream);

/* Per-row least-squares scale clamp(sum(q w) / max(sum(q q), 1e-8), min 1e-5)
 * (converter/ldlq.py:227-231, 262-265), both row sums of fp32 products in
 * torch's CPU inner-sum order (thread-count independent for rows >= 2, and
 * for one row below 32768 columns), so the scales equal the reference's. */
int ic_ls_scales(const int8_t* Q, const float* W, int64_t rows, int64_t cols, float* out, void* stream);

/* Full-rank greedy coordinate descent on the integer grid minimising
 * tr((Q s - W) H (Q s - W)^T), `passes` sweeps over all columns; scales
 * per row (scale_kind 0: scale[rows]) or per element (scale_kind 1:
 * scale[rows, cols], the reference's scale_2d), H [cols, cols] fp32;
 * Q (int8 [rows, cols]) updated in place.
 * Column blocks of 64 take their cross terms from one fp32-MFMA GEMM plus
 * exact in-block corrections.  workspace: ic_greedy_workspace_bytes().
 * Replaces converter/greedy.py:487-541 (greedy_local_search_pytorch) and
 * 207-285 (greedy_local_search_triton). */
int64_t ic_greedy_workspace_bytes(int64_t rows, int64_t cols);
int ic_greedy(const float* W, int8_t* Q, const float* scale, int scale_kind, const float* H, int64_t rows,
              int64_t cols, int passes, int bits, void* workspace, void* stream);

/* The p largest eigenpairs of a symmetric positive semi-definite H [n, n]
 * (fp32): seeded subspace iteration (`iters` steps of (H + mu I) Q with
 * shifted-CholeskyQR3 orthonormalisation, mu = 1e-3 x a power-iteration
 * estimate of the largest eigenvalue), then Rayleigh-Ritz with an fp64
 * cyclic Jacobi eigensolver.  evals [p] fp32 in descending order; evecs
 * [n, p] fp32, column i the eigenvector of evals[i].  2 <= p <= min(n, 4096),
 * p even; with p == n, iters = 0 gives the full eigendecomposition.
 * refuse_rel > 0 enables an early exit: after min(iters, 2) steps, if
 * Q^T H Q - refuse_rel ||H||_F I is positive definite (Cholesky), then H has
 * at least p eigenvalues above refuse_rel x its largest (interlacing, and
 * lambda_max <= ||H||_F), and the call returns IC_LOWRANK_REFUSED without
 * eigenpairs.  *sweeps (host, may be NULL) receives the Jacobi sweep count.
 * Synchronous: returns after the stream has finished (the Jacobi sweeps test
 * convergence on the host).  IC_ERR_RANGE if the orthonormalisation loses
 * positive definiteness (the caller falls back to the full-rank search).
 * workspace: ic_lowrank_workspace_bytes(n, p).
 * Replaces converter/greedy.py:293-366 (_lowrank_decompose: torch.svd_lowrank
 * with q = N/2, then torch.linalg.eigh); the rank cut and its refusal gates
 * stay with the caller, as in greedy.py:330-341. */
int64_t ic_lowrank_workspace_bytes(int64_t n, int64_t p);
int ic_lowrank_eigs(const float* H, int64_t n, int64_t p, int iters, unsigned long long seed, float refuse_rel,
                    float* evals, float* evecs, int* sweeps, void* workspace, void* stream);

/* Low-rank greedy search: the greedy of ic_greedy (same scale / scale_kind)
 * with the cross terms taken from Hk = U_k diag(s_k) U_k^T (U [cols, >= k]
 * pitch ldu, s [k]) and the
 * exact diagonal H_jj, i.e. cross_j = err . Hk[:, j] - err_j H_jj; after
 * every pass but the last, the proxy sum((err @ H) * err) with the full H
 * ends the search once it is >= 0.99 x the previous pass's (from the second
 * pass on).  *passes_run (host, may be NULL) receives the passes made.
 * Synchronous (one host read of the proxy per pass).
 * workspace: ic_greedy_lowrank_workspace_bytes(rows, cols, k).
 * Replaces converter/greedy.py:369-479 (greedy_lowrank_triton) and its
 * kernel 99-199 (_greedy_lowrank_kernel). */
int64_t ic_greedy_lowrank_workspace_bytes(int64_t rows, int64_t cols, int64_t k);
int ic_greedy_lowrank(const float* W, int8_t* Q, const float* scale, int scale_kind, const float* H,
                      const float* U, int64_t ldu, const float* s, int64_t k, int64_t rows, int64_t cols,
                      int passes, int bits, int* passes_run, void* workspace, void* stream);

/* ---------------------------------------------------------------- PermuQuant */

/* Channel second moments mu2[j] = mean(W[:, j]^2) (converter/permuquant.py:
 * 13-23, channel_second_moments), fp32 [rows, cols] at pitch ld, summed in
 * the order torch's CPU reduction uses, so the result is bit-exact with the
 * reference's CPU path.  cpu_vec (16 for AVX-512 torch builds, 8 for AVX2)
 * is the vector width of that reduction: the last cols % cpu_vec columns take
 * its scalar loop.  Workspace: ic_col_moments_workspace_bytes. */
int64_t ic_col_moments_workspace_bytes(int64_t rows, int64_t cols);
int ic_col_moments(const float* W, int64_t rows, int64_t cols, int64_t ld, int cpu_vec, float* mu2,
                   void* workspace, void* stream);

/* perm = argsort(v, descending=True) (permuquant.py:38-40, 61-64): a stable
 * sort, ties in increasing index, NaN first, -0 equal to +0.  torch's CPU
 * argsort is not stable from 100 elements on, so on exact ties its order
 * may differ.  perm: int64 [n].  Workspace: ic_argsort_workspace_bytes. */
int64_t ic_argsort_workspace_bytes(int64_t n);
int ic_argsort_desc(const float* v, int64_t n, int64_t* perm, void* workspace, void* stream);

/* compute_group_quant_error (permuquant.py:67-111) of W[:, perm] (perm may
 * be null: W itself): symmetric RTN with fp16 scales per row (bits 8) or per
 * group of `group` columns (bits 4, the last group zero-padded), then
 * sum((W - q s)^2) in the order torch's CPU sum uses with `threads` threads,
 * bit-exact with the reference run with that many threads.  out: one fp32 on
 * the device.  perm entries must lie in [0, cols).  Workspace:
 * ic_group_quant_error_workspace_bytes. */
int64_t ic_group_quant_error_workspace_bytes(int64_t rows, int64_t cols, int64_t group, int bits, int threads);
int ic_group_quant_error(const float* W, int64_t rows, int64_t cols, int64_t ld, const int64_t* perm, int64_t group,
                         int bits, int threads, float* out, void* workspace, void* stream);

/* torch.sum(x) of n contiguous fp32 values as torch's CPU kernel computes it
 * with `threads` threads (the reduction inside ic_group_quant_error). */
int64_t ic_torch_sum_workspace_bytes(int64_t n, int threads);
int ic_torch_sum(const float* x, int64_t n, int threads, float* out, void* workspace, void* stream);

/* Gathers that apply a permutation (pipeline.py:588-590, 609, 737;
 * permuquant.py:208-244): dst[r][j] = src[r][perm[j]] for j < n_perm, and
 * out[i][j] = H[perm[i]][perm[j]] (H[perm][:, perm]).  Indices outside the
 * source are not read; their outputs are 0. */
int ic_permute_cols(const float* src, int64_t rows, int64_t src_cols, int64_t ld_src, const int64_t* perm,
                    int64_t n_perm, float* dst, int64_t ld_dst, void* stream);
int ic_permute_sym(const float* H, int64_t n, int64_t ld, const int64_t* perm, int64_t n_perm, float* out,
                   int64_t ld_out, void* stream);

/* ---------------------------------------------------------------- DLR Hessians */

/* Damped inverse of a diagonal + low-rank Hessian H = diag(D) + U U^T by the
 * Woodbury identity (converter/dlr.py:70-119, woodbury_inverse):
 * D' = D + damping * max(mean(D + rowsum(U^2)), 1e-6) (damping > 0, else D),
 * Dinv = 1 / max(D', 1e-12), Z = Dinv U, M = I + U^T Z,
 * Hinv = diag(Dinv) - (Z M^-1) Z^T.  D fp32 [n], U fp32 [n, r] at pitch ldu
 * (r may be 0), Hinv fp32 [n, n] at pitch ldh.  M^-1 is the Cholesky inverse
 * of M; when that factorisation meets a non-positive pivot info[0] is set to
 * its 1-based column and Hinv is not meaningful: the caller then inverts M
 * (written to M_out [r, r] when M_out is not null) another way and calls
 * again with Minv_in (then U^T Z and the factorisation are skipped).
 * upper_only: only entries on and above the diagonal are computed; entries
 * less than 128 below the diagonal are set to 0, the rest of the lower
 * triangle is left as it was (for the GPTQ / LDLQ sweeps, which read rows j
 * from column j on).  info: 2 ints on the device.  Workspace:
 * ic_woodbury_workspace_bytes(n, r). */
int64_t ic_woodbury_workspace_bytes(int64_t n, int64_t r);
int ic_woodbury_inverse(const float* D, const float* U, int64_t n, int64_t r, int64_t ldu, float damping,
                        const float* Minv_in, int upper_only, float* Hinv, int64_t ldh, float* M_out, int* info,
                        void* workspace, void* stream);

/* H = diag(D) + U U^T as a dense fp32 [n, n] matrix at pitch ldh
 * (converter/dlr.py:122-127, dlr_to_dense; rotation.py:181-184 densifies a
 * DLR Hessian this way before rotating it). */
int ic_dlr_to_dense(const float* D, const float* U, int64_t n, int64_t r, int64_t ldu, float* H, int64_t ldh,
                    void* stream);

/* ---------------------------------------------------------------- PiSO */

/* PiSO per-row scales (converter/piso.py:28-183, the PyTorch path of
 * compute_piso_scales_int8 / _int8_asymmetric / _int4 / _int4_asymmetric):
 * for each row of W (fp32 [rows, cols], pitch ld) the error
 * sum_d (w_d - dq(w_d; s))^2 h_d (h fp32 [cols]) is evaluated for
 * s = s_ref * coarse[c], c < num_coarse, the first minimum picks s_best, then
 * for s_best * fine[f], f < num_fine, whose first minimum is the result.
 * Symmetric (asym 0): s_ref = max(absmax / qmax, 1e-10), dq = clamp(rhaz(
 * w / s)) s.  Asymmetric: s_ref = max((max - min) / (qmax - qmin), 1e-10),
 * s clamped at 1e-10, zp = clamp(rhaz(qmin - min / s)), dq = (clamp(rhaz(
 * w / s + zp)) - zp) s.  Grid [qmin, qmax] = [-8, 7] (bits 4) or
 * [-128, 127] (bits 8).  The sums follow torch's CPU order, so scales (fp32
 * [rows]) and zero-points (int8 [rows], asym only) equal the reference's CPU
 * path bit for bit.  coarse / fine: the factor tables on the device (the
 * reference's torch.linspace values), 1 to 1024 entries each. */
int ic_piso_scales(const float* W, int64_t rows, int64_t cols, int64_t ld, const float* h, int bits, int asym,
                   const float* coarse, int num_coarse, const float* fine, int num_fine, float* scales,
                   int8_t* zp, void* stream);

/* ---------------------------------------------------------------- profiling */

/* HBM ceiling probes (measurement only; no counterpart in the reference):
 * kind 0 copies `bytes` from src to dst, 1 reads them (dst: a float the
 * kernel may write), 2 writes `bytes` to dst, 3 converts bf16 src (`bytes`)
 * to fp32 dst (2 x bytes); 16-byte coalesced accesses, four loads in flight
 * per thread.  bench.py --hbm-ceiling times them. */
int ic_hbm_stream(int kind, const void* src, void* dst, int64_t bytes, void* stream);

/* Launch profiler (no reference counterpart; measurement support).  While
 * enabled, library launches are bracketed by HIP events on their stream and
 * tagged with a phase: 0 trailing-update GEMM, 1 Cholesky GEMMs, 2 inverse
 * GEMMs, 3 diagonal-block factor, 4 sweep, 5 weight rotation, 6 Hessian
 * rotation, 7 RTN quantise / INT4 pack, 8 greedy block kernel, 9 other, 10 greedy
 * cross-term GEMMs, 11 Cholesky panel solve, 12 RTN scales / clip search,
 * 13 fp64 verification, 14 PermuQuant (moments, sort, error scales,
 * gathers), 15 PermuQuant ordered error sums, 16 DLR r x r products,
 * 17 DLR n x n product, 18 PiSO scale search.  Enabling resets the record.
 * ic_profile_read synchronises the events and returns, per phase, the summed
 * kernel time (ms), algorithmic flops and bytes, and the launch count (arrays
 * of at least 19 entries). */
int ic_profile_enable(int on);
int ic_profile_read(double* ms, double* flops, double* bytes, int64_t* launches, int ntags);

#ifdef __cplusplus
}
#endif

#endif /* IC_ABI_H */
