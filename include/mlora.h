/*
 * mlora.h — C ABI of the MI355X (gfx950) grouped MoE-LoRA operator library, libmlora.so.
 *
 * Every entry point is plain C: raw device pointers, element counts and element strides, a HIP
 * stream passed as `void*` (NULL = the default stream), and an `int` status (0 = success).  On a
 * non-zero status `mlora_last_error()` returns a message naming the argument or condition that was
 * refused; the message is per host thread.  No entry point allocates device memory: a scratch
 * buffer, where one is needed, is passed in by the caller and its required size is returned by a
 * `*_workspace_bytes` query.  Nothing synchronises the host with the device; all work is enqueued
 * on the given stream in order.
 *
 * Dtype codes (`MLORA_DT_*`) describe element types of tensors whose type can vary.
 *
 * Reference interfaces replaced (paths into thinkube/meepsquared; `TF:` = transformers 5.x):
 *   routing     — TF:models/qwen3_moe/modeling_qwen3_moe.py:258-267 (router top-k softmax) and
 *                 src/meepsquared/_moe.py:77-87 (sort, histc, cumsum offsets, sentinel mask)
 *   tile map    — src/meepsquared/_grouped.py:83-103 (max_tiles, tile_map)
 *   products    — src/meepsquared/_grouped.py:120-221 (_grouped_gemm_kernel) via _launch :313-345
 *   reduction   — src/meepsquared/_grouped.py:232-256 (_grouped_reduce_kernel) via _reduce :362-370
 *   layer glue  — src/meepsquared/_moe.py:80-81 (gather), TF:integrations/moe.py:509-520 (SwiGLU gate),
 *                 src/meepsquared/_moe.py:123-126 (weight, un-permute, sum over k)
 *   fp8 stacks  — src/meepsquared/_fp8.py:68-79,111-134 (_grouped_scale_kernel, quantize_stack,
 *                 dequantize_stack), extended with one scale per output row
 *   nf4 stacks  — src/meepsquared/_vendor/axolotl/quantize.py:52-101,202-235 (the NF4 double-quant
 *                 format, there for dense layers only), applied here to expert stacks
 */
#ifndef MLORA_H
#define MLORA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  MLORA_DT_BF16 = 0,
  MLORA_DT_F32 = 1,
  MLORA_DT_F16 = 2,
  MLORA_DT_FP8_E4M3 = 3, /* OCP float8 e4m3fn, torch.float8_e4m3fn */
  MLORA_DT_NF4 = 4,      /* two 4-bit NF4 codes per byte, first element in the high nibble */
  MLORA_DT_NF4_KT = 5    /* NF4 codes of a stack read with k contiguous whose absmax varies along k
                            (mlora_nf4_transpose's layout): nf4_absmax2 is the fp32 table (E, N/64, K),
                            nf4_code the 16 codes; the other NF4 arguments are unused */
};

enum {
  MLORA_SCALE_NONE = 0,
  MLORA_SCALE_EXPERT = 1, /* scale[e]: one fp32 per expert (the reference's fp8 stacks) */
  MLORA_SCALE_ROW = 2     /* scale[e * scale_se + o]: one fp32 per output row o of the stack */
};

/* Library identity and the last error of this host thread ("" when none). */
const char* mlora_version(void);
const char* mlora_last_error(void);

/* ---------------------------------------------------------------------------------------------
 * Routing
 * ------------------------------------------------------------------------------------------- */

/* Router: probs = softmax(logits, fp32) over E, the k largest in the order torch.topk returns them
 * on the GPU, ties included (equal probabilities at the k-th place taken in ascending expert order;
 * for k <= 32 the k sorted descending by torch's 32-wide bitonic network, which places equal values
 * in an order of its own; for k > 32 equal values in ascending expert order), weights = probs
 * (renorm=0) or probs / sum of the k (renorm=1), cast to
 * w_dtype (MLORA_DT_BF16 or MLORA_DT_F32).  logits: (T, E) of logits_dtype (bf16/f16/f32) with
 * row stride ld_logits; out_idx (T, k) int64; out_w (T, k).  E <= 1024, 1 <= k <= min(E, 64).
 * Replaces TF:models/qwen3_moe/modeling_qwen3_moe.py:262-266 (Mixtral: TF:models/mixtral/
 * modeling_mixtral.py:104-111). */
int mlora_route_topk(const void* logits, int logits_dtype, int64_t ld_logits, int64_t T, int E, int k,
                     int renorm, int64_t* out_idx, void* out_w, int w_dtype, void* stream);

/* Scratch bytes mlora_route_sort needs for S ids over E experts. */
size_t mlora_route_sort_workspace_bytes(int64_t S, int E);

/* Counting sort of S expert ids (int64; an id outside [0, E) is a sentinel and sorts to the tail).
 * perm (S,) int64: the stable order, perm[p] = flat index of the p-th row in expert order;
 * inv (S,) int64: inv[perm[p]] = p (may be NULL); offsets (E,) int32: the end of each expert's
 * rows (cumsum of the per-expert counts, sentinels excluded).  When tile_expert is not NULL the
 * tile map of `mlora_tile_map` for (offsets, rows=S, block_m, max_tiles) is written as well.  E <= 2048.
 * Replaces src/meepsquared/_moe.py:77-87 (torch.sort, histc, cumsum) and _grouped.py:88-103. */
int mlora_route_sort(const int64_t* ids, int64_t S, int E, int64_t* perm, int64_t* inv, int32_t* offsets,
                     int block_m, int32_t* tile_expert, int32_t* tile_row, int32_t* tiles, int64_t max_tiles,
                     void* workspace, size_t workspace_bytes, void* stream);

/* mlora_route_sort without a workspace argument, for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No counterpart in
 * the reference.  The histograms live in a 4 MiB array of the library's own, one per GPU (the device
 * current on the calling thread), held until the process ends: S and E must satisfy
 * mlora_route_sort_workspace_bytes(S, E) <= 4194304 (e.g. S <= 2,080,768 ids at E = 128), else the call is
 * refused.  It calls no hipMalloc or hipFree.  Calls on one GPU share the array: calls that overlap
 * (concurrent streams) race; calls in sequence on one stream do not.  Results are those of
 * mlora_route_sort. */
int mlora_route_sort_noalloc(const int64_t* ids, int64_t S, int E, int64_t* perm, int64_t* inv, int32_t* offsets,
                             int block_m, int32_t* tile_expert, int32_t* tile_row, int32_t* tiles,
                             int64_t max_tiles, void* stream);

/* The tile map of src/meepsquared/_grouped.py:88-103: each expert's rows cut into block_m-row
 * tiles; tile_expert/tile_row (max_tiles,) int32, tiles a single int32 (the real count).  Spare
 * entries hold the last expert and the row the reference's formula gives.  E <= 4096. */
int mlora_tile_map(const int32_t* offsets, int E, int64_t rows, int block_m, int32_t* tile_expert,
                   int32_t* tile_row, int32_t* tiles, int64_t max_tiles, void* stream);

/* ---------------------------------------------------------------------------------------------
 * The grouped product with the fused LoRA (forward and input-gradient passes)
 * ------------------------------------------------------------------------------------------- */

/* out[row, n] = c · sum_k x[row, k] W_e[k, n] + scaling · bf16(x[row,:] · A_e)[:] · B_e[:, n] + bias[e, n]
 * for every row of expert e (rows offsets[e-1] .. offsets[e]-1; rows past offsets[E-1] untouched).
 *   x      (rows, K) bf16, row stride ldx, unit column stride, ldx % 8 == 0, 16-byte aligned.
 *   w      the stack addressed as W_e[k, n] = w[e*w_se + k*w_sk + n*w_sn], w_sk == 1 or w_sn == 1,
 *          in w_dtype: MLORA_DT_BF16, MLORA_DT_FP8_E4M3 or MLORA_DT_NF4 (NF4: a contiguous stack,
 *          the strides in elements, blocks of 64 along the unit-stride axis, whose length is a
 *          multiple of 64; nf4_absmax_q (uint8, one per block), nf4_absmax2 (fp32, one per 256
 *          blocks), nf4_code2 (256 fp32, the second-level code), nf4_offset: block b's absmax is
 *          code2[absmax_q[b]] * absmax2[b / 256] + nf4_offset[0]; nf4_code (16 fp32) the NF4 code
 *          book; all of these on the device).
 *   c      1, scale[e] (MLORA_SCALE_EXPERT), or scale[e*scale_se + o] for output row o of the
 *          stack (MLORA_SCALE_ROW); scale_on_k = 1 says the stack's output rows run along k here
 *          (the input-gradient pass), 0 along n.
 *   at, bt the LoRA factors as A_e^T and B_e^T, bf16: A_e[k, r] = at[e*at_se + r*at_sr + k] (k contiguous)
 *          and B_e[r, n] = bt[e*bt_se + n*bt_sn + r] (r contiguous); rank is 16, 32, 48 or 64 (a
 *          smaller rank is padded with zero rows/columns by the caller, as src/meepsquared/
 *          _grouped.py:275-282 does); at == NULL: no adapters.
 *   low    (rows, rank) bf16 row stride ldl, receives bf16(x · A_e) (NULL: not stored).
 *   bias   (E, N) bf16 with expert stride bias_se, or NULL.
 *   out    (rows, N) bf16, row stride ldo, unit column stride.
 * K % 8 == 0, N % 8 == 0.  Replaces _grouped_gemm_kernel (src/meepsquared/_grouped.py:120-221). */
int mlora_grouped_gemm(const void* x, int64_t ldx, int64_t rows, int K, int N,
                       const void* w, int w_dtype, int64_t w_se, int64_t w_sk, int64_t w_sn,
                       const float* scale, int scale_kind, int64_t scale_se, int scale_on_k,
                       const uint8_t* nf4_absmax_q, const float* nf4_absmax2, const float* nf4_code2,
                       const float* nf4_offset, const float* nf4_code,
                       const void* at, int64_t at_se, int64_t at_sr,
                       const void* bt, int64_t bt_se, int64_t bt_sn, int rank, float scaling,
                       const void* bias, int64_t bias_se,
                       void* out, int64_t ldo, void* low, int64_t ldl,
                       const int32_t* offsets, int E, void* stream);

/* mlora_grouped_gemm with the rows of x gathered: row r of the product is row gather[r] / k of x
 * (x_rows rows, row stride ldx), so the expert-sorted copy h[perm // k] of the layer's input
 * (src/meepsquared/_moe.py:80) is never written.  With row_scale (MLORA_DT_BF16 or MLORA_DT_F32),
 * output row r is (c · x W + scaling · bf16(x A) B) · row_scale[gather[r]] + bias: the input gradient
 * of the down product straight from the layer's output gradient, the combine weights applied per row
 * (src/meepsquared/_moe.py:123-126 and the down projection's backward, without the weighted copy of
 * the gradient); low stays bf16(x A) of the unscaled rows.  rows < 2^32; the other arguments as
 * mlora_grouped_gemm's (no NF4 stack and no per-row stack scale along k here: mlora_grouped_gemm_gather_q
 * takes those); a stack layout the DMA-fed product does not take is refused. */
int mlora_grouped_gemm_gather(const void* x, int64_t ldx, int64_t x_rows, const int64_t* gather, int k,
                              const void* row_scale, int row_scale_dtype, int64_t rows,
                              int K, int N, const void* w, int w_dtype, int64_t w_se, int64_t w_sk, int64_t w_sn,
                              const float* scale, int scale_kind, int64_t scale_se,
                              const void* at, int64_t at_se, int64_t at_sr,
                              const void* bt, int64_t bt_se, int64_t bt_sn, int rank, float scaling,
                              const void* bias, int64_t bias_se, void* out, int64_t ldo, void* low, int64_t ldl,
                              const int32_t* offsets, int E, void* stream);

/* mlora_grouped_gemm_gather for every stack type the DMA-fed product takes: mlora_grouped_gemm's stack
 * arguments (w_dtype bf16, fp8 e4m3 with its scale, per-row scales along k with scale_on_k, NF4 with its
 * tables; k contiguous for the quantised ones, rows of whole 16-byte chunks, NF4 rows of whole 64-code
 * blocks) with the rows of x gathered and optionally weighted as mlora_grouped_gemm_gather reads them;
 * a stack layout that product does not take is refused.  The layer's gathered gate_up product and the
 * down product's input-gradient pass over fp8 and NF4 stacks (src/meepsquared/_moe.py:80 and :123-126
 * folded into the products, as for bf16 stacks). */
int mlora_grouped_gemm_gather_q(const void* x, int64_t ldx, int64_t x_rows, const int64_t* gather, int k,
                                const void* row_scale, int row_scale_dtype, int64_t rows, int K, int N,
                                const void* w, int w_dtype, int64_t w_se, int64_t w_sk, int64_t w_sn,
                                const float* scale, int scale_kind, int64_t scale_se, int scale_on_k,
                                const uint8_t* nf4_absmax_q, const float* nf4_absmax2, const float* nf4_code2,
                                const float* nf4_offset, const float* nf4_code,
                                const void* at, int64_t at_se, int64_t at_sr, const void* bt, int64_t bt_se,
                                int64_t bt_sn, int rank, float scaling, const void* bias, int64_t bias_se,
                                void* out, int64_t ldo, void* low, int64_t ldl, const int32_t* offsets, int E,
                                void* stream);

/* mlora_grouped_gemm_gather_q's forward product (no row scale, no scale along k) of a gate_up stack, N = 2 I
 * columns (gate, then up), with SwiGLU formed in the same pass:
 *   act[r, c] = bf16(g · sigmoid(g) · u),  g = out[r, c], u = out[r, I + c]  (the stored bf16 values),
 * the values mlora_swiglu(out) writes, row stride lda (>= I, a multiple of 8, 16-byte aligned base).  out
 * and low are written as mlora_grouped_gemm_gather_q writes them.  Needs N a multiple of 256, adapters of
 * rank 16 or none, and a stack the DMA-fed product takes (bf16; fp8 and NF4 k contiguous).  Replaces, in the layer's forward,
 * _grouped_gemm_kernel's gate_up launch and the SwiGLU pass after it (src/meepsquared/_moe.py:80-84,
 * TF integrations/moe.py:509-520), so that gu is not read back. */
int mlora_grouped_gemm_gather_swiglu(const void* x, int64_t ldx, int64_t x_rows, const int64_t* gather, int k,
                                     int64_t rows, int K, int N, const void* w, int w_dtype, int64_t w_se,
                                     int64_t w_sk, int64_t w_sn, const float* scale, int scale_kind, int64_t scale_se,
                                     const uint8_t* nf4_absmax_q, const float* nf4_absmax2, const float* nf4_code2,
                                     const float* nf4_offset, const float* nf4_code, const void* at, int64_t at_se,
                                     int64_t at_sr, const void* bt, int64_t bt_se, int64_t bt_sn, int rank,
                                     float scaling, const void* bias, int64_t bias_se, void* out, int64_t ldo,
                                     void* low, int64_t ldl, void* act, int64_t lda, const int32_t* offsets, int E,
                                     void* stream);

/* Scratch bytes mlora_grouped_gemm_db needs for (rows, K, E): fp32 partial sums, 16 x K per 256-row tile
 * (E + rows / 256 + 1 tile slots; 16-byte aligned, contents on entry ignored). */
size_t mlora_grouped_gemm_db_workspace_bytes(int64_t rows, int K, int E);

/* The input-gradient product with the adapter gradient that reads the same rows fused into it:
 * mlora_grouped_gemm_gather's product (gather may be NULL: rows of x read in order, x_rows = rows; a
 * bf16 stack, adapters at rank 16, at most 256 experts), plus
 *   db_out[e, k, r] = bf16(scaling · sum over expert e's rows of x[row, k] · l[row, r]),  k < K, r < 16,
 * the sum mlora_grouped_reduce(_gather) forms over x's rows (g = x; with gather, row r is row
 * gather[r] / k of x), so that the output gradient is read once, by the product.  l (rows, 16) bf16 row
 * stride db_ldl (rows weighted as the caller needs them: mlora_grouped_reduce_gather's row_scale
 * corresponds to l[row] = bf16(row_scale[scale_index[row]] · l[row])); db_out written by its strides
 * (db_o_se, db_o_sk, db_o_sr).  fp32 partial sums per 256-row tile go to workspace
 * (mlora_grouped_gemm_db_workspace_bytes) and a second launch adds each expert's tiles in row order:
 * deterministic, no atomics.  Replaces, for the pass that reads the output gradient,
 * _grouped_gemm_kernel's input-gradient launch and the _grouped_reduce_kernel launch for B's gradient
 * (src/meepsquared/_grouped.py:398-399, :232-256). */
int mlora_grouped_gemm_db(const void* x, int64_t ldx, int64_t x_rows, const int64_t* gather, int k,
                          const void* row_scale, int row_scale_dtype, int64_t rows, int K, int N,
                          const void* w, int64_t w_se, int64_t w_sk, int64_t w_sn, const float* scale,
                          int scale_kind, int64_t scale_se, const void* at, int64_t at_se, int64_t at_sr,
                          const void* bt, int64_t bt_se, int64_t bt_sn, int rank, float scaling,
                          const void* bias, int64_t bias_se, void* out, int64_t ldo, void* low, int64_t ldl,
                          const void* db_l, int64_t db_ldl, void* db_out, int64_t db_o_se, int64_t db_o_sk,
                          int64_t db_o_sr, void* workspace, size_t workspace_bytes, const int32_t* offsets, int E,
                          void* stream);

/* Scratch bytes mlora_grouped_reduce(_gather) needs for (rows, N, R, E): the partial sums of split
 * experts (16-byte aligned, contents on entry ignored); 0 when no expert can be split (E > 32). */
size_t mlora_grouped_reduce_workspace_bytes(int64_t rows, int N, int R, int E);

/* out[e, n, r] = bf16(scaling · sum over expert e's rows of g[row, n] · l[row, r]), fp32
 * accumulation in a fixed order, no atomics: the adapters' gradients.  g (rows, N) bf16 row stride
 * ldg; l (rows, R) bf16 row stride ldl; out addressed out[e*o_se + n*o_sn + r*o_sr].  R <= 64,
 * rows < 2^32.  With E <= 32 an expert with more rows than a part (max(4096, the mean rows per expert
 * rounded up to a power of two)) is summed in parts whose fp32 partial sums go through the workspace and
 * are added in part order by a second launch.
 * Replaces _grouped_reduce_kernel (src/meepsquared/_grouped.py:232-256). */
int mlora_grouped_reduce(const void* g, int64_t ldg, const void* l, int64_t ldl, int64_t rows, int N, int R,
                         float scaling, const int32_t* offsets, int E,
                         void* out, int64_t o_se, int64_t o_sn, int64_t o_sr, void* workspace, size_t workspace_bytes,
                         void* stream);

/* mlora_grouped_reduce with the rows of g gathered and/or weighted: with gather, row r is row
 * gather[r] / k of g (A's gradient of the gate_up product when its input rows are gathered, as
 * mlora_grouped_gemm_gather reads them); with row_scale, row r's term is weighted by
 * row_scale[scale_index[r]], applied as bf16(row_scale[...] · l[r]) — for the down product's
 * adapters, whose gradient rows the combine's backward (src/meepsquared/_moe.py:123-126) would have
 * weighted.  At least one of gather and row_scale is given. */
int mlora_grouped_reduce_gather(const void* g, int64_t ldg, const int64_t* gather, int k, const void* row_scale,
                                int row_scale_dtype, const int64_t* scale_index, const void* l, int64_t ldl,
                                int64_t rows, int N, int R, float scaling, const int32_t* offsets, int E,
                                void* out, int64_t o_se, int64_t o_sn, int64_t o_sr, void* workspace,
                                size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------------------------
 * The layer around the products: gather, SwiGLU, combine (bf16 activations)
 * ------------------------------------------------------------------------------------------- */

/* out[p, :] = h[perm[p] / k, :] for p < offsets[E-1], zero for the sentinel rows after it.
 * h (T, H) row stride ldh; out (S, H) contiguous.  H % 8 == 0.  Replaces _moe.py:80,85-87. */
int mlora_gather_rows(const void* h, int64_t ldh, int64_t H, const int64_t* perm, int64_t S, int k,
                      const int32_t* offsets, int E, void* out, void* stream);

/* The gather's gradient: dh[t, :] = sum over j < k of dsel[inv[t*k + j], :] (rows at or past
 * offsets[E-1] skipped), fp32 accumulation.  dsel (S, H) contiguous; dh (T, H) contiguous. */
int mlora_gather_rows_backward(const void* dsel, int64_t H, const int64_t* inv, int64_t T, int k,
                               const int32_t* offsets, int E, void* dh, void* stream);

/* act[r, i] = silu(gu[r, i]) · gu[r, I + i] (gate first, as TF:integrations/moe.py:509-520).
 * gu (S, 2I) contiguous, act (S, I) contiguous, I % 8 == 0. */
int mlora_swiglu(const void* gu, int64_t S, int64_t I, void* act, void* stream);

/* dgu from dact and gu: dgate = dact · up · silu'(gate), dup = dact · silu(gate). */
int mlora_swiglu_backward(const void* gu, const void* dact, int64_t S, int64_t I, void* dgu, void* stream);

/* The SwiGLU backward of the layer's down product fused with the combine weights' gradient (no
 * counterpart function in the reference: it replaces the autograd of src/meepsquared/_moe.py:123-126
 * (the weighted combine) and of the SwiGLU gate when the down stack has no bias).
 * g (S, I) bf16 is the down product's input gradient computed WITHOUT the combine weights (the output
 * gradient read through perm); row p of the expert order has the weight w[perm[p]] (w: T*k, bf16 or
 * fp32, w_dtype).  Writes dgu (S, 2I) = the SwiGLU backward of (w[perm[p]] · g[p]) and
 * dw[perm[p]] = <g[p], act[p]> (act recomputed from gu as mlora_swiglu rounds it), which equals
 * <dout[t], y[p]> for y = the down product without bias.  Rows p >= offsets[E-1] (sentinels): dgu = 0,
 * dw = 0.  I % 8 == 0. */
int mlora_swiglu_backward_weighted(const void* gu, const void* g, int64_t S, int64_t I, const void* w, int w_dtype,
                                   const int64_t* perm, const int32_t* offsets, int E, void* dgu, void* dw,
                                   void* stream);

/* mlora_swiglu_backward_weighted fused with the two adapter reductions that read its operands (no
 * counterpart function in the reference: it replaces, in one pass over each expert's rows, the SwiGLU
 * gate's backward and the weighted combine's (src/meepsquared/_moe.py:118-126) and two of the
 * _reduce calls of src/meepsquared/_grouped.py:362-370, 398-399):
 *   dgu, dw             as mlora_swiglu_backward_weighted (dgu bit-identical; dw summed per 64 columns,
 *                       then over the column blocks in order);
 *   dA[e, n, r]         = bf16(scaling2 · sum over expert e's rows p of act[p, n] · bf16(w[perm[p]] · low2[p, r]))
 *                         (the down adapter's A gradient: act as mlora_swiglu rounds it, low2 (S, 16) the
 *                         down input-gradient product's low, unweighted, row stride ld2);
 *   dB[e, n, r]         = bf16(scaling_gu · sum over expert e's rows p of dgu[p, n] · lowgu[p, r]) for n < 2I
 *                         (the gate_up adapter's B gradient: lowgu (S, 16) the gate_up product's low);
 * each the same bits as mlora_grouped_reduce_gather(act, low2, row_scale w) and mlora_grouped_reduce(dgu,
 * lowgu) give.  dA and dB are written by their strides (se, sn, sr).  Rank 16 (padded) only; I % 8 == 0;
 * bf16 tensors 16-byte aligned.  The workspace (256-byte aligned) holds per-row parts of dw and, when an
 * expert's rows can be split over several workgroups, their partial sums:
 * mlora_swiglu_backward_reduce_workspace_bytes gives its size. */
size_t mlora_swiglu_backward_reduce_workspace_bytes(int64_t S, int64_t I, int E);
int mlora_swiglu_backward_reduce(const void* gu, const void* g, int64_t S, int64_t I, const void* w, int w_dtype,
                                 const int64_t* perm, const int32_t* offsets, int E, const void* low2, int64_t ld2,
                                 float scaling2, void* dA, int64_t a_se, int64_t a_sn, int64_t a_sr,
                                 const void* lowgu, int64_t ldu, float scaling_gu, void* dB, int64_t b_se,
                                 int64_t b_sn, int64_t b_sr, void* dgu, void* dw, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* out[t, :] = sum over j < k of bf16(y[inv[t*k+j], :] · w[t*k+j]) with fp32 accumulation; rows at
 * or past offsets[E-1] (sentinels) contribute nothing.  y (S, H) contiguous, w (T*k) of w_dtype
 * (MLORA_DT_BF16 or MLORA_DT_F32), out (T, H) contiguous.  Replaces _moe.py:123-126. */
int mlora_combine(const void* y, int64_t H, const void* w, int w_dtype, const int64_t* inv, int64_t T, int k,
                  const int32_t* offsets, int E, void* out, void* stream);

/* The combine's gradients: dy[inv[t*k+j], :] = bf16(dout[t, :] · w[t*k+j]) (zero for sentinel
 * rows) and dw[t*k+j] = sum_h dout[t, h] · y[inv[t*k+j], h] (zero for sentinel rows), in w_dtype.
 * dy may be NULL (dw only: the down product then reads dout through mlora_grouped_gemm_gather). */
int mlora_combine_backward(const void* dout, const void* y, int64_t H, const void* w, int w_dtype,
                           const int64_t* inv, int64_t T, int k, const int32_t* offsets, int E,
                           void* dy, void* dw, void* stream);

/* out[r, :] = bf16(w[index[r]] · l[r, :]) for r < rows (l, out (rows, R) bf16, row strides ldl, ldo; R and
 * the strides multiples of 8, 16-byte aligned bases; w bf16/f32): the down product's low weighted by each
 * routed row's combine weight, the form mlora_grouped_gemm_db takes for B's gradient (the weighting
 * mlora_grouped_reduce_gather's row_scale applies; src/meepsquared/_moe.py:123 weights the rows). */
int mlora_scale_rows(const void* l, int64_t ldl, int64_t rows, int64_t R, const void* w, int w_dtype,
                     const int64_t* index, void* out, int64_t ldo, void* stream);

/* The adapters' roles in the input-gradient product (src/meepsquared/_grouped.py:304-310, _Adapters.swapped)
 * in one launch: at_out (E, R, N) contiguous = bt's transpose, bt_out (E, K, R) contiguous = at's transpose,
 * for at = A^T (E, R, K) and bt = B^T (E, N, R) as mlora_grouped_gemm takes them (unit stride along K and
 * R; strides at_se, at_sr, bt_se, bt_sn multiples of 8, 16-byte aligned).  R (the padded rank) 16 or 32,
 * K and N multiples of 8 above R; other shapes take two mlora_transpose calls. */
int mlora_swap_adapters(const void* at, int64_t at_se, int64_t at_sr, const void* bt, int64_t bt_se, int64_t bt_sn,
                        int64_t E, int64_t R, int64_t K, int64_t N, void* at_out, void* bt_out, void* stream);

/* mlora_swap_adapters for two projections in one launch (the layer's down and gate_up adapters, swapped at
 * the first input-gradient product of the backward; _grouped.py:304-310 swaps each projection's factors
 * when its own backward runs): the first projection's arguments, then the second's, each as
 * mlora_swap_adapters takes them. */
int mlora_swap_adapters_two(const void* at, int64_t at_se, int64_t at_sr, const void* bt, int64_t bt_se,
                            int64_t bt_sn, int64_t E, int64_t R, int64_t K, int64_t N, void* at_out, void* bt_out,
                            const void* at2, int64_t at2_se, int64_t at2_sr, const void* bt2, int64_t bt2_se,
                            int64_t bt2_sn, int64_t E2, int64_t R2, int64_t K2, int64_t N2, void* at2_out,
                            void* bt2_out, void* stream);

/* dst[e][b][a] = src[e*s_e + a*s_a + b*s_b] (bf16): a batched transpose into a contiguous (E, B, A)
 * tensor, for the adapters' roles in the input-gradient product, which
 * src/meepsquared/_grouped.py:304-310 (_Adapters.swapped) addresses by strides. */
int mlora_transpose(const void* src, int64_t E, int64_t A, int64_t B, int64_t s_e, int64_t s_a, int64_t s_b,
                    void* dst, void* stream);

/* The same for 1-byte elements (an fp8 stack's transposed copy for the fp8 products). */
int mlora_transpose_u8(const void* src, int64_t E, int64_t A, int64_t B, int64_t s_e, int64_t s_a, int64_t s_b,
                       void* dst, void* stream);

/* ---------------------------------------------------------------------------------------------
 * fp8 products (an fp8 stack times activations quantised to e4m3 on the block-scaled fp8 MFMA)
 * ------------------------------------------------------------------------------------------- */

/* Activations for the fp8 products, one pass over x (rows, K) bf16: for every row and every 64
 * columns a power-of-two scale 2^e with amax·2^-e <= 448, stored as E8M0 (127 + e) in byte 0 of
 * xs[block * ldxs + row] (int32), and the 64 values e4m3(x·2^-e) rounded to nearest even.  terms = 1:
 * x8[row * ld8 + k] (ld8 >= K rounded up to 64; the columns past K of the last block are zero).
 * terms = 2: also the residual r = x - e4m3 value·2^e (exact in fp32) quantised the same way with its
 * own scale 2^e2 (byte 1 of the xs word): row r's bytes of block b are the first term's 64 at
 * x8[row * ld8 + 128b ..] and the residual's 64 after them (ld8 >= 2 · K rounded up to 64); x is
 * then represented to within 2^-7 of each block's amax instead of 2^-4.  colscale (NULL or per
 * expert colscale[e * cs_se + k]) multiplies the values before quantisation (a per-row stack scale
 * along k).  With at != NULL (A_e^T, as mlora_grouped_gemm's) low = bf16(x · A_e) from the bf16
 * values, fp32 accumulation.  K % 16 == 0.  Replaces the X_FP8 quantisation inside
 * src/meepsquared/_grouped.py:191-194 (per row and BLOCK_K tile, scale amax/448, one term), with the
 * tile 64 and the scale rounded up to a power of two. */
int mlora_fp8_prep(const void* x, int64_t ldx, int64_t rows, int K, int terms, const float* colscale, int64_t cs_se,
                   void* x8, int64_t ld8, int32_t* xs, int64_t ldxs, const void* at, int64_t at_se, int64_t at_sr,
                   int rank, void* low, int64_t ldl, const int32_t* offsets, int E, void* stream);

/* out[row, n] = c · sum_k x̃[row, k] W8_e[n][k] + scaling · low[row,:] · B_e[:, n] + bias[e, n] on
 * v_mfma_scale_f32_32x32x64_f8f6f4, x̃ the activations of mlora_fp8_prep with the same terms (two
 * terms: one MFMA per term, each with its own scale byte); w the fp8 e4m3 stack with k contiguous,
 * W8_e[n][k] = w[e*w_se + n*w_sn + k] (bytes); c = 1, scale[e] or scale[e*scale_se + n]; low
 * (rows, rank) bf16 and bt = B_e^T as in mlora_grouped_gemm, or low = NULL.  Rows past offsets[E-1]
 * untouched.  E <= 4096 (one term) or 3328 (two).  Replaces _grouped_gemm_kernel with X_FP8
 * (src/meepsquared/_grouped.py:120-221). */
int mlora_fp8_gemm(const void* x8, int64_t ld8, const int32_t* xs, int64_t ldxs, int64_t rows, int K, int terms, int N,
                   const void* w, int64_t w_se, int64_t w_sn, const float* scale, int scale_kind, int64_t scale_se,
                   const void* low, int64_t ldli, const void* bt, int64_t bt_se, int64_t bt_sn, int rank,
                   float scaling, const void* bias, int64_t bias_se, void* out, int64_t ldo,
                   const int32_t* offsets, int E, void* stream);

/* ---------------------------------------------------------------------------------------------
 * Frozen stack formats
 * ------------------------------------------------------------------------------------------- */

/* fp8 e4m3 stack with fp32 scales: x (E, R, C) contiguous of x_dtype (bf16/f32).  group =
 * MLORA_SCALE_EXPERT: one scale per expert over its R*C values; MLORA_SCALE_ROW with
 * rows_on_last = 0: one per (e, r) over C values; rows_on_last = 1: one per (e, c) over R values
 * (the stack (E, in, out), whose output rows are its columns).  scale = max(amax, 1e-12) / 448,
 * q = e4m3(x / scale) rounded to nearest even.  Replaces _fp8.py:122-128 (one scale per expert). */
int mlora_fp8_quantize(const void* x, int x_dtype, int64_t E, int64_t R, int64_t C, int group, int rows_on_last,
                       uint8_t* q, float* scale, void* stream);

/* y = fp8 · scale in y_dtype (bf16/f32), the same grouping.  Replaces _fp8.py:131-134. */
int mlora_fp8_dequantize(const uint8_t* q, const float* scale, int64_t E, int64_t R, int64_t C, int group,
                         int rows_on_last, void* y, int y_dtype, void* stream);

/* Scratch bytes mlora_nf4_quantize needs for n values. */
size_t mlora_nf4_workspace_bytes(int64_t n);

/* NF4 with double quantization of x (n values, bf16/f32, n % 64 == 0), blocks of 64: absmax per
 * block; offset = mean of the absmaxes; (absmax - offset) quantised with code2 in blocks of 256
 * (absmax2 = max |absmax - offset| per 256 blocks, absmax_q = nearest code2 index); each value's
 * code = nearest entry of `code` (16 fp32) to x / decoded absmax.  packed (n/2) uint8, absmax_q
 * (n/64) uint8, absmax2 (ceil(n/64/256)) fp32, offset (1) fp32, all on the device. */
int mlora_nf4_quantize(const void* x, int x_dtype, int64_t n, const float* code, const float* code2,
                       uint8_t* packed, uint8_t* absmax_q, float* absmax2, float* offset,
                       void* workspace, size_t workspace_bytes, void* stream);

/* y = code[nibble] · (code2[absmax_q[b]] · absmax2[b/256] + offset[0]) in y_dtype (bf16/f32), the absmax
 * rounded to fp32 after the product and again after the sum (no fused multiply-add). */
int mlora_nf4_dequantize(const uint8_t* packed, const uint8_t* absmax_q, const float* absmax2,
                         const float* offset, const float* code, const float* code2, int64_t n,
                         void* y, int y_dtype, void* stream);

/* An NF4 stack (E, R, C) (blocks of 64 along C, contiguous) read the other way: out_packed (E, C, R/2)
 * holds its transpose's codes two per byte along R (first in the high nibble), out_absmax (E, C/64, R)
 * every block's decoded absmax (code2[q] · absmax2 + offset, two roundings).  The grouped product takes
 * them as MLORA_DT_NF4_KT for the input-gradient pass, where R is k.  R even, C % 64 == 0.  No reference
 * counterpart: the reference has no NF4 stack path. */
int mlora_nf4_transpose(const uint8_t* packed, const uint8_t* absmax_q, const float* absmax2, const float* offset,
                        const float* code2, int64_t E, int64_t R, int64_t C, uint8_t* out_packed, float* out_absmax,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLORA_H */
