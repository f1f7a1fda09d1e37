/*
 * mlops_mi355x.h -- C ABI of the MI355X (gfx950) block-FP8 MoE expert path.
 *
 * One shared library, libmlops_mi355x.so. Every entry point takes raw device
 * pointers, sizes and a hipStream_t (passed as void* so this header needs no
 * HIP include), enqueues its kernels on that stream and returns 0, or a
 * negative code with a message in mi355x_last_error(). No entry point
 * allocates device memory, synchronizes the stream or reads device memory on
 * the host; scratch space, where needed, is a caller-provided workspace whose
 * size the matching *_workspace_size() function returns.
 *
 * Layout conventions (all row-major, contiguous):
 *   bf16      : uint16 storage of bfloat16
 *   e4m3      : uint8 storage of OCP float8_e4m3fn
 *   A         : routed rows = tokens * top_k, in expert-sorted order
 *   offsets   : int32 [E+1], rows of expert e are [offsets[e], offsets[e+1])
 *   1x128 activation scales are stored K-block major: scale[kb][row]
 *   128x128 weight scales: scale[e][out/128][in/128] (DeepSeek layout)
 *
 * The reference (als244/mlops) is pure Python; each entry point below names
 * the reference function whose behaviour it reproduces.
 */
#ifndef MLOPS_MI355X_H
#define MLOPS_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI355X_OK 0
#define MI355X_EINVAL (-1)
#define MI355X_ELAUNCH (-2)

/* Routing modes (reference: src/mlops/kernels/moe_router.py:19, :290). */
#define MI355X_ROUTE_TOPK_THEN_SOFTMAX 0
#define MI355X_ROUTE_SOFTMAX_THEN_TOPK 1
#define MI355X_ROUTE_SIGMOID_NOAUX_TC 2

const char* mi355x_last_error(void);
int mi355x_abi_version(void);

/* ------------------------------------------------------------ router ---- */

/* Top-k selection and route weights from fp32 logits [T,E].
 * Replaces route() / _topk_kernel / route_torch
 * (src/mlops/kernels/moe_router.py:235-344, :106-171, :347-400).
 * Selection is a stable descending sort: ties go to the lower expert id.
 * bias may be NULL (sigmoid mode only). forced_ids (NULL or int32 [T,k])
 * replaces the selection, as routing_override does (moe_router.py:272-289).
 * weights: fp32 [T,k]; ids: int32 [T,k]. */
int mi355x_router_topk(const float* logits, int tokens, int experts, int top_k, int mode,
                       const float* bias, int n_group, int topk_group, float routed_scaling,
                       const int32_t* forced_ids, float* weights, int32_t* ids, void* stream);

/* Routing statistics: aux loss, probability column sums and per-segment
 * counts. Replaces routing_statistics (src/mlops/providers/moe_common.py:32-71).
 * segments == 1 with seg_offsets/chunk_table NULL covers all tokens;
 * otherwise seg_offsets int32 [S+1] and chunk_table int32 [nchunks][2] =
 * (first token, segment) of each chunk of at most 64 tokens of one segment.
 * aux: fp32 [1]; prob_sum: fp32 [E]; seg_counts: int32 [S,E]. */
size_t mi355x_router_stats_workspace_size(int nchunks, int experts);
int mi355x_router_stats(const float* logits, const int32_t* ids, int tokens, int experts,
                        int top_k, int mode, int segments, const int32_t* seg_offsets,
                        const int32_t* chunk_table, int nchunks, float* aux, float* prob_sum,
                        int32_t* seg_counts, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Logit gradient from the per-sorted-row score gradient dscore [A] (gathered
 * to [T,k] through slots), grad_aux [1] and grad_prob_sum [E] (either may be
 * NULL = zero); expert counts are read from offsets [E+1] (permute plan).
 * Replaces routing_gradient + route_backward +
 * add_aux_gradient_ + add_sequence_aux_gradient_
 * (moe_common.py:74-124, moe_router.py:403-502). grad_logits: fp32 [T,E]. */
int mi355x_router_topk_bwd(const float* logits, const float* weights, const int32_t* ids,
                           const float* dscore, const int32_t* slots, int tokens, int experts,
                           int top_k, int mode, const float* grad_aux,
                           const float* grad_prob_sum, const int32_t* offsets, int segments,
                           const int32_t* seg_offsets, const int32_t* seg_counts,
                           float* grad_logits, void* stream);
/* mi355x_router_topk_bwd that also writes the two bf16 pieces of the logit
 * gradient g the router GEMMs consume, pieces bf16 [T, 2E]: row t holds
 * hi = bf16(g[t, :]) then mid = bf16(g[t, :] - hi) (round to nearest even).
 * hi is the input gradient's operand (grad_hidden += hi @ W) and [hi | mid]
 * the weight gradient's (dW = hi^T x + mid^T x); grad_logits may be NULL.
 * Replaces the casts of kernels/router.py:92-113 (and moe_common.py:142). */
int mi355x_router_topk_bwd_split(const float* logits, const float* weights, const int32_t* ids,
                                 const float* dscore, const int32_t* slots, int tokens,
                                 int experts, int top_k, int mode, const float* grad_aux,
                                 const float* grad_prob_sum, const int32_t* offsets,
                                 int segments, const int32_t* seg_offsets,
                                 const int32_t* seg_counts, float* grad_logits, void* pieces,
                                 void* stream);

/* Router weight gradient from those pieces: grad_weight fp32 [E, H] =
 * hi^T x + mid^T x with fp32 sums, x bf16 [T, H], on the bf16 MFMA over
 * token ranges whose partials are summed in range order (deterministic).
 * E a multiple of 8, H a multiple of 256; workspace of
 * mi355x_router_weight_grad_workspace_size bytes. Replaces the two products
 * of router_weight_gradient (kernels/router.py:91-110). */
size_t mi355x_router_weight_grad_workspace_size(int tokens, int experts, int hidden);
int mi355x_router_weight_grad(const void* pieces, const void* x, int tokens, int experts,
                              int hidden, float* grad_weight, void* workspace,
                              size_t workspace_bytes, void* stream);

/* ----------------------------------------------------------- permute ---- */

/* Stable counting sort of the flat expert ids [A] into expert order.
 * Replaces sort_assignments (src/mlops/kernels/moe_dispatch.py:106-119):
 * order = argsort(ids, stable), offsets = [0, cumsum(bincount)],
 * slots[order[i]] = i. counts: int64 [E]. */
size_t mi355x_permute_plan_workspace_size(int assignments, int experts);
int mi355x_permute_plan(const int32_t* ids, int assignments, int experts, int64_t* counts,
                        int32_t* offsets, int32_t* order, int32_t* slots, void* workspace,
                        size_t workspace_bytes, void* stream);

/* Allocation-free variant of mi355x_permute_plan, with the same outputs. It
 * has no counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Its histogram scratch is a fixed 4 MiB file-scope
 * device array, one per GPU, held until the process ends, so it never calls
 * hipMalloc/hipFree. Sizes beyond that scratch (chunks of 1024 assignments x
 * experts above 2^20 - 64 int32) are refused with MI355X_EINVAL;
 * mi355x_permute_plan_noalloc_max_assignments(E) gives the largest A for E.
 * Calls that overlap on one GPU share the scratch and race. */
size_t mi355x_permute_plan_noalloc_max_assignments(int experts);
int mi355x_permute_plan_noalloc(const int32_t* ids, int assignments, int experts, int64_t* counts,
                                int32_t* offsets, int32_t* order, int32_t* slots, void* stream);

/* Dispatch + quantize: token rows x bf16 [T,H] read once, written as e4m3 to
 * each of their k routed rows slots[t,j] with one fp32 descale per 1x128
 * block: s = max(amax * (1/448), 1e-12), q = e4m3(clip(x / s, +-448)).
 * Replaces dispatch + quantize_rows_fp8(gather=...)
 * (moe_dispatch.py:122-124; kernels/quack_moe/quantize_rows.py:34-60,140-207)
 * with 1x128 instead of per-row scales. q: [A,H]; scales: [H/128][A]. */
int mi355x_permute_quantize_fp8(const void* x, int tokens, int width, int top_k,
                                const int32_t* slots, uint8_t* q, float* scales, void* stream);

/* Row quantizer with 1x128 scales for rows already in routed order; with
 * gate_up != 0 an interleaved [gate_0, up_0, ...] row is stored gate columns
 * first (quantize_rows.py:63-111 gate_up=True). q: [rows,width];
 * scales: [width/128][rows]. */
int mi355x_quantize_rows_fp8(const void* x, int rows, int width, int64_t pitch, int gate_up,
                             uint8_t* q, float* scales, void* stream);

/* SwiGLU of the interleaved pre-activation h [rows, 2I], clamped at limit
 * when limit > 0, quantized to e4m3 with 1x128 scales.
 * Replaces swiglu_quantize_rows_fp8 (kernels/quack_moe/swiglu_rows.py:246-258,
 * _swiglu_rows :50-76). q: [rows,I]; scales: [I/128][rows]. act (NULL to
 * skip): the activation itself, bf16 [rows,I], for a consumer that needs it
 * unquantized (the expert-LoRA rank projection, lora/experts.py:162-163). */
int mi355x_swiglu_quantize_fp8(const void* h, int rows, int width, float limit, uint8_t* q,
                               float* scales, void* act, void* stream);

/* 128x128 block quantizer of expert weights [E,out,in] (bf16, or fp32 when
 * is_fp32): s = max(amax / 448, 1e-12) (true division), zero-padded partial
 * blocks. q_t (NULL or [E,in,out]) also receives the transposed e4m3 copy.
 * Replaces quantize_blocks (src/mlops/kernels/block_fp8.py:47-93). */
int mi355x_quantize_weight_blocks(const void* w, int is_fp32, int experts, int out, int in,
                                  uint8_t* q, float* scale, uint8_t* q_t, void* stream);

/* e4m3 [E,rows,cols] -> [E,cols,rows]: the MN-major weight operand of the
 * input-gradient GEMMs. Stands in for the in-shared-memory tile transposer of
 * block_fp8_transposed_gemm (kernels/quack_moe/block_fp8_gemm.py:154-195). */
int mi355x_transpose_fp8(const uint8_t* q, int experts, int rows, int cols, uint8_t* q_t,
                         void* stream);

/* Padded 128-row block table of the weight-gradient layout: each expert's
 * sorted rows start at a 128-aligned padded offset; for padded block pb of
 * padded/128, blocks[2 pb] = its first sorted row and blocks[2 pb + 1] the
 * number of those rows it holds (1..128; 0 past the last expert's blocks).
 * Computed once per routing and read by the kernels that write that layout.
 * No reference counterpart (the reference sizes its transposes per expert on
 * the host, quack_moe/fp8.py:129-157). */
size_t mi355x_wgrad_padded_rows(int assignments, int experts);
int mi355x_padded_row_blocks(const int32_t* offsets, int experts, int padded, int32_t* blocks,
                             void* stream);

/* Feature-major e4m3 operand of the weight-gradient GEMM: routed rows of x
 * (bf16, row pitch `pitch`; with gather != NULL sorted row r reads source row
 * gather[r] / gather_div) are written transposed, [width][padded], each
 * padded block pb holding rows row_blocks[2 pb] .. + row_blocks[2 pb + 1]
 * (mi355x_padded_row_blocks) and zeros after them, with one descale per
 * (feature, 128-row block): max(amax / 448, 1e-12) rounded up to a power of
 * two, so that the weight-gradient GEMM can apply it as an MFMA E8M0 block
 * scale. gate_up de-interleaves columns as in mi355x_quantize_rows_fp8.
 * Replaces quantize_transpose_fp8 (kernels/quack_moe/quantize_transpose.py
 * :126-313) with per-128-token power-of-two instead of per-expert fp32
 * scales. scales: [padded/128][width]. */
int mi355x_quantize_transpose_fp8(const void* x, int64_t pitch, int width, const int32_t* gather,
                                  int gather_div, int gate_up, const int32_t* row_blocks,
                                  int padded, uint8_t* qt, float* scales, void* stream);

/* out[t] = bf16(residual[t] + sum_j weights[t,j] * y[slots[t,j]]), fp32 sum in
 * j order. Replaces combine (moe_dispatch.py:21-72, :168-196). */
int mi355x_unpermute_combine(const void* y, const int32_t* slots, const float* weights,
                             const void* residual, int tokens, int top_k, int width, void* out,
                             void* stream);

/* out[t] = bf16(sum_j dx[slots[t,j]]). Replaces dispatch_backward
 * (moe_dispatch.py:136-165). */
int mi355x_unpermute_sum(const void* dx, const int32_t* slots, int tokens, int top_k,
                         int width, void* out, void* stream);

/* Routed SwiGLU backward over sorted rows: from r = dy @ W2 [A,I] (bf16),
 * h [A,2I] interleaved and the route score of each sorted row
 * (weights[order[row]]): dscore = <r, act> (fp32), dh = dSwiGLU(score * r)
 * interleaved (bf16), a' = score * act (bf16; not written when a_prime is
 * null). dh may be h itself (written in place). Replaces
 * routed_swiglu_rows_backward
 * (kernels/quack_moe/swiglu_rows.py:101-146, :278-318). */
int mi355x_routed_swiglu_bwd(const void* r, const void* h, const float* weights,
                             const int32_t* order, int rows, int width, float limit, void* dh,
                             void* a_prime, float* dscore, void* stream);

/* mi355x_routed_swiglu_bwd that also row-quantizes dh, gate-first, from its
 * bf16 values: dhq e4m3 [A, 2I] and dh_scales [2I/128][A], equal to
 * mi355x_quantize_rows_fp8 (gate_up = 1) on the dh it writes, without reading
 * dh back (expert LoRA needs the bf16 dh too, for its rank products). I must
 * be a multiple of 128. Replaces routed_swiglu_rows_backward followed by
 * quantize_rows_fp8(gate_up=True) (kernels/quack_moe/swiglu_rows.py:278-318;
 * quantize_rows.py:140). */
int mi355x_routed_swiglu_bwd_rows_fp8(const void* r, const void* h, const float* weights,
                                      const int32_t* order, int rows, int width, float limit,
                                      void* dh, void* a_prime, float* dscore, uint8_t* dhq,
                                      float* dh_scales, void* stream);

/* Fused routed SwiGLU backward and the quantizers its outputs feed, from
 * r = dy @ W2 [rows, I] (bf16), h [rows, 2I] interleaved and the route score
 * of each sorted row (weights[order[row]]), with dh and a' rounded to bf16 as
 * mi355x_routed_swiglu_bwd stores them:
 *   dhq, dh_scales: dh row-quantized gate-first, as mi355x_quantize_rows_fp8
 *                   (gate_up = 1) would from that dh;
 *   dh_t, dh_t_scales / ap_t, ap_t_scales: dh (gate-first) and a' in the
 *                   weight-gradient layout of mi355x_quantize_transpose_fp8
 *                   (each may be NULL, with its scales, to skip it);
 *   dscore[rows]:   <r, act> per sorted row (fp32, summed per 128 columns in
 *                   a fixed order).
 * workspace: mi355x_swiglu_bwd_quantize_workspace_size(rows, I) bytes. Replaces
 * the dSwiGLU epilogue of block_fp8_gemm's dgrad-down (kernels/quack_moe/
 * block_fp8_gemm.py:1215-1258, :1520) with the row quantizer of
 * quantize_rows.py:140 and the transposing quantizer of quantize_transpose.py
 * :126 fused behind it: one read of r and h instead of four passes. */
size_t mi355x_swiglu_bwd_quantize_workspace_size(int rows, int width);
int mi355x_swiglu_bwd_quantize(const void* r, const void* h, const float* weights,
                               const int32_t* order, const int32_t* row_blocks, int rows,
                               int width, int padded, float limit, uint8_t* dhq,
                               float* dh_scales, uint8_t* dh_t, float* dh_t_scales,
                               uint8_t* ap_t, float* ap_t_scales, float* dscore,
                               void* workspace, size_t workspace_bytes, void* stream);

/* mi355x_swiglu_bwd_quantize with bf16 dh [rows, 2I] in h's interleaved
 * order (2j = gate j, 2j + 1 = up j) in place of dhq / dh_scales, the
 * values mi355x_routed_swiglu_bwd writes; dh_t / ap_t and dscore as there.
 * The fp8_current backward needs dh in bf16 for its per-row quantizer
 * (quantize_rows.py:35-207) and the transposed operands for the weight
 * gradients (sonicmoe/moe.py:346-358, 408-419); this is one read of r and h
 * for all three instead of the SwiGLU backward plus two transposing passes. */
int mi355x_swiglu_bwd_bf16(const void* r, const void* h, const float* weights,
                           const int32_t* order, const int32_t* row_blocks, int rows, int width,
                           int padded, float limit, void* dh, uint8_t* dh_t, float* dh_t_scales,
                           uint8_t* ap_t, float* ap_t_scales, float* dscore, void* workspace,
                           size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------- GEMMs ---- */

/* Ragged grouped block-FP8 GEMM, fp8 MFMA with fp32 accumulation:
 *   out[r, n] = sum_kb (sum_{k in kb} a[r,k] * W[e][n,k]) * a_scale[kb][r] * ws
 * for rows r of expert e, ws the weight block's scale, plus addend when
 * given. w is e4m3 [E,N,K]. w_scale_t == 0: w_scale is [E,N/128,K/128] (a
 * projection, y = x @ W^T); w_scale_t == 1: w is the transposed copy of a
 * weight [E,K,N] and w_scale is that weight's [E,K/128,N/128] (an input
 * gradient, dx = dy @ W). interleave != 0 writes output column n < N/2 to 2n
 * and n >= N/2 to 2(n-N/2)+1 (gate/up interleaved h). out, addend: bf16 [M,N].
 * Replaces grouped_block_gemm / block_fp8_gemm / block_fp8_transposed_gemm
 * (src/mlops/kernels/block_fp8.py:120-336; kernels/quack_moe/block_fp8_gemm.py
 * :1424-1482). */
int mi355x_gemm_fp8_block(const uint8_t* a, const float* a_scale, int rows, const uint8_t* w,
                          const float* w_scale, int w_scale_t, int experts, int n, int k,
                          const int32_t* offsets, int interleave, const void* addend, void* out,
                          void* stream);
/* The input-gradient GEMM on the weight as stored, without a transposed
 * copy: w is e4m3 [E,K,N] with its own block scales w_scale [E,K/128,N/128]
 * (for dx = dh @ W13: W13 [E,2I,H]; for r = dy @ W2: W2 [E,H,I]), out bf16
 * [rows,N]; N a multiple of 256, K of 128. Bitwise equal to
 * mi355x_gemm_fp8_block with w_scale_t = 1 on the transposed copy. The
 * weight tile is copied K-major and its MFMA operand gathered with gfx950's
 * transposing LDS read (ds_read_b64_tr_b8). Replaces
 * block_fp8_transposed_gemm (kernels/quack_moe/block_fp8_gemm.py:1424, which
 * reads the weight MN-major as well). */
int mi355x_gemm_fp8_block_kmajor(const uint8_t* a, const float* a_scale, int rows,
                                 const uint8_t* w, const float* w_scale, int experts, int n, int k,
                                 const int32_t* offsets, void* out, void* stream);

/* mi355x_gemm_fp8_block / mi355x_gemm_fp8_block_kmajor whose GEMM row r
 * (expert-sorted rows, offsets) is row a_rows[r] of a [a_total, K] e4m3 with
 * 1x128 scales a_scale [a_total][K/128] (token-major, as
 * mi355x_quantize_token_rows_fp8 writes them): the activation (x forward, dy for
 * r = dy @ W2) quantized once per token and read by each of its k routed
 * rows, instead of a permuted copy of k rows per token. Routed row r reads
 * token a_rows[r] / a_rows_div: a_rows int32 [rows] is the plan's sorted
 * slot order with a_rows_div = top_k (no token-id pass), or token ids with
 * a_rows_div = 1; every token in [0, a_total), a_total * a_rows_div < 2^31:
 * the kernel reads the rows they name unchecked, as it reads offsets. N a multiple of
 * 256; no addend. Bitwise
 * equal to the routed-row forms on mi355x_permute_quantize_fp8's copy.
 * Replaces permute_quantize_rows followed by block_fp8_gemm /
 * block_fp8_transposed_gemm (kernels/quack_moe/quantize_rows.py:35,
 * block_fp8_gemm.py:1458 and :1424; the reference's GEMM takes no gather,
 * block_fp8_gemm.py:392). */
/* Token rows quantized for the gathered GEMMs: x bf16 [rows, width] ->
 * e4m3 q [rows, width] with 1x128 scales [rows][width/128] (row-major: a
 * row's scales together), the same values as mi355x_quantize_rows_fp8. */
int mi355x_quantize_token_rows_fp8(const void* x, int rows, int width, uint8_t* q, float* scales,
                                   void* stream);
int mi355x_gemm_fp8_block_gathered(const uint8_t* a, const float* a_scale, int a_total,
                                   const int32_t* a_rows, int a_rows_div, int rows, const uint8_t* w,
                                   const float* w_scale, int experts, int n, int k,
                                   const int32_t* offsets, int interleave, void* out,
                                   void* stream);
int mi355x_gemm_fp8_block_kmajor_gathered(const uint8_t* a, const float* a_scale, int a_total,
                                          const int32_t* a_rows, int a_rows_div, int rows, const uint8_t* w,
                                          const float* w_scale, int experts, int n, int k,
                                          const int32_t* offsets, void* out, void* stream);

/* mi355x_gemm_fp8_block with a rank-r term in place of the addend:
 *   out[r, n] = (block-FP8 product as above) + sum_j lora_z[r, j] * lora_b[e][n', j]
 * for rows r of expert e, where n' is the weight row feeding output column n
 * (the same row the product reads: n itself, or in gate/up mode the
 * gate-first row of the interleaved column). The rank term is a bf16 MFMA
 * with fp32 sums that initialises the accumulators, so no [rows, N] addend
 * is materialized. lora_z: bf16 [rows, R]; lora_b: bf16 [E, N, R]; R (the
 * rank padded with zero columns) a multiple of 16 up to 256. N must be a
 * multiple of 256. Replaces the LoRA C input of the expert-LoRA up and down
 * GEMMs and the in-place LoRA branch of their row gradients
 * (providers/sonicmoe/lora.py:1-45, _up_forward :189, _down_forward :540;
 * block_fp8_gemm(c=) at kernels/quack_moe/block_fp8_gemm.py:1458). */
int mi355x_gemm_fp8_block_lora(const uint8_t* a, const float* a_scale, int rows, const uint8_t* w,
                               const float* w_scale, int w_scale_t, int experts, int n, int k,
                               const int32_t* offsets, int interleave, const void* lora_z,
                               const void* lora_b, int lora_rank, void* out, void* stream);

/* ---- "fp8_current": one e4m3 descale per operand row (current scaling) ----
 * Row-scaled grouped GEMM: out[r, n] = bf16((acc * a_scale[r]) * w_scale[e, n])
 * with acc = sum_k e4m3(a[r, k]) e4m3(w[e][n, k]) in fp32, for the rows r of
 * expert e. a: e4m3 [rows, K], a_scale fp32 [rows]; w: e4m3 [E, N, K]
 * (the weight's rows, or its transposed copy for an input gradient), w_scale
 * fp32 [E, N]. N a multiple of 256, K of 128. Replaces the scale-aware
 * epilogue GEMMs of the fp8_current path (kernels/quack_moe/fp8.py;
 * providers/sonicmoe/fp8.py:226-247 _project_down, :330-357
 * input_gradient_rows, the products of :205-224 up_projection and :271-309
 * down_backward_activations). */
/* mi355x_gemm_fp8_rowwise whose row r is row a_rows[r] of per-token e4m3
 * a [a_total, K] with descales a_scale [a_total] (the fp8_current activation
 * quantized once per token; see mi355x_gemm_fp8_block_gathered). Bitwise
 * equal to the routed-row form on mi355x_permute_quantize_current_fp8's copy. */
int mi355x_gemm_fp8_rowwise_gathered(const uint8_t* a, const float* a_scale, int a_total,
                                     const int32_t* a_rows, int a_rows_div, int rows, const uint8_t* w,
                                     const float* w_scale, int experts, int n, int k,
                                     const int32_t* offsets, void* out, void* stream);
int mi355x_gemm_fp8_rowwise(const uint8_t* a, const float* a_scale, int rows, const uint8_t* w,
                            const float* w_scale, int experts, int n, int k,
                            const int32_t* offsets, void* out, void* stream);

/* mi355x_gemm_fp8_rowwise with a rank-r term: out[r, n] = (row-scaled product)
 * + sum_j lora_z[r, j] lora_b[e][n, j], the rank term a bf16 MFMA that starts
 * the accumulators (divided by the row and column descales the epilogue
 * applies). lora_z bf16 [rows, R], lora_b bf16 [E, N, R] in the weight's
 * stored row order, R a multiple of 16 in [16, 256]. Replaces the LoRA C
 * input of the fp8_current expert-LoRA GEMMs (providers/sonicmoe/lora.py
 * :189-262, :540-600 through fp8.py's scale-aware epilogues). */
int mi355x_gemm_fp8_rowwise_lora(const uint8_t* a, const float* a_scale, int rows,
                                 const uint8_t* w, const float* w_scale, int experts, int n, int k,
                                 const int32_t* offsets, const void* lora_z, const void* lora_b,
                                 int lora_rank, void* out, void* stream);

/* Per-row e4m3 quantizer: q[r] = e4m3(clip(x[src] / s, +-448)), scales[r] =
 * s = max(amax(x[src]) * (1/448), 1e-12), src = gather[r] / gather_div (a
 * routed row's token) or r. x bf16 rows of the given pitch. Replaces
 * quantize_rows_fp8 (kernels/quack_moe/quantize_rows.py:140-207). */
int mi355x_quantize_rows_current_fp8(const void* x, int rows, int width, int64_t pitch,
                                     const int32_t* gather, int gather_div, uint8_t* q,
                                     float* scales, void* stream);

/* The per-row quantizer above for the routed copies of token rows: row t of
 * x [tokens, width] (bf16) quantized once and stored, with its scale, at
 * each of its sorted slots slots[t, 0..top_k). Equals
 * mi355x_quantize_rows_current_fp8 over the gathered rows (gather = order,
 * gather_div = top_k). Replaces quantize_rows_fp8(..., gather=)
 * (kernels/quack_moe/quantize_rows.py:140-207) as the fp8_current path calls
 * it (providers/sonicmoe/fp8.py:214, :295). */
int mi355x_permute_quantize_current_fp8(const void* x, int tokens, int width, int top_k,
                                        const int32_t* slots, uint8_t* q, float* scales,
                                        void* stream);

/* SwiGLU of interleaved h [rows, 2I] (gate from above and up on both sides
 * clamped at limit when limit > 0), quantized per row as above: q [rows, I],
 * scales [rows]; act (bf16 [rows, I]) receives the activation too when not
 * null. Replaces swiglu_quantize_rows_fp8
 * (kernels/quack_moe/swiglu_rows.py:246-276). */
int mi355x_swiglu_quantize_rows_current_fp8(const void* h, int rows, int width, float limit,
                                            uint8_t* q, float* scales, void* act, void* stream);

/* Both orientations of expert weights w [E, out, in] (bf16, or fp32 when
 * is_fp32): q [E, out, in] with scales [E, out] (per row), qt [E, in, out]
 * with scales_t [E, in] (per column of w), each as the per-row quantizer
 * above; with interleave the out rows of both are stored gate/up-adjacent
 * (stored 2j = gate row j, 2j + 1 = up row j). in a multiple of 8, out of 16.
 * Replaces quantize_weights_fp8 (kernels/quack_moe/quantize_transpose.py
 * :316-339) behind QuackFP8Weight.quantize
 * (expert_parallel/quack/parameters/fp8.py:36-54, 111-121). */
int mi355x_quantize_weights_current_fp8(const void* w, int is_fp32, int experts, int out, int in,
                                        int interleave, uint8_t* q, float* scales, uint8_t* qt,
                                        float* scales_t, void* workspace, size_t workspace_bytes,
                                        void* stream);
/* Bytes of device workspace mi355x_quantize_weights_current_fp8 needs (the
 * row and column maxima of each 128 x 128 tile, and the reciprocals of both
 * scale vectors). */
size_t mi355x_quantize_weights_current_workspace_size(int experts, int out, int in);

/* Thin grouped product of expert LoRA: out[r, 0:R] = sum_k a[r, k] *
 * bt[e][0:R, k] for the rows r of expert e (offsets[E+1]), a bf16 [rows, K],
 * bt bf16 [E, R, K], out bf16 [rows, R], fp32 sums; K a multiple of 32, R a
 * multiple of 16 up to 64. Replaces the rank projections of expert LoRA that
 * stream routed rows (lora/grouped.py grouped_linear of lora/experts.py:47,
 * :49; sonicmoe/lora.py _low :87, _through :98). */
int mi355x_rank_product(const void* a, int rows, int k, const void* bt, int rank,
                        const int32_t* offsets, int experts, void* out, void* stream);
/* mi355x_rank_product with its K range split over `splits` blocks per 32-row
 * block (K a multiple of 128, splits <= K / 128), for few rows: each split
 * writes fp32 partial sums to the workspace
 * (mi355x_rank_product_workspace_size(rows, R, splits) bytes) and a second
 * pass adds them in split order and rounds once to bf16. splits = 1 is
 * mi355x_rank_product. */
size_t mi355x_rank_product_workspace_size(int rows, int rank, int splits);
int mi355x_rank_product_split(const void* a, int rows, int k, const void* bt, int rank,
                              const int32_t* offsets, int experts, int splits, void* out,
                              void* workspace, size_t workspace_bytes, void* stream);

/* Expert LoRA factor gradients as grouped reductions over routed rows:
 * out[e][m][n] = sum over expert e's rows j of big[j][m] * small[j][n], fp32
 * sums, with big bf16 [rows, M] (M a multiple of 8), small bf16 [rows, R] (R a
 * multiple of 16 up to 64), offsets int32 [E+1], out fp32 [E, M, R] (or
 * [E, R, M] with transposed = 1). Rows are taken in chunks of `chunk` rows of
 * one expert; workspace: mi355x_rank_grad_workspace_size(rows, E, M, R,
 * chunk) bytes. No host synchronization. Replaces the per-expert loops of the
 * factor gradients dB13 = s * sum dh z13^T and dA2 = sum u2 a'^T
 * (src/mlops/lora/experts.py:53-167; providers/sonicmoe/lora.py:1062). */
size_t mi355x_rank_grad_workspace_size(int rows, int experts, int m, int rank, int chunk);
int mi355x_rank_grad(const void* big, int rows, int m, const void* small, int rank,
                     const int32_t* offsets, int experts, int chunk, int transposed, float* out,
                     void* workspace, size_t workspace_bytes, void* stream);
/* mi355x_rank_grad with token rows and a row weight: row j of big is
 * big[gather[j] / gather_div] (big bf16 [big_rows, M]; the routed row's token
 * when gather is the routed order and gather_div = k; gather null: row j,
 * big_rows = rows), and, when weight is given, row j of small is
 * bf16(small[j] * (weight[weight_index[j]] * alpha)) (weight_index null:
 * weight[j]). The factor gradients dB2 = s * sum (score dy) z2^T,
 * dA13 = sum u13 x^T and dA2 = sum (score u2) a^T as reductions over each
 * expert's routed rows (src/mlops/lora/experts.py:53-167;
 * providers/sonicmoe/lora.py:1062). Workspace as for mi355x_rank_grad with
 * `rows` routed rows. */
int mi355x_rank_grad_gather(const void* big, int big_rows, int m, const void* small, int rows,
                            int rank, const int32_t* offsets, int experts, int chunk,
                            const int32_t* gather, int gather_div, const float* weight,
                            const int32_t* weight_index, float alpha, int transposed, float* out,
                            void* workspace, size_t workspace_bytes, void* stream);

/* The up projection with SwiGLU fused: mi355x_gemm_fp8_block in gate/up mode
 * (w13 [E, 2I, K], interleave = 1) writing h [rows, 2I] bf16 interleaved, and
 * from the same bf16 values act = silu(min(g, L)) * clamp(u, +-L) (limit <=
 * 0: no clamp), row-quantized 1x128 into act_q [rows, I] e4m3 with
 * act_scales [I/128][rows], bit-identical to mi355x_swiglu_quantize_fp8 on h.
 * 2I must be a multiple of 256. Replaces the SwiGLU epilogue of the up GEMM
 * (kernels/quack_moe/block_fp8_gemm.py:1196, :1484) with the row quantizer
 * of swiglu_rows.py:246 behind it. */
int mi355x_gemm_fp8_block_swiglu(const uint8_t* a, const float* a_scale, int rows,
                                 const uint8_t* w, const float* w_scale, int experts, int n,
                                 int k, const int32_t* offsets, const void* addend, float limit,
                                 void* h, uint8_t* act_q, float* act_scales, void* stream);

/* Grouped weight-gradient GEMM over feature-major e4m3 operands of the same
 * padded layout (see mi355x_quantize_transpose_fp8):
 *   out[e][m][n] = sum_{rows of e} p[m][row] q[n][row], block-scaled,
 * fp32 accumulation, written as bf16 (out_fp32 == 0) or fp32. p_scale
 * [padded/128][m_features], q_scale [padded/128][n_features]: powers of two
 * (as written by mi355x_quantize_transpose_fp8; other values are truncated to
 * their power-of-two exponent when both feature counts are multiples of 256,
 * where the MFMA applies the scales in hardware). Experts with no
 * rows get zeros. Replaces the varlen-K wgrad GEMMs
 * (providers/sonicmoe/moe.py:351-365, :404-419; quack_moe/wgrad.py:30). */
int mi355x_gemm_fp8_block_wgrad(const uint8_t* p, const float* p_scale, int m_features,
                                const uint8_t* q, const float* q_scale, int n_features,
                                int padded, const int32_t* offsets, int experts, void* out,
                                int out_fp32, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MLOPS_MI355X_H */
