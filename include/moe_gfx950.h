/* C ABI of libmoe_gfx950.so — the gfx950 (MI355X) MoE expert pipeline.
 *
 * Every entry point takes plain device pointers, element counts and a hipStream_t passed as
 * `void* stream` (NULL = the default stream). Nothing here allocates: the caller owns every
 * buffer, including the dispatch workspace. Calls are stream-ordered and asynchronous; none of
 * them synchronises with the host. Each returns MOE_OK or one of the MOE_ERR_* codes below; a
 * failed call launches nothing.
 *
 * Shapes (reference layout, /root/reference/kernels/sm75/moe.py:65-68):
 *   hidden         (N, H)        row-major, dtype = the model dtype
 *   top_k_indices  (N, k)        int64 expert ids
 *   top_k_weights  (N, k)        model dtype
 *   gate_up_proj   (E_glu, 2I, H) rows [0, I) = gate, rows [I, 2I) = up
 *   down_proj      (E_glu, H, I)
 *   act_codes      (E,) int32    E = E_glu + number of weightless special experts
 * M = N*k routed rows. "Sorted" rows are ordered by (expert id, flat index t*k+j): stable.
 */
#ifndef MOE_GFX950_H
#define MOE_GFX950_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOE_OK 0
#define MOE_ERR_SHAPE 1     /* a size is out of range or inconsistent */
#define MOE_ERR_ALIGN 2     /* a pointer or row length breaks the 16-byte rule */
#define MOE_ERR_CODE 3      /* an activation code the entry point does not implement */
#define MOE_ERR_DTYPE 4     /* unknown dtype code */
#define MOE_ERR_LAUNCH 5    /* the HIP launch itself failed */
#define MOE_ERR_WORKSPACE 6 /* workspace missing or too small */

#define MOE_DT_F32 0
#define MOE_DT_F16 1
#define MOE_DT_BF16 2

/* Library version string. */
const char* moe_version(void);

/* Rows per token tile of the grouped GEMMs; tile_offsets below count tiles of this height. */
int moe_tile_rows(void);

/* Bytes of device workspace moe_dispatch needs. */
size_t moe_get_workspace_size(int64_t n_tokens, int top_k, int n_experts);

/* Dispatch: histogram, prefix scan and stable permutation of the routed rows.
 * Replaces `_sort_by_expert` (kernels/sm75/moe.py:564-572), `_build_schedule` (:535-543) and the
 * sort / bincount / cumsum of kernels/sm120/moe_grouped.py:94-100, with no host sync.
 * Outputs: counts[E], offsets[E+1] (exclusive prefix of counts), tile_offsets[E+1] (exclusive
 * prefix of ceil(counts/moe_tile_rows())), expert_order[E] (expert ids by descending count, ties
 * by id), sorted_token[M] (token id t of each sorted row),
 * sorted_flat[M] (flat index t*k+j of each sorted row), flat_to_sorted[M] (inverse permutation;
 * -1 for an index outside [0, E)), status[0] += number of such out-of-range indices. Such indices
 * are dropped, so only offsets[E] <= M rows are routed: sorted_token and sorted_flat hold -1 at
 * positions [offsets[E], M). */
int moe_dispatch(const int64_t* top_k_indices, int64_t n_tokens, int top_k, int n_experts,
                 int32_t* counts, int32_t* offsets, int32_t* tile_offsets, int32_t* expert_order,
                 int32_t* sorted_token, int32_t* sorted_flat, int32_t* flat_to_sorted,
                 int32_t* status, void* workspace, size_t workspace_bytes, void* stream);

/* Allocation-free moe_dispatch: no counterpart in the reference. For callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops): same arguments,
 * outputs and results as moe_dispatch, minus the workspace, which is a 4 MiB file-scope device
 * array per GPU instead (held until the process ends). Limit: ceil(N*k / 1024) * E <= 2^20
 * (moe_get_workspace_size(...) <= 4 MiB; e.g. E = 64: N*k <= 16M rows), else MOE_ERR_WORKSPACE
 * and nothing is launched. Every call on one GPU shares that array: calls that overlap on one GPU
 * (different streams without ordering) race. Nothing in the array needs clearing between calls. */
int moe_dispatch_noalloc(const int64_t* top_k_indices, int64_t n_tokens, int top_k, int n_experts,
                         int32_t* counts, int32_t* offsets, int32_t* tile_offsets,
                         int32_t* expert_order, int32_t* sorted_token, int32_t* sorted_flat,
                         int32_t* flat_to_sorted, int32_t* status, void* stream);

/* Grouped gate/up projection with the GLU epilogue.
 * gate_up[m] = hidden[sorted_token[m]] @ gate_up_proj[e]^T for every sorted row m of a GLU expert
 * e < E_glu; inter[m, i] = act_e(gate) * up (act code 0 = SiLU, 1 = ReLU^2; the two codes the
 * epilogue fuses). inter_out may be NULL: then only gate_up is written (any act code).
 * top_k_weights non-NULL (model dtype; 16-bit dtypes, H % 64 == 0, inter_out given): inter is the
 * gate-weighted w * act(gate) * up with w = top_k_weights[sorted_flat[m]], or top_k_weights[m]
 * when sorted_flat is NULL (gates already in sorted-row order), so the down projection yields
 * w * eo and moe_combine_fwd with glu_rows_weighted = 1 only sums. NULL: unweighted.
 * Replaces `_grouped_mm` + `_glu_fwd` (kernels/sm75/moe.py:590-591), torch._grouped_mm +
 * BatchedGLU (kernels/sm120/moe_grouped.py:106-107) and the per-expert `@` + `_glu_fwd`
 * (kernels/sm75/moe.py:765-769). */
int moe_grouped_gateup_swiglu_fwd(int dtype, const void* hidden, int64_t n_tokens, int64_t H,
                                  const void* gate_up_proj, int E_glu, int64_t I,
                                  const int32_t* act_codes, const int32_t* offsets,
                                  const int32_t* tile_offsets, const int32_t* sorted_token,
                                  int64_t n_rows, void* gate_up_out, void* inter_out,
                                  const void* top_k_weights, const int32_t* sorted_flat,
                                  void* stream);

/* Grouped down projection: eo[m] = inter[m] @ down_proj[e]^T.
 * Replaces `_grouped_mm(inter, down_proj, ...)` (kernels/sm75/moe.py:592), the per-expert
 * `it @ down_proj[e].t()` (:770) and torch._grouped_mm (kernels/sm120/moe_grouped.py:108). */
int moe_grouped_down_fwd(int dtype, const void* inter, const void* down_proj, int E_glu, int64_t H,
                         int64_t I, const int32_t* offsets, const int32_t* tile_offsets,
                         int64_t n_rows, void* eo_out, void* workspace, size_t workspace_bytes,
                         void* stream);

/* Optional workspace of moe_grouped_down_fwd and moe_grouped_gateup_dx (no counterpart in the
 * reference): bytes for the current device, 256-byte aligned, zero-filled once by the caller and
 * left zero by every call; calls that share one workspace must be stream-ordered. With it, 16-bit
 * GEMMs whose K spans at least 40 steps of 64 cut each XCD's last partial wave of tiles along K
 * (partial tiles summed in a fixed order: results do not depend on timing). NULL: no split. */
size_t moe_token_split_workspace_size(void);

/* Gate-weighted combine: out[t] = sum_j w[t,j] * row(t,j), fp32 accumulation in slot order, where
 * row = eo[flat_to_sorted[t*k+j]] for GLU experts, hidden[t] for Identity (code 3), nothing for
 * Zero (code 4); experts e >= E_glu are the weightless specials, n_experts = len(act_codes).
 * glu_rows_weighted = 1: the GLU rows of eo already carry their gate (weight 1 here).
 * Replaces `_combine_scatter` (kernels/sm75/moe.py:673-682,704-709), the grouped
 * index_add_ (:593-595) and kernels/sm120/moe_grouped.py:110-121. Deterministic (no atomics). */
int moe_combine_fwd(int dtype, const void* eo, const void* hidden, const void* top_k_weights,
                    const int64_t* top_k_indices, const int32_t* act_codes, int n_experts, int E_glu,
                    const int32_t* flat_to_sorted, int64_t n_tokens, int top_k, int64_t H,
                    int glu_rows_weighted, void* out, void* stream);

/* Combine backward: grad_eo[m] = grad_out[t] * w (GLU rows), grad_wt[flat] = sum_h grad_out[t,h] *
 * row[h] (fp32 reduction; row = eo[m] for GLU, hidden[t] for Identity, 0 for Zero).
 * grad_out rows are `grad_out_ld` elements apart. Sorted rows with sorted_flat = -1 (past the
 * routed count) are skipped; grad_wt entries of dropped slots are left as the caller set them.
 * Replaces `_combine_bwd`
 * (kernels/sm75/moe.py:688-701,712-720) and the grouped bwd prologue (:606-608,616-617). */
int moe_combine_bwd(int dtype, const void* grad_out, int64_t grad_out_ld, const void* eo,
                    const void* hidden, const void* top_k_weights, const int64_t* top_k_indices,
                    const int32_t* act_codes, int n_experts, int E_glu, const int32_t* sorted_token,
                    const int32_t* sorted_flat, int64_t n_rows, int top_k, int64_t H,
                    void* grad_eo_out, void* grad_wt_out, void* stream);

/* Down-projection dX with the GLU-backward epilogue:
 * grad_inter[m] = grad_eo[m] @ down_proj[e]; ggu[m] = [d gate, d up] of act_e(gate)*up.
 * grad_inter_out may be NULL; when it is given (any act code) grad_inter is written and ggu_out
 * may be NULL. Replaces `_grouped_mm(..., trans_w=True)` + `_glu_bwd` (kernels/sm75/moe.py:609-611)
 * and the per-expert `ge @ down_proj[e]` + `_glu_bwd` (:807,817-819). */
int moe_grouped_down_dx_swiglu_bwd(int dtype, const void* grad_eo, const void* down_proj, int E_glu,
                                   int64_t H, int64_t I, const void* gate_up,
                                   const int32_t* act_codes, const int32_t* offsets,
                                   const int32_t* tile_offsets, int64_t n_rows, void* ggu_out,
                                   void* grad_inter_out, void* stream);

/* Gate/up dX: grad_x_s[m] = ggu[m] @ gate_up_proj[e]. Replaces `_grouped_mm(grad_gate_up,
 * gate_up_proj, ..., trans_w=True)` (kernels/sm75/moe.py:612) and `grad_gate_up @
 * gate_up_proj[e]` (:822). */
int moe_grouped_gateup_dx(int dtype, const void* ggu, const void* gate_up_proj, int E_glu, int64_t H,
                          int64_t I, const int32_t* offsets, const int32_t* tile_offsets,
                          int64_t n_rows, void* grad_xs_out, void* workspace,
                          size_t workspace_bytes, void* stream);

/* Grouped weight gradient over each expert's ragged row range [offsets[e], offsets[e+1]):
 *   out[e, c, r] = sum_m  rsrc[rrow(m), r] * csrc[crow(m), c]
 * rrow(m) = r_gather ? r_gather[m] : m (same for c). Rows of rsrc are r_ld elements apart, rows of
 * csrc c_ld apart. out is (E_glu, C, R) contiguous; experts with no rows get zeros.
 * expert_order (optional, from moe_dispatch, n_experts entries) lists the experts by descending
 * row count so the longest reductions are scheduled first; entries >= E_glu are skipped.
 * down:    out = grad_down_proj (E,H,I): rsrc = inter (R=I), csrc = grad_eo (C=H).
 * gate_up: out = grad_gate_up_proj (E,2I,H): rsrc = hidden gathered by sorted_token (R=H),
 *          csrc = ggu (C=2I).
 * workspace (optional, moe_token_split_workspace_size() bytes, 256-byte aligned, zero-filled
 * once; the same workspace as the token GEMMs'): when the experts' output tiles fill at most half
 * of the CUs, each tile's row range is split into pieces whose fp32 partials meet there and are
 * summed in a fixed order (deterministic); the workspace is left zero. NULL: no split. Calls that
 * share a workspace must be stream-ordered.
 * Replaces `_grouped_wgrad` (kernels/sm75/moe.py:507-532,556-561) and the per-expert
 * `ge.t() @ it`, `grad_gate_up.t() @ x_s[s:en]` (:808,821). */
int moe_grouped_wgrad(int dtype, const void* rsrc, int64_t r_ld, const int32_t* r_gather,
                      const void* csrc, int64_t c_ld, const int32_t* c_gather, int64_t R, int64_t C,
                      const int32_t* offsets, const int32_t* expert_order, int n_experts, int E_glu,
                      void* out, void* workspace, size_t workspace_bytes, void* stream);

/* Down-projection dX for fused codes (0 SiLU, 1 ReLU^2) with the combine backward folded in.
 * For sorted row m of GLU expert e, token t = sorted_token[m], w = top_k_weights[sorted_flat[m]]
 * (sorted_flat NULL: top_k_weights is already in sorted-row order, w = top_k_weights[m]):
 * s = grad_out[t] @ down_proj[e] (grad_out rows gathered, grad_out_ld elements apart);
 * ggu_out[m] = GLU backward of w*s; inter_w_out[m] = w * act(gate)*up (the down weight gradient's
 * row operand, so grad_eo = w*grad_out is never materialised; may be NULL when the forward kept
 * the gate-weighted intermediate); wt_partial[p*n_rows + m] = the
 * partial dot sum over channel slice p of s*inter, p < moe_gate_grad_parts(I).
 * Replaces moe_combine_bwd + moe_grouped_down_dx_swiglu_bwd for these codes: grad_eo = w*go and
 * grad_w = <go, eo> = <go @ W_d, inter> (kernels/sm75/moe.py:606-611,712-720). H % 64 == 0,
 * dtype bf16 or f16. */
int moe_grouped_down_dx_gated_bwd(int dtype, const void* grad_out, int64_t grad_out_ld,
                                  const void* down_proj, int E_glu, int64_t H, int64_t I,
                                  const void* gate_up, const int32_t* act_codes,
                                  const void* top_k_weights, const int32_t* offsets,
                                  const int32_t* sorted_token, const int32_t* sorted_flat,
                                  int64_t n_rows, void* ggu_out, void* inter_w_out,
                                  float* wt_partial, void* stream);

/* Number of channel slices (rows of wt_partial) moe_grouped_down_dx_gated_bwd writes for I. */
int moe_gate_grad_parts(int64_t I);

/* Gate-weight gradient from the partials above: grad_wt[t*k+j] = sum_p wt_partial[p*n_rows + pos]
 * (GLU slot, pos = flat_to_sorted[t*k+j], p ascending), <grad_out[t], hidden[t]> (Identity),
 * 0 (Zero or invalid index); fp32 accumulation (kernels/sm75/moe.py:712-720). */
int moe_gate_grad(int dtype, const float* wt_partial, int n_parts, int64_t n_rows,
                  const void* grad_out, int64_t grad_out_ld, const void* hidden,
                  const int64_t* top_k_indices, const int32_t* act_codes, int n_experts, int E_glu,
                  const int32_t* flat_to_sorted, int64_t n_tokens, int top_k, int64_t H,
                  void* grad_wt_out, void* stream);

/* Un-permute backward: grad_x[t] = sum_j contribution(t,j) in slot order, fp32 accumulation;
 * contribution = grad_xs[flat_to_sorted[t*k+j]] (GLU), w * grad_out[t] (Identity), 0 (Zero).
 * Replaces grad_x.index_add_(0, st, grad_x_s) (kernels/sm75/moe.py:614-615,822) and the Identity
 * backward (:796-799). */
int moe_unpermute_bwd(int dtype, const void* grad_xs, const void* grad_out, int64_t grad_out_ld,
                      const void* top_k_weights, const int64_t* top_k_indices,
                      const int32_t* act_codes, int n_experts, int E_glu,
                      const int32_t* flat_to_sorted,
                      int64_t n_tokens, int top_k, int64_t H, void* grad_x_out, void* stream);

/* Row-wise PolyGLU activation (BatchedGLU, kernels/sm75/moe.py:450-474): for every row m with
 * code c = row_act[m]: out[m] = act_c(gate) * up, codes 0,1,2,5,6,7 (kernels/sm75/moe.py:163-184).
 * gate_up rows are gu_ld elements apart, out rows out_ld apart. alpha/gamma: per-row fp32 SiTU
 * scalars with stride ap_stride (0 = one value for every row); NULL means 1.0. */
int moe_glu_fwd(int dtype, const void* gate_up, int64_t gu_ld, const int32_t* row_act,
                const float* alpha, const float* gamma, int ap_stride, int64_t n_rows, int64_t I,
                void* out, int64_t out_ld, void* stream);

/* Row-wise PolyGLU backward (kernels/sm75/moe.py:187-232): ggu = [d gate, d up]; when da/dg are
 * non-NULL, the per-row SiTU parameter gradients (0 for rows whose code is not 5). grad_out
 * elements are (go_row_stride, go_col_stride) apart, so broadcast grads need no copy. */
int moe_glu_bwd(int dtype, const void* grad_out, int64_t go_row_stride, int64_t go_col_stride,
                const void* gate_up, int64_t gu_ld, const int32_t* row_act, const float* alpha,
                const float* gamma, int ap_stride, int64_t n_rows, int64_t I, void* ggu_out,
                int64_t ggu_ld, float* da_out, float* dg_out, void* stream);

/* fp8-e4m3 forward (inference; BASELINE config 4; no counterpart in the reference, which has no
 * fp8 path — the algorithm is the bf16 pipeline of moe_grouped_gateup_swiglu_fwd /
 * moe_grouped_down_fwd with quantised operands). x_q (N,H) e4m3 + x_scale (N) fp32 (per token);
 * w13_q (E,2I,H) e4m3 + w13_scale (E,2I) fp32 and w2_q (E,H,I) + w2_scale (E,H) fp32 (per
 * output channel). Writes inter_q (M,I) e4m3 = SiLU(gate)*up re-quantised with one E8M0 scale
 * per routed row and 128-channel block (the smallest power of two 2^e with 448 * 2^e >= the
 * block's absmax), those scales into inter_bscale (a table of moe_fp8_inter_bscale_bytes bytes,
 * layout private to the library), and eo (M,H) bf16; moe_combine_fwd (bf16) makes the output.
 * H and I must be multiples of 128. */
int moe_fp8_fwd(const void* x_q, const float* x_scale, int64_t n_tokens, int64_t H,
                const void* w13_q, const float* w13_scale, const void* w2_q, const float* w2_scale,
                int E, int64_t I, const int32_t* offsets, const int32_t* sorted_token,
                int64_t n_rows, void* inter_q, void* inter_bscale, void* eo, void* stream);

/* Bytes of moe_fp8_fwd's inter_bscale for I, n_rows routed rows and E experts (0 for invalid
 * sizes). No counterpart in the reference. */
int64_t moe_fp8_inter_bscale_bytes(int64_t I, int64_t n_rows, int E);

/* Per-row absmax fp8 quantisation: scale[m] = absmax(x[m,:]) / 448 (1 for a zero row),
 * q = e4m3(x / scale), round to nearest even. x (n_rows, K) bf16, K a multiple of 8. */
int moe_rowquant_fp8(const void* x, int64_t n_rows, int64_t K, void* q, float* scale,
                     void* stream);

/* MXFP8-weight forward for decode batches (no counterpart in the reference).
 * hidden (N,H) bf16; w13_q (E,2I,H) e4m3 + w13_scale (E,2I,H/32) E8M0 bytes; w2_q (E,H,I) e4m3 +
 * w2_scale (E,H,I/32) E8M0 (value 2^(s-127), OCP MX). Writes inter (M,I) bf16 and eo (M,H) bf16;
 * moe_combine_fwd (bf16) makes the output. H and I must be multiples of 512 and at most 32256;
 * the scale tensors 4-byte aligned. */
int moe_mxfp8_fwd(const void* hidden, int64_t n_tokens, int64_t H, const void* w13_q,
                  const void* w13_scale, const void* w2_q, const void* w2_scale, int E, int64_t I,
                  const int32_t* offsets, const int32_t* sorted_token, int64_t n_rows, void* inter,
                  void* eo, void* stream);

/* Router epilogue forward (the fused epilogue of kernels/sm75/router.py:40-103,110-127): for
 * each token row n of logits (N,E; rows ld elements apart; dtype f32/f16/bf16): scores s =
 * sigmoid(logits) (softmax = 0) or softmax over the E experts (softmax = 1); selection on s + bias
 * (bias fp32 (E) or NULL; selection only); top_k picks in descending order, ties to the lower
 * expert; w = s at the picks, divided by (sum + 1e-20) when norm, times scale. Writes idx_out
 * (N,top_k) int64 and w_out (N,top_k) fp32; when counts (E) int32 is non-NULL the picks per expert
 * are added to it (the caller zeroes it). E <= 1024, top_k <= min(32, E). */
int moe_router_topk_fwd(int dtype, const void* logits, int64_t ld, int64_t n_tokens, int n_experts,
                        const float* bias, int top_k, int softmax, int norm, float scale,
                        int64_t* idx_out, float* w_out, int32_t* counts, void* stream);

/* Router epilogue backward (kernels/sm75/router.py:105-150): grad_logits (N,E), rows out_ld
 * apart, in the logits dtype, from grad_w (N,top_k) fp32 and the forward's idx; the picked raw
 * scores are recomputed from the logits. */
int moe_router_topk_bwd(int dtype, const void* logits, int64_t ld, int64_t n_tokens, int n_experts,
                        const int64_t* idx, const float* grad_w, int top_k, int softmax, int norm,
                        float scale, void* grad_logits_out, int64_t out_ld, void* stream);

/* Auxiliary-loss-free bias update, in place: bias[e] += u * sign(mean(counts) - counts[e]) in
 * fp32; no-op for u <= 0. counts must already be the global load
 * (replaces router_bias_update, kernels/sm75/router.py:293-301). */
int moe_router_bias_update(float* bias, const int32_t* counts, int n_experts, float u,
                           void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOE_GFX950_H */
