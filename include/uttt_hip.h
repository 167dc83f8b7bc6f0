/*
 * uttt_hip.h - C ABI of libuttt_hip.so, the gfx950 (MI355X) implementation of
 * uTTT's fast-weight hot path: routing, token permute/unpermute by expert,
 * the grouped SwiGLU fast-weight apply and its dot-product-loss update, and
 * the norm-preserving write.
 *
 * Conventions shared by every entry point
 *   - Plain pointers to device memory, sizes and element strides; no torch
 *     types.  `stream` is a hipStream_t (passed as void*; NULL = default).
 *   - Every call is asynchronous on `stream`, never synchronises the host and
 *     never allocates: scratch memory is passed in by the caller, sized by the
 *     matching *_workspace_bytes() query.
 *   - Return value: UTTT_OK (0) or a negative UTTT_ERR_* code; the message of
 *     the last failure on the calling thread is uttt_last_error().
 *   - dtype codes: UTTT_F32, UTTT_BF16, UTTT_F16.
 *   - Layouts are the reference's: activations [B, T, H] with H contiguous,
 *     row_id_map [B, T, 2E+1] int32, routing masks / probs [B, E, T] addressed
 *     by (batch, expert, token) element strides, fast weights [B, E, rows, cols].
 *
 * Reference interfaces are cited as paths under
 * uttt_llm/flame/custom_models/uttt_moe/ (abbreviated L/ for its
 * lact_moe_triton/ sub-package).
 */
#ifndef UTTT_HIP_H_
#define UTTT_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define UTTT_OK 0
#define UTTT_ERR_ARG (-1)         /* shape / dtype / pointer contract violated */
#define UTTT_ERR_HIP (-2)         /* a HIP runtime call or launch failed       */
#define UTTT_ERR_UNSUPPORTED (-3) /* valid request outside what is built       */

#define UTTT_F32 0
#define UTTT_BF16 1
#define UTTT_F16 2

/* Version of this ABI (bumped on any signature change). */
int uttt_abi_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char* uttt_last_error(void);

/* ------------------------------------------------------------------------ */
/* Router                                                                   */
/* ------------------------------------------------------------------------ */

/* Scratch bytes for uttt_router_select (D = 0) or uttt_route_tokens (D =
 * the feature size) at (B, T, E). */
size_t uttt_router_workspace_bytes(int B, int T, int E, int D);

/* Replaces create_router_mask_sizes_probs (M/moe_routing.py:7-75), M =
 * uttt_llm/flame/custom_models/uttt_moe.  logits fp32 addressed
 * logits[b*l_sb + e*l_se + t*l_st]; bias: optional fp32 [E] per batch
 * (bias_sb = 0: shared), added to the selection scores only.
 * router_type: 0 softmax, 1 norm_softmax, 2 norm_relu; combine_mode:
 * 0 selected_prob, 1 topk_renorm; router_scale <= 0 means sqrt(E).
 * Outputs (contiguous): mask [B,E,T] uint8 0/1 (torch.bool), group_sizes
 * [B,E] int32 (optional), combine and balance [B,E,T] fp32, lb_loss fp32
 * scalar (optional; its kernel is skipped when NULL), balance_sum [B,E] fp32
 * = sum over t of balance (optional: the sums of _make_lb_info,
 * M/modeling_recurrent_lact.py:171-176, added in a fixed order).  Top-k picks
 * the lower expert index among equal scores.  E <= 128, 1 <= topk <= E. */
int uttt_router_select(const float* logits, int64_t l_sb, int64_t l_se, int64_t l_st,
                       const float* bias, int64_t bias_sb, int B, int E, int T, int topk,
                       int router_type, int combine_mode, float alpha, float router_scale,
                       float norm_eps, void* mask, int32_t* group_sizes, float* combine,
                       float* balance, float* lb_loss, float* balance_sum, void* workspace,
                       size_t workspace_bytes, void* stream);

/* Replaces FastWeightMLPSubNN._route_tokens (M/modeling_recurrent_lact.py:147-169):
 * logits[b,e,t] = sum_d router_w[b,e,d] x[b,t,d] in fp32 (x [B,T,D]
 * contiguous of x_dtype, router_w fp32 [E,D] with batch stride w_sb, 0 =
 * shared), then the selection of uttt_router_select (32 tokens per
 * workgroup, whose waves take slices of D summed in a fixed order).
 * logits_out: optional fp32 [B,E,T]; lb_loss and balance_sum as in
 * uttt_router_select. */
int uttt_route_tokens(const void* x, int x_dtype, const float* router_w, int64_t w_sb, int B,
                      int T, int D, int E, const float* bias, int64_t bias_sb, int topk,
                      int router_type, int combine_mode, float alpha, float router_scale,
                      float norm_eps, float* logits_out, void* mask, int32_t* group_sizes,
                      float* combine, float* balance, float* lb_loss, float* balance_sum,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Scratch bytes for uttt_route_tokens_map at (B, T, E, D). */
size_t uttt_route_tokens_map_workspace_bytes(int B, int T, int E, int D);

/* The routing and the row map of one routed read in one call:
 * FastWeightMLPSubNN._route_tokens (M/modeling_recurrent_lact.py:147-169) as
 * uttt_route_tokens (no logits_out, no lb_loss; balance_sum required), then
 * make_row_id_map (lact_moe_triton/triton_permute.py:283-393) of its mask as
 * uttt_make_row_id_map, as _apply_moe_fast_weights_grouped (:296-349) calls
 * them in turn.  The outputs are those two calls' (the row map, mask, group
 * sizes, gates and balances bit-identical; balance_sum the same sums added
 * in another fixed order).  For T % 16 == 0, T <= 4096 and E <= 64 the row
 * map's one-launch kernel also adds the selection blocks' balance partials,
 * so the call is two launches instead of four.  src_rows (optional, int32
 * [B, T * topk]; only where uttt_route_tokens_map_src_rows(T, E) is 1, with
 * 16-byte aligned mask and row map): the inverse of the row map, src_rows[b,
 * row] = the token routed to that row, for uttt_grouped_gate_up_gather.  The
 * reference has no such output (its permute reads the row map). */
int uttt_route_tokens_map_src_rows(int T, int E);
int uttt_route_tokens_map(const void* x, int x_dtype, const float* router_w, int64_t w_sb, int B,
                          int T, int D, int E, const float* bias, int64_t bias_sb, int topk,
                          int router_type, int combine_mode, float alpha, float router_scale,
                          float norm_eps, void* mask, int32_t* group_sizes, float* combine,
                          float* balance, float* balance_sum, int32_t* row_id_map,
                          int32_t* src_rows, void* workspace, size_t workspace_bytes,
                          void* stream);

/* Loss-free balancing counts.  Replaces _store_loss_free_counts with
 * _loss_free_counts_for_scope (M/modeling_recurrent_lact.py:1646-1654,
 * 1695-1712) on one GPU (the all-reduce of :1657-1660 is the caller's):
 * apply_freqs, update_freqs fp32 [L, B, E] (per-layer row counts);
 * pending_counts fp32 [L, E] (pool = 0) or [E] (pool = 1) +=
 * sum over b (and over l when pool) of apply + update; *steps += 1 (int64). */
int uttt_loss_free_store_counts(const float* apply_freqs, const float* update_freqs, int L, int B,
                                int E, int pool, float* pending_counts, long long* steps,
                                void* stream);

/* Loss-free bias step.  Replaces the tensor part of _maybe_update_loss_free_bias
 * (M/modeling_recurrent_lact.py:1662-1693); the caller keeps the step
 * counter's warm-up / interval logic.  bias, counts fp32 [rows, E] (rows = 1
 * for the pool scope).  When the counts sum to > 0: mode 1 clears them (warm-up);
 * mode 2 does, per row, bias += rate * sign(mean(counts) - counts),
 * bias -= mean(bias), clamp to [-bias_max, bias_max] if bias_max >= 0,
 * then clears the counts and adds 1 to *num_updates (int64).  Means are the
 * fp32 sum times fp32(1 / E), as torch's GPU mean computes them. */
int uttt_loss_free_bias_step(float* bias, float* counts, int rows, int E, int mode, float rate,
                             float bias_max, long long* num_updates, void* stream);

/* ------------------------------------------------------------------------ */
/* Routing map                                                              */
/* ------------------------------------------------------------------------ */

/* Scratch bytes for uttt_make_row_id_map at (B, T, E). */
size_t uttt_row_id_map_workspace_bytes(int B, int T, int E);

/* Replaces make_row_id_map (L/triton_permute.py:283-393).
 * routing_map: 0/1 mask, element size mask_bytes (1 = bool/uint8, 4 = int32),
 *   addressed as map[b*s_b + e*s_e + t*s_t].
 * row_id_map: out [B, T, 2E+1] int32, bit-identical to the reference's,
 *   including the stale entries it leaves in columns [n, E).
 * group_sizes: optional out [B, E] int32 (tokens routed to each expert);
 *   may be NULL.
 * E <= 128. */
int uttt_make_row_id_map(const void* routing_map, int mask_bytes, int64_t s_b,
                         int64_t s_e, int64_t s_t, int B, int T, int E,
                         int32_t* row_id_map, int32_t* group_sizes,
                         void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------ */
/* Permute / unpermute                                                      */
/* ------------------------------------------------------------------------ */

/* Replaces triton_permute_with_mask_map / _permute_kernel
 * (L/triton_permute.py:396-571).  inp [B, T, H] contiguous of `dtype`;
 * out [B, num_out, H]; for every token t and slot j < n_routed(t):
 * out[row_j] = inp[t], or zeros if probs is given and probs[e_j, t] == 0.
 * probs: optional fp32, strides (p_sb, p_se, p_st); permuted_probs: optional
 * out [B, num_out] fp32 (required iff probs is given).  Rows >= num_out are
 * never written. */
int uttt_permute_fwd(const void* inp, int dtype, int B, int T, int H,
                     const int32_t* row_id_map, int E, const float* probs,
                     int64_t p_sb, int64_t p_se, int64_t p_st, void* out,
                     int num_out, float* permuted_probs, void* stream);

/* Replaces triton_permute_with_mask_map_bwd_batched
 * (L/triton_permute.py:579-762).  grad_inp[t] = sum_j grad_out[row_j]
 * (fp32 sum in slot order, one rounding); if grad_permuted_probs is given,
 * grad_probs [B, E, T] (contiguous) gets grad_permuted_probs[row_j] at
 * (e_j, t) and 0 elsewhere. */
int uttt_permute_bwd(const void* grad_out, int dtype, int B, int T, int H,
                     const int32_t* row_id_map, int E, int num_out,
                     const float* grad_permuted_probs, void* grad_inp,
                     float* grad_probs, void* stream);

/* Replaces triton_unpermute_with_mask_map / _unpermute_kernel
 * (L/triton_permute.py:765-930).  out[t] = cast(sum_j fma(inp[row_j], p_j))
 * accumulated in fp32 in slot order, p_j = probs[e_j, t] (fp32, strided);
 * probs may be NULL (plain sum). */
int uttt_unpermute_fwd(const void* inp, int dtype, int B, int num_out, int H,
                       const int32_t* row_id_map, int T, int E,
                       const float* probs, int64_t p_sb, int64_t p_se,
                       int64_t p_st, void* out, void* stream);

/* Replaces triton_unpermute_with_mask_map_bwd_with_merging_probs
 * (L/triton_permute.py:931-1141).  grad_inp[row_j] = cast(g[t] * p_j);
 * grad_probs[e_j, t] = sum_h fwd_inp[row_j, h] * g[t, h] (fp32), 0 for
 * experts not routed; grad_probs uses strides (gp_sb, gp_se, gp_st). */
int uttt_unpermute_bwd(const void* grad_out, const void* fwd_inp, int dtype,
                       int B, int T, int H, const int32_t* row_id_map, int E,
                       int num_out, const float* probs, int64_t p_sb,
                       int64_t p_se, int64_t p_st, void* grad_inp,
                       float* grad_probs, int64_t gp_sb, int64_t gp_se,
                       int64_t gp_st, void* stream);

/* Replaces _permute_kv_with_lrs_kernel (L/triton_permute.py:1333-1493) as
 * launched by PermuteKVAndLRs.forward (:1732-1900).  k, v [B, T, H]
 * contiguous (k_dtype, v_dtype); lr0/1/2 [B, T] with element size lr_bytes
 * (2 or 4) and token stride 1, batch stride T.  Outputs: k_out [B, num_out, H]
 * (k_dtype), v_out [B, num_out, H] (k_dtype) = cast(fp32(v) * p),
 * lr*_out [B, num_out] (copies). */
int uttt_permute_kv_lrs_fwd(const void* k, int k_dtype, const void* v,
                            int v_dtype, const void* lr0, const void* lr1,
                            const void* lr2, int lr_bytes, int B, int T, int H,
                            const int32_t* row_id_map, int E,
                            const float* probs, int64_t p_sb, int64_t p_se,
                            int64_t p_st, void* k_out, void* v_out,
                            void* lr0_out, void* lr1_out, void* lr2_out,
                            int num_out, void* stream);

/* Replaces _permute_kv_with_lrs_bwd_kernel (L/triton_permute.py:1496-1727).
 * gk, gv [B, num_out, H] (k_dtype); glr* [B, num_out] (glr_dtype, F32 or
 * BF16/F16).  Writes grad_k [B,T,H] (k_dtype), grad_v [B,T,H] (v_dtype),
 * grad_lr* [B,T] (glr_dtype), grad_probs [B,E,T] fp32 contiguous. */
int uttt_permute_kv_lrs_bwd(const void* gk, const void* gv, int k_dtype,
                            const void* glr0, const void* glr1,
                            const void* glr2, int glr_dtype, const void* v,
                            int v_dtype, const float* probs, int64_t p_sb,
                            int64_t p_se, int64_t p_st, int B, int T, int H,
                            const int32_t* row_id_map, int E, int num_out,
                            void* grad_k, void* grad_v, void* grad_lr0,
                            void* grad_lr1, void* grad_lr2, float* grad_probs,
                            void* stream);


/* ------------------------------------------------------------------------ */
/* Grouped SwiGLU fast-weight GEMMs (bf16 operands, fp32 accumulation)      */
/* ------------------------------------------------------------------------ */
/* Common contract: group_sizes [B, E] int32 on the device; the tokens of
 * expert e in batch b are the contiguous segment that starts after the
 * segments of experts < e (clamped to [0, N)).  Token columns past the last
 * segment are never written.  I, D, M, K must be multiples of 8 and every
 * tensor 16-byte aligned.  "token-major" intermediates are [B, N, rows]
 * (rows contiguous); the reference's layout is [B, rows, N]. */

/* APPLY, first GEMM pair.  Replaces fused_two_mm_swiglu_triton
 * (L/triton_grouped_swiglu_kernels.py:273-338; kernel :83-270).
 * w0_w2 [B, E, 2I, D] bf16, x [B, N, D] bf16 ->
 * hidden = silu(w0 x^T) * (w2 x^T) in bf16: [B, I, N] (token_major = 0, the
 * reference layout) or [B, N, I] (token_major = 1). */
int uttt_grouped_gate_up(const void* w0_w2, const void* x, const int32_t* group_sizes, int B,
                         int E, int I, int D, int N, void* hidden, int token_major,
                         void* stream);

/* uttt_grouped_gate_up (token-major hidden) reading its token rows straight
 * from the unpermuted x [B, T, D] through the inverse row map src_rows
 * [B, src_sb] (uttt_route_tokens_map's src_rows): routed row n of batch b is
 * x[b, src_rows[b, n]], so the permuted copy of x (permute_with_expert_mask,
 * L/triton_permute.py:1169-1248, fused_two_mm_swiglu_triton's input) is not
 * made.  Bit-identical to permuting then calling uttt_grouped_gate_up.  Only
 * for the sizes that take the skinny tiles: uttt_grouped_gate_up_gathers(N, E)
 * is 1 (else an error).  Indices outside [0, T) read row T - 1; T * D must be
 * below 2^30.  No counterpart in the reference: the routed read's glue
 * (_apply_moe_fast_weights_grouped, M:296-349) calls it where no gradient
 * flows through the read. */
int uttt_grouped_gate_up_gathers(long long N, int E);
int uttt_grouped_gate_up_gather(const void* w0_w2, const void* x, int T, const int32_t* src_rows,
                                long long src_sb, const int32_t* group_sizes, int B, int E, int I,
                                int D, int N, void* hidden, void* stream);

/* APPLY, down projection (and every "W times token rows" product).
 * Replaces grouped_gemm_transpose_triton (L/triton_grouped_gemm.py:170-243;
 * kernel :50-167) with its X operand token-major: w [B, E, M, K] bf16,
 * x [B, N, K] bf16 -> y [B, N, M] bf16, y[b, n] = w[b, e(n)] x[b, n]. */
int uttt_grouped_gemm_nt(const void* w, const void* x, const int32_t* group_sizes, int B, int E,
                         int M, int K, int N, void* y, void* stream);

/* Transposed-weight variant: w [B, E, K, M] (the product with w^T), e.g. the
 * APPLY backward's grad_X = W0_W2^T DY, which the reference computes as
 * grouped_gemm_transpose_triton(W0_W2.transpose(2, 3).contiguous(), DY0_DY2)
 * (L/lact_swiglu_ffn.py:94-96): x [B, N, K] -> y [B, N, M],
 * y[b, n] = w[b, e(n)]^T x[b, n]. */
int uttt_grouped_gemm_tn(const void* w, const void* x, const int32_t* group_sizes, int B, int E,
                         int M, int K, int N, void* y, void* stream);

/* Scratch bytes for uttt_grouped_update_stage1 at (B, I, N). */
size_t uttt_update_stage1_workspace_bytes(int B, int I, int N);

/* UPDATE, stage 1.  Replaces swiglu_backward_three_bmm_grouped_with_lr_triton
 * (L/triton_grouped_swiglu_bwd_with_lr_kernels.py:255-353; kernel :49-252).
 * w0_w2 [B,E,2I,D], w1 [B,E,D,I], k, v [B,N,D] (bf16); lr0/1/2 [B,N] of
 * lr_dtype (UTTT_F32/BF16/F16, widened to fp32) ->
 * dy0_dy2 ([B,2I,N] or token-major [B,N,2I]) and hidden ([B,I,N] or
 * [B,N,I]), bf16:
 *   Y0 = w0 k, Y2 = w2 k, DH = w1^T v (fp32, as the reference keeps it);
 *   DY0 = lr0 sig(Y0) Y2 DH (1 + Y0 (1 - sig(Y0))), DY2 = lr2 silu(Y0) DH,
 *   hidden = lr1 silu(Y0) Y2.
 * lr0 = lr1 = lr2 = NULL means lr = 1: the APPLY backward's three-GEMM pass
 * (swiglu_backward_three_bmm_grouped_triton,
 * L/triton_grouped_swiglu_bwd_kernels.py:49-320, with v = grad_out).
 * y0_y2_save [B,N,2I] and dh_save [B,N,I] (optional, both or neither):
 * bf16(Y0 | Y2) and bf16(DH), token-major, for uttt_grouped_update_bwd.
 * workspace: uttt_update_stage1_workspace_bytes(B, I, N) bytes (DH). */
int uttt_grouped_update_stage1(const void* w0_w2, const void* w1, const void* k, const void* v,
                               const void* lr0, const void* lr1, const void* lr2, int lr_dtype,
                               const int32_t* group_sizes, int B, int E, int I, int D, int N,
                               void* dy0_dy2, void* hidden, int token_major, void* y0_y2_save,
                               void* dh_save, void* workspace, size_t workspace_bytes,
                               void* stream);

/* UPDATE, stage 2 (weight gradients).  Replaces grouped_two_gemm_fw_bwd_triton
 * (L/triton_lact_bwd_grouped_two_mm_grad_fw.py:231-312; kernel :55-225) with
 * token-major intermediates: dy0_dy2_tok [B,N,2I], hidden_tok [B,N,I],
 * k, v [B,N,D] (bf16) -> dw0_w2 [B,E,2I,D] = DY[seg]^T K[seg] and
 * dw1 [B,E,D,I] = V[seg]^T Hid[seg], bf16; an empty expert gets zeros. */
int uttt_grouped_wgrad_pair(const void* dy0_dy2_tok, const void* k, const void* hidden_tok,
                            const void* v, const int32_t* group_sizes, int B, int E, int I,
                            int D, int N, void* dw0_w2, void* dw1, void* workspace,
                            size_t workspace_bytes, void* stream);
/* Workspace of uttt_grouped_wgrad_pair: fp32 split-K partials when the
 * output tiles fill under half of the GPU (a single expert with small
 * weights, as uTTT-Dense), else 0 (workspace may then be NULL). */
size_t uttt_grouped_wgrad_pair_workspace_bytes(int B, int E, int I, int D, int N);

/* One weight-gradient product.  Replaces grouped_gemm_bwd_triton
 * (L/triton_grouped_gemm.py:349-404; kernel :251-346) with token-major
 * operands: a_tok [B,N,R], b_tok [B,N,C] (bf16) ->
 * out[b,e] = A[seg]^T B[seg], [B,E,R,C] (transposed = 0) or [B,E,C,R]
 * (transposed = 1), bf16; an empty expert gets zeros. */
int uttt_grouped_wgrad(const void* a_tok, const void* b_tok, const int32_t* group_sizes, int B,
                       int E, int R, int C, int N, void* out, int transposed, void* stream);

/* Two chained products in one pass (fp32 accumulation, one bf16 rounding):
 *   nt2: y[b, n] = wa[b, e(n)] xa[b, n] + wb[b, e(n)] xb[b, n],  w [B,E,M,K]
 *   tn2: y[b, n] = wa[b, e(n)]^T xa[b, n] + wb[b, e(n)]^T xb[b, n], w [B,E,K,M]
 * x token-major [B, N, K], y [B, N, M], bf16.  Together they replace
 * fused_grouped_grad_kv (L/triton_lact_bwd_grouped_grad_kv.py:227-340):
 * grad_K = tn2(G_W0_W2, DY_lr, W0_W2, dY_02), grad_V = nt2(W1, dH, G_W1, H_lr). */
int uttt_grouped_gemm_nt2(const void* wa, const void* xa, const void* wb, const void* xb,
                          const int32_t* group_sizes, int B, int E, int M, int K, int N, void* y,
                          void* stream);
int uttt_grouped_gemm_tn2(const void* wa, const void* xa, const void* wb, const void* xb,
                          const int32_t* group_sizes, int B, int E, int M, int K, int N, void* y,
                          void* stream);

/* Scratch bytes for uttt_swiglu_bwd_bwd at (B, D, L). */
size_t uttt_swiglu_bwd_bwd_workspace_bytes(int B, int D, int L);

/* Second-order SwiGLU pointwise pass.  Replaces
 * triton_swiglu_bwd_bwd_fused_cat_inp_out / ref_pytorch_swiglu_bwd_bwd_fused_cat_inp_out
 * (L/triton_pointwise_kernels.py:240-436).  dh, grad_hidden_lr1, grad_dh,
 * hidden_lr1 [B, D, L]; x0_x2, grad_dx0_dx2, grad_x0_x2, dx0_x2 [B, 2D, L]
 * (x_dtype); lr0/1/2 and grad_lr0/1/2 [B, L] (lr_dtype).  fp32 arithmetic;
 * grad_lr* summed over D deterministically.  workspace:
 * uttt_swiglu_bwd_bwd_workspace_bytes(B, D, L) bytes. */
int uttt_swiglu_bwd_bwd(const void* dh, const void* x0_x2, int x_dtype, const void* lr0,
                        const void* lr1, const void* lr2, int lr_dtype, const void* grad_dx0_dx2,
                        const void* grad_hidden_lr1, int B, int D, int L, void* grad_dh,
                        void* grad_x0_x2, void* grad_lr0, void* grad_lr1, void* grad_lr2,
                        void* dx0_x2, void* hidden_lr1, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Scratch bytes for uttt_grouped_update_bwd at (B, I, N). */
size_t uttt_update_bwd_workspace_bytes(int B, int I, int N);

/* UPDATE backward.  Replaces FusedLactSwiGLUFFNBwd.backward
 * (L/lact_fw_grad.py:116-300): grouping_four_grouped_gemm_triton
 * (L/triton_lact_bwd_grouped_four_mm.py:300-439),
 * ref_pytorch_swiglu_bwd_bwd_fused_cat_inp_out (L/triton_pointwise_kernels.py:354-436),
 * fused_grouped_grad_kv (L/triton_lact_bwd_grouped_grad_kv.py:227-340) and
 * grouped_two_gemm_fw_bwd_triton, as five launches with no host sync.
 * Inputs: the forward's w0_w2, w1, k, v, lr0/1/2 (lr_dtype), group_sizes and
 * the upstream gradients grad_dw0_w2 [B,E,2I,D], grad_dw1 [B,E,D,I] (bf16).
 * Outputs: grad_w0_w2 [B,E,2I,D], grad_w1 [B,E,D,I], grad_k, grad_v [B,N,D]
 * (bf16), grad_lr0/1/2 [B,N] (lr_dtype; zero past the routed tokens).
 * y0_y2_saved / dh_saved (optional, both or neither): the forward's saved
 * bf16(Y0 | Y2) and bf16(DH) (uttt_grouped_update_stage1); with them the
 * backward does not recompute Y0, Y2 and DH, which the reference's backward
 * recomputes and rounds to bf16 (L/lact_fw_grad.py:131-176): GD = gw1^T v
 * runs alone and GY = gw0_w2 k carries the second-order pass in its
 * epilogue (6 N*I*D FLOP in place of 12).
 * workspace: uttt_update_bwd_workspace_bytes(B, I, N) bytes. */
int uttt_grouped_update_bwd(const void* w0_w2, const void* w1, const void* k, const void* v,
                            const void* lr0, const void* lr1, const void* lr2, int lr_dtype,
                            const int32_t* group_sizes, const void* grad_dw0_w2,
                            const void* grad_dw1, const void* y0_y2_saved, const void* dh_saved,
                            int B, int E, int I, int D, int N,
                            void* grad_w0_w2, void* grad_w1, void* grad_k, void* grad_v,
                            void* grad_lr0, void* grad_lr1, void* grad_lr2, void* workspace,
                            size_t workspace_bytes, void* stream);

/* Layout helper (no reference counterpart; used to accept the reference's
 * [B, rows, N] intermediates): out[b, c, r] = in[b, r, c], 2-byte elements. */
int uttt_transpose_2byte(const void* in, int B, int R, int C, void* out, void* stream);

/* Row preprocessing of the fast-weight inputs, forward.  Replaces the steps
 * of _preprocess_update_inputs (uttt_llm/flame/custom_models/uttt_moe/
 * modeling_recurrent_lact.py:630-657) and of the read's q path (ibid.
 * :588-601): optional F.silu (silu = 1), then an optional parameter-free norm
 * over each row of D elements (norm = 0 none, 1 l2_norm x / (|x| + 1e-5),
 * 2 rms_norm x * rsqrt(mean(x^2) + 1e-5); ref_base.py:181-195, fp32 inside,
 * the result rounded to dtype), then, when rope_dim > 0, the rotary
 * embedding of ref_base.py:342-355 (rotary.py:83-104, non-interleaved): the
 * value cast to bf16 and each pair (j, j + rope_dim / 2) of every rope_dim
 * block of the token's features rotated with the bf16 tables
 * rope_cos / rope_sin [table_rows, rope_dim / 2] at position
 * (token % seq_len) + pos_offset, token = row / rows_per_token.  Output:
 * bf16 with the rotary, else dtype; row r at out + r * ld_out.  dtype:
 * UTTT_BF16, UTTT_F16 or UTTT_F32; D and the strides multiples of 8,
 * D <= 4096, rope_dim one of 16 .. 256 (a power of two) dividing D, rows a
 * multiple of rows_per_token * seq_len, 16-byte aligned tensors. */
int uttt_rows_preprocess(const void* in, int dtype, int64_t rows, int D, int64_t ld_in,
                         int silu, int norm, const void* rope_cos, const void* rope_sin,
                         int rope_dim, int rows_per_token, int seq_len, int pos_offset,
                         int table_rows, void* out, int64_t ld_out, void* stream);

/* Backward of uttt_rows_preprocess: grad_in [rows, ld_in] (dtype) from the
 * forward's input `in` and grad_out [rows, ld_out] (the forward output's
 * dtype), with the reference autograd's rounding points: the conjugate
 * rotation (RotaryEmbeddingFunction.backward, rotary.py:244-266) stored bf16,
 * the compiled norm's backward and F.silu's backward stored in dtype.
 * Same arguments and limits as the forward. */
int uttt_rows_preprocess_bwd(const void* in, int dtype, const void* grad_out, int64_t rows,
                             int D, int64_t ld_in, int64_t ld_out, int silu, int norm,
                             const void* rope_cos, const void* rope_sin, int rope_dim,
                             int rows_per_token, int seq_len, int pos_offset, int table_rows,
                             void* grad_in, void* stream);

/* Test hook (no reference counterpart): grids of the token-grouped GEMMs
 * with at least `min_tiles` workgroup tiles take the XCD super-tile order
 * (default 2048, one value per process; a negative value restores it).
 * Returns the previous value.  Results do not depend on it: tests lower it
 * to run small problems down the path the large ones take. */
long long uttt_debug_set_supertile_min_tiles(long long min_tiles);

/* Test hook: which kernel runs the weight-streaming APPLY products
 * (uttt_grouped_gate_up with token_major, uttt_grouped_gemm_nt): -1 by the
 * sizes (gate/up on the skinny-tile three-stage kernel when N <= 256 * E;
 * uttt_grouped_gemm_nt on it when also the general 256x256 tiles would not
 * fill the 256 CUs once), 0 the general tiles, 1 the skinny tiles (128-row
 * down-projection tiles), 2 the skinny tiles with 256-row down-projection
 * tiles.  Results are identical on every path.  Returns the previous value. */
int uttt_debug_set_apply_path(int path);

/* Test hook (no reference counterpart): the wave layout of the token-grouped
 * and weight-gradient GEMM kernels, process-wide.  0: each product family's
 * default; 2: four waves per 256x256 tile (one per SIMD, 128x128 per wave);
 * 1: eight waves (two per SIMD, 64x128 per wave; families whose eight-wave
 * kernel does not fit the register file keep four).  Both layouts
 * accumulate every output in the same k order with the same MFMA, so
 * results are identical.  Returns the previous value. */
int uttt_debug_set_gemm_layout(int na);

/* Test hook (no reference counterpart): which path uttt_newton_schulz5 takes.
 * 0: by the sizes (one launch for the small matrices it covers), 1: always
 * the multi-launch path.  Both give identical results.  Returns the previous
 * value. */
int uttt_debug_set_ns_path(int path);

/* Test hook (no reference counterpart): which kernel runs the fused uTTT-Dense
 * stage 1 (uttt_dense_update_stage1, uttt_dense_update_stage1_layers) for
 * heads of D <= 192.  0: by the grid (the staged eight-wave kernel, weights
 * through LDS, for grids of at least 256 workgroups; the four-wave kernel
 * with register prefetch below that), 1: always the staged kernel, 2: always
 * the four-wave kernel.  Both give identical results.  Returns the previous
 * mode. */
int uttt_debug_set_s1_staged(int mode);

/* WRITE step of the fast weights.  Replaces the write of
 * _apply_moe_update_dense (uttt_llm/flame/custom_models/uttt_moe/
 * modeling_recurrent_lact.py:754-825; seg = C, norm_from_fast = 0,
 * renorm_master = 1) and of uTTT-Dense's _apply_shared_update
 * (uttt_llm/flame/custom_models/uttt_dense/modeling_recurrent_lact.py:1109-1240;
 * seg = d, nu from the fast weight unless master renorm is on), without Muon.
 * Tensors are [B, rows_per_batch, C] row-major; each row is cut into C / seg
 * segments and for each segment, with nu = |segment of master (or of
 * fast_in, bf16, when norm_from_fast)| taken before the step:
 *   G = grad (+ mom_in * m_coeff[b] when mom_in; then mom_out = G)
 *   U = master + G * lr_scale
 *   P = U / (|U| + 1e-5) * nu
 *   master_out = renorm_master ? P : U,   fast_out = bf16(P).
 * grad: grad_dtype (fp32, bf16 or fp16); master, mom, master_out fp32;
 * m_coeff fp32 [B].  master_out may be master and mom_out may be mom_in (in
 * place).  seg must be a multiple of 4, at most 4096, and divide C. */
int uttt_write_step(const float* master, const void* fast_in, const void* grad, int grad_dtype,
                    const float* mom_in, const float* m_coeff, float lr_scale, int B,
                    int64_t rows_per_batch, int C, int seg, int norm_from_fast, int renorm_master,
                    float* master_out, void* fast_out, float* mom_out, void* stream);

/* Sequence-start row norms of the single-layer LaCT's prenorm write
 * (w0_norm = w0.norm(dim=2) etc., uttt_nvs/models/kernels/ttt_operation.py:
 * 258-260): norms[r] = |w row r| in fp32 for `rows` rows of C elements
 * (dtype UTTT_F32, UTTT_BF16 or UTTT_F16; C a multiple of 4, at most 4096;
 * w 16-byte aligned). */
int uttt_row_norms(const void* w, int dtype, int64_t rows, int C, float* norms, void* stream);

/* Prenorm WRITE of the single-layer LaCT (prenorm_block_causal_lact_swiglu,
 * uttt_nvs/models/kernels/ttt_operation.py:217-367; the write at :341-353):
 * per row r of C elements, U = main + grad (fp32; the step carries its
 * learning rates, no scale), main_out = U and
 * fast_out = bf16(U / (|U| + 1e-5) * norms[r]), norms being the row norms
 * captured at the start of the sequence (uttt_row_norms).  main and
 * main_out fp32 (may alias), grad fp32 / bf16 / fp16, fast_out bf16; C a
 * multiple of 4, at most 4096. */
int uttt_write_prenorm(const float* main_w, const void* grad, int grad_dtype,
                       const float* norms, int64_t rows, int C, float* main_out,
                       void* fast_out, void* stream);

/* Unit-row WRITE of the NVS block.  Replaces the write of apply_raw_update
 * (uttt_nvs/models/uttt_moe_block.py:665-714; Muon, when on, runs before it
 * through uttt_newton_schulz5):
 *   U = master + grad              (fp32; grad fp32, bf16 or fp16)
 *   master_out = U,   fast_out = bf16(U / max(|U|, 1e-5))   (F.normalize)
 * per row of C elements.  The tensors hold `groups` groups of R rows; row r
 * of group g starts at g * <tensor>_gs + r * C elements, so the w0 / w2
 * halves of a packed [B, E, 2I, D] gradient or fast weight are addressed in
 * place (gs = 2I * D, offset 0 or I * D).  master_out may be master (same
 * strides).  C must be a multiple of 4, at most 4096; strides multiples of 4. */
int uttt_write_unit_rows(const float* master, int64_t master_gs, const void* grad, int grad_dtype,
                         int64_t grad_gs, int64_t groups, int R, int C, float* master_out,
                         int64_t master_out_gs, void* fast_out, int64_t fast_gs, void* stream);

/* Momentum step of the Muon write on its own: out = raw + m_coeff[b] * mom
 * (fp32; raw fp32 or bf16; B batches of per_batch elements).  Replaces the
 * momentum lines of _apply_moe_update_dense (uttt_llm/flame/custom_models/
 * uttt_moe/modeling_recurrent_lact.py:767-775) and of _apply_shared_update
 * (uttt_llm/flame/custom_models/uttt_dense/modeling_recurrent_lact.py:1175-1185),
 * whose result is both the new momentum buffer and the input of the
 * Newton-Schulz step.  out may be mom (in place). */
int uttt_momentum_add(const void* raw, int raw_dtype, const float* mom, const float* m_coeff,
                      int B, int64_t per_batch, float* out, void* stream);

/* Muon orthogonalisation: zeropower_via_newtonschulz5 (uttt_llm/flame/
 * custom_models/uttt_moe/ttt_operation.py:19-46), called by the Muon writes
 * (uttt_moe/modeling_recurrent_lact.py:777-810 with steps = 5;
 * uttt_dense/modeling_recurrent_lact.py:1192-1203 per d x d slice).  For each
 * of BE matrices G [rows, cols] (fp32 or bf16): X = bf16(G), transposed to
 * [min, max] when rows > cols; X = X / (||X||_F + 1e-7); five steps of
 * A = X X^T, B = b A + (c A) A (Python's `c * A @ A`), X = a X + B X with the reference's (a, b, c)
 * table, every operation rounded to bf16 as the reference's bf16 tensors are;
 * out = bf16(X * out_scale) [BE, rows, cols] bf16 (out_scale = the write's
 * step size, which the reference applies to the bf16 result; 1 leaves X).
 * rows and cols must be multiples of 8; the workspace is
 * uttt_newton_schulz5_workspace_bytes(BE, rows, cols) bytes.  Matrices whose
 * sides are multiples of 32 with min * (max + 8) <= 38400 (the uTTT-Dense
 * d x d slices up to d = 192) and a 16-byte aligned g run in one launch, one
 * workgroup per matrix with the whole computation in LDS, with the same
 * result bits as the multi-launch path (the workspace is then unused). */
size_t uttt_newton_schulz5_workspace_bytes(int BE, int rows, int cols);
int uttt_newton_schulz5(const void* g, int g_dtype, int BE, int rows, int cols, float out_scale,
                        void* out, void* workspace, size_t workspace_bytes, void* stream);

/* Routed SwiGLU read for a few tokens per sequence (generation): the part of
 * FastWeightMLPSubNN._apply_moe_fast_weights_grouped (uttt_llm/flame/
 * custom_models/uttt_moe/modeling_recurrent_lact.py:330-349) after routing --
 * _permute_with_expert_mask, _grouped_swiglu_ffn_fwd (L/lact_swiglu_ffn.py:
 * 37-61) and _unpermute_and_merge_with_probs -- fused for T <= 64 tokens per
 * batch, with no row map or permuted copy.  x [B, T, D] bf16; w0_w2
 * [B, E, 2I, D] and w1 [B, E, D, I] bf16 (contiguous); expert_mask [B, E, T]
 * (element size mask_bytes = 1 or 4, any strides), probs [B, E, T] fp32 (any
 * strides).  out[b, t] = bf16(sum over the token's experts in descending order
 * of fma(bf16(w1 h), p)), h = bf16(silu(w0 x) * (w2 x)): the reference's
 * rounding points.  E <= 64, T <= 64, D and I multiples of 8 and at most 4096;
 * topk sets the launch width (any number of selected experts is handled).
 * The workspace is uttt_moe_decode_read_workspace_bytes(B, T, E, I) bytes. */
size_t uttt_moe_decode_read_workspace_bytes(int B, int T, int E, int I);
int uttt_moe_decode_read(const void* x, int B, int T, int D, const void* w0_w2, const void* w1,
                         int E, int I, const void* expert_mask, int mask_bytes, int64_t m_sb,
                         int64_t m_se, int64_t m_st, const float* probs, int64_t p_sb,
                         int64_t p_se, int64_t p_st, int topk, void* out, void* workspace,
                         size_t workspace_bytes, void* stream);

/* No counterpart in the reference: uttt_moe_decode_read for callers that
 * cannot allocate (code under HIP graph capture, serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and results without the workspace:
 * the hidden buffer lives in a file-scope device array of 8 MiB that each GPU
 * the library runs on holds until the process ends, so B*E*T*I*2 must be at
 * most 8 MiB (larger problems are refused with UTTT_ERR_ARG).  Calls no
 * hipMalloc or hipFree.  The stream must belong to the current device.  Calls
 * that overlap on one GPU (other streams or threads) share the array and
 * race; calls ordered on one stream do not. */
int uttt_moe_decode_read_noalloc(const void* x, int B, int T, int D, const void* w0_w2,
                                 const void* w1, int E, int I, const void* expert_mask,
                                 int mask_bytes, int64_t m_sb, int64_t m_se, int64_t m_st,
                                 const float* probs, int64_t p_sb, int64_t p_se, int64_t p_st,
                                 int topk, void* out, void* stream);

/* uTTT-Dense read, fused for small heads: out = W1 (silu(W0 x) * (W2 x))
 * per head (_apply_fast_weights, uttt_dense/modeling_recurrent_lact.py:241-261,
 * with the rearranges of :251 and :261 folded in).  x [b, l, H*D] bf16,
 * w0_w2 [b*H, 2I, D] (w0 rows then w2 rows), w1 [b*H, D, I] bf16 ->
 * out [b, l, H*D] bf16 (fp32 products, bf16 hidden, as the grouped APPLY).
 * Shapes: uttt_dense_read_supported(D, I) != 0 (D in {64, 96, 128, 192, 256},
 * I a multiple of 32 up to 512), b*H <= 65535, 16-byte aligned tensors. */
int uttt_dense_read_supported(int D, int I);
int uttt_dense_read(const void* x, int b, int l, int H, int D, const void* w0_w2, const void* w1,
                    int I, void* out, void* stream);
/* The same read from a fragment-ordered copy of the weights (no reference
 * counterpart: a layout of this build for the shared fast-weight bank, whose
 * twelve reads per chunk share one copy).  uttt_dense_pack_weights writes
 * packed [BH, 3 I D] bf16 (the bytes of w0_w2 [BH, 2I, D] and w1 [BH, D, I]
 * regrouped so that each fragment load of the read is 64 lanes x 16
 * consecutive bytes); uttt_dense_read_packed(x, b, l, H, D, packed, I, out)
 * gives bit-identical results to uttt_dense_read on the weights packed.
 * Shapes and alignment as uttt_dense_read, BH = b*H. */
int uttt_dense_pack_weights(const void* w0_w2, const void* w1, int BH, int D, int I, void* packed,
                            void* stream);
int uttt_dense_read_packed(const void* x, int b, int l, int H, int D, const void* packed, int I,
                           void* out, void* stream);

/* uTTT-Dense UPDATE stage 1, fused for small heads (replaces the two grouped
 * products of uttt_grouped_update_stage1 with E = 1 for the dense write:
 * uttt_dense/modeling_recurrent_lact.py:409-432, gate_before_act,
 * hidden_before_mul, dhidden and silu_backprop, the lr factors of :425-432
 * applied to DY0 / Hid / DY2).  k, v [BH, N, D] bf16 (one head per BH, the
 * layers' tokens concatenated), lr0/1/2 [BH, N] fp32 (all three or none:
 * none means 1), dy [BH, N, 2I] and hid [BH, N, I] bf16, token-major as
 * uttt_grouped_update_stage1's token_major output.  The weights come as a
 * fragment-ordered copy [BH, 3 I D] bf16 written by
 * uttt_dense_pack_update_weights from w0_w2 [BH, 2I, D] and w1 [BH, D, I]
 * (a layout of this build, no reference counterpart).  D in {64, 96, 128,
 * 192, 256}, I a multiple of 32 in [32, 512] (uttt_dense_update_supported). */
int uttt_dense_update_supported(int D, int I);
int uttt_dense_pack_update_weights(const void* w0_w2, const void* w1, int BH, int D, int I,
                                   void* packed, void* stream);
int uttt_dense_update_stage1(const void* k, const void* v, const void* lr0, const void* lr1,
                             const void* lr2, int BH, int N, int D, int I, const void* packed,
                             void* dy, void* hid, void* stream);

/* uTTT-Dense head layout (uttt_dense/modeling_recurrent_lact.py, D:).
 * Gather: the head split 'b l (h d) -> (b h) l d' of k and v and
 * 'b l h -> (b h) l 1' of the three lr columns in compute_update (D:370-398;
 * of the read input at D:251), for L layers at once, the layers' tokens
 * concatenated per head (the aggregate write's batching of
 * _aggregate_memory_update, D:1302-1386):
 *   kh [b*H, L*l, d] (bf16; vh likewise) from k_layers[li] [b, l, H*d] bf16,
 *   lr0/1/2 [b*H, L*l] fp32 from lr_layers[li] [b, l, 3] (lr_per_head = 0,
 *   shared by the heads) or [b, l, H*3] (lr_per_head = 1), dtype lr_dtype.
 * k_layers, v_layers, lr_layers are HOST arrays of L device pointers
 * (L <= 64); v_layers/vh and lr_layers/lr* may be NULL.  d % 8 == 0, k, v
 * and the outputs 16-byte aligned. */
int uttt_dense_gather_heads(const void* const* k_layers, const void* const* v_layers,
                            const void* const* lr_layers, int lr_dtype, int lr_per_head, int L,
                            int b, int l, int H, int d, void* kh, void* vh, float* lr0,
                            float* lr1, float* lr2, void* stream);
/* The aggregate write's UPDATE without the per-head copy: stage 1
 * (uttt_dense_update_stage1) and the weight gradients (uttt_grouped_wgrad_pair,
 * one expert per head) reading every layer's own k_layers[li], v_layers[li]
 * [b, l, H*D] bf16 and lr_layers[li] (as uttt_dense_gather_heads takes them;
 * NULL for no lr) instead of kh, vh, lr0/1/2.  Token li*l + t of head
 * bb*H + hh is row bb*l + t of layer li at column hh*D, as the gather lays
 * it out.  The weight gradients split K once per layer (L runs; fp32
 * partials in the workspace, uttt_dense_wgrad_pair_layers_workspace_bytes,
 * summed in layer order), so they are bit-identical to the gathered path
 * wherever its split count is L (configs[1]: 12 layers, 12 runs).  dy, hid
 * as uttt_dense_update_stage1's outputs [b*H, L*l, 2I] / [b*H, L*l, I].
 * l must be a multiple of 64 (of 32 for stage 1), L <= 64, pointer arrays
 * on the host, every tensor 16-byte aligned.  No reference counterpart: the
 * reference rearranges per layer and loops over the layers (D:370-398,
 * D:1302-1386). */
int uttt_dense_update_stage1_layers(const void* const* k_layers, const void* const* v_layers,
                                    const void* const* lr_layers, int lr_dtype, int lr_per_head,
                                    int L, int b, int l, int H, int D, int I, const void* packed,
                                    void* dy, void* hid, void* stream);
size_t uttt_dense_wgrad_pair_layers_workspace_bytes(int L, int b, int H, int I, int D);
int uttt_dense_wgrad_pair_layers(const void* dy0_dy2_tok, const void* const* k_layers,
                                 const void* hidden_tok, const void* const* v_layers, int L,
                                 int b, int l, int H, int I, int D, void* dw0_w2, void* dw1,
                                 void* workspace, size_t workspace_bytes, void* stream);

/* Scatter: '(b h) l hd -> b l (h hd)' of the read output (D:261):
 * y [b*H, l, d] bf16 -> out [b, l, H*d] bf16; d % 8 == 0, 16-byte aligned. */
int uttt_dense_scatter_heads(const void* y, int b, int l, int H, int d, void* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* UTTT_HIP_H_ */
