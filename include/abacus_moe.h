/*
 * libabacus_moe — C ABI of the MI355X (gfx950) MoE layer kernels.
 *
 * The reference (satyaki-up/abacus) has no native layer: its MoE layer is the
 * torch-op sequence of abacus/moe/router.py and abacus/moe/moe.py.  Each entry
 * point below replaces the span of reference ops named in its comment
 * (file:line relative to the abacus tree); the Python modules in
 * abacus_amd/moe.py call them in order through ctypes.
 *
 * Conventions
 *   - All pointers are device pointers (HIP, same device), row-major,
 *     contiguous and 16-byte aligned.  Nothing here allocates, frees or
 *     synchronises; every launch goes to `stream` (a hipStream_t).
 *   - dtype: ABACUS_F32 (0) or ABACUS_BF16 (1) for activations and weights
 *     (the host build also ABACUS_F64 and ABACUS_F16); index tensors are int32
 *     unless named *_i64; score / dlogit buffers are fp32 (fp64 with fp64).
 *   - Return 0 on success, nonzero on a rejected argument (1) or launch
 *     failure (2); abacus_moe_last_error() gives the message (per thread).
 *   - Sizes: T tokens, D model dim, E experts (<= 1024), K slots per token
 *     (<= min(E, 64)), M expert hidden dim, R = T*K routed rows.  D and M must
 *     be multiples of 8 (bf16) or 4 (fp32).  Up to 256 experts and 16 slots
 *     the router is one fused kernel; beyond, a logits pass and a top-k pass
 *     (same results: the routing depends only on the stored logits).
 *   - offsets_E1[e] .. offsets_E1[e+1] are the routed rows of expert e in every
 *     expert-contiguous (R, .) buffer; rows are expert-major and, inside an
 *     expert, in ascending token order (moe.py:72-77).
 */
#ifndef ABACUS_MOE_H
#define ABACUS_MOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABACUS_F64 and ABACUS_F16 are taken by the host build only (CPU tensors; the
 * HIP library rejects them).  The acc side buffers (score and
 * dlogit) hold fp32 elements, fp64 ones for ABACUS_F64; scalar factors
 * (route_scale, bias speeds) are cast to that type, as torch casts a Python
 * scalar meeting a tensor of the dtype.  The load-balancing loss computes in
 * fp32 for every dtype (load_balancing.py:30 casts the probabilities to
 * float), so its f_E and fp32 loss stay fp32. */
enum { ABACUS_F32 = 0, ABACUS_BF16 = 1, ABACUS_F64 = 2, ABACUS_F16 = 3 };

/* int32 elements of the tile-counter workspace (tile_ctr) that the weight-gradient
 * entry points take: device memory the call clears on its stream and then uses
 * for the launch's work counters.  Calls in flight at the same time need
 * separate workspaces; its contents after the call are unspecified. */
#define ABACUS_MOE_TILE_CTR_INTS 16

/* ---- library / sizing queries ------------------------------------------ */
const char* abacus_moe_last_error(void);
/* 5: scalar factors are double and the acc side buffers void* (ABACUS_F64 and
 * ABACUS_F16 in the host build).  4: abacus_moe_router_wgrad_ws_bytes takes the
 * dtype (the partial-sum plan differs by dtype).  3: abacus_moe_router_ws_bytes
 * also covers the small-batch router's partial logits (size workspaces by the
 * queries, never by a formula). */
int abacus_moe_abi_version(void);
/* int32 elements of the per-token-block expert histogram (and of `base`). */
int64_t abacus_moe_hist_len(int64_t T, int64_t E);
/* bytes of the router workspace used by router_fwd / unpermute_bwd: the
 * transposed router weight and, for bf16 with E <= 256, room for the partial
 * logits of router_fwd's split small-batch pass (T <= 1024); independent of T. */
int64_t abacus_moe_router_ws_bytes(int64_t D, int64_t E, int dtype);
/* bytes of the fp32 partial-sum scratch used by router_wgrad for this dtype
 * (-1 for an unknown dtype). */
int64_t abacus_moe_router_wgrad_ws_bytes(int64_t T, int64_t D, int64_t E, int dtype);
/* bytes of the split-tail workspace of down_fwd (0: that shape runs no split, which
 * includes small batches, R <= 128 * E, and short reductions, M < 2560). */
int64_t abacus_moe_down_fwd_ws_bytes(int64_t R, int64_t M, int64_t D, int64_t E, int dtype);
/* bytes of the per-block partial sums and counts used by load_balancing_fwd. */
int64_t abacus_moe_load_balancing_ws_bytes(int64_t T, int64_t E);

/* ---- forward ------------------------------------------------------------ */

/* Replaces router.py:45-51 (logits GEMM, sigmoid, + expert_bias_E, topk,
 * gather, renormalise, * route_scale) and the bincount of router.py:65.
 * Outputs: logits_TE (dtype, the exact logits routing used), weights_TK
 * (dtype), indices_TK_i64 (descending selection, ties -> lower expert),
 * idx_TK (int32 copy), score_TK (fp32 value of the dtype-rounded selected
 * sigmoid scores), hist (abacus_moe_hist_len ints).  Every output is
 * required (past 256 experts or 16 slots the top-k pass reads logits_TE). */
int abacus_moe_router_fwd(const void* x_TD, const void* w_DE, const void* bias_E, int64_t T, int64_t D, int64_t E,
                          int64_t K, double route_scale, int dtype, void* logits_TE, void* weights_TK,
                          int64_t* indices_TK_i64, int32_t* idx_TK, void* score_TK, int32_t* hist, void* wt_ws,
                          void* stream);

/* Replaces the per-expert counting of moe.py:73-76 and, when bias_E is not
 * NULL, Router.update_bias (router.py:57-70) in place.  Produces counts_E,
 * offsets_E1 and base (per token-block first row of each expert). */
int abacus_moe_route_scan(const int32_t* hist, int64_t T, int64_t E, int64_t K, void* bias_E,
                          double bias_update_speed, int dtype, int32_t* base, int32_t* counts_E,
                          int32_t* offsets_E1, void* stream);

/* Replaces the boolean-mask gather x_TD[selected_T] of moe.py:77 for all
 * experts at once: pos_TK[t,k] = routed row of (t,k), perm_R[r] = token of
 * row r, x_perm_RD[pos] = x_TD[t]. */
int abacus_moe_permute_gather(const void* x_TD, const int32_t* idx_TK, const int32_t* base, int64_t T, int64_t D,
                              int64_t E, int64_t K, int dtype, int32_t* pos_TK, int32_t* perm_R, void* x_perm_RD,
                              void* stream);

/* Replaces moe.py:72-77 (the per-expert counting, the optional bias step of
 * router.py:57-70, and the gather) in one call: abacus_moe_route_scan then
 * abacus_moe_permute_gather, with the same outputs.  When the router's block
 * histograms hold at most 4096 ints (ceil(T / 16) * E) the gather blocks
 * scan them themselves and there is one launch; base_ws (hist-length ints)
 * is then unused. */
int abacus_moe_dispatch(const int32_t* hist, const void* x_TD, const int32_t* idx_TK, int64_t T, int64_t D,
                        int64_t E, int64_t K, void* bias_E, double bias_update_speed, int dtype, int32_t* counts_E,
                        int32_t* offsets_E1, int32_t* pos_TK, int32_t* perm_R, void* x_perm_RD, int32_t* base_ws,
                        void* stream);

/* Replaces moe.py:78-79 for every expert: gate = x @ w_gate[e],
 * up = x @ w_up[e], h = silu(gate) * up.  gate_RM / up_RM may be NULL
 * (inference: only h is written). */
int abacus_moe_gateup_fwd(const void* x_perm_RD, const void* w_gate_EDM, const void* w_up_EDM,
                          const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M, int64_t E, int dtype,
                          void* gate_RM, void* up_RM, void* h_RM, void* stream);

/* Replaces moe.py:80: y = h @ w_down[e] for every expert.  With a workspace of
 * abacus_moe_down_fwd_ws_bytes bytes (bf16, and fp32 batches large enough for
 * the pipelined kernel; reductions M >= 2560), the tiles beyond the whole rounds
 * of the GPU's CUs run as slices of the reduction, whose fp32 partials the
 * workspace holds; ws = NULL (or too small) runs every tile whole.  Either way
 * the same products are summed, in a fixed order: repeated calls agree bit
 * for bit. */
int abacus_moe_down_fwd(const void* h_RM, const void* w_down_EMD, const int32_t* offsets_E1, int64_t R, int64_t M,
                        int64_t D, int64_t E, int dtype, void* y_RD, void* ws, int64_t ws_bytes, void* stream);

/* Replaces moe.py:81-85: out[t] = sum over the token's experts (ascending)
 * of y[pos(t,k)] * weights_TK[t,k]. */
int abacus_moe_combine_fwd(const void* y_RD, const void* weights_TK, const int32_t* idx_TK, const int32_t* pos_TK,
                           int64_t T, int64_t D, int64_t K, int dtype, void* out_TD, void* stream);

/* ---- backward (autograd of the ops above) -------------------------------- */

/* Backward of moe.py:81-85 and router.py:45,49-51: dy_RD[pos] =
 * w * dout[t]; dL/dweights = <dout[t], y>; then renormalise and sigmoid
 * backward to dlogit_TK (fp32, one value per selected expert). */
int abacus_moe_combine_bwd(const void* dout_TD, const void* y_RD, const void* weights_TK, const void* score_TK,
                           const int32_t* pos_TK, int64_t T, int64_t D, int64_t K, double route_scale, int dtype,
                           void* dy_RD, void* dlogit_TK, void* stream);

/* Backward of moe.py:80 (dgrad) fused with the SwiGLU backward of moe.py:78-79:
 * dh = dy @ w_down[e]^T; dgate = dh*up*silu'(gate); dup = dh*silu(gate). */
int abacus_moe_down_bwd_dgrad(const void* dy_RD, const void* w_down_EMD, const void* gate_RM, const void* up_RM,
                              const int32_t* offsets_E1, int64_t R, int64_t M, int64_t D, int64_t E, int dtype,
                              void* dgate_RM, void* dup_RM, void* stream);

/* Backward of moe.py:80 (wgrad): dw_down[e] = h_e^T dy_e; zero for empty experts.
 * tile_ctr: ABACUS_MOE_TILE_CTR_INTS ints of workspace. */
int abacus_moe_down_bwd_wgrad(const void* h_RM, const void* dy_RD, const int32_t* offsets_E1, int64_t R, int64_t M,
                              int64_t D, int64_t E, int dtype, void* dw_down_EMD, int32_t* tile_ctr, void* stream);

/* Backward of moe.py:80, both halves in one launch: abacus_moe_down_bwd_dgrad
 * and abacus_moe_down_bwd_wgrad on the same operands (the weight gradient's
 * short per-expert tiles fill the CUs the data gradient's last round leaves
 * idle).  Outputs are those two calls' outputs, bit for bit.  tile_ctr: as above. */
int abacus_moe_down_bwd(const void* dy_RD, const void* w_down_EMD, const void* gate_RM, const void* up_RM,
                        const void* h_RM, const int32_t* offsets_E1, int64_t R, int64_t M, int64_t D, int64_t E,
                        int dtype, void* dgate_RM, void* dup_RM, void* dw_down_EMD, int32_t* tile_ctr,
                        void* stream);

/* Backward of moe.py:78-79 (dgrad): dx_perm = dgate @ w_gate[e]^T + dup @ w_up[e]^T. */
int abacus_moe_gateup_bwd_dgrad(const void* dgate_RM, const void* dup_RM, const void* w_gate_EDM,
                                const void* w_up_EDM, const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M,
                                int64_t E, int dtype, void* dx_perm_RD, void* stream);

/* Backward of moe.py:78-79 (wgrad): dw_gate[e] = x_e^T dgate_e, dw_up[e] = x_e^T dup_e.
 * tile_ctr: ABACUS_MOE_TILE_CTR_INTS ints of workspace. */
int abacus_moe_gateup_bwd_wgrad(const void* x_perm_RD, const void* dgate_RM, const void* dup_RM,
                                const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M, int64_t E, int dtype,
                                void* dw_gate_EDM, void* dw_up_EDM, int32_t* tile_ctr, void* stream);

/* Backward of moe.py:78-79, both halves in one launch: abacus_moe_gateup_bwd_dgrad
 * and abacus_moe_gateup_bwd_wgrad on the same operands.  Outputs are those two
 * calls' outputs, bit for bit.  tile_ctr: as above. */
int abacus_moe_gateup_bwd(const void* dgate_RM, const void* dup_RM, const void* w_gate_EDM, const void* w_up_EDM,
                          const void* x_perm_RD, const int32_t* offsets_E1, int64_t R, int64_t D, int64_t M,
                          int64_t E, int dtype, void* dx_perm_RD, void* dw_gate_EDM, void* dw_up_EDM,
                          int32_t* tile_ctr, void* stream);

/* Backward of the gather of moe.py:77 plus the router GEMM of router.py:45
 * (dgrad): dx[t] = sum_k dx_perm[pos(t,k)] + sum_k dlogit(t,k) w_DE[:, e(t,k)].
 * dx_perm_RD may be NULL (router used on its own).  wt_ws receives the
 * transposed router weights; with w_DE NULL it must already hold them, as
 * abacus_moe_router_fwd left them for the same weights. */
int abacus_moe_unpermute_bwd(const void* dx_perm_RD, const void* dlogit_TK, const int32_t* idx_TK,
                             const int32_t* pos_TK, const void* w_DE, void* wt_ws, int64_t T, int64_t D, int64_t E,
                             int64_t K, int dtype, void* dx_TD, void* stream);

/* Backward of the router GEMM of router.py:45 (wgrad): dw_DE = x^T dlogit. */
int abacus_moe_router_wgrad(const void* x_TD, const void* dlogit_TK, const int32_t* idx_TK, int64_t T, int64_t D,
                            int64_t E, int64_t K, int dtype, float* partial_ws, void* dw_DE, void* stream);

/* No counterpart in the reference: abacus_moe_router_wgrad for callers that cannot
 * allocate (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  The same kernels and the same result bit for bit, with the partial
 * sums in a static 32 MiB device array of the library (one per GPU, held until the
 * process ends) instead of partial_ws.  Shapes whose partial sums need more than
 * 32 MiB are rejected (1) before any launch; abacus_moe_router_wgrad_ws_bytes(T, D, E,
 * dtype) is that need.  The array used is the one of the stream's device, which must be
 * the current device (a stream of another device is rejected (1); the null stream is the
 * current device's).  Calls that overlap on one GPU share that array and race. */
int abacus_moe_router_wgrad_noalloc(const void* x_TD, const void* dlogit_TK, const int32_t* idx_TK, int64_t T,
                                    int64_t D, int64_t E, int64_t K, int dtype, void* dw_DE, void* stream);

/* Backward of router.py:49-51 and the sigmoid of :45 when Router.forward is
 * used on its own: dL/dweights -> dlogit_TK. */
int abacus_router_gating_bwd(const void* dweights_TK, const void* weights_TK, const void* score_TK, int64_t T,
                             int64_t K, double route_scale, int dtype, void* dlogit_TK, void* stream);

/* Router.update_bias (router.py:57-70) for an explicit int64 index tensor. */
int abacus_router_update_bias(const int64_t* indices_i64, int64_t N, int64_t E, double speed, int dtype,
                              void* bias_E, void* stream);

/* ---- auxiliary loss -------------------------------------------------------- */

/* load_balancing.py:30-41 (Switch-Transformer auxiliary loss) on (T, E) router
 * probabilities and (T, K) int64 expert slots: f_E = distinct-expert count per
 * token / (T*K) (one_hot(...).amax(1), :36-38), p_E = column mean in fp32 (:39),
 * loss = sum(f_E * p_E) * coeff_e (:40) with coeff_e = coeff * E as fp32,
 * written as fp32 and in `dtype` (:41).  f_E (E fp32) is kept for the backward.
 * Slots outside [0, E) set bad_index (bit 0: negative, bit 1: >= E) for the
 * caller to raise on, as torch.nn.functional.one_hot does; T must be > 0 (the
 * reference returns a zero without computing anything).  Deterministic. */
int abacus_moe_load_balancing_fwd(const void* probs_TE, const int64_t* slots_TK, int64_t T, int64_t E, int64_t K,
                                  double coeff_e, int dtype, void* ws, float* f_E, float* loss_f32, void* loss_out,
                                  int32_t* bad_index, void* stream);

/* Autograd of the above with respect to the probabilities: grad_probs[t, e] =
 * ((g * coeff_e) * f_E[e]) / T in fp32, rounded to `dtype`, g = the loss
 * gradient (one `dtype` element on the device). */
int abacus_moe_load_balancing_bwd(const void* grad_loss, const float* f_E, int64_t T, int64_t E, double coeff_e,
                                  int dtype, void* grad_probs_TE, void* stream);

/* ---- the decoder around the MoE layer ---------------------------------------- */

/* RMSNorm.forward (norm.py:26-31): y = gamma * x / sqrt(mean(x^2) + eps) over
 * the last dimension of `rows` contiguous rows of D elements (x, gamma and y
 * in `dtype`), in fp32 with one rounding per output; rstd (rows fp32) gets
 * 1 / sqrt(mean(x^2) + eps) for the backward.  D a multiple of 8 (bf16) or 4
 * (fp32), at most 4096 (bf16) or 2048 (fp32). */
int abacus_rmsnorm_fwd(const void* x, const void* gamma, int64_t rows, int64_t D, float eps, int dtype, void* y,
                       float* rstd, void* stream);

/* fp32 workspace bytes for abacus_rmsnorm_bwd. */
int64_t abacus_rmsnorm_bwd_ws_bytes(int64_t rows, int64_t D);

/* Autograd of RMSNorm.forward: dx = r * gamma * dy - x * r^3 * sum(gamma * dy * x) / D
 * per row (r = rstd), dgamma = sum over rows of dy * x * r (added in a fixed
 * order: deterministic). */
int abacus_rmsnorm_bwd(const void* dy, const void* x, const void* gamma, const float* rstd, int64_t rows, int64_t D,
                       int dtype, void* dx, void* dgamma, float* ws, int64_t ws_bytes, void* stream);

/* The attention's q/k norm followed by the rotary embedding
 * (attention.py:126-131, rope.py:36-46): for the rows = B*L*H rows (b, l, h)
 * of a contiguous (B, L, H, K) tensor, out = u * cos[l] + rotate_half(u) * sin[l]
 * with u = RMSNorm(row) as above and cos_LK, sin_LK (L, K) in `dtype`.  K/8 (bf16)
 * or K/4 (fp32) a power of two from 2 to 64. */
int abacus_rmsnorm_rope_fwd(const void* x, const void* gamma, const void* cos_LK, const void* sin_LK, int64_t rows,
                            int64_t L, int64_t H, int64_t K, float eps, int dtype, void* y, float* rstd,
                            void* stream);

/* Autograd of abacus_rmsnorm_rope_fwd: the transposed rotation of dy, then the
 * norm's backward (workspace: abacus_rmsnorm_bwd_ws_bytes(rows, K)). */
int abacus_rmsnorm_rope_bwd(const void* dy, const void* x, const void* gamma, const float* rstd, const void* cos_LK,
                            const void* sin_LK, int64_t rows, int64_t L, int64_t H, int64_t K, int dtype, void* dx,
                            void* dgamma, float* ws, int64_t ws_bytes, void* stream);

/* Causal attention forward (attention.py:136-141), flash style: for the
 * B*H (batch, head) pairs of q, k, v in (B, L, H, K) layout (token rows of
 * H*K contiguous elements, bf16, K = 64, L a multiple of 128),
 * o = softmax(mask(q k^T * scale)) v in the same layout, with the scores and
 * probabilities kept on chip in fp32 (the reference rounds them to the
 * activation dtype) and o rounded once; lse_BHL (fp32, (B, H, L)) gets each
 * query's log2-sum-exp2 of its base-2 scaled scores (max + log2(sum)), which
 * the backward uses to rebuild the probabilities. */
int abacus_attention_fwd(const void* q_BLHK, const void* k_BLHK, const void* v_BLHK, int64_t B, int64_t L, int64_t H,
                         int64_t K, float scale, int dtype, void* o_BLHK, float* lse_BHL, void* stream);

/* Bytes of fp32 workspace abacus_attention_bwd needs (one value per query). */
int64_t abacus_attention_bwd_ws_bytes(int64_t B, int64_t L, int64_t H);

/* Causal attention backward: the gradients of abacus_attention_fwd's o with
 * respect to q, k and v (what autograd derives for attention.py:136-141), from
 * q, k, v, the forward's o and lse_BHL, and dout = dL/do, all in the forward's
 * layouts and restrictions.  Probabilities are rebuilt from lse_BHL in fp32;
 * with D = rowsum(dout * o), dz = P (dout v^T - D), dq = scale dz k,
 * dk = scale dz^T q, dv = P^T dout, each rounded once to bf16.  ws: device
 * workspace of abacus_attention_bwd_ws_bytes bytes (16-byte aligned). */
int abacus_attention_bwd(const void* q_BLHK, const void* k_BLHK, const void* v_BLHK, const void* o_BLHK,
                         const void* dout_BLHK, const float* lse_BHL, int64_t B, int64_t L, int64_t H, int64_t K,
                         float scale, int dtype, void* dq_BLHK, void* dk_BLHK, void* dv_BLHK, float* ws,
                         int64_t ws_bytes, void* stream);

/* Cross-entropy of the decoder's logits (kernels/liger.py:12-47, called at
 * trainer.py:81-85), forward: for the N rows of logits_NV ((N, V), `dtype`)
 * with int64 targets_N, lse_N[i] = log(sum_j exp(x_ij)) and
 * loss_N[i] = lse_N[i] - x_i[t_i] in fp32, loss_N[i] = 0 where t_i equals
 * ignore_index (or lies outside [0, V)).  The mean loss is
 * sum(loss_N) / (number of rows not ignored), as the reference's reduction. */
int abacus_cross_entropy_fwd(const void* logits_NV, const int64_t* targets_N, int64_t N, int64_t V,
                             int64_t ignore_index, int dtype, float* lse_N, float* loss_N, void* stream);

/* Cross-entropy backward: dlogits_NV[i][j] = g * scale * (exp(x_ij - lse_N[i])
 * - [j == t_i]) with g = grad_loss[0] (device memory, fp32) and scale
 * 1 / (rows not ignored) for the mean; rows whose target is ignored get 0.
 * Rounded once to `dtype`. */
int abacus_cross_entropy_bwd(const void* logits_NV, const int64_t* targets_N, const float* lse_N,
                             const float* grad_loss, float scale, int64_t N, int64_t V, int64_t ignore_index,
                             int dtype, void* dlogits_NV, void* stream);

/* One AdamW step (optimizers/adamw.py:85-119, AdamW.step) over n tensors in
 * as few launches as possible: for tensor i, params[i], grads[i], exp_avgs[i]
 * and exp_avg_sqs[i] hold numels[i] contiguous elements of `dtype` (16-byte
 * aligned device memory), and steps[i] is its step count after this step's
 * increment.  params, grads, exp_avgs, exp_avg_sqs, numels and steps are host
 * arrays.  Every element goes through the reference's tensor-op sequence with
 * a rounding to `dtype` after each op:
 *   p = p*(1 - lr*wd); m = lerp(m, g, 1 - beta1); v = v*beta2 + (1 - beta2)*(g*g);
 *   d = sqrt(v) / sqrt(1 - beta2^step) + eps; p = p + (-lr / (1 - beta1^step)) * (m / d)
 * in fp32, in the forms of torch's device kernels: the lerp, the (1 - beta2)
 * product and the final update are fused multiply-adds, division by
 * sqrt(1 - beta2^step) is a product with its reciprocal (taken in double), and
 * the scalars are the double-precision values rounded to fp32. */
int abacus_adamw_step(void* const* params, const void* const* grads, void* const* exp_avgs, void* const* exp_avg_sqs,
                      const int64_t* numels, const int64_t* steps, int n, double lr, double beta1, double beta2,
                      double eps, double weight_decay, int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ABACUS_MOE_H */
