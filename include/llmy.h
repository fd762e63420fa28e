/*
 * libllmy — MI355X (gfx950) kernels for the LLMY hybrid-block inference hot
 * path, exported as a plain C ABI so ctypes (or any FFI) can bind them.
 *
 * Conventions shared by every entry point below:
 *   - All tensor pointers are device pointers to contiguous, caller-owned
 *     buffers.  bf16 tensors are passed as llmy_bf16 (the raw 16-bit word).
 *     No entry point allocates or frees device memory.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream); work is
 *     enqueued on it and the call returns without synchronising.
 *   - The return value is a hipError_t: 0 on success; hipErrorInvalidValue
 *     (1) when an argument fails validation, returned before anything is
 *     launched; otherwise the launch status (hipGetLastError).
 *   - A size of 0 along the token/batch axis is a valid no-op.
 *   Conventions follow the reference op hooks: llmy_cuda/include/llmy.h:74-88
 *   and their validation in llmy_cuda/src/llmy.cpp:213-240.
 */
#ifndef LLMY_H
#define LLMY_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t llmy_bf16;

/* --- Library identity ---------------------------------------------------- */

/* Version of this ABI; bumped when a signature changes.  No counterpart in
 * the reference (a probe for bindings). */
int32_t llmy_abi_version(void);

/* --- Router (model/layers/context_router.py:62,71-74) --------------------- */

/* logits[t,e] = (RMSNorm(x[t]) * norm_w) . w_router[e] in fp32 (norm skipped
 * when norm_w == NULL), then the k largest logits per token (descending,
 * ties -> lower expert index) and gates = softmax over those k values.
 * x [T,D] bf16, norm_w [D] fp32 or NULL, w_router [E,D] fp32,
 * logits_out [T,E] fp32 or NULL, idx [T,k] int32, gates [T,k] fp32.
 * Limits: D % 4 == 0, D <= 8192, E <= 256, k <= min(E, 32).
 * Replaces the router of SparseMoE.forward (model/layers/moe.py:180) and the
 * native router_topk_kernel (llmy_cuda/src/kernels/router.cu:14-132). */
int32_t llmy_router_topk_bf16(const llmy_bf16* x, const float* norm_w,
                              const float* w_router, float* logits_out,
                              int32_t* idx, float* gates, int32_t T, int32_t D,
                              int32_t E, int32_t k, float eps, void* stream);

/* Top-k + softmax of precomputed fp32 logits [T,E] (same tie rule).
 * Replaces torch.topk(...).softmax (context_router.py:73-74). */
int32_t llmy_router_topk_logits_f32(const float* logits, int32_t* idx,
                                    float* gates, int32_t T, int32_t E,
                                    int32_t k, void* stream);

/* --- MoE token permutation (model/layers/moe.py:39-66) -------------------- */

/* Stable counting sort of n_routes expert ids (flat route r = t*k + j):
 * counts [E], offsets [E+1] (exclusive cumsum, offsets[E] = n_routes),
 * sorted_routes [n_routes] (route ids grouped by expert, ascending r inside an
 * expert), route_pos [n_routes] (inverse: sorted position of route r).
 * Ids outside [0,E) are not placed.  E <= 1024. */
int32_t llmy_moe_permute(const int32_t* expert_ids, int32_t n_routes,
                         int32_t E, int32_t* counts, int32_t* offsets,
                         int32_t* sorted_routes, int32_t* route_pos,
                         void* stream);

/* --- Dense projections ---------------------------------------------------- */

/* Y[M,N] = X[M,K] . W[N,K]^T, bf16 operands, fp32 accumulation, with a fused
 * epilogue: 0 = store bf16 into out [M,N]; 1 = store fp32; 2 = out (fp32)
 * += Y (residual add); 3 = out (fp32) += Y * aux[M,N] (gated residual);
 * 4 = per-K-block partial products, M <= 64: out (fp32) [K/256, M, N], slice
 * s = X[:, 256s:256s+256] . W[:, 256s:256s+256]^T, for a consumer that folds
 * the slices in order (llmy_moe_route_decode).
 * weight_layout 0: W row-major [N,K] (nn.Linear); 1: W in the packed tile
 * order of llmy_pack_weights_bf16.  Limits: N % 16 == 0, K % 256 == 0.
 * M < 256 (decode batches): weight-streaming kernels; M >= 256 (prefill
 * sequences) with a 16-byte aligned out: MFMA tiles (128 x 128 per workgroup).
 * Replaces linear_forward / k_linear_gemv (llmy_cuda/src/model.cpp:1467-1515)
 * and nn.Linear on the decode and prefill paths. */
int32_t llmy_linear_bf16(const llmy_bf16* x, const llmy_bf16* w, void* out,
                         const float* aux, int32_t M, int32_t N, int32_t K,
                         int32_t epilogue, int32_t weight_layout, void* stream);

/* Re-lay batch row-major [N,K] bf16 matrices into the operand order the
 * weight-streaming kernels read (for each 16-row block and 256-wide K
 * block, 8 tiles of 64 lanes x 8 elements; tile j lane l element e =
 * W[16*nb + l%16][256*kb + 32*j + 8*(l/16) + e]), so a wavefront's operand
 * load is one contiguous KiB.  Same element count; out must not alias w.
 * No counterpart in the reference (a load-time layout transform). */
int32_t llmy_pack_weights_bf16(const llmy_bf16* w, llmy_bf16* out, int64_t batch,
                               int32_t N, int32_t K, void* stream);

/* --- SwiGLU MoE experts (model/layers/moe.py:72-81, expert.py:14-15) ------ */

/* For every route p (sorted by expert, from llmy_moe_permute):
 *   act[p] = bf16(silu(Wg[e] x[t]) * (Wu[e] x[t])),  t = sorted_routes[p] / k
 *   y[p]   = gates[sorted_routes[p]] * (Wd[e] act[p])           (fp32)
 * x [T,D] bf16; w_gate_up [E,2H,D] bf16 (gate rows then up rows, the packing
 * of llmy.h:80-82 in the reference); w_down [E,D,H] bf16; gates [T*k] fp32;
 * act [T*k,H] bf16 and y [T*k,D] fp32 are caller-provided scratch.  Experts
 * with no routes read no weights.  weight_layout as in llmy_linear_bf16
 * (packed: each expert's [2H,D] and [D,H] packed separately).
 * Limits: D % 256 == 0, H % 256 == 0. */
int32_t llmy_moe_experts_bf16(const llmy_bf16* x, const int32_t* offsets,
                              const int32_t* sorted_routes, const float* gates,
                              const llmy_bf16* w_gate_up, const llmy_bf16* w_down,
                              llmy_bf16* act, float* y, int32_t T, int32_t D,
                              int32_t H, int32_t E, int32_t k, int32_t weight_layout,
                              void* stream);

/* Route-indexed variant for small T*k (<= 2048, the decode path): no
 * permutation is materialised.  The workgroups of expert e derive the routes
 * {r : ids[r] == e} themselves (wavefront ballots over ids [T*k], ascending r)
 * and read x[r / k]; act [T*k,H] and y [T*k,D] are indexed by route id:
 *   act[r] = bf16(silu(Wg[e] x[r/k]) * (Wu[e] x[r/k])),  y[r] = gates[r] * (Wd[e] act[r]).
 * Same arithmetic as llmy_moe_experts_bf16. */
int32_t llmy_moe_experts_routed_bf16(const llmy_bf16* x, const int32_t* ids,
                                     const float* gates, const llmy_bf16* w_gate_up,
                                     const llmy_bf16* w_down, llmy_bf16* act, float* y,
                                     int32_t T, int32_t D, int32_t H, int32_t E,
                                     int32_t k, int32_t weight_layout, void* stream);

/* out[t] = sum_j y[route_pos[t*k + j]] (j ascending) — the un-permute /
 * combine of moe.py:78-81 without atomics.  mode 0: store bf16 out [T,D];
 * 1: store fp32; 2: fp32 out += sum (residual add).  D % 4 == 0. */
int32_t llmy_moe_combine(const float* y, const int32_t* route_pos, void* out,
                         int32_t T, int32_t D, int32_t k, int32_t mode,
                         void* stream);

/* --- Banded attention, prefill (runpod/kernels/fused_attention.py:6-41) --- */

/* o_i = sum_{j: 0 <= i-j < W} softmax_j(scale * q_i . k_j) v_j per (b, h), fp32
 * scores/accumulation.  q, k, v, o [B,T,H,head_dim] bf16; head_dim in {64,128}.
 * Replaces the Triton _banded_attn_fwd_kernel
 * (runpod/kernels/triton_banded_attention.py:23-90) and banded_attn_kernel
 * (llmy_cuda/src/kernels/attn.cu:17-126); rows whose window holds no valid
 * key cannot occur (every query sees itself). */
int32_t llmy_banded_attn_prefill_bf16(const llmy_bf16* q, const llmy_bf16* k,
                                      const llmy_bf16* v, llmy_bf16* o, int32_t B,
                                      int32_t T, int32_t H, int32_t head_dim, int32_t W,
                                      float scale, void* stream);

/* --- Banded attention, decode (model/layers/hca.py:119-128) --------------- */

/* One query per (b, h) against a ring-buffer cache k_cache/v_cache
 * [B,H,W,head_dim] bf16.  The new key/value are written to slot pos[b] % W,
 * then o = softmax(scale * q.K^T) V over the last min(pos[b] + 1, W) tokens
 * (the new one included).  q, k_new, v_new: head h of batch row b starts at
 * b*stride + h*head_dim (q_bstride / kv_bstride elements per batch row, so
 * a fused [B, 3*H*hd] projection can be passed directly).  out [B,H,hd] bf16.
 * head_dim in {64, 128}.  Replaces local_attn_decode_kernel
 * (llmy_cuda/src/kernels/attn.cu:135-229). */
int32_t llmy_banded_attn_decode_bf16(const llmy_bf16* q, const llmy_bf16* k_new,
                                     const llmy_bf16* v_new, int64_t q_bstride,
                                     int64_t kv_bstride, llmy_bf16* k_cache,
                                     llmy_bf16* v_cache, const int32_t* pos,
                                     llmy_bf16* out, int32_t B, int32_t H,
                                     int32_t head_dim, int32_t W, float scale,
                                     void* stream);
/* The same step with q, k_new and v_new given as the partial products of a
 * decode projection (llmy_linear_bf16 with epilogue 4): parts [nparts][B][row_stride]
 * fp32, part_stride floats apart; q at column 0, k at k_off, v at v_off.  The
 * slices are summed in order and rounded to bf16 -- the values the projection
 * would have stored as bf16 -- so it computes what the call above computes on
 * that projection.  No counterpart in the reference: it lets the decode step
 * run its q/k/v projection on the partial-product kernel. */
int32_t llmy_banded_attn_decode_parts_bf16(const float* parts, int32_t nparts,
                                           int64_t part_stride, int64_t row_stride,
                                           int32_t k_off, int32_t v_off, llmy_bf16* k_cache,
                                           llmy_bf16* v_cache, const int32_t* pos,
                                           llmy_bf16* out, int32_t B, int32_t H,
                                           int32_t head_dim, int32_t W, float scale,
                                           void* stream);

/* --- Gated delta rule, prefill (chunked; model/layers/gated_deltanet.py:140-149) */

/* Workspace (bytes) that llmy_gdn_prefill_bf16 needs for (B, T, H, dk, dv):
 * per 64-token chunk W [64,dk], U0 [64,dv], A [64,64] and 2 x 64 decay
 * factors, fp32.  No counterpart in the reference. */
int64_t llmy_gdn_prefill_workspace_bytes(int32_t B, int32_t T, int32_t H, int32_t dk,
                                         int32_t dv);

/* The recurrence over T tokens, chunked (C = 64) with the exact transition
 * A_t = g_t I - beta_t k_t k_t^T of the reference:
 *   S_t = g_t S_{t-1} + beta_t k_t (v_t - S_{t-1}^T k_t)^T,  out_t = S_t^T q_t.
 * q, k [B,T,H,dk], v [B,T,H,dv] bf16; beta, g [B,T,H] fp32 (g in (0,1]);
 * state [B,H,dk,dv] fp32 in/out (initial -> final); out [B,T,H,dv] bf16.
 * (dk,dv) in {(64,64),(128,128)}.  Replaces the sequential scans of
 * gated_deltanet.py:42-53,236-252 and runpod/kernels/triton_gdn.py:57-118. */
int32_t llmy_gdn_prefill_bf16(const llmy_bf16* q, const llmy_bf16* k, const llmy_bf16* v,
                              const float* beta, const float* g, float* state,
                              llmy_bf16* out, void* workspace, int64_t workspace_bytes,
                              int32_t B, int32_t T, int32_t H, int32_t dk, int32_t dv,
                              void* stream);

/* No counterpart in the reference: llmy_gdn_prefill_bf16 for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments, arithmetic and
 * results, without the workspace pair: the library keeps a fixed 64 MiB
 * workspace per GPU (a static device array, held from module load to process
 * end), enough for llmy_gdn_prefill_workspace_bytes(B, T, H, dk, dv) <= 64 MiB
 * (e.g. 1024 chunks of 64 tokens x heads at dk = dv = 64, 816 at 128).
 * Larger sizes return hipErrorOutOfMemory (2) before anything runs.  Calls
 * that overlap on one GPU (other streams, other threads) share that
 * workspace and race; each call fully rewrites the part it reads. */
int32_t llmy_gdn_prefill_bf16_noalloc(const llmy_bf16* q, const llmy_bf16* k,
                                      const llmy_bf16* v, const float* beta, const float* g,
                                      float* state, llmy_bf16* out, int32_t B, int32_t T,
                                      int32_t H, int32_t dk, int32_t dv, void* stream);

/* --- Gated delta rule, decode (model/layers/gated_deltanet.py:140-149) ---- */

/* pred = k^T S; S <- g S + beta k (v - pred)^T (in place); out = (q^T S) * gate.
 * q, k [B,H,dk], v [B,H,dv], gate [B,H,dv] or NULL (bf16); beta, g [B,H] fp32;
 * state [B,H,dk,dv] fp32; out [B,H,dv] bf16.  (dk,dv) in {(64,64),(128,128)}.
 * Replaces gdn_step_kernel (llmy_cuda/src/kernels/gdn.cu:22-87). */
int32_t llmy_gdn_step_bf16(const llmy_bf16* q, const llmy_bf16* k,
                           const llmy_bf16* v, const float* beta, const float* g,
                           const llmy_bf16* gate, float* state, llmy_bf16* out,
                           int32_t B, int32_t H, int32_t dk, int32_t dv,
                           void* stream);

/* The GDN block's step from its fused fp32 projection row
 * proj[b] = [q (H*dk) | k (H*dk) | v (H*dv) | gate logits (H*dv) | beta logits (H)]:
 * q, k L2-normalised per head (clamp 1e-12), beta = sigmoid(logit + beta_bias),
 * gate = sigmoid(logit), g = sigmoid(decay_logit[h]) (gated_deltanet.py:125-132),
 * then the step above; out [B, H*dv] bf16.  When conv_h != NULL the causal
 * conv gate of llmy_gdn_conv_gate is computed in the same launch
 * (conv_h [B,D] bf16 mixer input, conv_hist [B,3,D], conv_w [D,4],
 * conv_out [B,D] fp32; D % H == 0, conv_kernel == 4).  nparts in [1, 8]: proj
 * holds nparts slices [nparts, B, proj_ld] (the per-K-block partial products
 * of llmy_linear_bf16 epilogue 4), summed in slice order; 1 = the row itself. */
int32_t llmy_gdn_step_fused_f32(const float* proj, int64_t proj_ld, int32_t nparts,
                                const float* beta_bias, const float* decay_logit,
                                float* state, llmy_bf16* out, const llmy_bf16* conv_h,
                                llmy_bf16* conv_hist, const float* conv_w,
                                float* conv_out, int32_t D, int32_t conv_kernel,
                                int32_t B, int32_t H, int32_t dk, int32_t dv,
                                void* stream);

/* Causal depthwise conv gate for one new token (gated_deltanet.py:257-268):
 * out[b,d] = sigmoid(sum_j w[d,j] * [hist[b,0..K-2,d], h[b,d]]_j), then the
 * history [B,K-1,D] bf16 shifts by one.  kernel == 4. */
int32_t llmy_gdn_conv_gate(const llmy_bf16* h, llmy_bf16* hist, const float* w,
                           float* out, int32_t B, int32_t D, int32_t kernel,
                           void* stream);

/* --- Sequence prefill glue ------------------------------------------------
 * The reference prefills token by token through its decode step
 * (model_prefill, llmy_cuda/src/model.cpp:1955-1966, behind llmy_prefill,
 * llmy_cuda/include/llmy.h:51-53).  These entries let a caller prefill a
 * whole [B, T] prompt with the sequence kernels above instead. */

/* K/V rows of a prompt (k, v [B*T rows, ld] bf16, head h at columns
 * h*head_dim..) into the ring caches [B, H, W, head_dim] of
 * llmy_banded_attn_decode_bf16: position t in [max(0, T-W), T) goes to slot
 * t % W (the decode window of model/layers/hca.py:119-128). */
int32_t llmy_kv_cache_fill_bf16(const llmy_bf16* k, const llmy_bf16* v, int64_t ld,
                                llmy_bf16* k_cache, llmy_bf16* v_cache, int32_t B,
                                int32_t T, int32_t H, int32_t head_dim, int32_t W,
                                void* stream);

/* Per-token GDN inputs for llmy_gdn_prefill_bf16 from the fused fp32
 * projection rows of llmy_gdn_step_fused_f32 (proj [rows, ld]): q, k
 * [rows, H, dk] bf16 L2-normalised (clamp 1e-12), v [rows, H, dv] bf16,
 * beta = sigmoid(logit + beta_bias) and g = sigmoid(decay_logit[h]) as
 * [rows, H] fp32 (gated_deltanet.py:124-132).  dk in {64, 128, 256}. */
int32_t llmy_gdn_prefill_prep_f32(const float* proj, int64_t ld,
                                  const float* beta_bias, const float* decay_logit,
                                  llmy_bf16* q, llmy_bf16* k, llmy_bf16* v,
                                  float* beta, float* g, int32_t rows, int32_t H,
                                  int32_t dk, int32_t dv, void* stream);

/* Output gate of a GDN scan (gated_deltanet.py:176,247):
 * out[r, j] = bf16(o[r, j] * sigmoid(proj[r, gate_off + j])) for o
 * [rows, HV] bf16 (may alias out) and fp32 gate logits read in place from
 * proj [rows, ld].  HV % 8 == 0, ld and gate_off multiples of 4. */
int32_t llmy_gdn_gate_bf16(const llmy_bf16* o, const float* proj, int64_t ld,
                           int32_t gate_off, llmy_bf16* out, int32_t rows, int32_t HV,
                           void* stream);

/* Causal depthwise conv gate over a sequence with carried history
 * (gated_deltanet.py:254-269): h [B,T,D] bf16, hist [B,K-1,D] bf16 (read,
 * then set to the last K-1 entries of [hist, h]), w [D,K] fp32, out [B,T,D]
 * fp32 = sigmoid(conv).  Equal to T calls of llmy_gdn_conv_gate.  kernel == 4. */
int32_t llmy_gdn_conv_gate_prefill(const llmy_bf16* h, llmy_bf16* hist, const float* w,
                                   float* out, int32_t B, int32_t T, int32_t D,
                                   int32_t kernel, void* stream);

/* --- Per-row resets of the GDN recurrence (gated_deltanet.py:138-142,165-166:
 * the state is zeroed before token t's update where reset[b, t]; :56-78: conv
 * taps do not cross a reset, and :262-266: a reset clears the conv history).
 * reset arrays are device int32, nonzero = reset.  The reference's native
 * step takes a per-head mask for its one sequence (llmy_cuda/src/kernels/
 * gdn.cu:28,36-40); these take one flag per batch row (all heads).  Each is
 * the entry of the same name without "_reset" plus the mask, with the same
 * arithmetic where no reset is set. */

/* llmy_gdn_prefill_bf16 with reset [B, T]: a reset at token t starts a new
 * segment (the state entering token t is zero). */
int32_t llmy_gdn_prefill_reset_bf16(const llmy_bf16* q, const llmy_bf16* k, const llmy_bf16* v,
                                    const float* beta, const float* g, const int32_t* reset,
                                    float* state, llmy_bf16* out, void* workspace,
                                    int64_t workspace_bytes, int32_t B, int32_t T, int32_t H,
                                    int32_t dk, int32_t dv, void* stream);

/* llmy_gdn_step_bf16 with reset [B]: row b starts from a zero state. */
int32_t llmy_gdn_step_reset_bf16(const llmy_bf16* q, const llmy_bf16* k, const llmy_bf16* v,
                                 const float* beta, const float* g, const llmy_bf16* gate,
                                 const int32_t* reset, float* state, llmy_bf16* out, int32_t B,
                                 int32_t H, int32_t dk, int32_t dv, void* stream);

/* llmy_gdn_step_fused_f32 with reset [B]: row b starts from a zero state and
 * a zero conv history. */
int32_t llmy_gdn_step_fused_reset_f32(const float* proj, int64_t proj_ld, int32_t nparts,
                                      const float* beta_bias, const float* decay_logit,
                                      const int32_t* reset, float* state, llmy_bf16* out,
                                      const llmy_bf16* conv_h, llmy_bf16* conv_hist,
                                      const float* conv_w, float* conv_out, int32_t D,
                                      int32_t conv_kernel, int32_t B, int32_t H, int32_t dk,
                                      int32_t dv, void* stream);

/* llmy_gdn_conv_gate_prefill with reset [B, T]: the tap at position p counts
 * for token t only if no reset lies in (p, t] (history taps: none in [0, t]);
 * the new history is the last 3 inputs, zero where they precede the last
 * reset (what a token-by-token pass leaves). */
int32_t llmy_gdn_conv_gate_prefill_reset(const llmy_bf16* h, llmy_bf16* hist, const float* w,
                                         const int32_t* reset, float* out, int32_t B, int32_t T,
                                         int32_t D, int32_t kernel, void* stream);

/* Zero row b of a [rows, row_bytes] buffer wherever mask[b] != 0 (device int32
 * [rows]): the per-row state reset of model/recurrent_state.py:213-225 applied
 * to one state buffer (GDN states, conv histories, KV rings, router latent
 * rings, positions).  A kernel, so a captured graph may hold it; row_bytes a
 * multiple of 4. */
int32_t llmy_zero_rows(void* base, int64_t row_bytes, int32_t rows, const int32_t* mask,
                       void* stream);

/* --- Multi-stream hyper-connections (mHC) -------------------------------------
 * model/layers/mhc.py:156-231 around the block's sublayers (model/model.py:
 * 119-126,177-264); the reference's native twins are mhc_rmsnorm_flat,
 * mhc_gemv_small, mhc_activate, sinkhorn, mhc_read and mhc_write
 * (llmy_cuda/src/kernels/mhc.cu:26-443).  A token's residual is S streams
 * [S, D] fp32 (S = 2 or 4).  The maps' projection raw = theta . RMSNorm(X)
 * is the caller's: llmy_rmsnorm_f32_bf16 over the flattened [M, S*D] streams
 * (eps = fp32 epsilon, mhc.py:72) then llmy_linear_bf16 with theta. */

/* streams[m, s, :] = E[tokens[m], :] + seed[s, :]  (model.py:442-444) */
int32_t llmy_mhc_embed(const int32_t* tokens, const llmy_bf16* table, const float* seed,
                       float* streams, int32_t M, int32_t S, int32_t D, int32_t V,
                       void* stream);
/* Maps and read (mhc.py:156-206): from raw [M, raw_ld] (pre | post | residual
 * logits), pre = sigmoid(alpha[0] raw + pre_bias), post = 2 sigmoid(alpha[1] raw
 * + post_bias), R = Sinkhorn(alpha[2] raw + res_bias, iterations) -> maps
 * [M, S + S*S] (post, then R row-major); h [M, D] = bf16(RMSNorm(norm_w,
 * norm_eps)(LayerNorm(ln_w, ln_b, ln_eps)(sum_s pre_s X_s))), the sublayer
 * input.  D % 4 == 0, D <= 4096. */
int32_t llmy_mhc_read(const float* streams, const float* raw, int64_t raw_ld,
                      const float* pre_bias, const float* post_bias, const float* res_bias,
                      const float* alpha, int32_t iterations, const float* ln_w,
                      const float* ln_b, float ln_eps, const float* norm_w, float norm_eps,
                      float* maps, llmy_bf16* h, int32_t M, int32_t S, int32_t D, void* stream);
/* Write (mhc.py:208-227), in place: X_i += sigmoid(gating_logit[0]) scale[i] *
 * (sum_j R_ij X_j + post_i update[m]); update [M, update_ld] fp32. */
int32_t llmy_mhc_write(float* streams, const float* update, int64_t update_ld,
                       const float* maps, const float* scale, const float* gating_logit,
                       int32_t M, int32_t S, int32_t D, void* stream);
/* out[i] = bf16(x[i]), n % 4 == 0 (the collapse GEMM's operand, model.py:699). */
int32_t llmy_f32_to_bf16(const float* x, llmy_bf16* out, int64_t n, void* stream);
/* out [rows, Kp] = x [rows, K] with columns K .. Kp-1 zero (K <= Kp, both
 * even): the input of a GEMM whose weight was zero-padded from K inputs to
 * the kernels' multiple of 256 (the reference's mla.latent_dim 128 and
 * router query heads 4 x 32, runpod/config_a5000_moe24.yaml:47,50-51; the
 * reference's own GEMMs take any width, llmy_cuda/src/model.cpp:1497-1515). */
int32_t llmy_pad_cols_bf16(const llmy_bf16* x, llmy_bf16* out, int32_t rows, int32_t K,
                           int32_t Kp, void* stream);

/* --- Compressed-memory mixers, CSA and HCA (model/layers/csa.py:16-259,
 * hca.py:15-193, compressed_attention.py:82-211; the reference's native twins
 * are csa_local_attn_decode, csa_compress_step, csa_remote_attn_decode
 * (llmy_cuda/src/kernels/csa.cu) and hca_local_attn_decode, hca_compress_step,
 * hca_global_attn_decode, hca_global_topk_attn_decode (hca.cu:15-428), batch 1
 * only).  H heads of width head_dim score queries against keys (CSA: the index
 * heads; HCA: H = 1, head_dim = d_model), scale = 1/sqrt(head_dim); each head's
 * softmax probabilities are averaged over the heads and applied to one value
 * stream of width Dv.  q / k rows hold H*head_dim bf16, v rows Dv bf16, each at
 * its own row stride (elements, multiple of 8), outputs bf16 [rows, out_ld].
 * head_dim % 16 == 0, Dv % 8 == 0.  workspace: >= llmy_cmp_workspace_bytes,
 * 16-byte aligned.  Local branch: the last W tokens, the current one included.
 * Memory branch: summaries of complete ratio-token blocks, visible from the
 * block's last token on, dense softmax (top_k 0) or each head's top_k (<= 64;
 * ties to the lower index; no visible summary gives 0).  Decode memory: C
 * slots per row, keys [B, C, H*head_dim], values [B, C, Dv], tag [B, C] int32 =
 * position + 1 of the summary (0 = empty). */

/* Workspace bytes of one branch call for `queries` queries (prefill: B*T,
 * decode: B): slots = the local window W or the memory's entries / slots;
 * top_k 0 = dense lists (prefill with H > 1: plus the head-summed lists), else
 * top_k pairs; decode != 0 adds the raw scores the decode entries keep.  -1 on
 * bad sizes. */
int64_t llmy_cmp_workspace_bytes(int32_t queries, int32_t H, int32_t slots, int32_t top_k,
                                 int32_t decode);
/* Local branch over B fresh sequences of T tokens (rows b*T + t). */
int32_t llmy_cmp_local_prefill_bf16(const llmy_bf16* q, int64_t q_ld, const llmy_bf16* k,
                                    int64_t k_ld, const llmy_bf16* v, int64_t v_ld,
                                    llmy_bf16* out, int64_t out_ld, int32_t B, int32_t T,
                                    int32_t H, int32_t head_dim, int32_t Dv, int32_t W,
                                    float scale, void* workspace, int64_t workspace_bytes,
                                    void* stream);
/* Memory branch over B fresh sequences: n_entries = T / ratio summaries per row
 * (keys mk rows b*n + i, values mv rows b*n + i), summary i visible from
 * position (i + 1) ratio - 1 on; with slots_window > 0 (the decode memory's
 * slots per row) only while it is among the last slots_window summaries
 * emitted, as the token-by-token decode over that ring sees it (0: every
 * summary emitted so far, as csa.py:99-105 / hca.py:88-93).  n_entries <= 4000. */
int32_t llmy_cmp_memory_prefill_bf16(const llmy_bf16* q, int64_t q_ld, const llmy_bf16* mk,
                                     int64_t mk_ld, const llmy_bf16* mv, int64_t mv_ld,
                                     llmy_bf16* out, int64_t out_ld, int32_t B, int32_t T,
                                     int32_t n_entries, int32_t ratio, int32_t H,
                                     int32_t head_dim, int32_t Dv, int32_t top_k,
                                     int32_t slots_window, float scale, void* workspace,
                                     int64_t workspace_bytes, void* stream);
/* Local branch, one token per row at pos[b]: stores k_new / v_new (rows at
 * kv_ld) into ring slot pos % W of ring_k [B, W, H*head_dim] / ring_v [B, W, Dv]
 * and attends to keys max(0, pos - W + 1) .. pos. */
int32_t llmy_cmp_local_decode_bf16(const llmy_bf16* q, int64_t q_ld, const llmy_bf16* k_new,
                                   const llmy_bf16* v_new, int64_t kv_ld, llmy_bf16* ring_k,
                                   llmy_bf16* ring_v, const int32_t* pos, llmy_bf16* out,
                                   int64_t out_ld, int32_t B, int32_t H, int32_t head_dim,
                                   int32_t Dv, int32_t W, float scale, void* workspace,
                                   int64_t workspace_bytes, void* stream);
/* Memory branch, one token per row at pos[b], over the C slots (1 <= tag <= pos + 1). */
int32_t llmy_cmp_memory_decode_bf16(const llmy_bf16* q, int64_t q_ld, const llmy_bf16* mk,
                                    const llmy_bf16* mv, const int32_t* mtag, const int32_t* pos,
                                    llmy_bf16* out, int64_t out_ld, int32_t B, int32_t C,
                                    int32_t H, int32_t head_dim, int32_t Dv, int32_t top_k,
                                    float scale, void* workspace, int64_t workspace_bytes,
                                    void* stream);
/* Compressor, prefill (compressed_attention.py:105-123): means [B, T/ratio, D]
 * bf16 of the complete blocks of h (rows b*T + t); psum [B, D] fp32 / pcnt [B]
 * = the incomplete tail's sum and count. */
int32_t llmy_cmp_pool_prefill_bf16(const llmy_bf16* h, int64_t h_ld, llmy_bf16* means,
                                   float* psum, int32_t* pcnt, int32_t B, int32_t T, int32_t D,
                                   int32_t ratio, void* stream);
/* Compressor, decode (compressed_attention.py:177-207): psum += h, pcnt += 1,
 * mean = bf16(psum / pcnt); a row reaching ratio sets emit[b] = 1 and restarts
 * its sum and count (else emit[b] = 0). */
int32_t llmy_cmp_pool_step_bf16(const llmy_bf16* h, int64_t h_ld, float* psum, int32_t* pcnt,
                                llmy_bf16* mean, int32_t* emit, int32_t B, int32_t D,
                                int32_t ratio, void* stream);
/* Decode: rows with emit[b] store their summary kv[b] (Kw key channels, then
 * Dv value channels) at slot mcount[b] % C with tag pos[b] + 1; mcount += 1. */
int32_t llmy_cmp_commit_bf16(const llmy_bf16* kv, int64_t kv_ld, const int32_t* emit,
                             const int32_t* pos, llmy_bf16* mk, llmy_bf16* mv, int32_t* mtag,
                             int32_t* mcount, int32_t B, int32_t C, int32_t Kw, int32_t Dv,
                             void* stream);
/* Prefill: the last min(n, C) summaries of each row (kv rows b*n + i) into
 * slots i % C with tags (i + 1) * ratio; mcount[b] = n. */
int32_t llmy_cmp_memory_fill_bf16(const llmy_bf16* kv, int64_t kv_ld, llmy_bf16* mk,
                                  llmy_bf16* mv, int32_t* mtag, int32_t* mcount, int32_t B,
                                  int32_t n_entries, int32_t ratio, int32_t C, int32_t Kw,
                                  int32_t Dv, void* stream);
/* Prefill: the last min(T, W) rows of each sequence (src rows b*T + t) into
 * ring slots t % W of ring [B, W, width]. */
int32_t llmy_cmp_ring_fill_bf16(const llmy_bf16* src, int64_t src_ld, llmy_bf16* ring,
                                int32_t B, int32_t T, int32_t W, int32_t width, void* stream);

/* --- Glue (model/layers/norms.py:13-16, model/model.py:386) --------------- */

/* out[m] = bf16(x[m] * rsqrt(mean(x[m]^2) + eps) * w); x [M,D] fp32. */
int32_t llmy_rmsnorm_f32_bf16(const float* x, const float* w, llmy_bf16* out,
                              int32_t M, int32_t D, float eps, void* stream);

/* x[b] = float(table[tokens[b]]) (ids clamped to [0,V)); table [V,D] bf16. */
int32_t llmy_embed_bf16(const int32_t* tokens, const llmy_bf16* table, float* x,
                        int32_t B, int32_t D, int32_t V, void* stream);

/* x[b] = float(table[tokens[b]]); h[b] = bf16(RMSNorm(x[b]) * w) — embedding
 * gather fused with the first block's pre-norm.  D in {256,512,1024,2048}. */
int32_t llmy_embed_norm_bf16(const int32_t* tokens, const llmy_bf16* table,
                             const float* w, float* x, llmy_bf16* h, int32_t B,
                             int32_t D, int32_t V, float eps, void* stream);

/* MoE combine fused with the next pre-norm: x[t] += sum_j y[route_pos[t*k+j]]
 * (j ascending; route_pos == NULL means y is route-indexed, y[t*k+j]), then
 * h[t] = bf16(RMSNorm(x[t]) * w) unless w == NULL.
 * D in {256,512,1024,2048}. */
int32_t llmy_moe_combine_norm(const float* y, const int32_t* route_pos,
                              const float* w, float* x, llmy_bf16* h, int32_t T,
                              int32_t D, int32_t k, float eps, void* stream);

/* Shared experts (model/layers/moe.py:185-199; llmy_cuda/src/model.cpp:
 * 1205-1225 computes them in a loop after the routed ones) as always-on
 * routes: idx_out/gates_out [T, k+S] = the router's [T, k], then experts
 * E .. E+S-1 (the shared experts stacked after the routed ones in the expert
 * weights) with gate 1/sqrt(S) for every token.  The expert and combine
 * entries then run with k+S routes per token over E+S experts. */
int32_t llmy_moe_append_shared(const int32_t* idx, const float* gates, int32_t* idx_out,
                               float* gates_out, int32_t T, int32_t k, int32_t E,
                               int32_t S, void* stream);

/* Context-aware router, local-context branch (model/layers/context_router.py:
 * 59-76 for a prompt, :94-137 for a decode token; replaces the router half of
 * llmy_cuda/src/model.cpp:1110-1147 with its router_history_update_mean
 * :1253-1290).  Five launches route rows of h (the block's bf16 pre-MoE norm):
 *   1. llmy_router_context_latent_f32: local = RMSNorm(h) * norm_w (fp32
 *      [rows, D]); lat = LayerNorm(local . w_down^T) * ln_w + ln_b (fp32
 *      [rows, L], LayerNorm eps ln_eps = 1e-5, mla_memory.py:23-24).
 *      D in {256,512,768,1024}; L % 64 == 0, L <= 512.
 *   2. llmy_router_context_window: rows are B sequences of T tokens at
 *      absolute positions pos[b] + t (pos NULL: 0).  ring [B, W, L] fp32 holds
 *      each sequence's last W latents (slot p % W); ctx[b, t] = bf16(mean of
 *      the min(p+1, W) latents up to position p) (mla_memory.py:29-48), and
 *      the ring is updated.
 *   3. llmy_linear_bf16(ctx, W_lco [D, L]) -> bf16 [rows, D] (epilogue 0).
 *   4. llmy_linear_bf16(that, W_co [D, D]) -> c fp32 [rows, D] (epilogue 1).
 *   5. llmy_router_context_logits_f32: logits = (local + sigmoid(route_gate[0])
 *      * c) . w_router^T, fp32 [rows, E]; then llmy_router_topk_logits_f32. */
int32_t llmy_router_context_latent_f32(const llmy_bf16* h, const float* norm_w,
                                       const float* w_down, const float* ln_w,
                                       const float* ln_b, float* local, float* lat,
                                       int32_t rows, int32_t D, int32_t L, float eps,
                                       float ln_eps, void* stream);
int32_t llmy_router_context_window(const float* lat, float* ring, const int32_t* pos,
                                   llmy_bf16* ctx, int32_t B, int32_t T, int32_t W,
                                   int32_t L, void* stream);
int32_t llmy_router_context_logits_f32(const float* local, const float* c,
                                       const float* route_gate, const float* w_router,
                                       float* logits, int32_t rows, int32_t D, int32_t E,
                                       void* stream);
/* The router's global branch over an HCA block's summaries
 * (context_router.py:66-68,126-127; mla_memory.py:9-90; native
 * router_hca_latent_attention, llmy_cuda/src/model.cpp:972-1062).  Per summary,
 * once: latent = LayerNorm(down . value) (hca_latent, eps 1e-5) with
 * llmy_linear_bf16 + llmy_layernorm_f32_bf16, then its keys and values
 * [k; v] . latent (llmy_linear_bf16), stored in slots beside the summary's tag
 * (llmy_cmp_commit_bf16 / llmy_cmp_memory_fill_bf16).  Per query: q =
 * W_q . local (local = the router's RMSNorm of h, bf16), then
 * llmy_latent_attn_bf16, then W_o . that added to local_context_out(ctx)
 * before context_out. */
/* out[r] = bf16((x[r] - mean) / sqrt(var + eps) * w + b), x [rows, L] fp32. */
int32_t llmy_layernorm_f32_bf16(const float* x, const float* w, const float* b, llmy_bf16* out,
                                int32_t rows, int32_t L, float eps, void* stream);
/* Multi-head attention of q [B*T rows, heads*head_dim at q_ld] over each row's
 * C slots (keys / values [B, C, heads*head_dim] bf16); query row b*T + t is at
 * position pos[b] (pos NULL: t) and sees slots with 1 <= tag <= position + 1;
 * out [B*T, out_ld] bf16, 0 where nothing is visible.  scale = 1/sqrt(head_dim). */
int32_t llmy_latent_attn_bf16(const llmy_bf16* q, int64_t q_ld, const llmy_bf16* keys,
                              const llmy_bf16* vals, const int32_t* tag, const int32_t* pos,
                              llmy_bf16* out, int64_t out_ld, int32_t B, int32_t T, int32_t C,
                              int32_t heads, int32_t head_dim, float scale, void* stream);

/* Decode-time MoE front end (E*D <= 24576, D in {256,512,1024}, k <= 8):
 *   h2[t] = bf16(RMSNorm(x[t]) * ffn_w)   (the block's pre-MoE norm),
 *   logits = (RMSNorm(h2[t]) * router_w) . w_router^T in fp32, top-k (ties ->
 *   lower index) + softmax -> idx [T,k], gates [T,k],
 *   and (unless counts == NULL) the stable permutation of llmy_moe_permute —
 *   router with W_r staged in LDS, one wave per token, then the permutation.
 * Equivalent to llmy_rmsnorm_f32_bf16 + llmy_router_topk_bf16 +
 * llmy_moe_permute (context_router.py:62,71-74; moe.py:42-66).
 * nparts in [0, 8]: first complete the residual from the preceding
 * projection's partial products (llmy_linear_bf16 epilogue 4), parts
 * [nparts, T, D]: x[t] += sum_p parts[p][t] (p ascending), or, with gate
 * [T, D] non-NULL, x[t] += gate[t] * sum_p parts[p][t]; x is written back. */
int32_t llmy_moe_route_decode(float* x, const float* parts, int32_t nparts,
                              const float* gate, const float* ffn_w,
                              const float* router_w, const float* w_router,
                              llmy_bf16* h2, int32_t* idx, float* gates,
                              int32_t* counts, int32_t* offsets,
                              int32_t* sorted_routes, int32_t* route_pos, int32_t T,
                              int32_t D, int32_t E, int32_t k, float eps, void* stream);

/* --- The reference ABI's fp32 operator hooks (same signatures) ------------ */

/* One-token sparse MoE over the k selected experts, fp32 throughout; replaces
 * llmy_moe_selected_fp32 (llmy_cuda/include/llmy.h:80-88), called by
 * sample_standalone.py:3001-3075.  x [D], idx [k] int64, prob [k],
 * gate_up [E,2H,D] (gate rows then up rows), down [E,D,H]; scratch
 * activation [k,H] and route_output [k,D]; out [D]:
 *   activation[j] = silu(W_gate[e_j] x) * (W_up[e_j] x),
 *   route_output[j] = prob[j] * W_down[e_j] activation[j],
 *   out = sum over j (ascending) of route_output[j].
 * A route id outside [0, E) contributes zeros.  Returns 1 before any launch
 * for a null pointer or a non-positive size. */
int32_t llmy_moe_selected_fp32(const float* x, const int64_t* idx, const float* prob,
                               const float* gate_up, const float* down, float* activation,
                               float* route_output, float* out, int32_t D, int32_t H,
                               int32_t E, int32_t k, void* stream);

/* Out-of-place Sinkhorn on [matrices,4,4] fp32 in the log domain; replaces
 * llmy_mhc_sinkhorn4 (llmy_cuda/include/llmy.h:74-78), called by
 * sample_standalone.py:2544-2587: `iterations` rounds of subtracting each row's
 * logsumexp and then each column's, then output = exp.  matrices > 0,
 * iterations >= 0. */
int32_t llmy_mhc_sinkhorn4(const float* input, float* output, int32_t matrices,
                           int32_t iterations, void* stream);

/* --- Sampling (sample_standalone.py:5609-5636) ---------------------------- */

/* out[r] = first index of the maximum of logits[r, :V] (NaN counts as the
 * maximum), i.e. torch.argmax.  logits [rows,V] fp32, out [rows] int32. */
int32_t llmy_sample_argmax_f32(const float* logits, int32_t rows, int32_t V,
                               int32_t* out, void* stream);

/* Temperature + top-k + nucleus sampling with a caller-supplied uniform draw
 * per row; replaces the CPU sampler llmy_sample (llmy_cuda/include/llmy.h:64-67,
 * llmy_cuda/src/llmy.cpp:132-202), whose xorshift draw the caller makes and
 * passes as u[r] in [0, 1).  Per row: order ids by descending logit (equal
 * logits by ascending id); keep the first top_k (top_k <= 0 or >= V: all);
 * p = softmax(logit / temperature) over the kept ids; keep the shortest prefix
 * whose probability reaches top_p (top_p outside (0, 1): all); out[r] = the
 * first kept id whose cumulative renormalised probability exceeds u[r].
 * temperature <= 0 (or NaN) gives the greedy id of llmy_sample_argmax_f32.
 * logits [rows,V] fp32 with V <= 32768, u [rows] fp32, out [rows] int32.
 * Deterministic: probabilities are summed as exact 2^-47 fixed point. */
int32_t llmy_sample_top_p_f32(const float* logits, int32_t rows, int32_t V,
                              float temperature, int32_t top_k, float top_p,
                              const float* u, int32_t* out, void* stream);

/* In-place repetition penalty (sample_standalone.py:5601-5605; the C twin is
 * the penalty loop of llmy_sample, llmy_cuda/src/llmy.cpp:145-156): for each
 * distinct id in recent[r, :n_recent] inside [0, V), logits[r, id] is divided
 * by penalty if positive, else multiplied by it.  An id listed more than once
 * is penalised once (the Python sampler's set; the C twin would apply it per
 * listing).  Ids outside [0, V) (e.g. -1 padding) are ignored.  V <= 262144,
 * penalty > 0; penalty == 1 is a no-op. */
int32_t llmy_repetition_penalty_f32(float* logits, int32_t rows, int32_t V,
                                    const int32_t* recent, int32_t n_recent,
                                    float penalty, void* stream);

/* --- Engine handles (llmy_cuda/include/llmy.h:27-72) ----------------------
 * The reference engine API with the same signatures and meaning; the model
 * comes from a `.llmy` v1 file of this block stack (hybrid_llm_amd/checkpoint.py
 * writes one).  Replaces llmy_cuda/src/llmy.cpp:21-210 over model.cpp:1774-1972.
 * The model handle owns the device weights, the state handle the caches and
 * buffers; these entry points allocate device memory, the kernel entries
 * above never do.  No exception crosses the ABI: a failure returns NULL (load,
 * state_new) or is recorded for llmy_last_status / llmy_last_error. */
typedef struct llmy_model llmy_model;
typedef struct llmy_state llmy_state;

llmy_model* llmy_load(const char* path);                 /* llmy.h:31 */
void        llmy_free(llmy_model* m);                    /* llmy.h:32 */
int32_t llmy_vocab_size(const llmy_model* m);            /* llmy.h:35 */
int32_t llmy_d_model(const llmy_model* m);               /* llmy.h:36 */
/* loops a forward runs by default (set_num_loops, clamped to the built ones) */
int32_t llmy_num_loops(const llmy_model* m);             /* llmy.h:37 */
int32_t llmy_max_loops(const llmy_model* m);             /* llmy.h:38 */
/* residual streams per token: mhc.streams when mhc.enabled, else 1 */
int32_t llmy_mhc_streams(const llmy_model* m);           /* llmy.h:39 */
void    llmy_set_num_loops(llmy_model* m, int32_t n);    /* llmy.h:40 */
void    llmy_set_fixed_loops(llmy_model* m, int32_t n);  /* llmy.h:41 */
/* batch-1 state, as the reference */
llmy_state* llmy_state_new(llmy_model* m);               /* llmy.h:44 */
void        llmy_state_free(llmy_state* s);              /* llmy.h:45 */
/* zero every cache and state, position 0 (llmy.cpp:99-114) */
void        llmy_state_reset(llmy_state* s);             /* llmy.h:46 */
/* A fresh conversation of n_tokens from position 0 (the reference's
 * model_prefill runs it token by token, model.cpp:1955-1966; here it is one
 * sequence pass); logits of the last position into logits_out [vocab] on the
 * host or the device (llmy.h:49-53). */
void llmy_prefill(llmy_model* m, llmy_state* s, const int32_t* tokens,
                  int32_t n_tokens, float* logits_out);
/* One token at absolute position `position`; num_loops 0 = the model's
 * default (llmy.h:55-59). */
void llmy_decode(llmy_model* m, llmy_state* s, int32_t token, int32_t position,
                 int32_t num_loops, float* logits_out);
/* The CPU sampler (llmy.h:61-68, llmy.cpp:132-202): host logits, xorshift64
 * state; equal logits order by ascending id. */
int32_t llmy_sample(const float* logits, int32_t vocab_size, float temperature,
                    int32_t top_k, float top_p, float repetition_penalty,
                    const int32_t* recent_tokens, int32_t n_recent,
                    uint64_t* rng_state);
int32_t llmy_last_executed_loops(const llmy_state* s);   /* llmy.h:71 */
void    llmy_sync(void);                                 /* llmy.h:72 */

/* Batched forms — no counterpart in the reference, whose engine throws for
 * B > 1 (model.cpp:627,678): a state of `batch` sequences; prefill of
 * tokens [batch, n_tokens] (host or device) from position 0 and decode of
 * tokens [batch] at positions [batch] (NULL: one past the previous token),
 * logits_out [batch, vocab] (NULL: not copied).  Return 0 or 1 (see
 * llmy_last_error). */
llmy_state* llmy_state_new_batch(llmy_model* m, int32_t batch);
int32_t llmy_prefill_batch(llmy_model* m, llmy_state* s, const int32_t* tokens,
                           int32_t n_tokens, float* logits_out);
int32_t llmy_decode_batch(llmy_model* m, llmy_state* s, const int32_t* tokens,
                          const int32_t* positions, int32_t num_loops,
                          float* logits_out);
/* Reset the rows of a batched state where mask[b] != 0 (host or device int32
 * [batch]): their GDN states, conv histories, KV caches and router latent
 * rings are zeroed and their next position is 0, the reset_rows of
 * model/recurrent_state.py:213-225 that decode_step applies before a token
 * whose reset_mask is set (model/model.py:814-822).  Other rows keep their
 * state.  Returns 0 or 1 (see llmy_last_error). */
int32_t llmy_state_reset_rows(llmy_state* s, const int32_t* mask);
/* greedy (argmax) token of each row after the last forward into out [batch] */
int32_t llmy_greedy_tokens(const llmy_state* s, int32_t* out);
/* Status of the last engine call on this thread (0 ok) and its message — the
 * status query the reference lacks for prefill/decode (llmy.cpp:116-131). */
int32_t     llmy_last_status(void);
const char* llmy_last_error(void);
/* Parse a `.llmy` file without touching the GPU: config text, "--", then one
 * line per tensor "name dtype ndim d0 d1 d2 d3 nbytes" into buf. */
int32_t llmy_checkpoint_describe(const char* path, char* buf, int64_t buf_len);

#ifdef __cplusplus
}
#endif
#endif /* LLMY_H */
