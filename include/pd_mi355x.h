/*
 * pd_mi355x.h — C ABI of the MI355X (gfx950) masked-component kernels.
 *
 * The reference (goodfire-ai/param-decomp) is Python/JAX with no FFI layer; its seams
 * are Python functions. Each entry point below replaces the arithmetic of one of those
 * seams and cites it (paths relative to the reference root, pd/ =
 * param_decomp/param_decomp/). A jax.ffi custom-call handler or a ctypes stub binds
 * them one to one.
 *
 * Conventions (every entry point):
 *  - All tensor arguments are DEVICE pointers owned by the caller; outputs are
 *    preallocated by the caller. Row-major, densely packed unless a leading dimension
 *    is given. Entry points that need scratch take a caller-provided `workspace` whose
 *    size comes from the matching *_workspace_size query; nothing allocates.
 *  - `stream` is a hipStream_t (NULL = the default stream). Calls only enqueue work;
 *    none synchronizes the host. The stack steps (pd_moe_stack_step*, pd_lm_stack_step*)
 *    run independent parts of their work on a helper stream of the
 *    same priority, one per device, created with its events on the first call on that
 *    device (make that first call outside any stream capture); the helper stream waits
 *    on `stream` before it starts and `stream` waits on it before the call's last work,
 *    so anything later enqueued on `stream` sees every output.
 *  - Threading: every entry point is reentrant. Host threads may call any of them at the
 *    same time, on one device or several, each with its own stream, outputs and
 *    workspace. The stack steps hold a per-device lock while they enqueue (never while
 *    the GPU runs), so concurrent stack-step calls on one device enqueue one after
 *    another and their helper-stream work runs in that order; each call's results are
 *    those of the call alone. Calls that share an output or a workspace, and calls of
 *    pd_masked_linear_bwd_noalloc on one device (one shared scratch region), must be
 *    ordered by the caller.
 *  - Return PD_OK (0) or a PD_E* code; pd_last_error() gives the message (thread-local).
 *    Invalid shapes are rejected on the host before any launch.
 *  - Random keys are JAX threefry2x32 key words (k0, k1) as jax.random.PRNGKey /
 *    split / fold_in produce them; draws follow jax.random.uniform in the chosen
 *    counter layout.
 */
#ifndef PD_MI355X_H
#define PD_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PD_OK 0
#define PD_EINVAL 1
#define PD_ELAUNCH 2
#define PD_EUNSUPPORTED 3
#define PD_EWORKSPACE 4

#define PD_DTYPE_F32 0
#define PD_DTYPE_BF16 1
#define PD_DTYPE_U16 2 /* unit-interval fixed point u / 65535 (adversarial source storage) */

#define PD_PGD_SGD 0      /* source optimizers, pd/core/adversary.py:392-470 */
#define PD_PGD_MOMENTUM 1
#define PD_PGD_ADAM 2
#define PD_PGD_SIGN 3     /* fresh-PGD sign ascent, pd/core/train.py:788-800 */

#define PD_LAYOUT_PARTITIONABLE 0 /* jax_threefry_partitionable=True (JAX >= 0.5 default) */
#define PD_LAYOUT_ORIGINAL 1

#define PD_IMPMIN_PNORM 0     /* (upper+eps)^p, paper / nano_param_decomp/run.py:413-429 */
#define PD_IMPMIN_SMOOTH_L0 1 /* c^2/(c^2+gamma^2), pd/core/losses.py:388-394 */

#define PD_BLOCK_FUSED_OUTPUT 0 /* BlockContraction "fused_output", pd/core/linear_plan.py:134-146 */
#define PD_BLOCK_FUSED_INPUT 1  /* BlockContraction "fused_input" */

const char* pd_last_error(void);
int pd_abi_version(void);

/* ---- mask draw: jax.random.uniform (pd/core/linear_plan.py:80-106 uniform_like) ---- */
/* out[i] = uniform(key)[i], i < n, drawn in draw_dtype, stored in out_dtype. */
int pd_uniform(uint32_t k0, uint32_t k1, int64_t n, int draw_dtype, int layout, void* out, int out_dtype,
               void* stream);

/* ---- squashing: pd/core/ci_fn/squashing.py:8-45, CI.from_preactivations
 *      (pd/core/ci_fn/interface.py:35-41). lower/upper may be NULL. ---- */
int pd_squash_fwd(const void* pre, int dtype, int64_t n, void* lower, void* upper, void* stream);
/* d_pre = lower_vjp(pre, g_lower) + upper_vjp(pre, g_upper); either g may be NULL. */
int pd_squash_bwd(const void* pre, const void* g_lower, const void* g_upper, int dtype, int64_t n, void* d_pre,
                  void* stream);

/* ---- component mask: pd/core/masking.py:135-136 sample_component_mask
 *      m = ci + (1-ci)*uniform(key, ci.shape, draw_dtype). ---- */
int pd_component_mask_fwd(const void* ci, int dtype, int64_t n, uint32_t k0, uint32_t k1, int draw_dtype,
                          int layout, void* mask, void* stream);
/* d_ci = g_mask * (1 - u). */
int pd_component_mask_bwd(const void* g_mask, int dtype, int64_t n, uint32_t k0, uint32_t k1, int draw_dtype,
                          int layout, void* d_ci, void* stream);
/* The same two with the key in device memory (two uint32 words, read when the kernel
 * runs): the form a captured graph replays with a fresh key per step, written into that
 * buffer before each replay (pd/core/masking.py:135-136 as above). */
int pd_component_mask_fwd_dkey(const void* ci, int dtype, int64_t n, const uint32_t* key, int draw_dtype,
                               int layout, void* mask, void* stream);
int pd_component_mask_bwd_dkey(const void* g_mask, int dtype, int64_t n, const uint32_t* key, int draw_dtype,
                               int layout, void* d_ci, void* stream);

/* ---- per-component gate MLP (paper form, spd_paper.md appendix; engine GELU is exact
 *      erf, pd/core/ci_fn/implementations/mlp.py:77):
 *      g_raw[r,c] = b_out[c] + sum_j w_out[c,j]*GELU(w_in[c,j]*h[r,c] + b_in[c,j]).
 *      h is [rows, C] (dtype), params fp32 [C,H] / [C]; H must be 16. ---- */
int pd_gate_fwd(const void* h, int dtype, int64_t rows, int64_t C, int H, const float* w_in, const float* b_in,
                const float* w_out, const float* b_out, int precise, float* g_raw, void* stream);
size_t pd_gate_bwd_workspace_size(int64_t rows, int64_t C, int H);
/* dh (dtype) and fp32 parameter grads (overwritten) from dg_raw (fp32). */
int pd_gate_bwd(const void* h, int dtype, int64_t rows, int64_t C, int H, const float* w_in, const float* b_in,
                const float* w_out, const float* b_out, const float* dg_raw, int precise, void* dh, float* dw_in,
                float* db_in, float* dw_out, float* db_out, void* workspace, size_t workspace_bytes, void* stream);

/* ---- importance minimality over ci_upper [rows, C] (pd/core/losses.py:357-485;
 *      nano_param_decomp/run.py:413-429). kind PD_IMPMIN_PNORM uses (p, eps, beta,
 *      world_size); PD_IMPMIN_SMOOTH_L0 uses gamma, normalize_at_one and, when
 *      ref_count > 0, the frequency term. out[0] = activity, out[1] = frequency term
 *      (fp32, overwritten). grad (nullable, dtype of ci) = coeff_act*d act/d ci +
 *      coeff_freq*d freq/d ci. freq_ema_in (nullable, fp32 [C]): the frequency term
 *      reads the EMA estimate instead of the batch's (the rule under pd_dense_step;
 *      out[2] = the batch penalty; freq_ema_out [C] receives the new estimate). ---- */
size_t pd_impmin_workspace_size(int64_t rows, int64_t C);
int pd_impmin(const void* ci_upper, int dtype, int64_t rows, int64_t C, int kind, float p, float eps, float beta,
              float world_size, float gamma, int normalize_at_one, float ref_count, const float* freq_ema_in,
              float* freq_ema_out, float ema_count, float ema_halflife, float coeff_act, float coeff_freq, float* out,
              void* grad, void* workspace, size_t workspace_bytes, void* stream);

/* ---- recon losses ----
 * MSE: pd/targets/tms.py:380-388, pd/targets/resid_mlp.py:411-418: mean((a-b)^2).
 * out[0] = loss; grad_a (nullable, dtype) = coeff * 2(a-b)/n. */
size_t pd_mse_workspace_size(int64_t n);
int pd_mse(const void* a, const void* b, int dtype, int64_t n, float coeff, float* out, void* grad_a, void* workspace,
           size_t workspace_bytes, void* stream);
/* KL(clean || masked) per position, averaged over rows (pd/core/losses.py:80-92,
 * pd/targets/losses.py:50-60). logits are [rows, V]; grad (nullable, dtype) =
 * coeff * (softmax(masked) - softmax(clean)) / rows. */
size_t pd_kl_workspace_size(int64_t rows);
int pd_kl(const void* masked_logits, const void* clean_logits, int dtype, int64_t rows, int64_t vocab, float coeff,
          float* out, void* grad, void* workspace, size_t workspace_bytes, void* stream);
/* Streamed-vocab KL (pd/targets/losses.py:101-170 streamed_position_kl): per-position
 * KL(softmax(act_clean @ head_clean^T) || softmax(act_masked @ head_masked^T)) streamed over
 * n_chunks equal vocab chunks (V % n_chunks == 0) with the paired online-softmax
 * accumulators; the logits never materialize. act [N,d], head [V,d] in `dtype` (bf16: d
 * a multiple of 8; bf16 chunks are V/n_chunks rounded up to a multiple of 8, the last one
 * ragged, which the KL does not depend on). fwd writes position_kl [N] and stats [N,5] =
 * (m_p, s_p, a, m_q, s_q); bwd writes d_act_masked [N,d] fp32 = sum_v (q - p) g[n]
 * head_masked[v] for the per-position cotangent g (the clean side is the target). */
size_t pd_streamed_kl_workspace_size(int dtype, int64_t N, int64_t d, int64_t V, int n_chunks);
int pd_streamed_kl_fwd(int dtype, int64_t N, int64_t d, int64_t V, int n_chunks, const void* act_masked,
                       const void* head_masked, const void* act_clean, const void* head_clean, float* position_kl,
                       float* stats, void* workspace, size_t workspace_bytes, void* stream);
int pd_streamed_kl_bwd(int dtype, int64_t N, int64_t d, int64_t V, int n_chunks, const void* act_masked,
                       const void* head_masked, const void* act_clean, const void* head_clean, const float* stats,
                       const float* g_position, float* d_act_masked, void* workspace, size_t workspace_bytes,
                       void* stream);

/* ---- GEMM: C[M,N] = alpha * op(A) @ op(B) + beta * C, fp32 accumulation.
 *      dtype PD_DTYPE_BF16 runs bf16 MFMA (A/B bf16; C bf16 or fp32 via c_dtype);
 *      PD_DTYPE_F32 runs an fp32 kernel (A/B/C fp32). trans_a: A stored [K,M];
 *      trans_b: B stored [N,K]. Backs every x@V, (xV*m)@U and their transposes in
 *      site_forward (pd/core/decomposed_linear.py:142-175). ---- */
int pd_gemm(int dtype, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda, int trans_a, const void* B,
            int64_t ldb, int trans_b, void* C, int64_t ldc, int c_dtype, float alpha, float beta, void* stream);
/* Strided-batched pd_gemm: C[z] = alpha op(A[z]) op(B[z]) + beta C[z] for z < batch, each
 * operand at base + z * stride (stride 0 = shared). The per-block einsums of the
 * block-factored linears (pd/core/linear_plan.py:149-160). bf16: strides % 8 == 0. */
int pd_gemm_strided_batched(int dtype, int64_t batch, int64_t M, int64_t N, int64_t K, const void* A, int64_t lda,
                            int64_t stride_a, int trans_a, const void* B, int64_t ldb, int64_t stride_b, int trans_b,
                            void* C, int64_t ldc, int64_t stride_c, int c_dtype, float alpha, float beta,
                            void* stream);

/* ---- masked decomposed linear: pd/core/decomposed_linear.py:142-175 site_forward,
 *      ((x@V)*(m-d))@U blended with d*(x@W^T) and route (:65-85).
 *      x [T,d_in], V [d_in,C], U [C,d_out], W [d_out,d_in] (only read when delta or
 *      route is given), mask [T,C], delta [T] (nullable), route [T] uint8 (nullable).
 *      Outputs: out [T,d_out], xV [T,C]; acts [T,C] is the caller's residual buffer
 *      holding (x@V)*(m-d) for the backward. ---- */
int pd_masked_linear_fwd(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, const void* x, const void* V,
                         const void* U, const void* W, const void* mask, const void* delta, const uint8_t* route,
                         void* out, void* xV, void* acts, void* stream);
/* VJP: given d_out_grad [T,d_out] -> dx [T,d_in], dV, dU, dmask [T,C] and d_delta [T]
 * (each nullable, of `dtype`; an adversarial source ascent asks for dmask and d_delta
 * alone). d_delta[t] = routed ? sum_o g*(x@W^T) - sum_c (g@U^T)*xV : 0 is the weight-delta
 * cotangent the reference's autodiff forms for delta sources (pd/core/source_mask.py:61-63,
 * pd/core/adversary.py:74-82); it needs W, and is the gradient at d = 0 when delta is
 * NULL. workspace holds two [T,C] and one [T,d_out] tensors of `dtype`. */
size_t pd_masked_linear_bwd_workspace_size(int dtype, int64_t T, int64_t d_out, int64_t C);
int pd_masked_linear_bwd(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, const void* x, const void* V,
                         const void* U, const void* W, const void* mask, const void* delta, const uint8_t* route,
                         const void* xV, const void* acts, const void* g_out, void* dx, void* dV, void* dU,
                         void* dmask, void* d_delta, void* workspace, size_t workspace_bytes, void* stream);
/* pd_masked_linear_bwd without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference. Same arguments, kernels and results as
 * pd_masked_linear_bwd; its scratch is a fixed device region of
 * PD_MASKED_LINEAR_BWD_NOALLOC_MAX_BYTES per GPU inside the library, located once per
 * device on the first call and held until the process ends. Calls whose
 * pd_masked_linear_bwd_workspace_size exceeds it return PD_EUNSUPPORTED. No allocation
 * happens in the call. Every call on one GPU shares that GPU's region: calls that overlap
 * on one GPU (different streams, or host threads without ordering) race, and so do two
 * captured graphs containing it whose replays overlap. Under graph capture, make one
 * eager call on the device first (it looks the region up); the call itself launches
 * kernels only (no memset, no host synchronization). Loading the library reserves the
 * region on every GPU it runs on, whether or not the entry point is called. */
#define PD_MASKED_LINEAR_BWD_NOALLOC_MAX_BYTES ((size_t)64 << 20)
int pd_masked_linear_bwd_noalloc(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, const void* x,
                                 const void* V, const void* U, const void* W, const void* mask, const void* delta,
                                 const uint8_t* route, const void* xV, const void* acts, const void* g_out, void* dx,
                                 void* dV, void* dU, void* dmask, void* d_delta, void* stream);

/* ---- block-factored site, dense over every block: pd/core/decomposed_linear.py:209-271
 *      blocked_site_forward with the einsums of pd/core/linear_plan.py:149-160.
 *      V [E,d_in,c], U [E,c,d_out] per block; mask [T,E*c] block-major; delta [T], route
 *      [T] uint8 nullable (W read only with them).
 *      PD_BLOCK_FUSED_OUTPUT (gate/up): x [T,d_in], W [E*d_out,d_in], out [T,E*d_out]
 *        (block outputs concatenated); PD_BLOCK_FUSED_INPUT (down): x [T,E*d_in],
 *        W [d_out,E*d_in], out [T,d_out] (block outputs summed).
 *      Outputs xV [T,E*c] (the flat component activation) and acts [T,E*c] for the bwd.
 *      bwd: dx (nullable, x's shape), dV, dU, dmask (nullable), d_delta [T] (nullable; needs
 *      W): the delta cotangent over the whole site output, as pd_masked_linear_bwd forms it.
 *      bf16: d_in, d_out, c % 8. */
int pd_blocked_site_fwd(int dtype, int contraction, int64_t T, int64_t E, int64_t d_in, int64_t d_out, int64_t c,
                        const void* x, const void* V, const void* U, const void* W, const void* mask, const void* delta,
                        const uint8_t* route, void* out, void* xV, void* acts, void* stream);
size_t pd_blocked_site_bwd_workspace_size(int dtype, int contraction, int64_t T, int64_t E, int64_t d_in,
                                          int64_t d_out, int64_t c);
int pd_blocked_site_bwd(int dtype, int contraction, int64_t T, int64_t E, int64_t d_in, int64_t d_out, int64_t c,
                        const void* x, const void* V, const void* U, const void* W, const void* mask, const void* delta,
                        const uint8_t* route, const void* xV, const void* acts, const void* g_out, void* dx, void* dV,
                        void* dU, void* dmask, void* d_delta, void* workspace, size_t workspace_bytes, void* stream);

/* ---- fused single-site stochastic-recon step (the dense hot path) ----
 * One fwd+bwd of: clean target y_t = x@W^T (detached, pd/core/train.py:578-606);
 * h = x@V; paper-form gate g_raw = gate(h); lower/upper squashing; mask
 * m = lower + (1-lower)*uniform(mask key) (pd/core/masking.py:148-167); optional
 * delta d = uniform(delta key, [T]); y = (h*(m-d))@U + d*y_t; recon = mean((y-y_t)^2);
 * imp-min (imp_kind): PD_IMPMIN_PNORM imp = sum_c mean_t (upper)^p, loss = recon_coeff*recon
 * + imp_coeff*imp; PD_IMPMIN_SMOOTH_L0 the engine's term imp_coeff * sum_c f_c +
 * freq_coeff * sum_c f_c log2(1 + ref_count f_c), f_c = mean_t psi(upper), psi =
 * c^2/(c^2 + gamma^2) (times 1 + gamma^2 when normalize_at_one; pd/core/losses.py:340-394,
 * pd/core/objective.py:101-131; ref_count 0 = no frequency term).
 * Gradients (overwritten, fp32 for the fp32 masters): dV [d_in,C], dU [C,d_out], gate grads.
 * losses[4] = {loss, recon, activity, frequency} fp32. mask_key / delta_key are the site's
 * keys (already split/folded). dtype bf16: x,W,V,U bf16.
 * The bf16 step evaluates each component's gate from a per-step table (32 bins over the
 * observed h range, degree-7 Chebyshev interpolant of g per bin: |g error| <= 8.3e-7 *
 * sum_j |w_out_j|) and takes the gate-parameter gradients from 8 Chebyshev moments of the
 * gate cotangent on 16 bins (the exact pullback of 128 weighted nodes per component;
 * interpolation error <= 7.5e-4 of each summand's scale). A component for which some
 * |w_in_j| * (moment-bin width) > 3 gets the exact per-element gate in both passes. The
 * fp32 step evaluates the gate exactly everywhere.
 * The EMA frequency estimate (this and every fused step; pd/core/losses.py:425-458,
 * EmaFrequency :522-543, ema_halflife_steps pd/core/configs.py:165-182): freq_ema_in NULL
 * is the single-batch estimate above. Otherwise (smooth-L0 with ref_count > 0 only) each
 * component's estimate becomes new = in + alpha (f_c - in) and the frequency term reads
 * f_hat = new / debias, alpha = -expm1(-ln 2 / ema_halflife), debias = -expm1(-ln 2 /
 * ema_halflife * (ema_count + 1)) (ema_count = earlier observations >= 0, ema_halflife in
 * (0, 1e6]): value sum Phi(f_hat), CI gradient freq_coeff Phi'(f_hat) df_c (the
 * reference's first-order surrogate; no gradient reaches the estimate); losses then has a
 * fifth entry, the batch penalty sum Phi(f_c) (EmaFrequencyPenalty.batch_value), and
 * freq_ema_out (nullable, may equal freq_ema_in) receives new. Estimate layouts: dense
 * step [C]; MoE stack [L, 3, E*c] (site order gate, up, down; expert-major components);
 * LM stack [L][kind][C_kind], layer-major, kinds in KIND_ORDER. */
size_t pd_dense_step_workspace_size(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H);
int pd_dense_step(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H, const void* x, const void* W,
                  const void* V, const void* U, const float* w_in, const float* b_in, const float* w_out,
                  const float* b_out, uint32_t mask_k0, uint32_t mask_k1, uint32_t delta_k0, uint32_t delta_k1,
                  int use_delta, int draw_dtype, int layout, int imp_kind, float p, float gamma, int normalize_at_one,
                  float imp_coeff, float freq_coeff, float ref_count, const float* freq_ema_in, float* freq_ema_out,
                  float ema_count, float ema_halflife, float recon_coeff, float* losses, float* dV, float* dU,
                  float* dw_in, float* db_in, float* dw_out, float* db_out, void* workspace, size_t workspace_bytes,
                  void* stream);

/* pd_dense_step with phase timing for measurement harnesses: `events` holds
 * PD_DENSE_STEP_PHASES + 1 hipEvent_t handles recorded on `stream` at the phase
 * boundaries: 0 delta draw, 1 target GEMM x@W^T, 2 GEMM h=x@V, 3 gate/mask fwd
 * (bf16: h range, gate table, forward), 4 GEMM (h*m)@U, 5 recon residual, 6 loss
 * finalize, 7 GEMM dU, 8 GEMM da=dy@U^T, 9 gate/mask bwd, 10 gate-parameter gradients
 * (bf16: moment finalize), 11 GEMM dV. Same arithmetic as pd_dense_step. */
#define PD_DENSE_STEP_PHASES 12
int pd_dense_step_timed(int dtype, int64_t T, int64_t d_in, int64_t d_out, int64_t C, int H, const void* x,
                        const void* W, const void* V, const void* U, const float* w_in, const float* b_in,
                        const float* w_out, const float* b_out, uint32_t mask_k0, uint32_t mask_k1, uint32_t delta_k0,
                        uint32_t delta_k1, int use_delta, int draw_dtype, int layout, int imp_kind, float p,
                        float gamma, int normalize_at_one, float imp_coeff, float freq_coeff, float ref_count,
                        const float* freq_ema_in, float* freq_ema_out, float ema_count, float ema_halflife,
                        float recon_coeff, float* losses, float* dV, float* dU, float* dw_in, float* db_in,
                        float* dw_out, float* db_out, void* workspace, size_t workspace_bytes, void* stream,
                        void** events);

/* ---- site routing samplers: pd/core/recon.py:218-252 (which sites take the decomposed
 *      output at each position; AllRouting = no routes array). routes: uint8
 *      [n_sites, n_positions], 1 = routed. ----
 * UniformKRouting (:218-231): (k_key, perm_key) = split(key); k = randint(k_key, [N], 1,
 * n_sites + 1) (randint splits k_key into high/low 32-bit draws, offset = (hi*2^32 + lo)
 * mod n_sites); routes[j] = argsort(uniform_f32(perm_key, [n_sites, N]), axis 0, stable)[j]
 * < k. n_sites <= 64. */
int pd_route_uniform_k(uint32_t key0, uint32_t key1, int64_t n_positions, int n_sites, int layout, uint8_t* routes,
                       void* stream);
/* StaticProbabilityRouting (:233-244): routes[j] = uniform_f32(fold_in(key, j), [N]) < p. */
int pd_route_static_p(uint32_t key0, uint32_t key1, int64_t n_positions, int n_sites, float p, int layout,
                      uint8_t* routes, void* stream);

/* ---- MoE routing: pd/targets/qwen36_moe.py:473-514 (router softmax, select_experts
 *      stable-descending lowest-index ties, expert_mixing_weights renormalized). ----
 * logits [T,E] fp32 -> probs [T,E] fp32 (nullable), top_idx [T,k] int32,
 * weights [T,k] fp32. E <= 512, k <= min(E, 64). */
int pd_router_topk(const float* logits, int64_t T, int E, int k, float* probs, int32_t* top_idx, float* weights,
                   void* stream);

/* ---- bucketing: pd/routed/experts.py:115-123 routed_jobs: sort_idx = stable argsort
 *      of top_idx.reshape(-1), inv_sort_idx its inverse, group_sizes = bincount(E);
 *      group_offsets [E+1] exclusive prefix (int32). Bit-exact, deterministic. ---- */
size_t pd_routed_jobs_workspace_size(int64_t n_jobs, int E);
int pd_routed_jobs(const int32_t* top_idx, int64_t T, int k, int E, int32_t* sort_idx, int32_t* inv_sort_idx,
                   int32_t* group_sizes, int32_t* group_offsets, void* workspace, size_t workspace_bytes,
                   void* stream);

/* ---- job-space gathers (pd/routed/experts.py:127-206) ----
 * out[j,:] = src[idx[j] / div, :] for j < n_out (gather_tokens: idx=sort_idx, div=k;
 * sort_job_values / unsort: div=1). */
int pd_gather_rows(const void* src, int dtype, int64_t width, const int32_t* idx, int div, int64_t n_out, void* out,
                   void* stream);
/* gather_tokens VJP (:135-138): out[t,:] = sum_s grad[inv_sort_idx[t*k+s], :]. */
int pd_gather_rows_vjp(const void* grad, int dtype, int64_t width, const int32_t* inv_sort_idx, int64_t T, int k,
                       void* out, void* stream);
/* combine_jobs / sum_jobs (:202-206, :351-359): out[t,:] = sum_s w[t,s]*y[inv[t*k+s],:],
 * fp32 accumulation; weights NULL = sum_jobs. */
int pd_combine_jobs(const void* y, int dtype, int64_t width, const int32_t* inv_sort_idx, const float* weights,
                    int64_t T, int k, void* out, void* stream);

/* ---- grouped matmul: pd/routed/experts.py:326-348 grouped_matmul (backend "hip").
 *      out[rows_e] = lhs[rows_e] @ rhs[e] over contiguous groups; rhs [E,K,N]
 *      (trans_rhs=0) or [E,N,K] (trans_rhs=1, the d_input product). Rows past
 *      sum(group_sizes) are zero-filled. group_offsets [E+1] from pd_routed_jobs.
 *      bf16 operands, fp32 accumulation, out in out_dtype. ---- */
int pd_grouped_gemm(const void* lhs, const void* rhs, const int32_t* group_offsets, int64_t J, int E, int64_t K,
                    int64_t N, int trans_rhs, void* out, int out_dtype, void* stream);
/* transposed_grouped_matmul (:209-280): out[e] = lhs[rows_e]^T @ dout[rows_e],
 * [E,K,N]; empty groups are exactly zero. */
int pd_grouped_gemm_dw(const void* lhs, const void* dout, const int32_t* group_offsets, int64_t J, int E, int64_t K,
                       int64_t N, void* out, int out_dtype, void* stream);
/* The same weight cotangent from K-major (job-contiguous) operands, the fast MFMA path:
 * lhsT [K, J], doutT [N, J]; out[e] = lhsT[:, rows_e] @ doutT[:, rows_e]^T. J must be a
 * multiple of 8. */
int pd_grouped_gemm_dw_kmajor(const void* lhsT, const void* doutT, const int32_t* group_offsets, int64_t J, int E,
                              int64_t K, int64_t N, void* out, int out_dtype, void* stream);

/* ---- the decomposed MoE stack step (the routed-expert hot path end to end) ----
 * L layers of: h2 = rms_norm_zero_centered(r) (target_ports/qwen3_5_moe.py:33-41),
 * fp32 router softmax + top-k + renormalized weights (pd/targets/qwen36_moe.py:473-514),
 * stable expert bucketing (pd/routed/experts.py:115-123), the three decomposed expert
 * sites in job space (pd/targets/qwen36_moe.py:2752-2837: acts = gmm(x_jobs, V) * mask,
 * out = gmm(acts, U), routing weights folded into the down input in fp32,
 * :2272-2282), r += sum_jobs(down). A clean forward on the frozen expert weights W (its
 * routing weights applied in the fp32 combine) pins each masked layer's expert indices
 * (pd/targets/qwen36_moe.py:2923-2965). Masks m = lower(ci) + (1-lower(ci)) u are drawn
 * per (kind, layer) with key fold_in(fold_in(split(draw_key)[0], kind), layer), kind =
 * 11/12/13 for gate/up/down (pd/targets/qwen36_moe.py:3374-3401), over the selected-CI
 * values [T, k*c] in bf16. use_delta != 0 adds the frozen channel that the reference's
 * stochastic masking always draws (pd/targets/qwen36_moe.py:2151-2160, 2805-2815): a
 * per-token delta d = uniform_bf16(fold_in(fold_in(split(draw_key)[1], kind), layer), [T])
 * per site, component coefficients m - d and site output gmm(acts, U) + d * gmm(x_jobs,
 * W[e]) (pd/core/decomposed_linear.py:65-85); use_delta = 0 is d = 0. source_value < 0
 * draws as above (StochasticSources); source_value in [0, 1] is the reference's
 * ConstantSources(v) (pd/core/objective.py:435-449): u = v everywhere and, with
 * use_delta, d = v; 0 is the CI-masked reconstruction (m = lower(ci), d = 0).
 * Loss = recon_coeff * mean((r_L - rc_L)^2) + the imp-min term over every site/layer's
 * selected upper CI: imp_kind PD_IMPMIN_PNORM: imp_coeff * sum(upper^p) / T (the selected
 * arm of pd/core/losses.py:357-372); PD_IMPMIN_SMOOTH_L0: the engine's term
 * (pd/core/objective.py:101-131) imp_coeff * sum_c f_c + freq_coeff * sum_c f_c
 * log2(1 + ref_count f_c), f_c = sum psi(upper) / T over the site's [E*c] components
 * (values scattered to their expert's block, pd/core/losses.py:316-330), psi =
 * c^2/(c^2 + gamma^2) (times 1 + gamma^2 when normalize_at_one); ref_count = 0 drops
 * the frequency term; freq_ema_in as under pd_dense_step ([L, 3, E*c]).
 * routes (nullable) uint8 [L, 3, T]: per-token site routes (the recon term's routing,
 * pd/core/recon.py:219-252); an unrouted token's jobs take the frozen output at that site
 * (where(route, decomposed + d frozen, frozen), pd/targets/qwen36_moe.py:2822-2827), so
 * the frozen channel runs with routes even without the delta draws; NULL = every token
 * routed. pd_moe_stack_step_sources takes no routes.
 * Layouts (all bf16 unless noted): x0 [T,d]; ln fp32 [L,d]; router [L,E,d];
 * Wg, Wu [L,E,d,f]; Wd [L,E,f,d]; Vg, Vu [L,E,d,c]; Ug, Uu [L,E,c,f]; Vd [L,E,f,c];
 * Ud [L,E,c,d]; ci_pre [L,3,T,k,c] (site order gate, up, down; slot s = the token's
 * s-th selected expert). Outputs: losses[4] = {loss, recon, activity (the L_p sum or
 * sum f_c), frequency (0 for L_p)}; the six V/U
 * gradients fp32 in the V/U shapes; d_ci_pre bf16 [L,3,T,k,c]; top_idx_out int32
 * [L,T,k] (nullable). The stack input's gradient is not formed (layer 0 stops at its
 * weight and CI gradients).
 * E <= 512, k <= 64; d, f, c multiples of 8. */
size_t pd_moe_stack_workspace_size(int64_t T, int d, int f, int E, int k, int c, int L);
int pd_moe_stack_step(int64_t T, int d, int f, int E, int k, int c, int L, const void* x0, const float* ln,
                      const void* router, const void* Wg, const void* Wu, const void* Wd, const void* Vg,
                      const void* Ug, const void* Vu, const void* Uu, const void* Vd, const void* Ud,
                      const void* ci_pre, uint32_t draw_k0, uint32_t draw_k1, int use_delta, const uint8_t* routes,
                      float source_value, int layout, int imp_kind, float p, float gamma, int normalize_at_one,
                      float imp_coeff, float freq_coeff, float ref_count, const float* freq_ema_in,
                      float* freq_ema_out, float ema_count, float ema_halflife, float recon_coeff, float* losses,
                      float* dVg, float* dUg, float* dVu, float* dUu, float* dVd, float* dUd, void* d_ci_pre,
                      int32_t* top_idx_out, void* workspace, size_t workspace_bytes, void* stream);
/* pd_moe_stack_step with persistent (adversarial) source tables in place of the draws:
 * the reference's SourceMaskIngredients arm (pd/targets/qwen36_moe.py:2151-2163,
 * pd/core/source_mask.py:56-63) over block-factored sources read at each selected value's
 * expert (pd/core/masking.py:43-68), the source half of persistent PGD
 * (pd/core/train.py:693-811, pd/core/adversary.py:463-567). src [L, 3, S, E, c]
 * (src_dtype F32, BF16 or U16 = u / 65535), every source row covering rows_per_source
 * consecutive tokens (S = T / rows_per_source: rows_per_source = T is the `c` shape, the
 * positions of a sample `bc`, 1 `bsc`); m = lower + (1 - lower) bf16(src[t / rps, e, :]);
 * src_delta [L, 3, S] (its own dtype; NULL = no delta channel) gives each token's delta,
 * d = bf16(src_delta[t / rps]). Outputs as pd_moe_stack_step (the weight gradients only
 * when want_weight_grads; NULL allowed otherwise: the warmup ascents need only the
 * sources' gradient), plus d_src fp32 [L, 3, S, E, c] = the sum over each row's selected
 * values of dm (1 - lower) (unselected entries 0), and d_src_delta fp32 [L, 3, S] = the sum
 * over each row's tokens and their jobs of the delta cotangent sum_o g_out frozen -
 * sum_c dm. Every sum is in a fixed order. Workspace:
 * pd_moe_stack_sources_workspace_size. reuse_clean = 1 takes the frozen clean pass (the
 * clean routing of every layer, its final residual and the frozen weights' copies) from
 * the workspace as the previous call on it left it: the adversary's warmup ascents and
 * final step within one PGD step, where x0, ln, router, Wg, Wu, Wd and the dimensions are
 * unchanged and no other call used the workspace in between (results are then identical
 * to reuse_clean = 0). */
size_t pd_moe_stack_sources_workspace_size(int64_t T, int d, int f, int E, int k, int c, int L,
                                           int64_t rows_per_source);
int pd_moe_stack_step_sources(int64_t T, int d, int f, int E, int k, int c, int L, const void* x0, const float* ln,
                              const void* router, const void* Wg, const void* Wu, const void* Wd, const void* Vg,
                              const void* Ug, const void* Vu, const void* Uu, const void* Vd, const void* Ud,
                              const void* ci_pre, const void* src, int src_dtype, const void* src_delta,
                              int delta_dtype, int64_t rows_per_source, int imp_kind, float p, float gamma,
                              int normalize_at_one, float imp_coeff, float freq_coeff, float ref_count,
                              const float* freq_ema_in, float* freq_ema_out, float ema_count, float ema_halflife,
                              float recon_coeff, int want_weight_grads, int reuse_clean, float* losses, float* dVg,
                              float* dUg, float* dVu, float* dUu, float* dVd, float* dUd, void* d_ci_pre,
                              float* d_src, float* d_src_delta, int32_t* top_idx_out, void* workspace,
                              size_t workspace_bytes, void* stream);
/* pd_moe_stack_step recording a hipEvent_t before each launch group and one at the
 * end; categories[i] labels the interval [i, i+1): 0 clean forward, 1 masked norm /
 * router / bucketing / gather, 2 grouped GEMMs fwd, 3 mask fwd, 4 SwiGLU fold,
 * 5 combine / loss / gathers, 6 grouped GEMMs d_input, 7 grouped GEMMs d_weight,
 * 8 mask bwd, 9 router+norm token backward, 10 waiting for the helper stream, 11 grouped
 * d_acts GEMMs with the mask backward as their epilogue; the last event ends the final
 * interval. *n_recorded = events used. */
int pd_moe_stack_step_timed(int64_t T, int d, int f, int E, int k, int c, int L, const void* x0, const float* ln,
                            const void* router, const void* Wg, const void* Wu, const void* Wd, const void* Vg,
                            const void* Ug, const void* Vu, const void* Uu, const void* Vd, const void* Ud,
                            const void* ci_pre, uint32_t draw_k0, uint32_t draw_k1, int use_delta,
                            const uint8_t* routes, float source_value, int layout, int imp_kind, float p, float gamma,
                            int normalize_at_one, float imp_coeff, float freq_coeff, float ref_count,
                            const float* freq_ema_in, float* freq_ema_out, float ema_count, float ema_halflife,
                            float recon_coeff, float* losses, float* dVg, float* dUg, float* dVu, float* dUu,
                            float* dVd, float* dUd, void* d_ci_pre, int32_t* top_idx_out, void* workspace,
                            size_t workspace_bytes, void* stream, void** events, int32_t* categories, int capacity,
                            int* n_recorded);

/* ---- the TMS toy decomposition step as one fused launch (pd/targets/tms.py:254-388) ----
 * target hid = x W1^T, out = relu(hid W1 + b2); both sites (linear1: W1 [H,F], linear2:
 * W1^T) decomposed with the paper-form gate on the clean input's x @ V, fp32 Threefry
 * masks m = lower + (1 - lower) u under the site keys fold_in(split(draw_key)[0], site)
 * (pd/core/masking.py:148-167), the delta channel under fold_in(split(draw_key)[1], site)
 * when use_delta, routes [2, B] uint8 (NULL = every row routed); loss = recon_coeff mse(out,
 * clean) + imp_coeff sum_sites sum_c mean_b upper^p. x [B,F], W1 [H,F], b2 [F], V1 [F,C],
 * U1 [C,H], V2 [H,C], U2 [C,F] fp32; gates = 8 pointers (per site w_in [C,16], b_in
 * [C,16], w_out [C,16], b_out [C]). grads fp32 (pd_tms_step_grads_size floats): dV1 |
 * dU1 | dV2 | dU2 | site 1 gate (w_in, b_in, w_out, b_out) | site 2 gate; losses[3] =
 * {loss, recon, imp}. Deterministic. Compiled for F = 5, H = 2, C = 20. */
size_t pd_tms_step_workspace_size(int64_t B, int F, int H, int C);
int pd_tms_step_grads_size(int F, int H, int C);
int pd_tms_step(int64_t B, int F, int H, int C, const float* x, const float* W1, const float* b2, const float* V1,
                const float* U1, const float* V2, const float* U2, const float* const* gates, uint32_t draw_k0,
                uint32_t draw_k1, int use_delta, int layout, const uint8_t* routes, float p, float imp_coeff,
                float recon_coeff, float* grads, float* losses, void* workspace, size_t workspace_bytes,
                void* stream);

/* ---- the ResidMLP toy decomposition step as one native call (pd/targets/resid_mlp.py:266-418) ----
 * target r_0 = x W_E, per layer r += relu(r W_in[l]^T) W_out[l]^T (no biases), out = r W_U;
 * every mlp_in (W_in [M,D]) and mlp_out (W_out [D,M]) decomposed (sites in the order
 * layers.0.mlp_in, layers.0.mlp_out, ...) with the paper-form gate on the clean input's
 * a @ V and fp32 Threefry masks m = lower + (1 - lower) u under the site keys
 * fold_in(split(draw_key)[0], site) (pd/core/masking.py:148-167); loss = recon_coeff
 * mse(out, clean) + imp_coeff sum_sites sum_c mean_b upper^p, fwd + bwd. x [B,F],
 * W_E [F,D], W_U [D,F] fp32; W_in, W_out: L pointers each; V, U: 2L pointers (V [din,C],
 * U [C,dout]); gates: 8L pointers (per site w_in [C,16], b_in [C,16], w_out [C,16],
 * b_out [C]). grads fp32 (pd_resid_mlp_step_grads_size floats): per site dV | dU | gate
 * (w_in, b_in, w_out, b_out); losses[3] = {loss, recon, imp}; out [B,F] (the masked
 * output) or NULL. Deterministic. No weight-delta channel or routes (the composed step
 * in param_decomp_amd/toys.py has them). */
size_t pd_resid_mlp_step_workspace_size(int64_t B, int F, int D, int M, int C, int L);
int64_t pd_resid_mlp_step_grads_size(int D, int M, int C, int L);
int pd_resid_mlp_step(int64_t B, int F, int D, int M, int C, int L, const float* x, const float* W_E,
                      const float* W_U, const float* const* W_in, const float* const* W_out, const float* const* V,
                      const float* const* U, const float* const* gates, uint32_t draw_k0, uint32_t draw_k1,
                      int layout, float p, float imp_coeff, float recon_coeff, float* grads, float* losses,
                      float* out, void* workspace, size_t workspace_bytes, void* stream);

/* ---- the decomposed Llama-style LM step (one stochastic-recon KL step, fwd + bwd) -----
 * The pre-RMSNorm transformer of pd/targets/transformer.py:1031-1140 in its
 * LlamaSimpleMLP form (pd/targets/llama_simple_mlp.py: rotate-half RoPE, causal GQA
 * attention, GELU-tanh MLP c_fc -> down_proj, tied embedding/head, no biases), with every
 * one of the six matrices per layer (KIND_ORDER q_proj, k_proj, v_proj, o_proj, c_fc,
 * down_proj = kinds 0..5) decomposed: site = ((x@V) * (m - d)) @ U + d * (x @ W^T)
 * (pd/core/decomposed_linear.py:142-175). Masks are drawn in-block per (kind, layer):
 * m = lower(ci) + (1 - lower(ci)) uniform(fold_in(fold_in(split(draw_key)[0], kind),
 * layer), [N, C]) and d = uniform(fold_in(fold_in(split(draw_key)[1], kind), layer), [N])
 * in bf16 (pd/targets/transformer.py:1048-1058, 1424-1451); use_delta = 0 is d = 0.
 * routes (nullable) uint8 [L, 6, N]: per-token site routes (the recon term's routing,
 * pd/core/recon.py:219-252); an unrouted token's site output is the target's x @ W^T
 * (where(route, masked, target), pd/core/decomposed_linear.py:72-85), so its masks take
 * no recon gradient; NULL = every token routed (AllRouting). Size the workspace of a
 * routed call with use_delta = 1 (the target segment of the site products).
 * Loss: recon_coeff * mean KL(softmax(clean logits) || softmax(masked logits)) (the
 * streamed form, pd/targets/losses.py:102-163, over n_kl_chunks vocab chunks) + the
 * imp-min term: PD_IMPMIN_PNORM: imp_coeff * sum_sites sum_c mean_tokens upper(ci)^p;
 * PD_IMPMIN_SMOOTH_L0: imp_coeff * sum_sites sum_c f_c + freq_coeff * sum f_c log2(1 +
 * ref_count f_c), f_c = mean_tokens psi(upper) (as pd_moe_stack_step, one component
 * block per site); freq_ema_in as under pd_dense_step ([L][kind][C_kind]).
 * Shapes: N = B*T tokens (int32 ids [N], T % 64 == 0); head_dim 64 (d = 64 n_head);
 * n_head % n_kv_head == 0; d, d_mlp % 64 == 0; C[6] each % 8 == 0; vocab % n_kl_chunks == 0.
 * wte [vocab, d] bf16 (embedding and head); ln1, ln2 [L, d], norm [d] fp32 (values the
 * bf16 weights hold); per kind k: W[k] [L, d_out, d_in], V[k] [L, d_in, C_k], U[k]
 * [L, C_k, d_out] bf16; ci_pre[k] [L, N, C_k] bf16. Outputs: losses [4] = (total, kl,
 * activity, frequency) fp32; dV[k], dU[k] fp32 in V/U's layouts; d_ci_pre[k] bf16 in
 * ci_pre's layout. */
size_t pd_lm_stack_workspace_size(int64_t B, int64_t T, int d, int n_head, int n_kv_head, int d_mlp, int64_t vocab,
                                  int L, const int32_t* C, int use_delta, int n_kl_chunks);
int pd_lm_stack_step(int64_t B, int64_t T, int d, int n_head, int n_kv_head, int d_mlp, int64_t vocab, int L,
                     const int32_t* C, const int32_t* tokens, const void* wte, const float* ln1, const float* ln2,
                     const float* norm, float eps, float rope_base, const void* const* W, const void* const* V,
                     const void* const* U, const void* const* ci_pre, uint32_t draw_k0, uint32_t draw_k1,
                     int use_delta, const uint8_t* routes, int layout, int imp_kind, float p, float gamma,
                     int normalize_at_one, float imp_coeff, float freq_coeff, float ref_count,
                     const float* freq_ema_in, float* freq_ema_out, float ema_count, float ema_halflife,
                     float recon_coeff, int n_kl_chunks, float* losses, float* const* dV, float* const* dU,
                     void* const* d_ci_pre, void* workspace, size_t workspace_bytes, void* stream);
/* pd_lm_stack_step with persistent (adversarial) source tables in place of the draws
 * (pd/core/source_mask.py:56-63; pd/core/masking.py:260-272), the source half of
 * persistent PGD (pd/core/train.py:693-811, pd/core/adversary.py:463-567). src[k] [L, S,
 * C_k] per kind (src_dtype F32, BF16 or U16 = u / 65535), every source row covering
 * rows_per_source consecutive tokens of the [B*T] order (S = B*T / rows_per_source:
 * B*T is the `c` shape, T the positions of a sample `bc`, 1 `bsc`; a pooled adversary's
 * per-sample draw of a pool particle is a `bc` table the caller gathers);
 * m = lower + (1 - lower) bf16(src[n / rps]); src_delta [L, 6, S] (its own dtype; NULL =
 * no delta channel) gives d = bf16(src_delta[n / rps]). No routes. Outputs as
 * pd_lm_stack_step (dV, dU only when want_weight_grads; NULL allowed otherwise: the
 * warmup ascents need only the sources' gradient), plus d_src[k] fp32 [L, S, C_k] = the
 * sum over each row's tokens of dm (1 - lower), and d_src_delta fp32 [L, 6, S] = the sum
 * over each row's tokens of sum_o g_out (x @ W^T) - sum_c dm; every sum in a fixed order.
 * reuse_clean = 1 takes the frozen forward's final activations from the workspace as the
 * previous call on it left them (the warmup ascents and final step of one PGD step:
 * tokens, wte and the frozen weights unchanged). Workspace:
 * pd_lm_stack_sources_workspace_size. */
size_t pd_lm_stack_sources_workspace_size(int64_t B, int64_t T, int d, int n_head, int n_kv_head, int d_mlp,
                                          int64_t vocab, int L, const int32_t* C, int use_delta, int n_kl_chunks,
                                          int64_t rows_per_source);
int pd_lm_stack_step_sources(int64_t B, int64_t T, int d, int n_head, int n_kv_head, int d_mlp, int64_t vocab, int L,
                             const int32_t* C, const int32_t* tokens, const void* wte, const float* ln1,
                             const float* ln2, const float* norm, float eps, float rope_base, const void* const* W,
                             const void* const* V, const void* const* U, const void* const* ci_pre,
                             const void* const* src, int src_dtype, const void* src_delta, int delta_dtype,
                             int64_t rows_per_source, int imp_kind, float p, float gamma, int normalize_at_one,
                             float imp_coeff, float freq_coeff, float ref_count, const float* freq_ema_in,
                             float* freq_ema_out, float ema_count, float ema_halflife, float recon_coeff,
                             int n_kl_chunks, int want_weight_grads, int reuse_clean, float* losses, float* const* dV,
                             float* const* dU, void* const* d_ci_pre, float* const* d_src, float* d_src_delta,
                             void* workspace, size_t workspace_bytes, void* stream);
/* pd_lm_stack_step recording HIP events at phase boundaries (categories: 0 per-step weight
 * copies and delta draws, 1 frozen forward, 2 site products fwd, 3 mask fwd, 4 attention,
 * 5 norms / adds / GELU / transposes, 6 streamed KL, 7 d_acts and d_input products, 8 dU
 * and dV products, 9 mask bwd, 10 end). */
int pd_lm_stack_step_timed(int64_t B, int64_t T, int d, int n_head, int n_kv_head, int d_mlp, int64_t vocab, int L,
                           const int32_t* C, const int32_t* tokens, const void* wte, const float* ln1,
                           const float* ln2, const float* norm, float eps, float rope_base, const void* const* W,
                           const void* const* V, const void* const* U, const void* const* ci_pre, uint32_t draw_k0,
                           uint32_t draw_k1, int use_delta, const uint8_t* routes, int layout, int imp_kind, float p,
                           float gamma, int normalize_at_one, float imp_coeff, float freq_coeff, float ref_count,
                           const float* freq_ema_in, float* freq_ema_out, float ema_count, float ema_halflife,
                           float recon_coeff, int n_kl_chunks, float* losses, float* const* dV, float* const* dU,
                           void* const* d_ci_pre, void* workspace, size_t workspace_bytes, void* stream,
                           void** events, int32_t* categories, int capacity, int* n_recorded);

/* ---- the engine's CI functions ------------------------------------------------------
 * SiteMLP (pd/core/ci_fn/implementations/mlp.py:57-78) of n_layers linears, as
 * LayerwiseMLPCIFn.site_preactivations runs it per site
 * (pd/core/ci_fn/implementations/layerwise_mlp.py:127-140): a_0 = x, z_i = a_i-1 @ W_i +
 * b_i, a_i = GELU_erf(z_i) for every layer but the last, preact = z_n. dims[0..n_layers]
 * are the widths (d_in, hidden..., C), each a positive multiple of 8; x bf16
 * [n_tokens, dims[0]]; weights[i] bf16 [dims[i], dims[i+1]] (the reference's "i o"
 * layout); biases[i] bf16 [dims[i+1]]; preact bf16 [n_tokens, dims[n]]. bf16 compute
 * with fp32 accumulation, every product, bias sum and GELU rounded to bf16 as the
 * engine's bf16 compute cast does. The forward keeps W^T copies and every hidden z_i and
 * a_i in the workspace; pd_ci_mlp_bwd reads them, so it takes the forward's workspace
 * unchanged. dims, weights, biases, d_weights and d_biases are HOST arrays of device
 * pointers. All tensors 16-byte aligned. n_layers <= 16. */
size_t pd_ci_mlp_workspace_size(int n_layers, const int64_t* dims, int64_t n_tokens);
int pd_ci_mlp_fwd(int n_layers, const int64_t* dims, int64_t n_tokens, const void* x, const void* const* weights,
                  const void* const* biases, void* preact, void* workspace, size_t workspace_bytes, void* stream);
/* Backward of pd_ci_mlp_fwd from d_preact bf16 [n_tokens, dims[n]]: d_weights[i] fp32
 * [dims[i], dims[i+1]], d_biases[i] fp32 [dims[i+1]] (overwritten; column sums in a fixed
 * order, so repeated calls are bit-identical), d_x bf16 [n_tokens, dims[0]] (nullable). */
int pd_ci_mlp_bwd(int n_layers, const int64_t* dims, int64_t n_tokens, const void* x, const void* const* weights,
                  const void* d_preact, float* const* d_weights, float* const* d_biases, void* d_x, void* workspace,
                  size_t workspace_bytes, void* stream);

/* ComponentActivationReadout (pd/core/ci_fn/implementations/transformer/
 * component_conditioning.py:215-245) with its ClampedAffineArm pair (:188-212):
 * out = base + s+ sig(a+ h + b+) + s- sig(a- (-h) + b-) + bias per component, sig the
 * symmetric leaky hard sigmoid (pd/core/ci_fn/squashing.py:25-38; forward clamp to
 * [0, 1]). h, base, out bf16 [n_tokens, C] (base nullable); params fp32 [7, C] rows
 * a+, b+, s+, a-, b-, s-, bias, each rounded to bf16 at use. */
int pd_ci_readout_fwd(int64_t n_tokens, int64_t C, const void* h, const float* params, const void* base, void* out,
                      void* stream);
/* Backward: d_h bf16 [n_tokens, C] (nullable) and d_params fp32 [7, C] (overwritten,
 * fixed-order sums) from d_out bf16; the d_base gradient is d_out itself. The clamp's
 * pullback is the symmetric leaky form: inside (0, 1) the gradient, at or below 0 only
 * a negative gradient scaled by 0.01, at or above 1 only a positive one scaled by 0.01. */
size_t pd_ci_readout_workspace_size(int64_t n_tokens, int64_t C);
int pd_ci_readout_bwd(int64_t n_tokens, int64_t C, const void* h, const float* params, const void* d_out, void* d_h,
                      float* d_params, void* workspace, size_t workspace_bytes, void* stream);

/* ---- adversarial sources (persistent and fresh PGD) ----------------------------------
 * Source masks m = ci + (1 - ci) s (pd/core/source_mask.py:56-63; the source read into
 * the CI's frame and dtype, pd/core/masking.py:260-272). ci and mask [rows, C] in dtype;
 * sources [rows / rows_per_source, C] stored as src_dtype (F32, BF16 or U16 = u / 65535,
 * pd/core/adversary.py:150-184). A source row covers rows_per_source consecutive CI rows:
 * the reference's source shapes `bsc`, `bc` and `c` over (batch, positions) are 1, the
 * positions of a sample, and every row. */
int pd_source_mask_fwd(const void* ci, int dtype, int64_t rows, int64_t C, const void* sources, int src_dtype,
                       int64_t rows_per_source, void* mask, void* stream);
/* d_sources fp32 [rows / rows_per_source, C] = sum over covered rows of g (1 - ci), in a
 * fixed order (overwritten); d_ci (nullable, dtype) = g (1 - s). */
size_t pd_source_mask_bwd_workspace_size(int64_t rows, int64_t C, int64_t rows_per_source);
int pd_source_mask_bwd(const void* g_mask, const void* ci, int dtype, int64_t rows, int64_t C, const void* sources,
                       int src_dtype, int64_t rows_per_source, float* d_sources, void* d_ci, void* workspace,
                       size_t workspace_bytes, void* stream);
/* One projected ascent of n source values in place (pd/core/adversary.py:392-470 and the
 * uint16 store with stochastic rounding, :186-214; fresh PGD's sign step,
 * pd/core/train.py:788-800), projected to [0, 1]. grad fp32 is the gradient w.r.t. the
 * float view. PD_PGD_SGD: s += lr g. PD_PGD_MOMENTUM: v = momentum v + g (state_a: fp32
 * velocity for fp32 sources, bf16 otherwise), s += lr v. PD_PGD_ADAM: state_a/state_b =
 * m, v at the source dtype (F32 or BF16), step_count = the step after this update (>= 1),
 * s += lr m_hat / (sqrt(v_hat) + eps); beta1/beta2 are doubles so that 1 - beta is formed in
 * double and rounded once, as the reference's Python-float arithmetic does.
 * PD_PGD_SIGN (F32 sources): s += lr sign(g). Bf16
 * storage rounds where the reference's bf16 arithmetic does; U16 storage quantizes with
 * uniforms of key (k0, k1) (the per-leaf fold of the caller's key) under `layout`. */
int pd_source_ascend(int opt, int src_dtype, int64_t n, void* sources, const float* grad, void* state_a,
                     void* state_b, float step_count, float lr, double beta1, double beta2, float eps, float momentum,
                     uint32_t k0, uint32_t k1, int layout, void* stream);

/* ---- faithfulness ---------------------------------------------------------------------
 * Relative squared weight error (pd/core/faithfulness.py:16-75) of the fp32 deltas
 * Delta = W - (V U)^T that the targets form per stack (pd/targets/transformer.py:2134-2184,
 * protocol pd/core/model.py:430-449). n_mats matrices W bf16 or fp32 [n_mats, d_out, d_in],
 * V fp32 [n_mats, d_in, C], U fp32 [n_mats, C, d_out]; every mats_per_site consecutive
 * matrices form one site (1 for dense stacks, the expert count for block-factored ones,
 * whose blocks partition the site matrix). w_sq_norms fp32 [n_mats / mats_per_site] =
 * ||W_site||^2. Outputs (device): loss[0] = scale * sum_site ||Delta_site||^2 /
 * ||W_site||^2 (scale = 1 / the number of sites of the whole model, so per-group calls
 * add up to the reference's mean); site_errors [n_sites] the relative errors (nullable);
 * delta fp32 [n_mats, d_out, d_in] (nullable; keep it for pd_faithfulness_bwd). fp32
 * products on the matrix cores (v_mfma_f32_32x32x2f32), split over C into at most 8
 * fixed chunks when the matrices alone fill fewer than 512 blocks; fixed-order
 * reductions, so results are bit-identical from call to call. */
size_t pd_faithfulness_workspace_size(int64_t n_mats, int64_t d_in, int64_t d_out, int64_t C);
int pd_faithfulness_fwd(int64_t n_mats, int64_t mats_per_site, int64_t d_in, int64_t d_out, int64_t C, const void* W,
                        int w_dtype, const float* V, const float* U, const float* w_sq_norms, float scale, float* loss,
                        float* site_errors, float* delta, void* workspace, size_t workspace_bytes, void* stream);
/* Gradients of pd_faithfulness_fwd's loss times *d_loss (a device scalar; NULL = 1):
 * dV = -2 scale d_loss / ||W_site||^2 Delta^T U^T, dU = -2 scale d_loss / ||W_site||^2
 * V^T Delta^T, fp32, overwritten. */
int pd_faithfulness_bwd(int64_t n_mats, int64_t mats_per_site, int64_t d_in, int64_t d_out, int64_t C,
                        const float* delta, const float* V, const float* U, const float* w_sq_norms, float scale,
                        const float* d_loss, float* dV, float* dU, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* PD_MI355X_H */
