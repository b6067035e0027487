/*
 * bssm.h — C ABI of the MI355X (gfx950) Bayesian-recurrence library.
 *
 * Every entry point takes raw device pointers (row-major, contiguous fp32),
 * sizes, scalar options and a HIP stream handle passed as `void*`
 * (a `hipStream_t`; NULL = the legacy default stream).  Nothing here
 * allocates device memory or synchronises the stream, and each call only
 * enqueues kernels.  Two exceptions to "keeps no state between calls":
 *   - bssm_small_batch_limit() sets process-wide tuning limits that pick the
 *     D = 4, M = 8 kernel layout for a sequence count (row-per-sequence or
 *     rotated).  The layouts round differently, so changing a limit changes
 *     the low bits of those results; set it once, before the calls whose
 *     bits must be reproducible, not concurrently with them.
 *   - bssm_causal_conv4_backward_noalloc() keeps its partial sums in one
 *     device scratch array per GPU: calls that overlap on one GPU race.
 * Every other entry point is safe under HIP graph capture and from several
 * host threads at once.
 *
 * Return value: BSSM_OK (0) or a BSSM_ERR_* code; bssm_last_error() returns
 * the message of the most recent failure on the calling host thread.
 *
 * Shapes follow the reference extension ABI (N sequences, T tokens, key dim
 * D, value dim M, nb = ceil(T / chunk)):
 *   keys, queries, decay  [N, T, D]      values, out, gy          [N, T, M]
 *   process, observation  [N, T]         mean0, mean_final, gm*   [N, D, M]
 *   cov0, cov_final, gc*  [N, D, D]      bmean [N, nb+1, D, M]   bcov [N, nb+1, D, D]
 * bmean[:, c] / bcov[:, c] hold the belief before token c*chunk; index nb
 * holds the final belief.
 *
 * Supported (D, M): (1, 8), (2, 8), (4, 8), (8, 8), (64, 64).  D = M = 64
 * replaces the pybind module of bayes_ssm/persistent_bayes_chunked.cu
 * (exports at :436: forward_chunked, forward_chunked_fixed, backward_chunked,
 * backward_chunked_lean, backward_chunked_fixed, backward_chunked_lean_fixed;
 * kernels at :175-343).  Its covariance adjoint follows that file's
 * convention: the u = P'k adjoint gu k^T enters symmetrized
 * (persistent_bayes_chunked.cu:329-333), so the initial-covariance gradient
 * is symmetric, where D <= 8 return the full asymmetric one.
 */
#ifndef BSSM_H_
#define BSSM_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  BSSM_OK = 0,
  BSSM_ERR_ARGUMENT = 1,     /* null pointer, bad size, chunk <= 0, ...      */
  BSSM_ERR_UNSUPPORTED = 2,  /* (D, M) outside the supported set             */
  BSSM_ERR_LAUNCH = 3,       /* the HIP runtime rejected a kernel launch     */
};

/* Message of the last failure on this host thread ("" if none). */
const char* bssm_last_error(void);

/* ABI revision of this library (bumped on any signature change or change of
 * the supported (D, M) set). */
int bssm_abi_version(void);

/* 1 if (key_dim, value_dim) has a kernel, else 0. */
int bssm_supported(int key_dim, int value_dim);

/* Checkpoint interval (tokens) at which bssm_backward_chunked* replays each
 * chunk exactly once from its checkpoint (the kernel's on-chip history
 * length for this key dimension); 0 if unsupported.  Larger chunks are
 * valid but re-replay each chunk prefix once per history-length piece.
 * No reference counterpart: the reference backward always replays whole
 * chunks through HBM history tensors (persistent_bayes_chunked_d4m8.cu:524-548). */
int bssm_preferred_checkpoint(int key_dim);

/* ------------------------------------------------------------------------
 * Dynamic-diagonal forward with chunk-boundary checkpoints.
 * Replaces the pybind function `forward_chunked`
 * (bayes_ssm/persistent_bayes_chunked_d4m8.cu:461-468; same contract in
 * _d1m8.cu:387-393, _d2m8.cu forward_chunked, _d8.cu forward_chunked).
 * Per token: P' = diag(d) P diag(d) + p I, u = P' k, s = max(r + k.u, floor),
 * e = v - (d*M)^T k, M <- d*M + u e^T / s, P <- P' - u u^T / s, y = M^T q.
 */
int bssm_forward_chunked(int key_dim, int value_dim,
                         const float* keys, const float* values, const float* queries,
                         const float* decay, const float* process, const float* observation,
                         const float* mean0, const float* cov0,
                         float* out, float* mean_final, float* cov_final,
                         float* bmean, float* bcov,
                         int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                         void* stream);

/* Fixed dynamics A = 0.97 I, Q = 0.1 I, R = 1: decay/process/observation are
 * not read (they may be NULL).  Replaces `forward_chunked_fixed`
 * (persistent_bayes_chunked_d4m8.cu:470-474). */
int bssm_forward_chunked_fixed(int key_dim, int value_dim,
                               const float* keys, const float* values, const float* queries,
                               const float* decay, const float* process, const float* observation,
                               const float* mean0, const float* cov0,
                               float* out, float* mean_final, float* cov_final,
                               float* bmean, float* bcov,
                               int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                               void* stream);

/* Forward that also writes the per-token replay history used by the D1
 * saved-history reverse: mp = d*M_prev [N,T,D,M], pp = P' [N,T,D,D],
 * uh = u [N,T,D], bh = 1/s [N,T], eh = e [N,T,M].  Requires chunk == t
 * (one full-sequence chunk, so nb = 1).  Replaces `forward_chunked_saved`
 * (persistent_bayes_chunked_d1m8.cu:387-414). */
int bssm_forward_chunked_saved(int key_dim, int value_dim,
                               const float* keys, const float* values, const float* queries,
                               const float* decay, const float* process, const float* observation,
                               const float* mean0, const float* cov0,
                               float* out, float* mean_final, float* cov_final,
                               float* bmean, float* bcov,
                               float* mp, float* pp, float* uh, float* bh, float* eh,
                               int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                               void* stream);

/* ------------------------------------------------------------------------
 * Chunk-replay reverse.  Each checkpoint chunk is replayed on chip from
 * bmean/bcov and then reversed; the adjoint of the belief is carried across
 * chunks inside the kernel (one launch per call).  For D = 4, M = 8 the
 * tiled kernels take checkpoint chunks of 8 tokens (the preferred interval)
 * or 16 (the start of each 16-token tile's second half re-advanced on chip);
 * other chunks run the generic kernels.
 *
 * gmf / gcf are the gradients of mean_final / cov_final; NULL means zero.
 * Output gradients: gk, gq, gd [N,T,D]; gv [N,T,M]; gp, gr [N,T];
 * gm0 [N,D,M]; gc0 [N,D,D].  gc0 keeps the full (asymmetric) derivative with
 * respect to the unconstrained initial covariance: (sym(G) + gu k^T) * d d^T.
 *
 * Replaces `backward_chunked` (persistent_bayes_chunked_d4m8.cu:556-559):
 * all eight gradients. */
int bssm_backward_chunked(int key_dim, int value_dim,
                          const float* keys, const float* values, const float* queries,
                          const float* decay, const float* process, const float* observation,
                          const float* mean0, const float* cov0,
                          const float* bmean, const float* bcov,
                          const float* gy, const float* gmf, const float* gcf,
                          float* gk, float* gv, float* gq, float* gd, float* gp, float* gr,
                          float* gm0, float* gc0,
                          int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                          void* stream);

/* Keys/values/queries gradients only.  Replaces `backward_chunked_lean`
 * (persistent_bayes_chunked_d4m8.cu:561-564). */
int bssm_backward_chunked_lean(int key_dim, int value_dim,
                               const float* keys, const float* values, const float* queries,
                               const float* decay, const float* process, const float* observation,
                               const float* mean0, const float* cov0,
                               const float* bmean, const float* bcov,
                               const float* gy, const float* gmf, const float* gcf,
                               float* gk, float* gv, float* gq,
                               int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                               void* stream);

/* Six gradients (no initial-state outputs).  Replaces
 * `backward_chunked_noinitial` (persistent_bayes_chunked_d2m8.cu:576-580). */
int bssm_backward_chunked_noinitial(int key_dim, int value_dim,
                                    const float* keys, const float* values, const float* queries,
                                    const float* decay, const float* process, const float* observation,
                                    const float* mean0, const float* cov0,
                                    const float* bmean, const float* bcov,
                                    const float* gy, const float* gmf, const float* gcf,
                                    float* gk, float* gv, float* gq, float* gd, float* gp, float* gr,
                                    int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                    void* stream);

/* Fixed-dynamics reverse (A = 0.97 I, Q = 0.1 I, R = 1).  gd, gp, gr are
 * written as zeros, as the reference fixed ABI returns them.  Replaces
 * `backward_chunked_fixed` (persistent_bayes_chunked_d4m8.cu:572-575). */
int bssm_backward_chunked_fixed(int key_dim, int value_dim,
                                const float* keys, const float* values, const float* queries,
                                const float* decay, const float* process, const float* observation,
                                const float* mean0, const float* cov0,
                                const float* bmean, const float* bcov,
                                const float* gy, const float* gmf, const float* gcf,
                                float* gk, float* gv, float* gq, float* gd, float* gp, float* gr,
                                float* gm0, float* gc0,
                                int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                void* stream);

/* Replaces `backward_chunked_lean_fixed` (persistent_bayes_chunked_d4m8.cu:566-569). */
int bssm_backward_chunked_lean_fixed(int key_dim, int value_dim,
                                     const float* keys, const float* values, const float* queries,
                                     const float* decay, const float* process, const float* observation,
                                     const float* mean0, const float* cov0,
                                     const float* bmean, const float* bcov,
                                     const float* gy, const float* gmf, const float* gcf,
                                     float* gk, float* gv, float* gq,
                                     int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                     void* stream);

/* Replaces `backward_chunked_noinitial_fixed` (persistent_bayes_chunked_d2m8.cu:597-600). */
int bssm_backward_chunked_noinitial_fixed(int key_dim, int value_dim,
                                          const float* keys, const float* values, const float* queries,
                                          const float* decay, const float* process, const float* observation,
                                          const float* mean0, const float* cov0,
                                          const float* bmean, const float* bcov,
                                          const float* gy, const float* gmf, const float* gcf,
                                          float* gk, float* gv, float* gq, float* gd, float* gp, float* gr,
                                          int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                          void* stream);

/* Saved-history reverse: consumes mp/pp/uh/bh/eh written by
 * bssm_forward_chunked_saved instead of replaying.  Requires chunk == t.
 * Replaces `backward_chunked_saved` (persistent_bayes_chunked_d1m8.cu:632-640)
 * and `backward_chunked_saved_d1` (:600-630), which return the same eight
 * gradients. */
int bssm_backward_chunked_saved(int key_dim, int value_dim,
                                const float* keys, const float* values, const float* queries,
                                const float* decay, const float* process, const float* observation,
                                const float* mean0, const float* cov0,
                                const float* bmean, const float* bcov,
                                const float* mp, const float* pp, const float* uh,
                                const float* bh, const float* eh,
                                const float* gy, const float* gmf, const float* gcf,
                                float* gk, float* gv, float* gq, float* gd, float* gp, float* gr,
                                float* gm0, float* gc0,
                                int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                void* stream);

/* Replaces `backward_chunked_saved_lean` (persistent_bayes_chunked_d1m8.cu:642-650). */
int bssm_backward_chunked_saved_lean(int key_dim, int value_dim,
                                     const float* keys, const float* values, const float* queries,
                                     const float* decay, const float* process, const float* observation,
                                     const float* mean0, const float* cov0,
                                     const float* bmean, const float* bcov,
                                     const float* mp, const float* pp, const float* uh,
                                     const float* bh, const float* eh,
                                     const float* gy, const float* gmf, const float* gcf,
                                     float* gk, float* gv, float* gq,
                                     int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                     void* stream);

/* ------------------------------------------------------------------------
 * bfloat16 keys, values and queries.
 * No reference counterpart: the reference promotes bfloat16 projections to
 * float32 before its extension (bayes_ssm/bayesian_layer.py:823-827); these
 * entry points read them as bfloat16 and widen them on chip, with results
 * identical to the float32 entry points on the widened values.  D = 4, M = 8
 * only, T a positive multiple of 4, 16-byte aligned streams; anything else
 * returns BSSM_ERR_UNSUPPORTED (the caller widens and uses the float32 ABI).
 */

/* Forward: as bssm_forward_chunked (fixed == 0) or
 * bssm_forward_chunked_fixed (fixed != 0); keys, values, queries are
 * bfloat16 [N,T,D] / [N,T,M] / [N,T,D]; out and all other tensors float32. */
int bssm_forward_chunked_bf16(int key_dim, int value_dim, int fixed,
                              const void* keys, const void* values, const void* queries,
                              const float* decay, const float* process, const float* observation,
                              const float* mean0, const float* cov0,
                              float* out, float* mean_final, float* cov_final,
                              float* bmean, float* bcov,
                              int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                              void* stream);

/* Reverse: gk, gv, gq are bfloat16, each the float32 gradient rounded to
 * nearest even (the gradient of a bfloat16 -> float32 widening).  gd, gp,
 * gr (float32) are given together or all NULL (then not computed; with
 * fixed != 0 they are written as zeros when given); gm0, gc0 may be NULL.
 * chunk must equal bssm_preferred_checkpoint(4). */
int bssm_backward_chunked_bf16(int key_dim, int value_dim, int fixed,
                               const void* keys, const void* values, const void* queries,
                               const float* decay, const float* process, const float* observation,
                               const float* mean0, const float* cov0,
                               const float* bmean, const float* bcov,
                               const float* gy, const float* gmf, const float* gcf,
                               void* gk, void* gv, void* gq, float* gd, float* gp, float* gr,
                               float* gm0, float* gc0,
                               int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                               void* stream);

/* float8 keys, values and queries (format 0: torch.float8_e4m3fn, 1:
 * torch.float8_e5m2, the OCP encodings), for D = 4, M = 8 under the same
 * conditions as the bfloat16 entry points.  The kernels widen each value to
 * float32 on chip (exactly), so outputs equal those of the float32 entry
 * points on the widened inputs, bit for bit; the gradients of keys, values
 * and queries leave as float8, the float32 gradient rounded to nearest even
 * with torch's overflow rules (bssm_round_float8).  Replaces the float32
 * promotion of float8 inputs (bayes_ssm/bayesian_layer.py:823-827) feeding
 * the float32 entry points; no counterpart in the reference library. */
int bssm_forward_chunked_fp8(int key_dim, int value_dim, int fixed, int format,
                             const void* keys, const void* values, const void* queries,
                             const float* decay, const float* process, const float* observation,
                             const float* mean0, const float* cov0,
                             float* out, float* mean_final, float* cov_final, float* bmean, float* bcov,
                             int64_t n, int64_t t, int64_t chunk, float denominator_floor, void* stream);
int bssm_backward_chunked_fp8(int key_dim, int value_dim, int fixed, int format,
                              const void* keys, const void* values, const void* queries,
                              const float* decay, const float* process, const float* observation,
                              const float* mean0, const float* cov0, const float* bmean, const float* bcov,
                              const float* gy, const float* gmf, const float* gcf,
                              void* gk, void* gv, void* gq, float* gd, float* gp, float* gr,
                              float* gm0, float* gc0,
                              int64_t n, int64_t t, int64_t chunk, float denominator_floor, void* stream);

/* Host-side float32 -> float8 rounding of the float8 gradients (format as
 * above): round to nearest even; e4m3fn gives the NaN code 0x7f (with the
 * sign) for magnitudes that round past 448, for infinities and NaN; e5m2
 * overflows to infinity and gives 0x7f for NaN.  This is torch's
 * float32 -> float8 conversion; no counterpart in the reference library. */
int bssm_round_float8(int format, const float* x, uint8_t* out, int64_t count);

/* Value statistics behind bayesian_layer's argument checks (finite entries,
 * variance signs; bayes_ssm/bayesian_layer.py:105-129, :798-985, where each
 * tensor is checked with its own reduction and synchronization).  For each of
 * `count` (at most 16) contiguous device tensors (float32, or float64 where
 * is_double[i] != 0) writes out[3i .. 3i+2] = (min, max, any non-finite) on
 * `stream`: min and max over the finite entries (float64 entries mapped to
 * float32 with their sign kept), the third 1 if any entry is NaN or
 * infinite.  workspace: bssm_value_stats_workspace(count, numels) floats
 * (-1: invalid arguments).  No counterpart in the reference library. */
int64_t bssm_value_stats_workspace(int count, const int64_t* numels);
int bssm_value_stats(int count, const void* const* tensors, const int64_t* numels, const int* is_double,
                     float* workspace, int64_t workspace_floats, float* out, void* stream);

/* ------------------------------------------------------------------------
 * Static (A = I, Q = 0) associative scan in information form.
 * Replaces the torch-op chain of `associative_static_bayesian`
 * (bayes_ssm/replay_ssm.py:251-270):
 *   L_t = inv(P0) + sum_{s<=t} k_s k_s^T / r_s,  N_t = inv(P0) M0 + sum k_s v_s^T / r_s,
 *   M_t = L_t^{-1} N_t (Cholesky), y_t = M_t^T q_t, P_T = L_T^{-1}.
 * keys/queries [B,T,D], values [B,T,M], observation [B,T] (>= floor, checked
 * by the caller), mean0 [B,D,M], cov0 [B,D,D] (SPD).  Outputs out [B,T,M],
 * mean_final [B,D,M], cov_final [B,D,D].  Supports D <= 32, M <= 64. */
int bssm_associative_static_scan(const float* keys, const float* values, const float* queries,
                                 const float* observation, const float* mean0, const float* cov0,
                                 float* out, float* mean_final, float* cov_final,
                                 int64_t b, int64_t t, int key_dim, int value_dim,
                                 void* stream);

/* Reverse of bssm_associative_static_scan.  Replaces the autograd of the
 * differentiable torch-op chain behind associative_static_bayesian_cuda
 * (bayes_ssm/replay_ssm.py:251-270, :276-339): given grad_out [B,T,M] and
 * the (optional, NULL = zero) grad_mean_final [B,D,M] / grad_cov_final
 * [B,D,D], writes the gradients of keys, values, queries [B,T,*],
 * observation [B,T], mean0 [B,D,M] and cov0 [B,D,D].  With
 * G_t = q_t gy_t^T (+ grad_mean_final at the last token):
 *   gq_t = M_t gy_t,  gN_t = L_t^{-1} G_t,
 *   gL_t = sym(-gN_t M_t^T) (+ sym(-P_T grad_cov_final P_T) at the last token),
 * suffix sums SL_s, SN_s of gL_t, gN_t over t >= s, and
 *   gk_s = (2 SL_s k_s + SN_s v_s) / r_s,  gv_s = SN_s^T k_s / r_s,
 *   gr_s = -(k_s^T SL_s k_s + k_s^T SN_s v_s) / r_s^2,
 *   gM0 = inv(P0)^T SN_0,  gP0 = -inv(P0)^T (SL_0 + SN_0 M0^T) inv(P0)^T.
 * workspace: B * T * (D * D + D * M) floats (the caller's).  Supports
 * key_dim <= 16, value_dim <= 64 and T >= 1. */
int bssm_associative_static_scan_backward(const float* keys, const float* values, const float* queries,
                                          const float* observation, const float* mean0, const float* cov0,
                                          const float* grad_out, const float* grad_mean_final,
                                          const float* grad_cov_final, float* workspace,
                                          float* grad_keys, float* grad_values, float* grad_queries,
                                          float* grad_observation, float* grad_mean0, float* grad_cov0,
                                          int64_t b, int64_t t, int key_dim, int value_dim, void* stream);

/* ------------------------------------------------------------------------
 * Producer-fused layer core of the Bayes mixer (D = 4, M = 8, learned
 * dynamics).  Replaces the torch-op chain between the projections and the
 * readout of example/train_6layer.py:627-693 and :702-709:
 *   q, k = normalize(silu(q_proj)), normalize(silu(k_proj))  (per head, eps 1e-12)
 *   v = silu(v_proj), decay = exp(-softplus(decay_logits)),
 *   process, observation = softplus(noise[.., 0]), softplus(noise[.., 1]) + 1e-4,
 *   the [B,T,H,.] -> [B*H,T,.] permutes, bayesian_layer, and the readout
 *   permute back to [B,T,H,8].
 * Inputs are bfloat16 [B, T, *] views with a row stride in elements (ld*):
 * q_proj, k_proj, decay_logits [.., H*4], v_proj [.., H*8], noise [.., H*2]
 * ((process, observation) per head); the innermost dimension is contiguous,
 * each ld* is a multiple of 8 and each base 16-byte aligned, so that one
 * fused projection output can be passed as five column views.  mean0 [B*H,4,8],
 * cov0 [B*H,4,4] float32 (sequence b*H + h).  Outputs: read [B,T,H*8] float32
 * (contiguous), mean_final, cov_final, and the checkpoints bmean
 * [B*H, nb+1, 4, 8], bcov [B*H, nb+1, 4, 4] with nb = ceil(T / chunk).
 * Needs H % 16 == 0, T a positive multiple of 4, chunk ==
 * bssm_preferred_checkpoint(4);
 * otherwise BSSM_ERR_UNSUPPORTED.  No counterpart in the reference library:
 * its mixer materialises every transformed and permuted tensor in float32. */
int bssm_mixer_forward(const void* q_proj, int64_t ldq, const void* k_proj, int64_t ldk,
                       const void* v_proj, int64_t ldv, const void* decay_logits, int64_t ldd,
                       const void* noise, int64_t ldn,
                       const float* mean0, const float* cov0,
                       float* read, float* mean_final, float* cov_final,
                       float* bmean, float* bcov,
                       int64_t batch, int64_t t, int64_t heads, int64_t chunk,
                       float denominator_floor, void* stream);

/* Reverse of bssm_mixer_forward: gradients of the five projections, written
 * contiguous ([B,T,H*4] for q, k, decay logits; [B,T,H*8] for v; [B,T,H*2]
 * for noise) as bfloat16, the float32 gradient rounded to nearest even (what
 * autograd through the reference's .float() widening yields); with
 * grad_f32 != 0 they are written as float32 instead (same shapes).
 * grad_decay_logits and grad_noise are given together or both NULL (then
 * not computed); grad_read [B,T,H*8] float32 contiguous; gmf, gcf, gm0, gc0
 * may be NULL. */
int bssm_mixer_backward(const void* q_proj, int64_t ldq, const void* k_proj, int64_t ldk,
                        const void* v_proj, int64_t ldv, const void* decay_logits, int64_t ldd,
                        const void* noise, int64_t ldn,
                        const float* mean0, const float* cov0,
                        const float* bmean, const float* bcov,
                        const float* grad_read, const float* gmf, const float* gcf,
                        void* grad_q, void* grad_k, void* grad_v, void* grad_decay_logits,
                        void* grad_noise, float* gm0, float* gc0,
                        int64_t batch, int64_t t, int64_t heads, int64_t chunk,
                        float denominator_floor, int grad_f32, void* stream);

/* ------------------------------------------------------------------------
 * Rotation dynamics: block-diagonal damped 2-D rotations.  Replaces the
 * reference's rotation core _core_loop_rotation (bayes_ssm/bayesian_layer.py
 * :254-323, run there through torch.compile, :326-340).  Per token, pair
 * j = state rows (2j, 2j+1) turns by [[c, -s], [s, c]], c = rho cos(angle),
 * s = rho sin(angle), rho = min(max(radius, FLT_MIN), 1); the pair's process
 * variance is added to covariance entry (2j, 2j); then the update of
 * bssm_forward_chunked.  keys/queries [N,T,D], values/out [N,T,M],
 * radii/angles/process [N,T,D/2], observation [N,T]; belief and checkpoint
 * tensors as bssm_forward_chunked.  Supports (D, M) in {(2,8), (4,8), (8,8)}.
 * No counterpart in the reference's CUDA extension. */
int bssm_forward_chunked_rotation(int key_dim, int value_dim,
                                  const float* keys, const float* values, const float* queries,
                                  const float* radii, const float* angles, const float* process,
                                  const float* observation, const float* mean0, const float* cov0,
                                  float* out, float* mean_final, float* cov_final,
                                  float* bmean, float* bcov,
                                  int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                  void* stream);

/* Reverse: all seven input gradients (g_radii is zero where the radius clamp
 * is active) and, when non-NULL, gm0 and the asymmetric gc0 (the convention
 * of bssm_backward_chunked).  Replays each chunk of `chunk` tokens from its
 * checkpoint; bssm_rotation_checkpoint(D) is the interval replayed in one
 * piece. */
int bssm_backward_chunked_rotation(int key_dim, int value_dim,
                                   const float* keys, const float* values, const float* queries,
                                   const float* radii, const float* angles, const float* process,
                                   const float* observation, const float* mean0, const float* cov0,
                                   const float* bmean, const float* bcov,
                                   const float* gy, const float* gmf, const float* gcf,
                                   float* gk, float* gv, float* gq, float* g_radii, float* g_angles,
                                   float* g_process, float* g_observation, float* gm0, float* gc0,
                                   int64_t n, int64_t t, int64_t chunk, float denominator_floor,
                                   void* stream);

/* Checkpoint interval of the rotation backward for key_dim (0 if unsupported).
 * No reference counterpart. */
int bssm_rotation_checkpoint(int key_dim);

/* Largest sequence count N for which the D = 4, M = 8 float32 forward
 * (direction 0) or backward (direction 1) uses the row-per-sequence kernels
 * (a 16-lane row per sequence, 4 per wave) instead of the rotated-layout ones
 * (a quad per sequence, 16 per wave).  Below about 1024 x 16 sequences the
 * waves of the latter do not fill the GPU and each wave's time is its own
 * instruction stream, which the row layout shortens; at large N the row
 * layout's extra lane work costs more than it saves (the backward first).
 * The backward also needs T a multiple of 16 and the preferred checkpoint
 * chunk.  Direction 2 (3): the largest N, within direction 0's (1's), for
 * which the row forward (backward) runs as two (three) waves per 4
 * sequences, the covariance and mean halves (the covariance replay, the
 * covariance reverse and the mean) on separate SIMDs, bitwise the one-wave
 * results.  bf16 and float8 keys, values and queries (the _bf16 / _fp8 entry
 * points) take the row kernels only within the two-wave (three-wave) limits
 * (widened on chip, bitwise the float32 split kernels on the widened values).
 * Direction 4: the largest N for which the D = 4 rotation forward
 * (bssm_forward_chunked_rotation) uses its row-per-sequence kernel (16-byte
 * aligned streams, T a multiple of 4).  Defaults: 24576, 8192, 2048, 2048,
 * 32768, the measured crossovers.
 * Sets the limit when limit >= 0 and returns the previous one; limit < 0
 * only reads it; -1 for any other direction.  Results of the row and
 * rotated layouts agree within float32 rounding, not bitwise.  With the
 * default limits the forward results of a sequence are the same bits for
 * every N up to 24576 (the row layout's one- and two-wave forwards are
 * bitwise one another); its gradients change layout above 8192 sequences
 * and then differ in the last bits: at config 3 (T = 512), the same
 * sequences inside N = 16384 and inside N = 2048 or 32 differ by at most
 * 1.2e-4 absolute (dL/dr) and 2e-5 for the other gradients, inside the
 * 1e-5 relative + 1e-4 absolute tolerance both meet against the float64
 * oracle (tests/test_gpu_batch_invariance.py).  No counterpart in the
 * reference (a tuning switch of this library). */
int64_t bssm_small_batch_limit(int direction, int64_t limit);

/* ------------------------------------------------------------------------
 * Length-four causal depthwise filter.  Replaces CausalDepthwise4.forward
 * (example/train_6layer.py:160-191) as the mixer applies it to each
 * projected stream (:474-480): per channel c and token t,
 *   y[t] = w[c,0] x[t-3] + w[c,1] x[t-2] + w[c,2] x[t-1] + w[c,3] x[t],
 * x = 0 before token 0.  Channels-last rows: x [B, T, C] with row stride ldx
 * (elements; a column view of a wider projection is fine), y [B, T, C]
 * contiguous.  bf16 != 0: bfloat16 streams (else float32), computed in
 * float32 and rounded once.  weight: float32 [C, 4] (the module's [C, 1, 4]).
 * C and ldx must be multiples of 16 bytes' worth of elements (8 bf16,
 * 4 float32) and the pointers 16-byte aligned. */
int bssm_causal_conv4_forward(int bf16, const void* x, int64_t ldx, const float* weight, void* y,
                              int64_t batch, int64_t t, int64_t channels, void* stream);

/* Reverse: grad_x[s] = sum_j w[c,j] grad_y[s+3-j] (contiguous [B, T, C],
 * same dtype) and the weight gradient as per-batch-entry partial sums
 * grad_weight_partials [B, C, 4] (float32; their sum over B is the
 * gradient of the [C, 1, 4] weight). */
int bssm_causal_conv4_backward(int bf16, const void* x, int64_t ldx, const float* weight,
                               const void* grad_y, void* grad_x, float* grad_weight_partials,
                               int64_t batch, int64_t t, int64_t channels, void* stream);

/* The reverse of bssm_causal_conv4_forward without any allocation: the same
 * grad_x, and the weight gradient itself, grad_weight [C, 4] (float32, the
 * sum over the batch of bssm_causal_conv4_backward's partials), with the
 * per-batch-entry partials kept in the library's own device scratch (a
 * file-scope array of 2^21 floats, 8 MiB, on every GPU the library runs on,
 * held until the process ends) instead of a caller buffer.  Needs
 * batch * channels <= 524288, else BSSM_ERR_ARGUMENT.  All calls on one GPU
 * share the scratch: calls that overlap on that GPU (other streams or
 * threads) race.  No counterpart in the reference library: it is for callers
 * that cannot allocate (code under HIP graph capture, serving loops,
 * harnesses that forbid hipMalloc). */
int bssm_causal_conv4_backward_noalloc(int bf16, const void* x, int64_t ldx, const float* weight,
                                       const void* grad_y, void* grad_x, float* grad_weight,
                                       int64_t batch, int64_t t, int64_t channels, void* stream);

/* ------------------------------------------------------------------------
 * The mixer core with its readout epilogue.  Replaces, after the op chain
 * of bssm_mixer_forward, the readout of example/train_6layer.py:719-729:
 *   out = read_norm(read.to(bf16)) * silu(gate)     (per head of 8 values)
 * with read_norm an RMSNorm over the head: x / sqrt(mean(x^2) + norm_eps) * w
 * (torch's rms_norm with eps None uses the float32 epsilon, 1.1920929e-7).
 * The product is formed in float32 from bf16(read) and rounded to bf16 once.
 * gate: bf16 [B, T, H*8] view with row stride ldg (a multiple of 8, 16-byte
 * aligned base); norm_weight: float32 [8].  Outputs: out [B, T, H*8] bf16
 * (float32 when precise != 0), read_bf16 = bf16(read) [B, T, H*8] (kept for
 * the backward), and the belief outputs of bssm_mixer_forward; read itself is
 * not written.  No counterpart in the reference library. */
int bssm_mixer_gated_forward(const void* q_proj, int64_t ldq, const void* k_proj, int64_t ldk,
                             const void* v_proj, int64_t ldv, const void* decay_logits, int64_t ldd,
                             const void* noise, int64_t ldn, const void* gate, int64_t ldg,
                             const float* norm_weight, float norm_eps,
                             const float* mean0, const float* cov0,
                             void* out, void* read_bf16, float* mean_final, float* cov_final,
                             float* bmean, float* bcov,
                             int64_t batch, int64_t t, int64_t heads, int64_t chunk,
                             float denominator_floor, int precise, void* stream);

/* Reverse of bssm_mixer_gated_forward from grad_out (bf16 [B, T, H*8]):
 * the readout gradient is formed on chip and never stored.  Writes the
 * projection gradients as bssm_mixer_backward does, grad_gate [B, T, H*8]
 * (bf16, contiguous) and the norm-weight gradient as per-wave partial sums
 * grad_norm_weight_partials [B*H/16, 8] (float32; their column sums are the
 * gradient).  precise != 0 writes every bf16 gradient as float32 instead. */
int bssm_mixer_gated_backward(const void* q_proj, int64_t ldq, const void* k_proj, int64_t ldk,
                              const void* v_proj, int64_t ldv, const void* decay_logits, int64_t ldd,
                              const void* noise, int64_t ldn, const void* gate, int64_t ldg,
                              const float* norm_weight, float norm_eps,
                              const float* mean0, const float* cov0,
                              const float* bmean, const float* bcov,
                              const void* read_bf16, const void* grad_out,
                              const float* gmf, const float* gcf,
                              void* grad_q, void* grad_k, void* grad_v, void* grad_decay_logits,
                              void* grad_noise, void* grad_gate, float* grad_norm_weight_partials,
                              float* gm0, float* gc0,
                              int64_t batch, int64_t t, int64_t heads, int64_t chunk,
                              float denominator_floor, int precise, void* stream);

/* ------------------------------------------------------------------------
 * Config 4's Bayes block in one call per direction.  Replaces the torch chain
 * of BayesianMixer.forward (example/train_6layer.py:583-729) from the fused
 * projection to out_proj's input, paper features with the fused Q/K/V/aux/gate
 * projection (:585-600), key dim 4, value dim 8:
 *   convolved = CausalDepthwise4(projected[..., :16H])      (:598, :474-480)
 *   q, k, v   = convolved split (4H, 4H, 8H)                (:599-601)
 *   aux       = projected[..., 16H:22H] + aux_bias          (:589-593)
 *   out       = bssm_mixer_gated_forward(q, k, v, aux[..., :4H], aux[..., 4H:],
 *                                        gate = projected[..., 22H:])
 * projected: bf16 [B, T, 30H] rows with stride ld_projected (>= 30H, a
 * multiple of 8, 16-byte aligned).  aux_bias: NULL (no bias) or bf16 [6H],
 * 16-byte aligned; the kernels add it to the aux columns as they read them,
 * in bf16 (one rounding to nearest even, as torch adds two bf16 tensors).
 * conv_weight: float32 [16H, 4].  convolved: bf16 [B, T, 16H] (written by the
 * forward, kept for the backward).  Other arguments as in the gated mixer
 * (heads a multiple of 16, T a positive multiple of 4). */
int bssm_mixer_block_forward(const void* projected, int64_t ld_projected, const float* conv_weight,
                             const void* aux_bias, const float* norm_weight, float norm_eps,
                             const float* mean0, const float* cov0, void* convolved, void* out,
                             void* read_bf16, float* mean_final, float* cov_final, float* bmean, float* bcov,
                             int64_t batch, int64_t t, int64_t heads, int64_t chunk,
                             float denominator_floor, void* stream);

/* Reverse of bssm_mixer_block_forward.  Writes every column of
 * grad_projected (bf16 [B, T, 30H], row stride ld_grad_projected): the
 * filter's input gradient into the core columns, the aux and gate gradients
 * into theirs (the aux gradient is also aux_bias's per token).  Workspace
 * grad_convolved: bf16 [B, T, 16H], and the float32 partial sums of the
 * weight gradients: grad_conv_weight_partials [B, 16H, 4] (over the first
 * axis), grad_norm_weight_partials [B*H/16, 8] and, when not NULL,
 * grad_aux_partials [B, 6H] (the aux gradient summed over T).  Each of
 * grad_conv_weight [16H, 4], grad_norm_weight [8] and grad_aux_bias [6H]
 * that is not NULL receives the column sums of its partials (grad_aux_bias
 * needs grad_aux_partials), bf16 when grad_bf16 != 0, else float32. */
int bssm_mixer_block_backward(const void* projected, int64_t ld_projected, const float* conv_weight,
                              const void* aux_bias, const void* convolved,
                              const float* norm_weight, float norm_eps,
                              const float* mean0, const float* cov0, const float* bmean, const float* bcov,
                              const void* read_bf16, const void* grad_out,
                              const float* gmf, const float* gcf,
                              void* grad_convolved, void* grad_projected, int64_t ld_grad_projected,
                              float* grad_conv_weight_partials, float* grad_norm_weight_partials,
                              float* grad_aux_partials, void* grad_conv_weight, void* grad_norm_weight,
                              void* grad_aux_bias, int grad_bf16, float* gm0, float* gc0,
                              int64_t batch, int64_t t, int64_t heads, int64_t chunk,
                              float denominator_floor, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BSSM_H_ */
