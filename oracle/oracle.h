/*
 * CPU oracle for the fused LoRA / RMSNorm / softmax hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare against.
 * The product (libmc_hip.so) never links, loads or calls it, and nothing on
 * the product path may fall back to it.
 *
 * It restates the candle CPU composites of GarthDB/metal-candle v1.3.0 in
 * their op order, with fp64 accumulation and fp32 storage:
 *   LoRA delta   src/training/lora.rs:320-339  (H = x.A; dropout(H); H.B; *s)
 *                src/graph/executor.rs:141-158  (same order, no dropout)
 *   base linear  candle_nn::Linear as used at src/models/transformer.rs:189-192
 *                (y = x.W^T + b, W stored [out, in])
 *   RMSNorm      src/backend/tensor.rs:111-117  (sqr, mean, +eps, sqrt, divide)
 *                src/models/qwen.rs:314-325     (then * weight)
 *   softmax      src/backend/tensor.rs:91-98    (max, sub, exp, sum, divide)
 *                src/models/transformer.rs:264-275 (causal -inf mask added first)
 *   AdamW        src/training/optimizer.rs:227-281 (fp32 op order of the step)
 *   LayerNorm    src/backend/custom_ops.rs LayerNormOp::cpu_fwd, tensor.rs:100-109,
 *                src/embeddings/metal_bert.rs:30-72 (weight, bias)
 *   log-softmax  candle_nn::ops::log_softmax (src/training/loss.rs:108)
 *   cross entropy src/training/loss.rs:58-245 (ignore_index, label smoothing)
 *   dropout      candle_nn::ops::dropout (candle-nn 0.9, not vendored): keep iff
 *                U >= p, kept values scaled by 1/(1-p); the mask itself comes
 *                from the Philox4x32-10 generator below, shared with the GPU path.
 * The reference has no backward for any of these ops; the backward functions
 * are the closed-form gradients of the composites above (candle autograd of
 * lora.rs:323-339, tensor.rs:91-117, qwen.rs:320-321).
 *
 * How each function is pinned (tests/test_oracle.py):
 *   oracle_lora_fwd      executor known answer (tests/executor_direct.rs:345-367),
 *                        numpy fp64 brute force, B = 0 => delta = 0, p = 0 => W-only
 *                        linearity, committed golden vectors.
 *   oracle_lora_bwd      central finite differences of <y, dY> in fp64,
 *                        shape contract of tests/gradient_verification.rs:57-62.
 *   oracle_rmsnorm_fwd   known answers tensor.rs:185-199, 321-336, 382-420,
 *                        executor_direct.rs:480-495, constant rows
 *                        rmsnorm_correctness.rs:205-265 closed form.
 *   oracle_rmsnorm_bwd   finite differences (dx and dw).
 *   oracle_softmax_fwd   known answers tensor.rs:126-162, 262-276, 400-420,
 *                        softmax_correctness.rs:200-243, shift invariance,
 *                        exact zeros under the mask.
 *   oracle_softmax_bwd   finite differences, rows of dS sum to 0, masked zeros.
 *   oracle_philox4x32_10 Random123 known-answer vectors (Salmon et al., SC'11).
 *   oracle_dropout_mask  fraction kept ~ 1-p, independence of (seed, element).
 *   oracle_attention_fwd closed forms (q = 0: uniform / prefix-mean rows of v;
 *                        S = 1: o = v; a dominant key: o = its v row), an
 *                        all-zero mask equals no mask (transformer.rs:469-480),
 *                        torch.nn.functional.scaled_dot_product_attention on
 *                        the CPU in fp64 as a library cross-check, GQA equal to
 *                        explicitly repeated K/V heads.
 *   oracle_adamw_step    the reference's own AdamW tests (optimizer.rs:395-509:
 *                        lr 0.1 on ones gives 0.899 after one step, five
 *                        default steps lower the sum), the constant-gradient
 *                        closed form (m_hat = g, v_hat = g^2 at every step),
 *                        torch.optim.AdamW as a library cross-check.
 *   oracle_layernorm_*   the reference's layer_norm tests (tensor.rs:165-300:
 *                        zero row means, zeros in -> zeros out) and a
 *                        hand-computed row; torch.nn.functional.layer_norm and
 *                        its autograd in fp64; finite differences.
 *   oracle_log_softmax_* torch.log_softmax and autograd in fp64; exp rows sum
 *                        to 1; shift invariance.
 *   oracle_cross_entropy_* the reference's loss tests (loss.rs:247-380) with
 *                        their closed forms; torch.nn.functional.cross_entropy
 *                        (ignore_index, label smoothing without ignored rows)
 *                        and its autograd; finite differences.
 *   oracle_attention_bwd central finite differences of <o, dO> in fp64 for
 *                        q, k and v, torch autograd of the fp64 composite.
 *
 * Attention (src/models/transformer.rs:258-283, repeat_kv 295-319) is the
 * first of the rows next to the hot path: the score row of the reference's
 * q.k^T / sqrt(d) + mask, softmax_stable, .v sequence.
 */
#ifndef MC_ORACLE_H
#define MC_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Philox4x32-10 block: ctr[4], key[2] -> out[4]. */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* Dropout keep-mask for a [rows, rank] hidden: mask[i] = (U_i >= p), with
 * U_i = (philox word >> 8) * 2^-24 and element i = t*rank + j drawn from
 * counter block i/4, word i%4, key = (seed lo, seed hi). */
void oracle_dropout_mask(uint64_t seed, float p, int64_t rows, int32_t rank, uint8_t* mask);

/* y[T,N] = x[T,K] . W[N,K]^T + bias[N] + scale * ((x.A) (.) mask / (1-p)) . B
 * W and bias may be NULL (delta only, like FusedLoRAOp). mask may be NULL
 * (no dropout). If hd_out is not NULL it receives Hd[T,r] (post-dropout,
 * pre-scale hidden). threads <= 0 means all OpenMP threads. */
void oracle_lora_fwd(int64_t T, int64_t K, int64_t N, int32_t r, float scale, float p,
                     const float* x, const float* W, const float* bias,
                     const float* A, const float* B, const uint8_t* mask,
                     float* y, float* hd_out, int threads);

/* Backward of oracle_lora_fwd with W frozen:
 *   G = s dY B^T, Gd = G (.) M/(1-p)
 *   dX = dY W + Gd A^T ; dA = x^T Gd ; dB = s Hd^T dY
 * W may be NULL (delta-only op). Any of dx, dA, dB may be NULL (skipped). */
void oracle_lora_bwd(int64_t T, int64_t K, int64_t N, int32_t r, float scale, float p,
                     const float* x, const float* W, const float* A, const float* B,
                     const uint8_t* mask, const float* dy,
                     float* dx, float* dA, float* dB, int threads);

/* y = x / sqrt(mean(x^2) + eps) * w ; w may be NULL (unweighted, as in
 * FusedRMSNormOp). rstd_out (may be NULL) receives 1/sqrt(mean+eps) per row. */
void oracle_rmsnorm_fwd(int64_t rows, int64_t D, float eps, const float* x, const float* w,
                        float* y, float* rstd_out, int threads);

/* dx_ij = r_i g_ij - x_ij r_i^3 (1/D) sum_k g_ik x_ik, g = dy (.) w ;
 * dw_j = sum_i dy_ij x_ij r_i. w may be NULL (then g = dy); dx / dw may be NULL. */
void oracle_rmsnorm_bwd(int64_t rows, int64_t D, float eps, const float* x, const float* w,
                        const float* dy, float* dx, float* dw, int threads);

/* Row softmax over the last dim. causal_rows = 0: no mask. causal_rows = S > 0:
 * row i is query q = i mod S and column j is masked (-inf) iff j > q + (D - S),
 * the bottom-right aligned causal mask (S = D gives the square causal mask). */
void oracle_softmax_fwd(int64_t rows, int64_t D, int64_t causal_rows, const float* s, float* p,
                        int threads);

/* dS = P (.) (dP - sum_j dP_j P_j) ; masked positions give exactly 0. */
void oracle_softmax_bwd(int64_t rows, int64_t D, int64_t causal_rows, const float* p,
                        const float* dp, float* ds, int threads);

/* Same as oracle_softmax_fwd / _bwd on n rows whose positions in the full
 * tensor are row_ids[i] (the causal mask of row i uses row_ids[i] mod S), so a
 * sample of rows of a large tensor can be checked on its own. */
void oracle_softmax_fwd_rows(int64_t n, int64_t D, int64_t causal_rows, const int64_t* row_ids,
                             const float* s, float* p, int threads);
void oracle_softmax_bwd_rows(int64_t n, int64_t D, int64_t causal_rows, const int64_t* row_ids,
                             const float* p, const float* dp, float* ds, int threads);

/* Round-to-nearest-even fp32 -> bf16 -> fp32 (the rounding the bf16 inputs get). */
/* Attention core: q [B, H, S, D], k, v [B, Hkv, S, D], mask [S, S] or NULL,
 * o [B, S, H * D], lse [B, H, S] or NULL (natural log-sum-exp of each row). */
void oracle_attention_fwd(int64_t B, int32_t H, int32_t Hkv, int64_t S, int32_t D, float scale, int causal,
                          const float* q, const float* k, const float* v, const float* mask, float* o,
                          float* lse, int threads);
/* dq [B, H, S, D], dk, dv [B, Hkv, S, D] from dout [B, S, H * D]. */
void oracle_attention_bwd(int64_t B, int32_t H, int32_t Hkv, int64_t S, int32_t D, float scale, int causal,
                          const float* q, const float* k, const float* v, const float* mask, const float* dout,
                          float* dq, float* dk, float* dv, int threads);

/* One AdamW::step over n fp32 values: m, v updated in place, the new
 * parameter written to param_out (may equal param). */
void oracle_adamw_step(int64_t n, float lr, float beta1, float beta2, float eps, float wd, int64_t step,
                       const float* param, const float* grad, float* m, float* v, float* param_out);

/* LayerNorm [rows, D] with optional weight / bias (NULL: none). */
void oracle_layernorm_fwd(int64_t rows, int64_t D, float eps, const float* x, const float* w, const float* b,
                          float* y, float* mean, float* rstd, int threads);
void oracle_layernorm_bwd(int64_t rows, int64_t D, float eps, const float* x, const float* w, const float* dy,
                          float* dx, float* dw, float* db, int threads);
/* log-softmax over the last dim and its backward. */
void oracle_log_softmax_fwd(int64_t rows, int64_t D, const float* x, float* y, int threads);
void oracle_log_softmax_bwd(int64_t rows, int64_t D, const float* y, const float* dy, float* dx, int threads);
/* Cross-entropy loss over logits [rows, V] and targets [rows]; ignore_index < 0: none. */
double oracle_cross_entropy_fwd(int64_t rows, int64_t V, const float* logits, const uint32_t* targets,
                                int64_t ignore_index, float smoothing, float* lse, double* count);
void oracle_cross_entropy_bwd(int64_t rows, int64_t V, const float* logits, const uint32_t* targets,
                              int64_t ignore_index, float smoothing, float dloss, float* dlogits);

void oracle_round_bf16(const float* in, float* out, int64_t n);

#ifdef __cplusplus
}
#endif

#endif
