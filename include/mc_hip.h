/*
 * mc_hip.h - C ABI of the MI355X (gfx950) fused LoRA / RMSNorm / softmax path.
 *
 * This is the drop-in boundary for the fused custom ops of GarthDB/metal-candle
 * v1.3.0. Each entry point replaces the Metal dispatch inside one candle
 * CustomOp (or the candle autograd of the composite the op stands for):
 *
 *   mc_lora_fwd      FusedLoRAOp::metal_fwd / metal_fwd_impl
 *                    (src/backend/custom_ops.rs:247-249, 359-430), extended
 *                    with the frozen base linear of candle_nn::Linear
 *                    (src/models/transformer.rs:189-192) and the dropout of
 *                    LoRALayer::forward (src/training/lora.rs:320-339).
 *   mc_lora_bwd      no reference kernel: candle autograd of lora.rs:323-339
 *                    (dX, dA, dB with W frozen). FusedLoRAOp leaves
 *                    CustomOp1::bwd at candle's default.
 *   mc_rmsnorm_fwd   FusedRMSNormOp::metal_fwd (custom_ops.rs:534-631), plus
 *                    the weight multiply of Qwen RMSNorm::forward
 *                    (src/models/qwen.rs:314-325).
 *   mc_rmsnorm_bwd   no reference kernel: autograd of tensor.rs:111-117 and
 *                    qwen.rs:320-321.
 *   mc_softmax_fwd   FusedSoftmaxOp::metal_fwd (custom_ops.rs:727-823), plus
 *                    the causal -inf mask that Attention::forward adds before
 *                    softmax_stable (src/models/transformer.rs:264-275).
 *   mc_softmax_bwd   no reference kernel: autograd of tensor.rs:91-98.
 *   mc_attention_fwd the attention core of Attention::forward
 *                    (src/models/transformer.rs:258-283) with repeat_kv
 *                    (295-319), without materialising the score matrix.
 *   mc_attention_bwd no reference kernel: autograd of the same composite.
 *   mc_adamw_step    AdamW::step (src/training/optimizer.rs:227-281) for many
 *                    parameter tensors per launch.
 *   mc_layernorm_*   LayerNormOp (custom_ops.rs:826-1079) with the weight and
 *                    bias of MetalLayerNorm (src/embeddings/metal_bert.rs).
 *   mc_log_softmax_*, mc_cross_entropy_*  cross_entropy_loss and its label
 *                    smoothing (src/training/loss.rs:58-245).
 *
 * Conventions (all entry points):
 *  - Device buffers are caller-owned, row-major and contiguous; inputs are
 *    read-only; outputs are fully written. Pointers must be 16-byte aligned.
 *  - All work is enqueued on `stream` (0 = the null stream); no call
 *    synchronises the device. Workspace is passed in explicitly and its size
 *    is given by the matching *_workspace_size() query.
 *  - Return value 0 (MC_OK) on success, otherwise an mc_status code; the
 *    message for the calling thread is in mc_last_error(). A caller that gets
 *    a non-zero status uses its fallback, as LoRALayer::forward does on any
 *    Err from the fused op (lora.rs:302-310).
 *  - Argument validation runs on the host before anything is enqueued, so
 *    every error path is testable without a GPU.
 */
#ifndef MC_HIP_H
#define MC_HIP_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mc_status {
    MC_OK = 0,
    MC_ERR_NULL = 1,        /* a required pointer is NULL */
    MC_ERR_SHAPE = 2,       /* sizes inconsistent, zero where not allowed, or unsupported */
    MC_ERR_DTYPE = 3,       /* dtype code not supported by this entry point */
    MC_ERR_LAYOUT = 4,      /* misaligned pointer / row stride */
    MC_ERR_VALUE = 5,       /* scalar argument out of range (eps, p, scale) */
    MC_ERR_WORKSPACE = 6,   /* workspace missing or smaller than the query */
    MC_ERR_HIP = 7,         /* HIP runtime error (launch failure, bad stream) */
} mc_status;

typedef enum mc_dtype {
    MC_F32 = 0,
    MC_BF16 = 1,
} mc_dtype;

/* LoRA linear, shapes in the reference's conventions:
 *   x [T, K] (T = product of the leading dims of the input, as
 *   FusedLoRAOp::extract_dimensions folds batch x seq, custom_ops.rs:254-270),
 *   W [N, K] (candle Linear), bias [N], A [K, r] (lora.rs:233-239),
 *   B [r, N] (lora.rs:241-247), y [T, N].
 * x, W, bias, y, dY, dX use act_dtype; A, B, dA, dB, the saved hidden are fp32.
 * dropout mask: uint8 [T, r], 1 = keep; required iff dropout_p > 0; kept
 * values are scaled by 1/(1 - p) (candle_nn::ops::dropout semantics). */
typedef struct mc_lora_desc {
    int64_t tokens;        /* T >= 1 */
    int64_t in_features;   /* K >= 1 */
    int64_t out_features;  /* N >= 1 */
    int32_t rank;          /* 1 <= r <= 8192 */
    float scale;           /* alpha / rank (LoRAConfig::scaling, lora.rs:84-87) */
    float dropout_p;       /* 0 <= p < 1 (LoRAConfig::validate, lora.rs:97-120) */
    int32_t act_dtype;     /* mc_dtype */
} mc_lora_desc;

/* Workspace bytes mc_lora_fwd / mc_lora_bwd need for this descriptor. */
size_t mc_lora_fwd_workspace_size(const mc_lora_desc* d);
size_t mc_lora_bwd_workspace_size(const mc_lora_desc* d);

/* y = x W^T + bias + scale * ((x A) (.) mask / (1-p)) B.
 * W == NULL: delta only (exactly what FusedLoRAOp computes); bias may be NULL.
 * h_save [r, T] fp32 (may be NULL) receives Hd^T = ((x A) (.) mask/(1-p))^T,
 * the saved activation mc_lora_bwd needs for dB. bf16 K or N not a multiple
 * of 8 runs on zero-padded copies in the workspace (mc_lora_bwd likewise). */
mc_status mc_lora_fwd(const mc_lora_desc* d, const void* x, const void* W, const void* bias,
                      const float* A, const float* B, const uint8_t* mask,
                      void* y, float* h_save, void* workspace, size_t workspace_bytes,
                      hipStream_t stream);

/* Backward with W frozen:
 *   G = scale dY B^T, Gd = G (.) mask/(1-p)
 *   dX = dY W + Gd A^T   (dY W omitted when W == NULL)
 *   dA = x^T Gd          [K, r]
 *   dB = scale Hd^T dY   [r, N]  (Hd^T from h_save of mc_lora_fwd)
 * dX, dA, dB may individually be NULL (not computed); h_save is required iff
 * dB is requested. Reductions over T are split in a fixed partition and
 * summed in a fixed order: results are bitwise reproducible run to run. */
mc_status mc_lora_bwd(const mc_lora_desc* d, const void* x, const void* W, const float* A,
                      const float* B, const uint8_t* mask, const float* h_save,
                      const void* dY, void* dX, float* dA, float* dB,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Grouped projections of one input: the LoRA linears that read the same x,
 * as the q, k and v projections of the attention's normalised input and the
 * gate and up projections of the MLP's (src/models/transformer.rs:241-243,
 * 389-395), each with its own frozen W, bias, A, B and mask, sharing T, K,
 * rank, scale, dropout_p and act_dtype (the layer's LoRAConfig). No
 * reference kernel: an additive entry point for a caller that holds a
 * layer's projections. bf16 only (MC_ERR_DTYPE otherwise); 1 <= count <=
 * MC_LORA_MAX_GROUP; desc->out_features is not used. */
#define MC_LORA_MAX_GROUP 4
typedef struct mc_lora_proj {
    int64_t out_features;   /* N_g >= 1, multiple of 8 */
    const void* W;          /* [N_g, K] frozen base weight, or NULL (delta only) */
    const void* bias;       /* [N_g] or NULL (requires W) */
    const float* A;         /* [K, r] */
    const float* B;         /* [r, N_g] */
    const uint8_t* mask;    /* [T, r] keep-mask, required iff dropout_p > 0 */
    const void* Wt;         /* [K, N_g] = W^T of the frozen W (mc_transpose_bf16, built once), or
                             * NULL: the backward then transposes W into its workspace on every call.
                             * Requires W; read by the backward's dX product only. */
} mc_lora_proj;

size_t mc_lora_group_fwd_workspace_size(const mc_lora_desc* d, const mc_lora_proj* projs, int32_t count);
size_t mc_lora_group_bwd_workspace_size(const mc_lora_desc* d, const mc_lora_proj* projs, int32_t count);

/* y[g] = x W_g^T + bias_g + scale ((x A_g) (.) mask_g / (1-p)) B_g for every
 * g < count; h_save (or any entry) may be NULL, else h_save[g] [r, T]
 * receives Hd_g^T as in mc_lora_fwd. The results equal count calls of
 * mc_lora_fwd bit for bit; x is read once per row-projection pass (up to 64
 * ranks of whole projections) and all the projections' base products run in
 * one GEMM launch. */
mc_status mc_lora_group_fwd(const mc_lora_desc* d, const void* x, const mc_lora_proj* projs, int32_t count,
                            void* const* y, float* const* h_save, void* workspace, size_t workspace_bytes,
                            hipStream_t stream);

/* Backward of mc_lora_group_fwd with every W frozen:
 *   dX    = sum_g (dY_g W_g + Gd_g A_g^T)   [T, K], the gradient of the shared
 *           input (candle autograd sums the projections' contributions), as
 *           one GEMM over the concatenated reduction; may be NULL
 *   dA[g] = x^T Gd_g, dB[g] = scale Hd_g^T dY_g, each equal bit for bit to
 *           mc_lora_bwd's; dA / dB or any entry may be NULL (not computed)
 * h_save[g] is required where dB[g] is requested, x where any dA is. */
mc_status mc_lora_group_bwd(const mc_lora_desc* d, const void* x, const mc_lora_proj* projs, int32_t count,
                            const float* const* h_save, const void* const* dY, void* dX, float* const* dA,
                            float* const* dB, void* workspace, size_t workspace_bytes, hipStream_t stream);

/* out[j][i] = in[i][j] for a bf16 matrix in [rows, cols] (out [cols, rows]),
 * both 16-byte aligned with rows and cols multiples of 8. No reference
 * counterpart: it builds the mc_lora_proj.Wt of a frozen base weight once
 * (at load), so that the backward does not transpose W on every call. */
mc_status mc_transpose_bf16(int64_t rows, int64_t cols, const void* in, void* out, hipStream_t stream);

/* RMSNorm over the last dim of x [rows, dim]:
 *   y = x / sqrt(mean(x^2) + eps) * w     (w == NULL: no weight, as FusedRMSNormOp)
 * x, w, y in dtype; rstd [rows] fp32 (may be NULL) receives 1/sqrt(mean + eps).
 * rows <= 67108860 (one wave per row; a launch holds at most 2^32 - 1
 * work-items), as for mc_layernorm_fwd; larger: MC_ERR_SHAPE. */
mc_status mc_rmsnorm_fwd(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x,
                         const void* w, void* y, float* rstd, hipStream_t stream);

size_t mc_rmsnorm_bwd_workspace_size(int64_t rows, int64_t dim);

/* dx = r g - x r^3 mean(g x), g = dy (.) w ; dw = sum_rows dy x r (fp32 [dim]).
 * rstd may be NULL (recomputed from x); dw may be NULL (not computed; then no
 * workspace is needed). dw is reduced in a fixed order (reproducible). */
mc_status mc_rmsnorm_bwd(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x,
                         const void* w, const float* rstd, const void* dy, void* dx, float* dw,
                         void* workspace, size_t workspace_bytes, hipStream_t stream);

/* mc_rmsnorm_bwd without a workspace: allocates nothing. It has no
 * counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops). The
 * dw partials go to a static device scratch of 16 MiB that the library
 * holds on each device it runs on until the process ends; shapes whose
 * partials need more (mc_rmsnorm_bwd_workspace_size(rows, dim) > 16 MiB,
 * e.g. dim > 8192 with rows >= 4096) are rejected with MC_ERR_SHAPE. Same
 * kernels and row partition as mc_rmsnorm_bwd, so the results are equal bit
 * for bit. Calls that overlap on one device share the scratch and race:
 * serialise them (one stream, or events). */
mc_status mc_rmsnorm_bwd_noalloc(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x,
                                 const void* w, const float* rstd, const void* dy, void* dx, float* dw,
                                 hipStream_t stream);

/* Softmax over the last dim of s [rows, dim]. causal_rows = 0: no mask;
 * causal_rows = S > 0 (S <= dim): row i is query q = i mod S and column j is
 * masked (-inf before the softmax, so p = 0 exactly) iff j > q + (dim - S).
 * 16-byte vectors of s lying wholly in the masked region are not read. */
mc_status mc_softmax_fwd(int64_t rows, int64_t dim, int64_t causal_rows, int32_t dtype,
                         const void* s, void* p, hipStream_t stream);

/* ds = p (.) (dp - sum_j dp_j p_j), same mask convention (masked ds = 0;
 * 16-byte vectors of p / dp lying wholly in the masked region are not read). */
mc_status mc_softmax_bwd(int64_t rows, int64_t dim, int64_t causal_rows, int32_t dtype,
                         const void* p, const void* dp, void* ds, hipStream_t stream);

/* Attention core: the part of Attention::forward between the rotary
 * embedding and o_proj (src/models/transformer.rs:258-283), with the K/V head
 * repetition of repeat_kv (transformer.rs:295-319) done by indexing:
 *   q [B, H, S, D], k, v [B, Hkv, S, D]   (after RoPE and transpose(1, 2))
 *   query head h reads K/V head h / (H / Hkv)
 *   scores = scale q.k^T  (+ mask[i, j])  (-inf where key j > query i if causal)
 *   o [B, S, H * D] = softmax_stable(scores) . v   (the reference's
 *                     transpose(1, 2) + reshape, transformer.rs:280-282)
 * scale is 1/sqrt(D) in the reference (transformer.rs:266). mask is an
 * optional fp32 [S, S] additive mask broadcast over B and H (the reference's
 * attention_mask of shape [1, 1, S, S]); S * S * 4 must stay below 2^31. A
 * row whose scores are all -inf gives NaN, as softmax_stable does. lse
 * [B, H, S] fp32 (may be NULL) receives the natural log-sum-exp of each score
 * row, which mc_attention_bwd takes.
 * bf16 with D = 64 or 128 runs the MFMA (flash) kernel and needs the
 * workspace of mc_attention_fwd_workspace_size(); other D (<= 256) and fp32
 * run a one-wave-per-row kernel with no workspace. */
typedef struct mc_attn_desc {
    int64_t batch;     /* B >= 1 */
    int64_t seq;       /* S >= 1: queries and keys (self-attention, no KV cache) */
    int32_t heads;     /* H >= 1 */
    int32_t kv_heads;  /* Hkv >= 1, H % Hkv == 0 */
    int32_t head_dim;  /* 1 <= D <= 256; bf16: D % 8 == 0 */
    int32_t causal;    /* 0 or 1 */
    float scale;       /* finite */
    int32_t dtype;     /* mc_dtype of q, k, v, o, dq, dk, dv, do */
} mc_attn_desc;

size_t mc_attention_fwd_workspace_size(const mc_attn_desc* d);

mc_status mc_attention_fwd(const mc_attn_desc* d, const void* q, const void* k, const void* v,
                           const float* mask, void* o, float* lse, void* workspace,
                           size_t workspace_bytes, hipStream_t stream);

size_t mc_attention_bwd_workspace_size(const mc_attn_desc* d);

/* Backward of mc_attention_fwd (no reference kernel: candle autograd of
 * transformer.rs:264-283): from o and lse of the forward and the output
 * gradient dout [B, S, H * D],
 *   P = exp(scores - lse), dP = dout.v^T, dS = P (.) (dP - rowsum(dout (.) o))
 *   dq = scale dS.k   [B, H, S, D]
 *   dk = scale dS^T.q, dv = P^T.dout   [B, Hkv, S, D], each summed over the
 *        H / Hkv query heads that read the K/V head (backward of repeat_kv)
 * Every reduction runs in a fixed order: results are bitwise reproducible. */
mc_status mc_attention_bwd(const mc_attn_desc* d, const void* q, const void* k, const void* v,
                           const float* mask, const void* o, const float* lse, const void* dout,
                           void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

/* AdamW (src/training/optimizer.rs:33-48 config, 227-281 step) over fp32
 * parameter tensors, typically the LoRA A and B of every projection. */
typedef struct mc_adamw_config {
    float learning_rate;  /* > 0 */
    float beta1;          /* [0, 1) */
    float beta2;          /* [0, 1) */
    float epsilon;        /* > 0 */
    float weight_decay;   /* >= 0 */
} mc_adamw_config;

typedef struct mc_adamw_tensor {
    const float* param;   /* theta_{t-1} [numel] */
    const float* grad;    /* g_t [numel] */
    float* m;             /* first moment, updated in place */
    float* v;             /* second moment, updated in place */
    float* param_out;     /* theta_t [numel]; may equal param (in place) */
    int64_t numel;        /* >= 0 */
    int64_t step;         /* t in 1 .. 2^31-1: the optimizer's step count for this update */
} mc_adamw_tensor;

/* One AdamW::step per tensor, all in one or a few launches:
 *   m = b1 m + (1-b1) g ;  v = b2 v + (1-b2) g^2
 *   theta_t = theta - lr (m/(1-b1^t)) / (sqrt(v/(1-b2^t)) + eps) - (wd lr) theta
 * in the reference's fp32 op order (each intermediate rounded to fp32, no
 * fused multiply-add; b^t as Rust's f32::powi), so results equal a CPU
 * evaluation of optimizer.rs:246-281 bit for bit. The tensor table is read
 * on the host; pointers must be 16-byte aligned. Validation messages are
 * AdamWConfig::validate's (optimizer.rs:67-103). */
mc_status mc_adamw_step(const mc_adamw_config* cfg, const mc_adamw_tensor* tensors, int32_t count,
                        hipStream_t stream);

/* LayerNorm over the last dim of x [rows, dim] (LayerNormOp,
 * src/backend/custom_ops.rs:826-1079; its CPU path cpu_fwd and
 * TensorExt::layer_norm, src/backend/tensor.rs:100-109; the weight and bias
 * of MetalLayerNorm::forward, src/embeddings/metal_bert.rs:30-72):
 *   mean = sum(x)/D, var = sum((x - mean)^2)/D, y = (x - mean)/sqrt(var + eps) * w + b
 * w, b may be NULL (none, as LayerNormOp); mean, rstd [rows] fp32 may be NULL. */
mc_status mc_layernorm_fwd(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x,
                           const void* w, const void* b, void* y, float* mean, float* rstd,
                           hipStream_t stream);

size_t mc_layernorm_bwd_workspace_size(int64_t rows, int64_t dim);

/* Backward (no reference kernel: autograd of the composite): with
 * xh = (x - mean) rstd and g = dy w,
 *   dx = rstd (g - mean(g) - xh mean(g xh)), dw = sum_rows dy xh, db = sum_rows dy
 * mean and rstd may be NULL (recomputed, both or neither); dw, db (fp32 [dim])
 * may be NULL; they are reduced in a fixed order (reproducible). */
mc_status mc_layernorm_bwd(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x,
                           const void* w, const float* mean, const float* rstd, const void* dy,
                           void* dx, float* dw, float* db, void* workspace, size_t workspace_bytes,
                           hipStream_t stream);

/* log-softmax over the last dim (candle_nn::ops::log_softmax as
 * cross_entropy_loss uses it, src/training/loss.rs:108):
 *   y = (x - max) - log(sum(exp(x - max)));  backward dx = dy - exp(y) sum(dy).
 * rows <= 16777215 (one 256-thread workgroup per row), as for the
 * cross-entropy calls; larger: MC_ERR_SHAPE. */
mc_status mc_log_softmax_fwd(int64_t rows, int64_t dim, int32_t dtype, const void* x, void* y,
                             hipStream_t stream);
mc_status mc_log_softmax_bwd(int64_t rows, int64_t dim, int32_t dtype, const void* y,
                             const void* dy, void* dx, hipStream_t stream);

/* Cross-entropy loss (cross_entropy_loss, src/training/loss.rs:58-148, and
 * cross_entropy_loss_with_smoothing, loss.rs:208-245) over logits
 * [rows, vocab] (rows = batch * seq_len) and uint32 targets [rows]:
 *   loss = -mean over counted rows of log_softmax(logits)[target]
 *   counted rows: target != ignore_index (every row when ignore_index < 0)
 *   smoothing s > 0: (1 - s) * loss + s * (-mean of every log-probability,
 *   ignored rows included, as the reference's log_probs.mean_all())
 * loss: fp32 [1], device. stats (fp32 [rows + 1], may be NULL): per-row
 * log-sum-exp, then the count of counted rows; mc_cross_entropy_bwd needs it.
 * Where the reference returns an error the loss is NaN instead (the count is
 * only known on the device): every row ignored, or a counted target >= vocab. */
typedef struct mc_xent_desc {
    int64_t rows;          /* 1 .. 16777215 */
    int64_t vocab;         /* >= 1 */
    int64_t ignore_index;  /* < 0: none (the reference's Option<u32> None) */
    float smoothing;       /* [0, 1) */
    int32_t dtype;         /* mc_dtype of logits and dlogits */
} mc_xent_desc;

size_t mc_cross_entropy_workspace_size(const mc_xent_desc* d);

mc_status mc_cross_entropy_fwd(const mc_xent_desc* d, const void* logits, const uint32_t* targets,
                               float* loss, float* stats, void* workspace, size_t workspace_bytes,
                               hipStream_t stream);

/* dlogits = dloss ((1 - s) [counted] (p - onehot(target)) / count + s (p - 1/vocab) / rows),
 * p = softmax(logits); dloss: fp32 [1] device (the loss gradient, usually 1). */
mc_status mc_cross_entropy_bwd(const mc_xent_desc* d, const void* logits, const uint32_t* targets,
                               const float* stats, const float* dloss, void* dlogits, hipStream_t stream);

/* Host-side dropout keep-mask [rows, rank] from a seed (Philox4x32-10; element
 * i = t*rank + j uses counter block i/4, word i%4, key = seed; keep iff
 * (word >> 8) * 2^-24 >= p). Both the GPU path and the CPU reference are fed
 * the same bytes. Writes host memory; touches no device. */
mc_status mc_dropout_mask(uint64_t seed, float p, int64_t rows, int32_t rank, uint8_t* mask_host);

/* Kernel timing hook. No counterpart in the reference (its benches time whole
 * candle calls); it is for callers that need per-kernel times on their own
 * stream, such as the roofline report of bench.py.
 * While enabled, every kernel launch of the entry points above is bracketed
 * by a hipEvent pair recorded on the launch stream and tagged with its class
 * and its algorithmic work (FLOPs, HBM bytes). mc_profile_collect() waits for
 * the recorded events and adds them to per-class totals; mc_profile_read()
 * returns the totals of one class. Classes: 0 = MFMA GEMM (FLOPs count the
 * base x.W^T / dY.W product only), 1 = rank-r kernels, 2 = RMSNorm,
 * 3 = softmax, 4 = attention (FLOPs of the unmasked score and P.V products),
 * 5 = AdamW (bytes: 28 per element), 6 = LayerNorm / log-softmax /
 * cross-entropy.
 * Enabling allocates hipEvents (not for allocation-free use). */
mc_status mc_profile_enable(int32_t on);
mc_status mc_profile_collect(void);
mc_status mc_profile_read(int32_t kind, double* elapsed_ms, int64_t* launches, double* flops, double* bytes);
mc_status mc_profile_reset(void);

/* Message for the last non-zero status returned on this thread. */
const char* mc_last_error(void);

/* Library version string. */
const char* mc_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MC_HIP_H */
