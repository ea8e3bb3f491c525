// C ABI of libmc_hip.so: argument validation, error reporting, dispatch.
//
// Validation mirrors the checks of the reference's fused ops and LoRA config
// (FusedLoRAOp::new, custom_ops.rs:118-148; compute_output_shape, 153-174;
// FusedRMSNormOp / FusedSoftmaxOp metal_fwd, 534-560 / 727-752;
// LoRAConfig::validate, lora.rs:97-120) and returns a status code instead of
// a candle error, with the message kept per thread in mc_last_error(). It runs
// on the host before anything is enqueued, so every error path can be
// exercised without a GPU.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "kernels.hpp"
#include "mc_hip.h"
#include "profile.hpp"

namespace {

thread_local std::string g_last_error;

mc_status fail(mc_status code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

mc_status ok() {
    g_last_error.clear();
    return MC_OK;
}

mc_status hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return ok();
    return fail(MC_ERR_HIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

#define MC_CHECK(cond, code, ...)                     \
    do {                                              \
        if (!(cond)) return fail(code, __VA_ARGS__);  \
    } while (0)

mc_status check_dtype(int32_t dtype, const char* op) {
    MC_CHECK(dtype == MC_F32 || dtype == MC_BF16, MC_ERR_DTYPE,
             "%s: unsupported dtype code %d (supported: 0 = f32, 1 = bf16)", op, (int)dtype);
    return MC_OK;
}

mc_status check_lora_desc(const mc_lora_desc* d) {
    MC_CHECK(d != nullptr, MC_ERR_NULL, "LoRA: descriptor is NULL");
    MC_CHECK(d->act_dtype == MC_F32 || d->act_dtype == MC_BF16, MC_ERR_DTYPE,
             "LoRA: unsupported act_dtype code %d (supported: 0 = f32, 1 = bf16)", (int)d->act_dtype);
    MC_CHECK(d->tokens >= 1 && d->in_features >= 1 && d->out_features >= 1, MC_ERR_SHAPE,
             "LoRA: tokens, in_features and out_features must be >= 1, got %lld, %lld, %lld",
             (long long)d->tokens, (long long)d->in_features, (long long)d->out_features);
    // LoRAConfig::validate: "LoRA rank must be greater than 0" (lora.rs:99-104)
    MC_CHECK(d->rank >= 1, MC_ERR_SHAPE, "LoRA rank must be greater than 0");
    MC_CHECK(d->rank <= 8192, MC_ERR_SHAPE, "LoRA: rank %d exceeds the supported maximum 8192", (int)d->rank);
    MC_CHECK(std::isfinite(d->scale), MC_ERR_VALUE, "LoRA: scale must be finite");
    // LoRAConfig::validate: "LoRA dropout must be in [0, 1)" (lora.rs:113-118)
    MC_CHECK(d->dropout_p >= 0.0f && d->dropout_p < 1.0f, MC_ERR_VALUE, "LoRA dropout must be in [0, 1)");
    if (d->act_dtype == MC_BF16) {
        // (K or N not a multiple of 8: mc_lora_fwd / mc_lora_bwd run the
        // kernels on zero-padded copies; grouped calls require multiples of 8.)
        // The bf16 kernels address a workgroup's block of rows (256 GEMM rows
        // of up to max(K, N) features, 32 rank rows of T fp32 values) through
        // buffer resources with 32-bit byte offsets.
        // The bound applies to the features rounded up to 8, the widths the
        // kernels see on the zero-padded path.
        MC_CHECK((d->in_features + 7) / 8 * 8 < (1 << 22) && (d->out_features + 7) / 8 * 8 < (1 << 22),
                 MC_ERR_SHAPE, "LoRA bf16: in_features (%lld) and out_features (%lld) must be below 2^22 - 7",
                 (long long)d->in_features, (long long)d->out_features);
        MC_CHECK(d->tokens < (1 << 24), MC_ERR_SHAPE, "LoRA bf16: tokens (%lld) must be below 2^24",
                 (long long)d->tokens);
    }
    return MC_OK;
}

// One launch holds at most 2^32 - 1 work-items. The RMSNorm and LayerNorm
// forward kernels run one 64-lane wave per row, four rows per 256-thread
// workgroup; log_softmax and cross-entropy one 256-thread workgroup per row.
// (Softmax splits its launches by rows and has no such bound.)
constexpr int64_t kMaxWaveRows = ((((int64_t)1 << 32) - 1) / 256) * 4;  // 67108860
constexpr int64_t kMaxBlockRows = (((int64_t)1 << 32) - 1) / 256;       // 16777215

mc_status check_rows(int64_t rows, int64_t dim, const char* op, int64_t max_rows = INT64_MAX) {
    MC_CHECK(rows >= 1 && dim >= 1, MC_ERR_SHAPE, "%s: rows and dim must be >= 1, got %lld x %lld", op,
             (long long)rows, (long long)dim);
    MC_CHECK(rows <= max_rows, MC_ERR_SHAPE, "%s: rows must be <= %lld, got %lld", op, (long long)max_rows,
             (long long)rows);
    return MC_OK;
}

// Elements a causal softmax reads: row i (query q = i mod S) reads columns
// 0 .. q + dim - S; summed over whole S-row blocks plus the partial block.
double unmasked(int64_t rows, int64_t dim, int64_t S) {
    if (S <= 0) return (double)rows * dim;
    auto block = [&](int64_t n) {  // first n queries of a block
        return (double)n * (dim - S) + (double)n * (n + 1) / 2.0;
    };
    return (double)(rows / S) * block(S) + block(rows % S);
}

mc_status check_attn_desc(const mc_attn_desc* d, const char* op) {
    MC_CHECK(d != nullptr, MC_ERR_NULL, "%s: descriptor is NULL", op);
    mc_status s = check_dtype(d->dtype, op);
    if (s != MC_OK) return s;
    MC_CHECK(d->batch >= 1 && d->seq >= 1 && d->heads >= 1 && d->kv_heads >= 1, MC_ERR_SHAPE,
             "%s: batch, seq, heads and kv_heads must be >= 1, got %lld, %lld, %d, %d", op, (long long)d->batch,
             (long long)d->seq, (int)d->heads, (int)d->kv_heads);
    // repeat_kv repeats each K/V head num_heads / num_kv_heads times (transformer.rs:258-259, 300-318)
    MC_CHECK(d->heads % d->kv_heads == 0, MC_ERR_SHAPE, "%s: heads (%d) must be a multiple of kv_heads (%d)", op,
             (int)d->heads, (int)d->kv_heads);
    MC_CHECK(d->head_dim >= 1 && d->head_dim <= 256, MC_ERR_SHAPE, "%s: head_dim must be in [1, 256], got %d", op,
             (int)d->head_dim);
    MC_CHECK(d->dtype != MC_BF16 || d->head_dim % 8 == 0, MC_ERR_SHAPE,
             "%s: bf16 head_dim must be a multiple of 8, got %d", op, (int)d->head_dim);
    MC_CHECK(d->causal == 0 || d->causal == 1, MC_ERR_VALUE, "%s: causal must be 0 or 1", op);
    MC_CHECK(std::isfinite(d->scale), MC_ERR_VALUE, "%s: scale must be finite", op);
    // buffer offsets inside one batch slice of [S, H, D] stay below 2^31 bytes
    MC_CHECK((double)d->seq * d->heads * d->head_dim * 4.0 < 2147483647.0, MC_ERR_SHAPE,
             "%s: S * H * D (%lld x %d x %d) too large for one batch slice", op, (long long)d->seq, (int)d->heads,
             (int)d->head_dim);
    const double elems = (double)d->batch * d->heads * d->seq * d->head_dim;
    MC_CHECK(elems < 9.0e15 && (double)d->batch * d->heads * d->seq < 2.0e9, MC_ERR_SHAPE,
             "%s: problem too large (B * H * S must stay below 2^31)", op);
    return MC_OK;
}

// Score-matrix entries an attention pass computes (causal: the lower triangle).
double attn_pairs(const mc_attn_desc* d) {
    const double S = (double)d->seq;
    return (double)d->batch * d->heads * (d->causal ? S * (S + 1) / 2 : S * S);
}

}  // namespace

extern "C" {

const char* mc_version(void) { return "mc_hip 0.1.0 (gfx950)"; }

mc_status mc_profile_enable(int32_t on) {
    mc::prof::set_enabled(on != 0);
    return ok();
}

mc_status mc_profile_collect(void) { return hip_status(mc::prof::collect(), "profile collect"); }

mc_status mc_profile_read(int32_t kind, double* elapsed_ms, int64_t* launches, double* flops, double* bytes) {
    MC_CHECK(kind >= 0 && kind < mc::prof::kNumKinds, MC_ERR_VALUE, "profile: unknown kernel class %d", (int)kind);
    long long n = 0;
    mc::prof::read(kind, elapsed_ms, &n, flops, bytes);
    if (launches) *launches = n;
    return ok();
}

mc_status mc_profile_reset(void) {
    mc::prof::reset();
    return ok();
}

const char* mc_last_error(void) { return g_last_error.c_str(); }

size_t mc_lora_fwd_workspace_size(const mc_lora_desc* d) {
    if (check_lora_desc(d) != MC_OK) return 0;
    return mc::lora_fwd_ws(*d).total;
}

size_t mc_lora_bwd_workspace_size(const mc_lora_desc* d) {
    if (check_lora_desc(d) != MC_OK) return 0;
    return mc::lora_bwd_ws(*d).total;
}

mc_status mc_lora_fwd(const mc_lora_desc* d, const void* x, const void* W, const void* bias,
                      const float* A, const float* B, const uint8_t* mask, void* y, float* h_save,
                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
    mc_status s = check_lora_desc(d);
    if (s != MC_OK) return s;
    MC_CHECK(x && A && B && y, MC_ERR_NULL, "LoRA forward: x, A, B and y must not be NULL");
    MC_CHECK(!bias || W, MC_ERR_NULL, "LoRA forward: bias given without W");
    MC_CHECK(d->dropout_p == 0.0f || mask, MC_ERR_NULL, "LoRA forward: dropout_p > 0 requires a mask");
    MC_CHECK(aligned16(x) && aligned16(y) && (!W || aligned16(W)) && (!h_save || aligned16(h_save)),
             MC_ERR_LAYOUT, "LoRA forward: x, W, y and h_save must be 16-byte aligned");
    const size_t need = mc::lora_fwd_ws(*d).total;
    MC_CHECK(workspace_bytes >= need && (need == 0 || workspace), MC_ERR_WORKSPACE,
             "LoRA forward: workspace of %zu bytes required, %zu given", need, workspace_bytes);
    MC_CHECK(aligned16(workspace), MC_ERR_LAYOUT, "LoRA forward: workspace must be 16-byte aligned");
    return hip_status(mc::launch_lora_fwd(*d, x, W, bias, A, B, mask, y, h_save, workspace, stream),
                      "LoRA forward");
}

mc_status mc_lora_bwd(const mc_lora_desc* d, const void* x, const void* W, const float* A, const float* B,
                      const uint8_t* mask, const float* h_save, const void* dY, void* dX, float* dA,
                      float* dB, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    mc_status s = check_lora_desc(d);
    if (s != MC_OK) return s;
    MC_CHECK(dY && A && B, MC_ERR_NULL, "LoRA backward: dY, A and B must not be NULL");
    MC_CHECK(!dA || x, MC_ERR_NULL, "LoRA backward: dA requires x");
    MC_CHECK(!dB || h_save, MC_ERR_NULL, "LoRA backward: dB requires h_save from the forward");
    MC_CHECK(d->dropout_p == 0.0f || mask, MC_ERR_NULL, "LoRA backward: dropout_p > 0 requires a mask");
    MC_CHECK(aligned16(dY) && (!x || aligned16(x)) && (!W || aligned16(W)) && (!dX || aligned16(dX)) &&
                 (!h_save || aligned16(h_save)),
             MC_ERR_LAYOUT, "LoRA backward: x, W, dY, dX and h_save must be 16-byte aligned");
    const size_t need = mc::lora_bwd_ws(*d).total;
    MC_CHECK(workspace_bytes >= need && (need == 0 || workspace), MC_ERR_WORKSPACE,
             "LoRA backward: workspace of %zu bytes required, %zu given", need, workspace_bytes);
    MC_CHECK(aligned16(workspace), MC_ERR_LAYOUT, "LoRA backward: workspace must be 16-byte aligned");
    if (!dX && !dA && !dB) return ok();
    return hip_status(mc::launch_lora_bwd(*d, x, W, A, B, mask, h_save, dY, dX, dA, dB, workspace, stream),
                      "LoRA backward");
}

}  // extern "C"

namespace {

// A grouped call's descriptor and projection table: the shared T, K, r,
// scale, p and dtype as for one projection, then every projection's N; the
// group runs the bf16 kernels only.
mc_status check_lora_group(const mc_lora_desc* d, const mc_lora_proj* projs, int32_t count, const char* op,
                           mc_lora_desc* per_proj, int64_t* Ns) {
    MC_CHECK(d != nullptr, MC_ERR_NULL, "%s: descriptor is NULL", op);
    MC_CHECK(projs != nullptr, MC_ERR_NULL, "%s: projection table is NULL", op);
    MC_CHECK(count >= 1 && count <= MC_LORA_MAX_GROUP, MC_ERR_SHAPE, "%s: count must be in [1, %d], got %d", op,
             MC_LORA_MAX_GROUP, (int)count);
    MC_CHECK(d->act_dtype == MC_BF16, MC_ERR_DTYPE,
             "%s: grouped projections run in bf16 only (act_dtype %d); use mc_lora_fwd / mc_lora_bwd per projection",
             op, (int)d->act_dtype);
    for (int32_t g = 0; g < count; ++g) {
        *per_proj = *d;
        per_proj->out_features = projs[g].out_features;
        mc_status s = check_lora_desc(per_proj);
        if (s != MC_OK) return s;
        MC_CHECK(d->in_features % 8 == 0 && projs[g].out_features % 8 == 0, MC_ERR_SHAPE,
                 "%s: projection %d: in_features (%lld) and out_features (%lld) must be multiples of 8 "
                 "(mc_lora_fwd / mc_lora_bwd take any size)",
                 op, (int)g, (long long)d->in_features, (long long)projs[g].out_features);
        MC_CHECK(projs[g].A && projs[g].B, MC_ERR_NULL, "%s: projection %d: A and B must not be NULL", op, (int)g);
        MC_CHECK(!projs[g].bias || projs[g].W, MC_ERR_NULL, "%s: projection %d: bias given without W", op, (int)g);
        MC_CHECK(d->dropout_p == 0.0f || projs[g].mask, MC_ERR_NULL,
                 "%s: projection %d: dropout_p > 0 requires a mask", op, (int)g);
        MC_CHECK(!projs[g].W || aligned16(projs[g].W), MC_ERR_LAYOUT, "%s: projection %d: W must be 16-byte aligned",
                 op, (int)g);
        MC_CHECK(!projs[g].Wt || projs[g].W, MC_ERR_NULL, "%s: projection %d: Wt given without W", op, (int)g);
        MC_CHECK(!projs[g].Wt || aligned16(projs[g].Wt), MC_ERR_LAYOUT,
                 "%s: projection %d: Wt must be 16-byte aligned", op, (int)g);
        Ns[g] = projs[g].out_features;
    }
    *per_proj = *d;
    per_proj->out_features = projs[0].out_features;
    return MC_OK;
}

void to_lora_proj(const mc_lora_proj* projs, int32_t count, mc::LoraProj* out) {
    for (int32_t g = 0; g < count; ++g)
        out[g] = mc::LoraProj{projs[g].out_features, projs[g].W, projs[g].bias, projs[g].A, projs[g].B, projs[g].mask,
                              projs[g].Wt};
}

// Projections whose W^T the backward builds in its workspace.
void need_wt_of(const mc_lora_proj* projs, int32_t count, bool* need) {
    for (int32_t g = 0; g < count; ++g) need[g] = projs[g].W && !projs[g].Wt;
}

}  // namespace

extern "C" {

size_t mc_lora_group_fwd_workspace_size(const mc_lora_desc* d, const mc_lora_proj* projs, int32_t count) {
    mc_lora_desc dd;
    int64_t Ns[MC_LORA_MAX_GROUP];
    if (check_lora_group(d, projs, count, "LoRA group forward", &dd, Ns) != MC_OK) return 0;
    return mc::lora_group_fwd_ws(dd, Ns, count).total;
}

size_t mc_lora_group_bwd_workspace_size(const mc_lora_desc* d, const mc_lora_proj* projs, int32_t count) {
    mc_lora_desc dd;
    int64_t Ns[MC_LORA_MAX_GROUP];
    if (check_lora_group(d, projs, count, "LoRA group backward", &dd, Ns) != MC_OK) return 0;
    bool need_wt[MC_LORA_MAX_GROUP];
    need_wt_of(projs, count, need_wt);
    return mc::lora_group_bwd_ws(dd, Ns, count, need_wt).total;
}

mc_status mc_lora_group_fwd(const mc_lora_desc* d, const void* x, const mc_lora_proj* projs, int32_t count,
                            void* const* y, float* const* h_save, void* workspace, size_t workspace_bytes,
                            hipStream_t stream) {
    mc_lora_desc dd;
    int64_t Ns[MC_LORA_MAX_GROUP];
    mc_status s = check_lora_group(d, projs, count, "LoRA group forward", &dd, Ns);
    if (s != MC_OK) return s;
    MC_CHECK(x && y, MC_ERR_NULL, "LoRA group forward: x and y must not be NULL");
    MC_CHECK(aligned16(x), MC_ERR_LAYOUT, "LoRA group forward: x must be 16-byte aligned");
    for (int32_t g = 0; g < count; ++g) {
        MC_CHECK(y[g], MC_ERR_NULL, "LoRA group forward: y[%d] must not be NULL", (int)g);
        MC_CHECK(aligned16(y[g]) && (!h_save || !h_save[g] || aligned16(h_save[g])), MC_ERR_LAYOUT,
                 "LoRA group forward: y[%d] and h_save[%d] must be 16-byte aligned", (int)g, (int)g);
    }
    const size_t need = mc::lora_group_fwd_ws(dd, Ns, count).total;
    MC_CHECK(workspace_bytes >= need && workspace, MC_ERR_WORKSPACE,
             "LoRA group forward: workspace of %zu bytes required, %zu given", need, workspace_bytes);
    MC_CHECK(aligned16(workspace), MC_ERR_LAYOUT, "LoRA group forward: workspace must be 16-byte aligned");
    mc::LoraProj lp[MC_LORA_MAX_GROUP];
    to_lora_proj(projs, count, lp);
    return hip_status(mc::launch_lora_group_fwd(dd, x, lp, count, y, h_save, workspace, stream), "LoRA group forward");
}

mc_status mc_lora_group_bwd(const mc_lora_desc* d, const void* x, const mc_lora_proj* projs, int32_t count,
                            const float* const* h_save, const void* const* dY, void* dX, float* const* dA,
                            float* const* dB, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    mc_lora_desc dd;
    int64_t Ns[MC_LORA_MAX_GROUP];
    mc_status s = check_lora_group(d, projs, count, "LoRA group backward", &dd, Ns);
    if (s != MC_OK) return s;
    MC_CHECK(dY, MC_ERR_NULL, "LoRA group backward: dY must not be NULL");
    bool any = dX != nullptr;
    for (int32_t g = 0; g < count; ++g) {
        MC_CHECK(dY[g], MC_ERR_NULL, "LoRA group backward: dY[%d] must not be NULL", (int)g);
        MC_CHECK(aligned16(dY[g]), MC_ERR_LAYOUT, "LoRA group backward: dY[%d] must be 16-byte aligned", (int)g);
        const bool wa = dA && dA[g], wb = dB && dB[g];
        MC_CHECK(!wa || x, MC_ERR_NULL, "LoRA group backward: dA requires x");
        MC_CHECK(!wb || (h_save && h_save[g]), MC_ERR_NULL,
                 "LoRA group backward: dB[%d] requires h_save[%d] from the forward", (int)g, (int)g);
        MC_CHECK(!wb || aligned16(h_save[g]), MC_ERR_LAYOUT, "LoRA group backward: h_save[%d] must be 16-byte aligned",
                 (int)g);
        any = any || wa || wb;
    }
    MC_CHECK((!x || aligned16(x)) && (!dX || aligned16(dX)), MC_ERR_LAYOUT,
             "LoRA group backward: x and dX must be 16-byte aligned");
    bool need_wt[MC_LORA_MAX_GROUP];
    need_wt_of(projs, count, need_wt);
    const size_t need = mc::lora_group_bwd_ws(dd, Ns, count, need_wt).total;
    MC_CHECK(workspace_bytes >= need && workspace, MC_ERR_WORKSPACE,
             "LoRA group backward: workspace of %zu bytes required, %zu given", need, workspace_bytes);
    MC_CHECK(aligned16(workspace), MC_ERR_LAYOUT, "LoRA group backward: workspace must be 16-byte aligned");
    if (!any) return ok();
    mc::LoraProj lp[MC_LORA_MAX_GROUP];
    to_lora_proj(projs, count, lp);
    return hip_status(mc::launch_lora_group_bwd(dd, x, lp, count, h_save, dY, dX, dA, dB, workspace, stream),
                      "LoRA group backward");
}

mc_status mc_transpose_bf16(int64_t rows, int64_t cols, const void* in, void* out, hipStream_t stream) {
    MC_CHECK(rows >= 1 && cols >= 1 && rows <= ((int64_t)1 << 40) / cols, MC_ERR_SHAPE,
             "transpose: rows and cols must be >= 1 with rows * cols <= 2^40 (got %lld x %lld)", (long long)rows,
             (long long)cols);
    MC_CHECK(rows % 8 == 0 && cols % 8 == 0, MC_ERR_SHAPE, "transpose: rows and cols must be multiples of 8 (got %lld x %lld)",
             (long long)rows, (long long)cols);
    MC_CHECK(in && out, MC_ERR_NULL, "transpose: in and out must not be NULL");
    MC_CHECK(aligned16(in) && aligned16(out), MC_ERR_LAYOUT, "transpose: in and out must be 16-byte aligned");
    MC_CHECK((rows + 63) / 64 * ((cols + 63) / 64) <= 0x7fffffff, MC_ERR_SHAPE, "transpose: too many 64 x 64 tiles");
    return hip_status(mc::launch_transpose_bf16(in, rows, cols, out, stream), "transpose");
}

mc_status mc_rmsnorm_fwd(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x, const void* w,
                         void* y, float* rstd, hipStream_t stream) {
    mc_status s = check_rows(rows, dim, "RMSNorm", kMaxWaveRows);
    if (s != MC_OK) return s;
    if ((s = check_dtype(dtype, "RMSNorm")) != MC_OK) return s;
    MC_CHECK(eps >= 0.0f && std::isfinite(eps), MC_ERR_VALUE, "RMSNorm: eps must be finite and >= 0");
    MC_CHECK(x && y, MC_ERR_NULL, "RMSNorm: x and y must not be NULL");
    MC_CHECK(aligned16(x) && aligned16(y) && (!w || aligned16(w)), MC_ERR_LAYOUT,
             "RMSNorm: x, w and y must be 16-byte aligned");
    const double es = dtype == MC_F32 ? 4.0 : 2.0;
    mc::prof::Scope sc(mc::prof::kRmsNorm, stream, 0.0,
                       es * (2.0 * rows * dim + (w ? dim : 0)) + (rstd ? 4.0 * rows : 0.0));
    return hip_status(mc::launch_rmsnorm_fwd(rows, dim, eps, dtype, x, w, y, rstd, stream), "RMSNorm forward");
}

size_t mc_rmsnorm_bwd_workspace_size(int64_t rows, int64_t dim) {
    if (rows < 1 || dim < 1) return 0;
    return (size_t)mc::rmsnorm_bwd_blocks(rows, dim) * (size_t)dim * sizeof(float);
}

}  // extern "C"

namespace {

mc_status check_rmsnorm_bwd(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x, const void* w,
                            const void* dy, void* dx) {
    mc_status s = check_rows(rows, dim, "RMSNorm backward");
    if (s != MC_OK) return s;
    if ((s = check_dtype(dtype, "RMSNorm backward")) != MC_OK) return s;
    MC_CHECK(eps >= 0.0f && std::isfinite(eps), MC_ERR_VALUE, "RMSNorm: eps must be finite and >= 0");
    MC_CHECK(x && dy && dx, MC_ERR_NULL, "RMSNorm backward: x, dy and dx must not be NULL");
    MC_CHECK(aligned16(x) && aligned16(dy) && aligned16(dx) && (!w || aligned16(w)), MC_ERR_LAYOUT,
             "RMSNorm backward: x, w, dy and dx must be 16-byte aligned");
    return MC_OK;
}

}  // namespace

extern "C" {

mc_status mc_rmsnorm_bwd(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x, const void* w,
                         const float* rstd, const void* dy, void* dx, float* dw, void* workspace,
                         size_t workspace_bytes, hipStream_t stream) {
    mc_status s = check_rmsnorm_bwd(rows, dim, eps, dtype, x, w, dy, dx);
    if (s != MC_OK) return s;
    if (dw) {
        const size_t need = mc_rmsnorm_bwd_workspace_size(rows, dim);
        MC_CHECK(workspace && workspace_bytes >= need, MC_ERR_WORKSPACE,
                 "RMSNorm backward: workspace of %zu bytes required for dw, %zu given", need, workspace_bytes);
    }
    const double es = dtype == MC_F32 ? 4.0 : 2.0;
    mc::prof::Scope sc(mc::prof::kRmsNorm, stream, 0.0,
                       es * (3.0 * rows * dim + (w ? dim : 0)) + (rstd ? 4.0 * rows : 0.0) + (dw ? 4.0 * dim : 0.0));
    return hip_status(mc::launch_rmsnorm_bwd(rows, dim, eps, dtype, x, w, rstd, dy, dx, dw,
                                             static_cast<float*>(workspace), stream),
                      "RMSNorm backward");
}

mc_status mc_rmsnorm_bwd_noalloc(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x,
                                 const void* w, const float* rstd, const void* dy, void* dx, float* dw,
                                 hipStream_t stream) {
    mc_status s = check_rmsnorm_bwd(rows, dim, eps, dtype, x, w, dy, dx);
    if (s != MC_OK) return s;
    float* partial = nullptr;
    if (dw) {
        const size_t need = mc_rmsnorm_bwd_workspace_size(rows, dim);
        MC_CHECK(need <= mc::kRmsNormScratchBytes, MC_ERR_SHAPE,
                 "RMSNorm backward (no-alloc): the dw partials of %lld x %lld need %zu bytes, above the "
                 "%zu-byte static scratch; use mc_rmsnorm_bwd with a workspace",
                 (long long)rows, (long long)dim, need, mc::kRmsNormScratchBytes);
        hipError_t e = mc::rmsnorm_scratch(&partial);
        if (e != hipSuccess) return hip_status(e, "RMSNorm backward (no-alloc): scratch address");
    }
    // No profiling scope here: the timing hook creates events when enabled.
    return hip_status(mc::launch_rmsnorm_bwd(rows, dim, eps, dtype, x, w, rstd, dy, dx, dw, partial, stream),
                      "RMSNorm backward (no-alloc)");
}

mc_status mc_softmax_fwd(int64_t rows, int64_t dim, int64_t causal_rows, int32_t dtype, const void* sc,
                         void* p, hipStream_t stream) {
    mc_status s = check_rows(rows, dim, "Softmax");
    if (s != MC_OK) return s;
    if ((s = check_dtype(dtype, "Softmax")) != MC_OK) return s;
    MC_CHECK(causal_rows >= 0 && causal_rows <= dim, MC_ERR_SHAPE,
             "Softmax: causal_rows must be in [0, dim], got %lld for dim %lld", (long long)causal_rows,
             (long long)dim);
    MC_CHECK(sc && p, MC_ERR_NULL, "Softmax: input and output must not be NULL");
    MC_CHECK(aligned16(sc) && aligned16(p), MC_ERR_LAYOUT, "Softmax: input and output must be 16-byte aligned");
    const double es = dtype == MC_F32 ? 4.0 : 2.0;
    mc::prof::Scope scope(mc::prof::kSoftmax, stream, 0.0, es * (unmasked(rows, dim, causal_rows) + (double)rows * dim));
    return hip_status(mc::launch_softmax_fwd(rows, dim, causal_rows, dtype, sc, p, stream), "Softmax forward");
}

mc_status mc_softmax_bwd(int64_t rows, int64_t dim, int64_t causal_rows, int32_t dtype, const void* p,
                         const void* dp, void* ds, hipStream_t stream) {
    mc_status s = check_rows(rows, dim, "Softmax backward");
    if (s != MC_OK) return s;
    if ((s = check_dtype(dtype, "Softmax backward")) != MC_OK) return s;
    MC_CHECK(causal_rows >= 0 && causal_rows <= dim, MC_ERR_SHAPE,
             "Softmax: causal_rows must be in [0, dim], got %lld for dim %lld", (long long)causal_rows,
             (long long)dim);
    MC_CHECK(p && dp && ds, MC_ERR_NULL, "Softmax backward: p, dp and ds must not be NULL");
    MC_CHECK(aligned16(p) && aligned16(dp) && aligned16(ds), MC_ERR_LAYOUT,
             "Softmax backward: p, dp and ds must be 16-byte aligned");
    const double es = dtype == MC_F32 ? 4.0 : 2.0;
    mc::prof::Scope scope(mc::prof::kSoftmax, stream, 0.0,
                          es * (2.0 * unmasked(rows, dim, causal_rows) + (double)rows * dim));
    return hip_status(mc::launch_softmax_bwd(rows, dim, causal_rows, dtype, p, dp, ds, stream),
                      "Softmax backward");
}

size_t mc_attention_fwd_workspace_size(const mc_attn_desc* d) {
    if (check_attn_desc(d, "Attention") != MC_OK) return 0;
    return mc::attention_fwd_ws(*d).total;
}

mc_status mc_attention_fwd(const mc_attn_desc* d, const void* q, const void* k, const void* v, const float* mask,
                           void* o, float* lse, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    mc_status s = check_attn_desc(d, "Attention");
    if (s != MC_OK) return s;
    MC_CHECK(q && k && v && o, MC_ERR_NULL, "Attention: q, k, v and o must not be NULL");
    MC_CHECK(!mask || (double)d->seq * d->seq * 4.0 < 2147483647.0, MC_ERR_SHAPE,
             "Attention: an explicit mask needs S * S * 4 < 2^31 bytes (S = %lld)", (long long)d->seq);
    MC_CHECK(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o), MC_ERR_LAYOUT,
             "Attention: q, k, v and o must be 16-byte aligned");
    const size_t need = mc::attention_fwd_ws(*d).total;
    MC_CHECK(workspace_bytes >= need && (need == 0 || workspace), MC_ERR_WORKSPACE,
             "Attention: workspace of %zu bytes required, %zu given", need, workspace_bytes);
    MC_CHECK(aligned16(workspace), MC_ERR_LAYOUT, "Attention: workspace must be 16-byte aligned");
    const double es = d->dtype == MC_F32 ? 4.0 : 2.0;
    const double qo = (double)d->batch * d->heads * d->seq * d->head_dim;
    const double kv = (double)d->batch * d->kv_heads * d->seq * d->head_dim;
    mc::prof::Scope sc(mc::prof::kAttention, stream, 4.0 * attn_pairs(d) * d->head_dim,
                       es * (2.0 * qo + 2.0 * kv) + (lse ? 4.0 * d->batch * d->heads * d->seq : 0.0));
    return hip_status(mc::launch_attention_fwd(*d, q, k, v, mask, o, lse, workspace, stream), "Attention forward");
}

size_t mc_attention_bwd_workspace_size(const mc_attn_desc* d) {
    if (check_attn_desc(d, "Attention backward") != MC_OK) return 0;
    return mc::attention_bwd_ws(*d).total;
}

mc_status mc_attention_bwd(const mc_attn_desc* d, const void* q, const void* k, const void* v, const float* mask,
                           const void* o, const float* lse, const void* dout, void* dq, void* dk, void* dv,
                           void* workspace, size_t workspace_bytes, hipStream_t stream) {
    mc_status s = check_attn_desc(d, "Attention backward");
    if (s != MC_OK) return s;
    MC_CHECK(q && k && v && o && lse && dout && dq && dk && dv, MC_ERR_NULL,
             "Attention backward: q, k, v, o, lse, dout, dq, dk and dv must not be NULL");
    MC_CHECK(!mask || (double)d->seq * d->seq * 4.0 < 2147483647.0, MC_ERR_SHAPE,
             "Attention backward: an explicit mask needs S * S * 4 < 2^31 bytes (S = %lld)", (long long)d->seq);
    MC_CHECK(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) && aligned16(dout) && aligned16(dq) &&
                 aligned16(dk) && aligned16(dv),
             MC_ERR_LAYOUT, "Attention backward: q, k, v, o, dout, dq, dk and dv must be 16-byte aligned");
    const size_t need = mc::attention_bwd_ws(*d).total;
    MC_CHECK(workspace_bytes >= need && (need == 0 || workspace), MC_ERR_WORKSPACE,
             "Attention backward: workspace of %zu bytes required, %zu given", need, workspace_bytes);
    MC_CHECK(aligned16(workspace), MC_ERR_LAYOUT, "Attention backward: workspace must be 16-byte aligned");
    const double es = d->dtype == MC_F32 ? 4.0 : 2.0;
    const double qo = (double)d->batch * d->heads * d->seq * d->head_dim;
    const double kv = (double)d->batch * d->kv_heads * d->seq * d->head_dim;
    // dS.K, dS^T.Q, P^T.dO and dO.V^T: four products over the computed score pairs
    mc::prof::Scope sc(mc::prof::kAttention, stream, 8.0 * attn_pairs(d) * d->head_dim,
                       es * (4.0 * qo + 4.0 * kv) + 4.0 * d->batch * d->heads * d->seq);
    return hip_status(mc::launch_attention_bwd(*d, q, k, v, mask, o, lse, dout, dq, dk, dv, workspace, stream),
                      "Attention backward");
}

// b^t as Rust's f32::powi lowers it for a run-time exponent: right-to-left
// binary exponentiation in fp32 (square the base, multiply the result in at
// every set bit of t).
static float powi_f32(float base, int32_t t) {
    float r = 1.0f;
    for (;;) {
        if (t & 1) r *= base;
        t /= 2;
        if (t == 0) break;
        base *= base;
    }
    return r;
}

mc_status mc_adamw_step(const mc_adamw_config* cfg, const mc_adamw_tensor* tensors, int32_t count,
                        hipStream_t stream) {
    MC_CHECK(cfg != nullptr, MC_ERR_NULL, "AdamW: config is NULL");
    // AdamWConfig::validate (optimizer.rs:67-103), with its comparisons
    MC_CHECK(!(cfg->learning_rate <= 0.0f), MC_ERR_VALUE, "learning rate must be positive");
    MC_CHECK(cfg->beta1 >= 0.0f && cfg->beta1 < 1.0f, MC_ERR_VALUE, "beta1 must be in [0, 1), got %g",
             (double)cfg->beta1);
    MC_CHECK(cfg->beta2 >= 0.0f && cfg->beta2 < 1.0f, MC_ERR_VALUE, "beta2 must be in [0, 1), got %g",
             (double)cfg->beta2);
    MC_CHECK(!(cfg->epsilon <= 0.0f), MC_ERR_VALUE, "epsilon must be positive");
    MC_CHECK(!(cfg->weight_decay < 0.0f), MC_ERR_VALUE, "weight decay must be non-negative");
    MC_CHECK(count >= 0, MC_ERR_SHAPE, "AdamW: tensor count must be >= 0, got %d", (int)count);
    MC_CHECK(count == 0 || tensors, MC_ERR_NULL, "AdamW: tensor table is NULL");
    double bytes = 0.0;
    for (int32_t i = 0; i < count; ++i) {
        const mc_adamw_tensor& t = tensors[i];
        MC_CHECK(t.numel >= 0 && t.numel < ((int64_t)1 << 40), MC_ERR_SHAPE, "AdamW: tensor %d: numel %lld out of range",
                 (int)i, (long long)t.numel);
        MC_CHECK(t.step >= 1 && t.step <= 2147483647, MC_ERR_VALUE, "AdamW: tensor %d: step must be in [1, 2^31), got %lld",
                 (int)i, (long long)t.step);
        if (t.numel == 0) continue;
        MC_CHECK(t.param && t.grad && t.m && t.v && t.param_out, MC_ERR_NULL,
                 "AdamW: tensor %d: param, grad, m, v and param_out must not be NULL", (int)i);
        MC_CHECK(aligned16(t.param) && aligned16(t.grad) && aligned16(t.m) && aligned16(t.v) && aligned16(t.param_out),
                 MC_ERR_LAYOUT, "AdamW: tensor %d: pointers must be 16-byte aligned", (int)i);
        bytes += 28.0 * (double)t.numel;
    }
    mc::prof::Scope sc(mc::prof::kAdamW, stream, 0.0, bytes);
    mc::AdamWBatch b{};
    b.b1 = cfg->beta1;
    b.b2 = cfg->beta2;
    b.omb1 = 1.0f - cfg->beta1;  // f64::from(1.0 - beta1): the difference is taken in fp32
    b.omb2 = 1.0f - cfg->beta2;
    b.eps = cfg->epsilon;
    b.lr = cfg->learning_rate;
    b.wdlr = cfg->weight_decay * cfg->learning_rate;
    int blocks = 0;
    for (int32_t i = 0; i < count; ++i) {
        const mc_adamw_tensor& t = tensors[i];
        if (t.numel == 0) continue;
        mc::AdamWSlot& sl = b.slot[b.count++];
        sl.p = t.param;
        sl.g = t.grad;
        sl.m = t.m;
        sl.v = t.v;
        sl.po = t.param_out;
        sl.n = t.numel;
        // m_hat = m / f64::from(1 - b1^t): affine(1 / x, 0) with the reciprocal in f64, applied in fp32
        sl.c1 = (float)(1.0 / (double)(1.0f - powi_f32(cfg->beta1, (int32_t)t.step)));
        sl.c2 = (float)(1.0 / (double)(1.0f - powi_f32(cfg->beta2, (int32_t)t.step)));
        sl.blk0 = blocks;
        blocks += mc::adamw_blocks(t.numel);
        if (b.count == mc::kAdamWSlots || i == count - 1) {
            hipError_t e = mc::launch_adamw(b, blocks, stream);
            if (e != hipSuccess) return hip_status(e, "AdamW");
            b.count = 0;
            blocks = 0;
        }
    }
    if (b.count > 0) {
        hipError_t e = mc::launch_adamw(b, blocks, stream);
        if (e != hipSuccess) return hip_status(e, "AdamW");
    }
    return ok();
}

size_t mc_layernorm_bwd_workspace_size(int64_t rows, int64_t dim) {
    if (rows < 1 || dim < 1) return 0;
    return 2 * (size_t)mc::layernorm_bwd_blocks(rows) * (size_t)dim * sizeof(float);
}

mc_status mc_layernorm_fwd(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x, const void* w,
                           const void* b, void* y, float* mean, float* rstd, hipStream_t stream) {
    mc_status s = check_rows(rows, dim, "LayerNorm", kMaxWaveRows);
    if (s != MC_OK) return s;
    if ((s = check_dtype(dtype, "LayerNorm")) != MC_OK) return s;
    MC_CHECK(eps >= 0.0f && std::isfinite(eps), MC_ERR_VALUE, "LayerNorm: eps must be finite and >= 0");
    MC_CHECK(x && y, MC_ERR_NULL, "LayerNorm: x and y must not be NULL");
    MC_CHECK(aligned16(x) && aligned16(y) && (!w || aligned16(w)) && (!b || aligned16(b)), MC_ERR_LAYOUT,
             "LayerNorm: x, w, b and y must be 16-byte aligned");
    const double es = dtype == MC_F32 ? 4.0 : 2.0;
    mc::prof::Scope sc(mc::prof::kRowOps, stream, 0.0,
                       es * (2.0 * rows * dim) + (mean ? 4.0 * rows : 0.0) + (rstd ? 4.0 * rows : 0.0));
    return hip_status(mc::launch_layernorm_fwd(rows, dim, eps, dtype, x, w, b, y, mean, rstd, stream),
                      "LayerNorm forward");
}

mc_status mc_layernorm_bwd(int64_t rows, int64_t dim, float eps, int32_t dtype, const void* x, const void* w,
                           const float* mean, const float* rstd, const void* dy, void* dx, float* dw, float* db,
                           void* workspace, size_t workspace_bytes, hipStream_t stream) {
    mc_status s = check_rows(rows, dim, "LayerNorm backward");
    if (s != MC_OK) return s;
    if ((s = check_dtype(dtype, "LayerNorm backward")) != MC_OK) return s;
    MC_CHECK(eps >= 0.0f && std::isfinite(eps), MC_ERR_VALUE, "LayerNorm: eps must be finite and >= 0");
    MC_CHECK(x && dy && dx, MC_ERR_NULL, "LayerNorm backward: x, dy and dx must not be NULL");
    MC_CHECK(!mean == !rstd, MC_ERR_NULL, "LayerNorm backward: pass both mean and rstd, or neither");
    MC_CHECK(aligned16(x) && aligned16(dy) && aligned16(dx) && (!w || aligned16(w)), MC_ERR_LAYOUT,
             "LayerNorm backward: x, w, dy and dx must be 16-byte aligned");
    if (dw || db) {
        const size_t need = mc_layernorm_bwd_workspace_size(rows, dim);
        MC_CHECK(workspace && workspace_bytes >= need, MC_ERR_WORKSPACE,
                 "LayerNorm backward: workspace of %zu bytes required for dw / db, %zu given", need, workspace_bytes);
        MC_CHECK(aligned16(workspace), MC_ERR_LAYOUT, "LayerNorm backward: workspace must be 16-byte aligned");
    }
    const double es = dtype == MC_F32 ? 4.0 : 2.0;
    mc::prof::Scope sc(mc::prof::kRowOps, stream, 0.0, es * 3.0 * rows * dim);
    return hip_status(mc::launch_layernorm_bwd(rows, dim, eps, dtype, x, w, mean, rstd, dy, dx, dw, db,
                                               static_cast<float*>(workspace), stream),
                      "LayerNorm backward");
}

mc_status mc_log_softmax_fwd(int64_t rows, int64_t dim, int32_t dtype, const void* x, void* y, hipStream_t stream) {
    mc_status s = check_rows(rows, dim, "log_softmax", kMaxBlockRows);
    if (s != MC_OK) return s;
    if ((s = check_dtype(dtype, "log_softmax")) != MC_OK) return s;
    MC_CHECK(x && y, MC_ERR_NULL, "log_softmax: x and y must not be NULL");
    const double es = dtype == MC_F32 ? 4.0 : 2.0;
    mc::prof::Scope sc(mc::prof::kRowOps, stream, 0.0, es * 2.0 * rows * dim);
    return hip_status(mc::launch_log_softmax_fwd(rows, dim, dtype, x, y, stream), "log_softmax forward");
}

mc_status mc_log_softmax_bwd(int64_t rows, int64_t dim, int32_t dtype, const void* y, const void* dy, void* dx,
                             hipStream_t stream) {
    mc_status s = check_rows(rows, dim, "log_softmax backward", kMaxBlockRows);
    if (s != MC_OK) return s;
    if ((s = check_dtype(dtype, "log_softmax backward")) != MC_OK) return s;
    MC_CHECK(y && dy && dx, MC_ERR_NULL, "log_softmax backward: y, dy and dx must not be NULL");
    const double es = dtype == MC_F32 ? 4.0 : 2.0;
    mc::prof::Scope sc(mc::prof::kRowOps, stream, 0.0, es * 3.0 * rows * dim);
    return hip_status(mc::launch_log_softmax_bwd(rows, dim, dtype, y, dy, dx, stream), "log_softmax backward");
}

static mc_status check_xent(const mc_xent_desc* d) {
    MC_CHECK(d != nullptr, MC_ERR_NULL, "cross_entropy: descriptor is NULL");
    mc_status s = check_dtype(d->dtype, "cross_entropy");
    if (s != MC_OK) return s;
    MC_CHECK(d->rows >= 1 && d->vocab >= 1 && d->rows <= kMaxBlockRows, MC_ERR_SHAPE,
             "cross_entropy: rows (%lld) and vocab (%lld) must be >= 1, rows <= %lld", (long long)d->rows,
             (long long)d->vocab, (long long)kMaxBlockRows);
    // cross_entropy_loss_with_smoothing: "smoothing must be in [0, 1), got {}" (loss.rs:214-219)
    MC_CHECK(d->smoothing >= 0.0f && d->smoothing < 1.0f, MC_ERR_VALUE, "smoothing must be in [0, 1), got %g",
             (double)d->smoothing);
    return MC_OK;
}

size_t mc_cross_entropy_workspace_size(const mc_xent_desc* d) {
    if (check_xent(d) != MC_OK) return 0;
    return (size_t)d->rows * 3 * sizeof(float);
}

mc_status mc_cross_entropy_fwd(const mc_xent_desc* d, const void* logits, const uint32_t* targets, float* loss,
                               float* stats, void* workspace, size_t workspace_bytes, hipStream_t stream) {
    mc_status s = check_xent(d);
    if (s != MC_OK) return s;
    MC_CHECK(logits && targets && loss, MC_ERR_NULL, "cross_entropy: logits, targets and loss must not be NULL");
    const size_t need = mc_cross_entropy_workspace_size(d);
    MC_CHECK(workspace && workspace_bytes >= need, MC_ERR_WORKSPACE,
             "cross_entropy: workspace of %zu bytes required, %zu given", need, workspace_bytes);
    MC_CHECK(aligned16(workspace), MC_ERR_LAYOUT, "cross_entropy: workspace must be 16-byte aligned");
    const double es = d->dtype == MC_F32 ? 4.0 : 2.0;
    mc::prof::Scope sc(mc::prof::kRowOps, stream, 0.0, es * (double)d->rows * d->vocab + 4.0 * d->rows);
    return hip_status(mc::launch_cross_entropy_fwd(*d, logits, targets, loss, stats, static_cast<float*>(workspace),
                                                   stream),
                      "cross_entropy forward");
}

mc_status mc_cross_entropy_bwd(const mc_xent_desc* d, const void* logits, const uint32_t* targets,
                               const float* stats, const float* dloss, void* dlogits, hipStream_t stream) {
    mc_status s = check_xent(d);
    if (s != MC_OK) return s;
    MC_CHECK(logits && targets && stats && dloss && dlogits, MC_ERR_NULL,
             "cross_entropy backward: logits, targets, stats, dloss and dlogits must not be NULL");
    const double es = d->dtype == MC_F32 ? 4.0 : 2.0;
    mc::prof::Scope sc(mc::prof::kRowOps, stream, 0.0, es * 2.0 * (double)d->rows * d->vocab + 4.0 * d->rows);
    return hip_status(mc::launch_cross_entropy_bwd(*d, logits, targets, stats, dloss, dlogits, stream),
                      "cross_entropy backward");
}

// Philox4x32-10 (Salmon et al., SC'11), 10 rounds of the two 32x32->64
// multiplies 0xD2511F53 / 0xCD9E8D57 with Weyl key steps 0x9E3779B9 /
// 0xBB67AE85.
static void philox_block(uint64_t blk, uint64_t seed, uint32_t out[4]) {
    uint32_t c0 = (uint32_t)blk, c1 = (uint32_t)(blk >> 32), c2 = 0, c3 = 0;
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    for (int i = 0; i < 10; ++i) {
        const uint64_t a = (uint64_t)0xD2511F53u * c0;
        const uint64_t b = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(b >> 32) ^ c1 ^ k0;
        const uint32_t n2 = (uint32_t)(a >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)b;
        c3 = (uint32_t)a;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

mc_status mc_dropout_mask(uint64_t seed, float p, int64_t rows, int32_t rank, uint8_t* mask_host) {
    MC_CHECK(rows >= 1 && rank >= 1, MC_ERR_SHAPE, "dropout mask: rows and rank must be >= 1");
    MC_CHECK(p >= 0.0f && p < 1.0f, MC_ERR_VALUE, "LoRA dropout must be in [0, 1)");
    MC_CHECK(mask_host != nullptr, MC_ERR_NULL, "dropout mask: output must not be NULL");
    const int64_t n = rows * (int64_t)rank;
    uint32_t w[4];
    for (int64_t i = 0; i < n; ++i) {
        if ((i & 3) == 0) philox_block((uint64_t)(i >> 2), seed, w);
        const float u = (float)(w[i & 3] >> 8) * (1.0f / 16777216.0f);
        mask_host[i] = (uint8_t)(u >= p);
    }
    return ok();
}

}  // extern "C"
