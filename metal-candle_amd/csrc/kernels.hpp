// Host-side launchers of the gfx950 kernels. Arguments are validated by the
// C ABI layer (abi.cpp) before any of these is called; the launchers assume
// consistent shapes, 16-byte aligned pointers and non-null required buffers.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mc_hip.h"

namespace mc {

// ------------------------------------------------------------- RMSNorm
hipError_t launch_rmsnorm_fwd(int64_t rows, int64_t dim, float eps, int dtype, const void* x,
                              const void* w, void* y, float* rstd, hipStream_t stream);
// Number of row blocks the dw reduction is split into (fixed for a shape).
int rmsnorm_bwd_blocks(int64_t rows, int64_t dim);
hipError_t launch_rmsnorm_bwd(int64_t rows, int64_t dim, float eps, int dtype, const void* x,
                              const void* w, const float* rstd, const void* dy, void* dx, float* dw,
                              float* partial, hipStream_t stream);
// Size of the static device scratch that mc_rmsnorm_bwd_noalloc uses in place
// of a workspace, and its device address on the current device (looked up
// once per device).
constexpr size_t kRmsNormScratchBytes = (size_t)16 << 20;
hipError_t rmsnorm_scratch(float** out);

// ------------------------------------------------------------- softmax
hipError_t launch_softmax_fwd(int64_t rows, int64_t dim, int64_t causal_rows, int dtype,
                              const void* s, void* p, hipStream_t stream);
hipError_t launch_softmax_bwd(int64_t rows, int64_t dim, int64_t causal_rows, int dtype,
                              const void* p, const void* dp, void* ds, hipStream_t stream);

// ---------------------------------------------------------------- LoRA
// Workspace layout of the LoRA entry points (byte offsets into workspace).
struct LoraFwdWs {
    size_t at_hilo;   // bf16 [2][r16][K]  A^T split into hi/lo (bf16 path)
    size_t bt_ext;    // bf16 [N][rext]    B^T, zero padded (GEMM extension operand)
    size_t hs_ext;    // bf16 [T][rext]    s*Hd, zero padded (GEMM extension operand)
    size_t hd_t;      // f32  [r][T]       Hd^T when the caller passes no h_save
    size_t total;
};
struct LoraBwdWs {
    size_t wt;        // bf16 [K][N]       W^T (dX GEMM operand; bf16 path with W)
    size_t at_ext;    // bf16 [K][rext]    A, zero padded columns (dX extension operand);
                      // fp32 path: f32 [r][K] A^T
    size_t gd_ext;    // bf16 [T][rext]    Gd, zero padded (dX extension operand)
    size_t gd_t;      // f32  [r][T]       Gd^T
    size_t part_a;    // f32  [S_a][r16][K] split-T partials of dA
    size_t part_b;    // f32  [S_b][r16][N] split-T partials of dB
    size_t total;
};
LoraFwdWs lora_fwd_ws(const mc_lora_desc& d);
LoraBwdWs lora_bwd_ws(const mc_lora_desc& d);

// Grouped projections of one input (bf16): up to kLoraMaxProj projections
// sharing x, T, K, r, scale and p. Workspace layouts (byte offsets).
constexpr int kLoraMaxProj = 4;
struct LoraProj {
    int64_t N;
    const void* W;
    const void* bias;
    const float* A;
    const float* B;
    const uint8_t* mask;
    const void* Wt = nullptr;  // W^T [K][N] built by the caller, or null (transposed into the workspace)
};
struct LoraGroupFwdWs {
    size_t at_hilo[kLoraMaxProj];  // per row-projection pass: bf16 [2][16 rc][K]
    size_t bt_ext[kLoraMaxProj];   // per projection: bf16 [N_g][rext]
    size_t hs_ext;                 // bf16 [T][G rext]: s Hd of every projection
    size_t part;                   // split row projection: f32 [passes][splits][T][16 rc] partials of H
    size_t total;
};
struct LoraGroupBwdWs {
    size_t wt[kLoraMaxProj];       // per projection with W and no caller W^T: bf16 [K][N_g] W_g^T
    size_t at_ext;                 // bf16 [K][G rext]: A of every projection
    size_t gd_ext;                 // bf16 [T][G rext]: Gd of every projection
    size_t gd_t;                   // f32 [G r][T]: Gd^T of every projection (or bf16 hi / lo planes [2][G r][T])
    size_t hd_hilo;                // column-split path: bf16 [2][G r][T] hi / lo planes of every Hd_g^T
    size_t part_a;                 // f32 [S_a][colreduce rows of G r][K]
    size_t part_b[kLoraMaxProj];   // f32 [S_b][colreduce rows of r][N_g]
    size_t gpart[kLoraMaxProj];    // G partials: f32 [column groups of N_g][T][r] of the fused dY pass, or
                                   // f32 [splits][T][16 rc] of the split row projection
    size_t total;
};
LoraGroupFwdWs lora_group_fwd_ws(const mc_lora_desc& d, const int64_t* N, int count);
// need_wt[g]: projection g's W^T is transposed into the workspace (null: all)
LoraGroupBwdWs lora_group_bwd_ws(const mc_lora_desc& d, const int64_t* N, int count, const bool* need_wt = nullptr);
hipError_t launch_lora_group_fwd(const mc_lora_desc& d, const void* x, const LoraProj* proj, int count,
                                 void* const* y, float* const* h_save, void* ws, hipStream_t stream);
// dX (may be null) receives the sum over the projections; dA / dB (arrays,
// or null; entries may be null) per projection; h_save[g] is required where
// dB[g] is requested.
hipError_t launch_lora_group_bwd(const mc_lora_desc& d, const void* x, const LoraProj* proj, int count,
                                 const float* const* h_save, const void* const* dY, void* dX, float* const* dA,
                                 float* const* dB, void* ws, hipStream_t stream);

// out [cols][rows] = in [rows][cols]^T, bf16
hipError_t launch_transpose_bf16(const void* in, int64_t rows, int64_t cols, void* out, hipStream_t stream);

hipError_t launch_lora_fwd(const mc_lora_desc& d, const void* x, const void* W, const void* bias,
                           const float* A, const float* B, const uint8_t* mask, void* y,
                           float* h_save, void* ws, hipStream_t stream);
hipError_t launch_lora_bwd(const mc_lora_desc& d, const void* x, const void* W, const float* A,
                           const float* B, const uint8_t* mask, const float* h_save,
                           const void* dY, void* dX, float* dA, float* dB, void* ws,
                           hipStream_t stream);

// ----------------------------------------------------------- attention
// Workspace of mc_attention_fwd: V^T [B, Hkv, D, Sp] bf16 for the MFMA path
// (Sp = S rounded up to 64), nothing for the generic path.
struct AttnWs {
    size_t vt;
    size_t total;
};
bool attention_uses_mfma(const mc_attn_desc& d);
AttnWs attention_fwd_ws(const mc_attn_desc& d);
hipError_t launch_attention_fwd(const mc_attn_desc& d, const void* q, const void* k, const void* v,
                                const float* mask, void* o, float* lse, void* ws, hipStream_t stream);
// Workspace of mc_attention_bwd (byte offsets). MFMA path: lse * log2 e and
// Delta per 64-query block (f32 [B, H, Sp/64, 2, 64], Sp = S rounded up to
// 64) and, when the dK/dV kernel splits a K/V head's query heads into more
// than one group (attn_dkdv_groups), the per-group dK / dV partials (f32
// [B, Hkv, groups, S, D]). Generic path: Delta (f32 [B, H, S]) at lsd.
struct AttnBwdWs {
    size_t lsd, dk_part, dv_part;
    size_t dst;  // bf16 dS^T [B, H, S, ldst] for the dQ pass (attention_dq_from_ds), else unused
    size_t total;
};
AttnBwdWs attention_bwd_ws(const mc_attn_desc& d);
int attn_dkdv_groups(const mc_attn_desc& d);
hipError_t launch_attention_bwd(const mc_attn_desc& d, const void* q, const void* k, const void* v,
                                const float* mask, const void* o, const float* lse, const void* dout, void* dq,
                                void* dk, void* dv, void* ws, hipStream_t stream);

// --------------------------------------------------------------- AdamW
// One launch of the AdamW kernel updates up to kAdamWSlots tensors; the
// table travels by value as a kernel argument (no device allocation).
// blk0: first workgroup of the slot; c1, c2: the bias-correction factors of
// the slot's step, as fp32.
constexpr int kAdamWSlots = 16;
struct AdamWSlot {
    const float* p;
    const float* g;
    float* m;
    float* v;
    float* po;
    int64_t n;
    float c1, c2;
    int blk0, pad;
};
struct AdamWBatch {
    AdamWSlot slot[kAdamWSlots];
    int count;
    float b1, b2, omb1, omb2, eps, lr, wdlr;
};
int adamw_blocks(int64_t n);  // workgroups one tensor of n elements takes
hipError_t launch_adamw(const AdamWBatch& batch, int blocks, hipStream_t stream);

// ------------------------------------------------ LayerNorm, log-softmax, CE
int layernorm_bwd_blocks(int64_t rows);  // dw / db partial rows in the workspace
hipError_t launch_layernorm_fwd(int64_t rows, int64_t dim, float eps, int dtype, const void* x, const void* w,
                                const void* b, void* y, float* mean, float* rstd, hipStream_t stream);
hipError_t launch_layernorm_bwd(int64_t rows, int64_t dim, float eps, int dtype, const void* x, const void* w,
                                const float* mean, const float* rstd, const void* dy, void* dx, float* dw, float* db,
                                float* ws, hipStream_t stream);
hipError_t launch_log_softmax_fwd(int64_t rows, int64_t dim, int dtype, const void* x, void* y, hipStream_t stream);
hipError_t launch_log_softmax_bwd(int64_t rows, int64_t dim, int dtype, const void* y, const void* dy, void* dx,
                                  hipStream_t stream);
hipError_t launch_cross_entropy_fwd(const mc_xent_desc& d, const void* logits, const uint32_t* targets, float* loss,
                                    float* stats, float* ws, hipStream_t stream);
hipError_t launch_cross_entropy_bwd(const mc_xent_desc& d, const void* logits, const uint32_t* targets,
                                    const float* stats, const float* dloss, void* dlogits, hipStream_t stream);

}  // namespace mc
