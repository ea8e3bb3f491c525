// LoRA linear forward / backward: workspace layout and launch sequence.
//
// Forward (bf16 activations), reference order lora.rs:320-339 plus the base
// candle Linear (transformer.rs:189-192), three launches:
//   1. A^T -> bf16 hi/lo, B^T -> bf16 ext operand          (one prep launch)
//   2. Hd = dropout(x.A) -> h_save (fp32 [r][T]) and s*Hd (bf16 ext operand)
//   3. y = [x | s*Hd] . [W | B^T]^T + b                    (one MFMA GEMM)
// Backward (W frozen; candle autograd of the same composite):
//   1. G = s dY.B^T, Gd = dropout'(G) -> Gd^T fp32, Gd bf16 (B read as
//      fp32, split hi/lo in registers), with A -> bf16 ext operand and
//      W -> W^T in the same launch
//   2. dX = [dY | Gd] . [W^T | A]^T                         (one MFMA GEMM)
//   3. dA = x^T.Gd and dB = s Hd^T.dY: split-T column reductions (one
//      launch) and their fixed-order split sums (one launch)
// The fp32 path runs the same sequence with fp32 operands and FMA kernels.
#include "common.hpp"
#include "kernels.hpp"
#include "lora_kernels.hpp"
#include "profile.hpp"

namespace mc {
namespace {

__global__ __launch_bounds__(256) void transpose_f32(const float* __restrict__ src, int64_t rows, int64_t cols,
                                                     float* __restrict__ dst) {
    // dst[j][i] = src[i][j]
    const int64_t n = rows * cols;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = idx / cols, j = idx % cols;
        dst[j * rows + i] = src[idx];
    }
}

hipError_t launch_transpose_f32(const float* src, int64_t rows, int64_t cols, float* dst, hipStream_t st) {
    int64_t blocks = (rows * cols + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    transpose_f32<<<dim3((unsigned)blocks), 256, 0, st>>>(src, rows, cols, dst);
    return hipGetLastError();
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct Dims {
    int64_t T, K, N;
    int r, r16, rext;
    bool bf16;
};

Dims dims_of(const mc_lora_desc& d) {
    Dims m;
    m.T = d.tokens;
    m.K = d.in_features;
    m.N = d.out_features;
    m.r = d.rank;
    // MFMA rank tiles: 16, 32, 64 or 128 rows (the rowproj instantiations)
    m.r16 = d.rank <= 16 ? 16 : d.rank <= 32 ? 32 : d.rank <= 64 ? 64 : 128;
    m.rext = (int)round_up(d.rank, 8);
    m.bf16 = d.act_dtype == MC_BF16;
    return m;
}

// Algorithmic work of one GEMM launch: FLOPs of the base product (the rank
// columns when there is no base), bytes of one read of each operand and one
// write of the output.
prof::Scope gemm_scope(hipStream_t st, int64_t M, int64_t N, int64_t kbase, int64_t kext, int r, int es) {
    const double k = (double)(kbase > 0 ? kbase : r);
    return prof::Scope(prof::kGemm, st, 2.0 * M * N * k,
                       (double)es * ((double)(M + N) * (double)(kbase + kext) + (double)M * N));
}

// rowproj / colreduce: one read of X (T x C, act dtype), the rank-r side in fp32.
prof::Scope lowrank_scope(hipStream_t st, int64_t T, int64_t C, int r, int es) {
    return prof::Scope(prof::kLowRank, st, 2.0 * T * C * r, (double)T * C * es + 4.0 * T * r);
}

#define MC_TRY(expr)                          \
    do {                                      \
        hipError_t e_ = (expr);               \
        if (e_ != hipSuccess) return e_;      \
    } while (0)

}  // namespace

LoraFwdWs lora_fwd_ws(const mc_lora_desc& d) {
    const Dims m = dims_of(d);
    LoraFwdWs w{};
    size_t off = 0;
    if (m.bf16) {
        w.at_hilo = off; off += align256((size_t)2 * m.r16 * m.K * 2);
        w.bt_ext = off;  off += align256((size_t)m.N * m.rext * 2);
        w.hs_ext = off;  off += align256((size_t)m.T * m.rext * 2);
    } else {
        w.bt_ext = off;  off += align256((size_t)m.N * m.r * 4);
        w.hs_ext = off;  off += align256((size_t)m.T * m.r * 4);
    }
    w.hd_t = 0;
    w.total = off;
    return w;
}

LoraBwdWs lora_bwd_ws(const mc_lora_desc& d) {
    const Dims m = dims_of(d);
    LoraBwdWs w{};
    size_t off = 0;
    if (m.bf16) {
        w.wt = off;     off += align256((size_t)m.K * m.N * 2);
        w.at_ext = off; off += align256((size_t)m.K * m.rext * 2);
        w.gd_ext = off; off += align256((size_t)m.T * m.rext * 2);
        w.gd_t = off;   off += align256((size_t)m.r * m.T * 4);
        w.part_a = off; off += align256((size_t)colreduce_splits(m.T, m.K) * m.r16 * m.K * 4);
        w.part_b = off; off += align256((size_t)colreduce_splits(m.T, m.N) * m.r16 * m.N * 4);
    } else {
        w.at_ext = off; off += align256((size_t)m.r * m.K * 4);
        w.gd_ext = off; off += align256((size_t)m.T * m.r * 4);
        w.gd_t = off;   off += align256((size_t)m.r * m.T * 4);
    }
    w.total = off;
    return w;
}

hipError_t launch_lora_fwd(const mc_lora_desc& d, const void* x, const void* W, const void* bias,
                           const float* A, const float* B, const uint8_t* mask, void* y,
                           float* h_save, void* ws, hipStream_t st) {
    const Dims m = dims_of(d);
    const LoraFwdWs w = lora_fwd_ws(d);
    char* base = static_cast<char*>(ws);
    const float keep = mask ? 1.0f / (1.0f - d.dropout_p) : 1.0f;
    const int64_t kbase = W ? m.K : 0;
    if (m.bf16) {
        uint16_t* at_hi = reinterpret_cast<uint16_t*>(base + w.at_hilo);
        uint16_t* at_lo = at_hi + (size_t)m.r16 * m.K;
        uint16_t* bt = reinterpret_cast<uint16_t*>(base + w.bt_ext);
        uint16_t* hs = reinterpret_cast<uint16_t*>(base + w.hs_ext);
        const uint16_t* xb = static_cast<const uint16_t*>(x);
        {
            auto sc = lowrank_scope(st, m.T, m.K, m.r, 2);
            const PrepJob ja{A, m.r, m.r, m.K, true, at_hi, at_lo, m.r16, m.K};   // A^T hi / lo
            const PrepJob jb{B, m.N, m.N, m.r, true, bt, nullptr, m.N, m.rext};   // B^T, zero-padded
            MC_TRY(launch_prep_bf16(ja, jb, st));
            MC_TRY(launch_rowproj_bf16(xb, m.T, m.K, at_hi, at_lo, m.r, 1.0f, mask, keep, h_save, hs, m.rext,
                                       d.scale, st));
        }
        GemmSeg s0{xb, m.K, static_cast<const uint16_t*>(W), m.K, kbase};
        GemmSeg s1{hs, m.rext, bt, m.rext, m.rext};
        auto sc = gemm_scope(st, m.T, m.N, kbase, m.rext, m.r, 2);
        return launch_gemm_bf16(m.T, m.N, s0, s1, static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(y),
                                m.N, st);
    }
    float* bt = reinterpret_cast<float*>(base + w.bt_ext);
    float* hs = reinterpret_cast<float*>(base + w.hs_ext);
    const float* xf = static_cast<const float*>(x);
    {
        auto sc = lowrank_scope(st, m.T, m.K, m.r, 4);
        MC_TRY(launch_rowproj_f32(xf, m.T, m.K, A, true, m.r, 1.0f, mask, keep, h_save, hs, d.scale, st));
        MC_TRY(launch_transpose_f32(B, m.r, m.N, bt, st));
    }
    GemmSegF32 s0{xf, m.K, static_cast<const float*>(W), m.K, kbase};
    GemmSegF32 s1{hs, m.r, bt, m.r, m.r};
    auto sc = gemm_scope(st, m.T, m.N, kbase, m.r, m.r, 4);
    return launch_gemm_f32(false, m.T, m.N, s0, s1, static_cast<const float*>(bias), static_cast<float*>(y),
                           m.N, st);
}

hipError_t launch_lora_bwd(const mc_lora_desc& d, const void* x, const void* W, const float* A,
                           const float* B, const uint8_t* mask, const float* h_save,
                           const void* dY, void* dX, float* dA, float* dB, void* ws,
                           hipStream_t st) {
    const Dims m = dims_of(d);
    const LoraBwdWs w = lora_bwd_ws(d);
    char* base = static_cast<char*>(ws);
    const float keep = mask ? 1.0f / (1.0f - d.dropout_p) : 1.0f;
    const bool need_g = dX || dA;
    const int64_t kbase = W ? m.N : 0;
    if (m.bf16) {
        const uint16_t* dyb = static_cast<const uint16_t*>(dY);
        uint16_t* at = reinterpret_cast<uint16_t*>(base + w.at_ext);
        uint16_t* gd = reinterpret_cast<uint16_t*>(base + w.gd_ext);
        float* gdt = reinterpret_cast<float*>(base + w.gd_t);
        uint16_t* wt = reinterpret_cast<uint16_t*>(base + w.wt);
        if (need_g) {
            // one launch: G = s dY.B^T (B read as fp32), A zero-padded to the
            // dX extension columns, and W^T for the dX GEMM
            const PrepJob ja{A, m.r, m.K, m.r, false, dX ? at : nullptr, nullptr, m.K, m.rext};
            const bool tw = dX && W;
            const double bytes = 2.0 * m.T * m.N + 4.0 * m.T * m.r + 4.0 * m.r * m.N +
                                 (dX ? 6.0 * m.r * m.K : 0.0) + (tw ? 4.0 * m.N * m.K : 0.0);
            auto sc = prof::Scope(prof::kLowRank, st, 2.0 * m.T * m.N * m.r, bytes);
            MC_TRY(launch_lora_bwd_operands(dyb, m.T, m.N, B, m.r, d.scale, mask, keep, dA ? gdt : nullptr,
                                            dX ? gd : nullptr, m.rext, ja, static_cast<const uint16_t*>(W), m.K,
                                            tw ? wt : nullptr, st));
        }
        if (dX) {
            GemmSeg s0{dyb, m.N, wt, m.N, kbase};
            GemmSeg s1{gd, m.rext, at, m.rext, m.rext};
            auto sc = gemm_scope(st, m.T, m.K, kbase, m.rext, m.r, 2);
            MC_TRY(launch_gemm_bf16(m.T, m.K, s0, s1, nullptr, static_cast<uint16_t*>(dX), m.K, st));
        }
        if (dA || dB) {
            // dA = x^T.Gd and dB = s Hd^T.dY: split-T column reductions in one
            // launch, then both fixed-order split sums in one launch
            const int sa = colreduce_splits(m.T, m.K), sb = colreduce_splits(m.T, m.N);
            float* pa = reinterpret_cast<float*>(base + w.part_a);
            float* pb = reinterpret_cast<float*>(base + w.part_b);
            const ColJob ca{dA ? static_cast<const uint16_t*>(x) : nullptr, m.K, gdt, sa, pa};
            const ColJob cb{dB ? dyb : nullptr, m.N, h_save, sb, pb};
            const SumJob ua{pa, sa, m.K, (int64_t)m.r16 * m.K, 1.0f, true, dA};
            const SumJob ub{pb, sb, m.N, (int64_t)m.r16 * m.N, d.scale, false, dB};
            const double bytes = (dA ? 2.0 * m.T * m.K + 4.0 * m.T * m.r : 0.0) +
                                 (dB ? 2.0 * m.T * m.N + 4.0 * m.T * m.r : 0.0);
            const double flops = (dA ? 2.0 * m.T * m.K * m.r : 0.0) + (dB ? 2.0 * m.T * m.N * m.r : 0.0);
            auto sc = prof::Scope(prof::kLowRank, st, flops, bytes);
            MC_TRY(launch_colreduce_bf16(m.T, m.r, ca, cb, st));
            MC_TRY(launch_split_sum(m.r, ua, ub, st));
        }
        return hipSuccess;
    }
    const float* dyf = static_cast<const float*>(dY);
    float* at = reinterpret_cast<float*>(base + w.at_ext);
    float* gd = reinterpret_cast<float*>(base + w.gd_ext);
    float* gdt = reinterpret_cast<float*>(base + w.gd_t);
    if (need_g) {
        auto sc = lowrank_scope(st, m.T, m.N, m.r, 4);
        MC_TRY(launch_rowproj_f32(dyf, m.T, m.N, B, false, m.r, d.scale, mask, keep, gdt, gd, 1.0f, st));
    }
    if (dX) {
        MC_TRY(launch_transpose_f32(A, m.K, m.r, at, st));
        GemmSegF32 s0{dyf, m.N, static_cast<const float*>(W), m.K, kbase};
        GemmSegF32 s1{gd, m.r, at, m.K, m.r};
        auto sc = gemm_scope(st, m.T, m.K, kbase, m.r, m.r, 4);
        MC_TRY(launch_gemm_f32(true, m.T, m.K, s0, s1, nullptr, static_cast<float*>(dX), m.K, st));
    }
    if (dA) {
        auto sc = lowrank_scope(st, m.T, m.K, m.r, 4);
        MC_TRY(launch_colreduce_f32(static_cast<const float*>(x), m.T, m.K, gdt, m.r, 1.0f, true, dA, st));
    }
    if (dB) {
        auto sc = lowrank_scope(st, m.T, m.N, m.r, 4);
        MC_TRY(launch_colreduce_f32(dyf, m.T, m.N, h_save, m.r, d.scale, false, dB, st));
    }
    return hipSuccess;
}

}  // namespace mc
