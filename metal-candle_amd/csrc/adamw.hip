// AdamW update of the LoRA parameters, gfx950.
//
// AdamW::step (src/training/optimizer.rs:227-281) updates one parameter
// tensor with candle fp32 tensor ops, each rounded to fp32 in this order
// (`tensor * f64` and `tensor + f64` are candle's affine(mul, add), which
// computes v * mul + add):
//
//   m1 = (m * b1 + 0) + (g * (1 - b1) + 0)
//   v1 = (v * b2 + 0) + ((g * g) * (1 - b2) + 0)
//   mh = m1 * c1 + 0            c1 = 1 / (1 - b1^t)  (f64 reciprocal, rounded to fp32)
//   vh = v1 * c2 + 0            c2 = 1 / (1 - b2^t)
//   u  = mh / (sqrt(vh) * 1 + eps)
//   p1 = (p - (u * lr + 0)) - (p * (wd * lr) + 0)
//
// adamw_kernel fuses the chain into one pass over (p, g, m, v): 16 bytes in
// and 12 out per element, HBM-bound (one float4 of each per thread: the
// LoRA parameter sets are small, so more workgroups keep more CUs loading).
// Contraction into FMA is off for this
// file, division and square root are the correctly rounded ones, so every
// value equals the fp32 op sequence above bit for bit. One launch updates up
// to kSlots tensors (a table passed by value); each workgroup finds its
// tensor from the table's block offsets.
#include "common.hpp"
#include "kernels.hpp"

#pragma clang fp contract(off)

namespace mc {
namespace {

constexpr int kThreads = 256;
constexpr int kPerBlock = kThreads * 4;  // elements per workgroup: one float4 per thread

__device__ __forceinline__ float affine0(float x, float mul) { return x * mul + 0.0f; }

__device__ __forceinline__ void adamw_elem(float& p, float g, float& m, float& v, float c1, float c2,
                                           const AdamWBatch& b) {
    const float m1 = affine0(m, b.b1) + affine0(g, b.omb1);
    const float v1 = affine0(v, b.b2) + affine0(g * g, b.omb2);
    const float mh = affine0(m1, c1);
    const float vh = affine0(v1, c2);
    const float den = sqrtf(vh) * 1.0f + b.eps;  // sqrtf: the correctly rounded square root
    const float u = mh / den;
    const float p1 = (p - affine0(u, b.lr)) - affine0(p, b.wdlr);
    p = p1;
    m = m1;
    v = v1;
}

__global__ __launch_bounds__(kThreads) void adamw_kernel(AdamWBatch bt) {
    int s = 0;
    for (int i = 1; i < bt.count; ++i)
        if ((int)blockIdx.x >= bt.slot[i].blk0) s = i;
    const AdamWSlot& t = bt.slot[s];
    const int64_t base = (int64_t)((int)blockIdx.x - t.blk0) * kPerBlock;
    {
        const int64_t e = base + (int64_t)threadIdx.x * 4;
        if (e + 4 <= t.n) {
            float4 p = *reinterpret_cast<const float4*>(t.p + e);
            const float4 g = *reinterpret_cast<const float4*>(t.g + e);
            float4 m = *reinterpret_cast<const float4*>(t.m + e);
            float4 v = *reinterpret_cast<const float4*>(t.v + e);
            adamw_elem(p.x, g.x, m.x, v.x, t.c1, t.c2, bt);
            adamw_elem(p.y, g.y, m.y, v.y, t.c1, t.c2, bt);
            adamw_elem(p.z, g.z, m.z, v.z, t.c1, t.c2, bt);
            adamw_elem(p.w, g.w, m.w, v.w, t.c1, t.c2, bt);
            *reinterpret_cast<float4*>(t.po + e) = p;
            *reinterpret_cast<float4*>(t.m + e) = m;
            *reinterpret_cast<float4*>(t.v + e) = v;
        } else {
            for (int64_t i = e; i < t.n; ++i) {
                float p = t.p[i], m = t.m[i], v = t.v[i];
                adamw_elem(p, t.g[i], m, v, t.c1, t.c2, bt);
                t.po[i] = p;
                t.m[i] = m;
                t.v[i] = v;
            }
        }
    }
}

}  // namespace

int adamw_blocks(int64_t n) { return (int)((n + kPerBlock - 1) / kPerBlock); }

hipError_t launch_adamw(const AdamWBatch& batch, int blocks, hipStream_t stream) {
    if (blocks <= 0) return hipSuccess;
    adamw_kernel<<<dim3((unsigned)blocks), kThreads, 0, stream>>>(batch);
    return hipGetLastError();
}

}  // namespace mc
