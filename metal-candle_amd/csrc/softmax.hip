// Last-dim softmax forward / backward with an optional causal mask, gfx950.
//
// Semantics: the candle composite softmax_stable (src/backend/tensor.rs:91-98:
// max, sub, exp, sum, divide) applied after Attention::forward adds the
// causal -inf mask (src/models/transformer.rs:264-275). Replaces the Metal
// kernel fused_softmax (src/backend/kernels.metal:187-261), which handles
// rank <= 3 only (custom_ops.rs:743-751) and has no mask and no backward.
//
// Design: one wave64 per row, the row held in registers as VPL 16-byte
// vectors per lane, so s is read once and p written once. Max and sum are
// DPP butterflies. exp is v_exp_f32 on (z - max) * log2(e); the normaliser
// is applied as a multiply by 1/sum. With a causal mask, 16-byte vectors that
// lie entirely past the row's last unmasked column are neither read nor
// computed; the kernel writes exact zeros there. Offsets are 64-bit: a
// [4,28,4096,4096] score tensor has 1.9e9 elements.
#include "common.hpp"
#include "kernels.hpp"

namespace mc {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Last unmasked column (inclusive) of a row.
__device__ __forceinline__ int64_t row_limit(int64_t row, int64_t dim, int64_t causal_rows) {
    return causal_rows > 0 ? row % causal_rows + (dim - causal_rows) : dim - 1;
}

// Vector path: the 4 rows of a workgroup through one buffer resource (a
// wave's row at a scalar byte offset); every load of the row is issued
// before any use, with wholly masked vectors and vectors past the row given
// out-of-range offsets (no memory traffic, zeros), and the masks applied as
// value selects.
template <typename T, int VPL>
__global__ __launch_bounds__(256) void softmax_fwd_vec(int64_t rows, int dim, int64_t causal_rows,
                                                       const T* __restrict__ s, T* __restrict__ p) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    const int lane = lane_id();
    const int wave = wave_id();
    const int64_t r0 = (int64_t)blockIdx.x * kRowsPerBlock;
    const int64_t row = r0 + wave;
    if (row >= rows) return;
    const int64_t nrows = rows - r0 < kRowsPerBlock ? rows - r0 : kRowsPerBlock;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(s + r0 * dim, nrows * dim * ES);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(p + r0 * dim, nrows * dim * ES);
    const int nvec = dim / N;
    const int lim = (int)row_limit(row, dim, causal_rows);
    const uint32_t rowoff = (uint32_t)(wave * dim * ES);
    float v[VPL][N];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
        const bool ok = vi < nvec && vi * N <= lim;
        BVec<T>::load(rs, ok ? rowoff + (uint32_t)(vi * N * ES) : kOOB, v[i]);
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const bool valid = vi < nvec && vi * N + e <= lim;
            v[i][e] = valid ? v[i][e] : -INFINITY;
            m = fmaxf(m, v[i][e]);
        }
    }
    m = wave_max(m);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float ex = fast_exp2((v[i][e] - m) * kLog2e);  // masked: exp2(-inf) = 0
            v[i][e] = ex;
            sum += ex;
        }
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
        float o[N];
#pragma unroll
        for (int e = 0; e < N; ++e) o[e] = v[i][e] * inv;
        BVec<T>::store(rp, vi < nvec ? rowoff + (uint32_t)(vi * N * ES) : kOOB, o);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_fwd_scalar(int64_t rows, int64_t dim, int64_t causal_rows,
                                                          const T* __restrict__ s, T* __restrict__ p) {
    const int lane = lane_id();
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t lim = row_limit(row, dim, causal_rows);
    const T* sr = s + row * dim;
    float m = -INFINITY;
    for (int64_t j = lane; j <= lim; j += kWave) m = fmaxf(m, Elem<T>::load(sr, j));
    m = wave_max(m);
    float sum = 0.f;
    for (int64_t j = lane; j <= lim; j += kWave) sum += fast_exp2((Elem<T>::load(sr, j) - m) * kLog2e);
    sum = wave_sum(sum);
    const float inv = 1.0f / sum;
    for (int64_t j = lane; j < dim; j += kWave) {
        float o = j <= lim ? fast_exp2((Elem<T>::load(sr, j) - m) * kLog2e) * inv : 0.f;
        Elem<T>::store(p + row * dim, j, o);
    }
}

template <typename T, int VPL>
__global__ __launch_bounds__(256) void softmax_bwd_vec(int64_t rows, int dim, int64_t causal_rows,
                                                       const T* __restrict__ p, const T* __restrict__ dp,
                                                       T* __restrict__ ds) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    const int lane = lane_id();
    const int wave = wave_id();
    const int64_t r0 = (int64_t)blockIdx.x * kRowsPerBlock;
    const int64_t row = r0 + wave;
    if (row >= rows) return;
    const int64_t nrows = rows - r0 < kRowsPerBlock ? rows - r0 : kRowsPerBlock;
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(p + r0 * dim, nrows * dim * ES);
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(dp + r0 * dim, nrows * dim * ES);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(ds + r0 * dim, nrows * dim * ES);
    const int nvec = dim / N;
    const int lim = (int)row_limit(row, dim, causal_rows);
    const uint32_t rowoff = (uint32_t)(wave * dim * ES);
    float pv[VPL][N], gv[VPL][N];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
        const uint32_t off = (vi < nvec && vi * N <= lim) ? rowoff + (uint32_t)(vi * N * ES) : kOOB;
        BVec<T>::load(rp, off, pv[i]);
        BVec<T>::load(rg, off, gv[i]);
    }
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            // masked: p = 0 by definition (and dp is not read there)
            pv[i][e] = (vi < nvec && vi * N + e <= lim) ? pv[i][e] : 0.f;
            dot += pv[i][e] * gv[i][e];
        }
    }
    dot = wave_sum(dot);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
        float o[N];
#pragma unroll
        for (int e = 0; e < N; ++e) o[e] = pv[i][e] * (gv[i][e] - dot);
        BVec<T>::store(rd, vi < nvec ? rowoff + (uint32_t)(vi * N * ES) : kOOB, o);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_bwd_scalar(int64_t rows, int64_t dim, int64_t causal_rows,
                                                          const T* __restrict__ p, const T* __restrict__ dp,
                                                          T* __restrict__ ds) {
    const int lane = lane_id();
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t lim = row_limit(row, dim, causal_rows);
    const T* pr = p + row * dim;
    const T* gr = dp + row * dim;
    float dot = 0.f;
    for (int64_t j = lane; j <= lim; j += kWave) dot += Elem<T>::load(pr, j) * Elem<T>::load(gr, j);
    dot = wave_sum(dot);
    for (int64_t j = lane; j < dim; j += kWave) {
        float o = j <= lim ? Elem<T>::load(pr, j) * (Elem<T>::load(gr, j) - dot) : 0.f;
        Elem<T>::store(ds + row * dim, j, o);
    }
}

template <typename T>
bool vec_ok(int64_t dim) {
    return dim % Vec16<T>::N == 0 && dim / Vec16<T>::N <= 16 * kWave;
}

template <typename T>
int vpl_for(int64_t dim) {
    const int64_t nvec = dim / Vec16<T>::N;
    const int64_t per = (nvec + kWave - 1) / kWave;
    return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : per <= 8 ? 8 : 16;
}

template <typename T>
hipError_t fwd_impl(int64_t rows, int64_t dim, int64_t causal, const void* s, void* p, hipStream_t st) {
    const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const T* sp = static_cast<const T*>(s);
    T* pp = static_cast<T*>(p);
    if (vec_ok<T>(dim)) {
        const int d = (int)dim;
        switch (vpl_for<T>(dim)) {
            case 1: softmax_fwd_vec<T, 1><<<grid, 256, 0, st>>>(rows, d, causal, sp, pp); break;
            case 2: softmax_fwd_vec<T, 2><<<grid, 256, 0, st>>>(rows, d, causal, sp, pp); break;
            case 4: softmax_fwd_vec<T, 4><<<grid, 256, 0, st>>>(rows, d, causal, sp, pp); break;
            case 8: softmax_fwd_vec<T, 8><<<grid, 256, 0, st>>>(rows, d, causal, sp, pp); break;
            default: softmax_fwd_vec<T, 16><<<grid, 256, 0, st>>>(rows, d, causal, sp, pp); break;
        }
    } else {
        softmax_fwd_scalar<T><<<grid, 256, 0, st>>>(rows, dim, causal, sp, pp);
    }
    return hipGetLastError();
}

template <typename T>
hipError_t bwd_impl(int64_t rows, int64_t dim, int64_t causal, const void* p, const void* dp, void* ds,
                    hipStream_t st) {
    const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const T* pp = static_cast<const T*>(p);
    const T* gp = static_cast<const T*>(dp);
    T* dsp = static_cast<T*>(ds);
    if (vec_ok<T>(dim)) {
        const int d = (int)dim;
        switch (vpl_for<T>(dim)) {
            case 1: softmax_bwd_vec<T, 1><<<grid, 256, 0, st>>>(rows, d, causal, pp, gp, dsp); break;
            case 2: softmax_bwd_vec<T, 2><<<grid, 256, 0, st>>>(rows, d, causal, pp, gp, dsp); break;
            case 4: softmax_bwd_vec<T, 4><<<grid, 256, 0, st>>>(rows, d, causal, pp, gp, dsp); break;
            case 8: softmax_bwd_vec<T, 8><<<grid, 256, 0, st>>>(rows, d, causal, pp, gp, dsp); break;
            default: softmax_bwd_vec<T, 16><<<grid, 256, 0, st>>>(rows, d, causal, pp, gp, dsp); break;
        }
    } else {
        softmax_bwd_scalar<T><<<grid, 256, 0, st>>>(rows, dim, causal, pp, gp, dsp);
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_softmax_fwd(int64_t rows, int64_t dim, int64_t causal_rows, int dtype,
                              const void* s, void* p, hipStream_t stream) {
    if (dtype == MC_F32) return fwd_impl<float>(rows, dim, causal_rows, s, p, stream);
    return fwd_impl<uint16_t>(rows, dim, causal_rows, s, p, stream);
}

hipError_t launch_softmax_bwd(int64_t rows, int64_t dim, int64_t causal_rows, int dtype,
                              const void* p, const void* dp, void* ds, hipStream_t stream) {
    if (dtype == MC_F32) return bwd_impl<float>(rows, dim, causal_rows, p, dp, ds, stream);
    return bwd_impl<uint16_t>(rows, dim, causal_rows, p, dp, ds, stream);
}

}  // namespace mc
