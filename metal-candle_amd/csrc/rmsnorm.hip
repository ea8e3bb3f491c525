// RMSNorm forward / backward for gfx950.
//
// Semantics follow the candle composite the reference uses on CPU:
//   src/backend/tensor.rs:111-117   x / sqrt(mean(x^2) + eps)
//   src/models/qwen.rs:314-325      ... * weight
// and replace the Metal kernel fused_rms_norm (src/backend/kernels.metal:281-330),
// which reduces a whole row with one thread (dispatch grid (1, seq, batch),
// custom_ops.rs:602-617).
//
// Design: one wave64 per row. A row of `dim` elements is held in registers as
// VPL 16-byte vectors per lane (vector v of the row goes to lane v % 64), so
// x is read from HBM exactly once; the sum of squares is a DPP butterfly.
// The backward reduces dw over rows in two fixed-order stages (per-block
// partials in the workspace, then a column sum), so it is bitwise
// reproducible. Longer rows take a workgroup of up to 1024 threads per row
// (forward) or per block of rows (backward), the row still held in
// registers; rows whose length is not a multiple of the vector width, or
// past those paths (forward 32768 fp32 / 65536 bf16 columns, backward 16384
// / 16384), use a scalar variant that reads x twice.
#include <mutex>

#include "column_sum.hpp"
#include "common.hpp"
#include "kernels.hpp"

// Scratch of mc_rmsnorm_bwd_noalloc: the per-block dw partials
// [rmsnorm_bwd_blocks][dim] fp32 that mc_rmsnorm_bwd keeps in the caller's
// workspace. Each device holds its own copy for the life of the process.
// Every element a call reads was written by the same call, so nothing in it
// needs clearing. Calls that overlap on one device race on it.
static __device__ __align__(256) float scratch[mc::kRmsNormScratchBytes / sizeof(float)];

namespace mc {

hipError_t rmsnorm_scratch(float** out) {
    // The host-side name `scratch` is not a device address: the device copy is
    // found once per device with hipGetSymbolAddress, with that device current
    // (it is the caller's current device here), and only that address is used.
    constexpr int kMaxDevices = 64;
    static std::mutex mu;
    static float* ptrs[kMaxDevices] = {};
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(mu);
    if (!ptrs[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        ptrs[dev] = static_cast<float*>(p);
    }
    *out = ptrs[dev];
    return hipSuccess;
}

namespace {

constexpr int kRowsPerBlock = 4;  // waves (rows) per 256-thread workgroup

// ------------------------------------------------------------- forward
// Vector path: the workgroup's 4 rows through one buffer resource (a wave's
// row at a scalar byte offset); the row and the weight are loaded before any
// use, vectors past the row through out-of-range offsets (zeros, stores
// dropped) instead of branches.
template <typename T, int VPL>
__global__ __launch_bounds__(256) void rmsnorm_fwd_vec(int64_t rows, int dim, float eps,
                                                       const T* __restrict__ x,
                                                       const T* __restrict__ w,
                                                       T* __restrict__ y,
                                                       float* __restrict__ rstd) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    const int lane = lane_id();
    const int wave = wave_id();
    const int64_t r0 = (int64_t)blockIdx.x * kRowsPerBlock;
    const int64_t row = r0 + wave;
    if (row >= rows) return;
    const int64_t nrows = rows - r0 < kRowsPerBlock ? rows - r0 : kRowsPerBlock;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + r0 * dim, nrows * dim * ES);
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(y + r0 * dim, nrows * dim * ES);
    const bool hw = w != nullptr;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, hw ? (int64_t)dim * ES : 0);
    const int nvec = dim / N;
    const uint32_t rowoff = (uint32_t)(wave * dim * ES);
    float v[VPL][N], wv[VPL][N];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
        const uint32_t off = vi < nvec ? (uint32_t)(vi * N * ES) : kOOB;
        BVec<T>::load(rx, off == kOOB ? kOOB : rowoff + off, v[i]);
        BVec<T>::load(rw, off, wv[i]);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int e = 0; e < N; ++e) ss += v[i][e] * v[i][e];
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)dim + eps);
    if (rstd && lane == 0) rstd[row] = r;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
        float o[N];
#pragma unroll
        for (int e = 0; e < N; ++e) o[e] = v[i][e] * r * (hw ? wv[i][e] : 1.f);
        BVec<T>::store(ry, vi < nvec ? rowoff + (uint32_t)(vi * N * ES) : kOOB, o);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void rmsnorm_fwd_scalar(int64_t rows, int64_t dim, float eps,
                                                          const T* __restrict__ x,
                                                          const T* __restrict__ w,
                                                          T* __restrict__ y,
                                                          float* __restrict__ rstd) {
    const int lane = lane_id();
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const T* xr = x + row * dim;
    float ss = 0.f;
    for (int64_t j = lane; j < dim; j += kWave) {
        float a = Elem<T>::load(xr, j);
        ss += a * a;
    }
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / (float)dim + eps);
    if (rstd && lane == 0) rstd[row] = r;
    for (int64_t j = lane; j < dim; j += kWave) {
        float o = Elem<T>::load(xr, j) * r;
        if (w) o *= Elem<T>::load(w, j);
        Elem<T>::store(y + row * dim, j, o);
    }
}

// ------------------------------------------------------------ backward
// Block b owns rows [b*chunk, min(rows, (b+1)*chunk)); wave k of the block
// takes rows k, k+4, ... of that range in order. dw partials: per lane in registers,
// accumulated in row order, then summed over the 4 waves in LDS in wave
// order, written to partial[b][dim].
template <typename T, int VPL, bool DW>
__global__ __launch_bounds__(256) void rmsnorm_bwd_vec(int64_t rows, int dim, float eps, int64_t chunk,
                                                       const T* __restrict__ x,
                                                       const T* __restrict__ w,
                                                       const float* __restrict__ rstd,
                                                       const T* __restrict__ dy,
                                                       T* __restrict__ dx,
                                                       float* __restrict__ partial) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    const int lane = lane_id();
    const int wave = wave_id();
    const int nvec = dim / N;
    const int64_t r0 = (int64_t)blockIdx.x * chunk;
    const int64_t r1 = r0 + chunk < rows ? r0 + chunk : rows;
    const int64_t nr = r1 > r0 ? r1 - r0 : 0;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + r0 * dim, nr * dim * ES);
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(dy + r0 * dim, nr * dim * ES);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(dx + r0 * dim, nr * dim * ES);
    const bool hw = w != nullptr;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, hw ? (int64_t)dim * ES : 0);
    float wv[VPL][N];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
        BVec<T>::load(rw, vi < nvec ? (uint32_t)(vi * N * ES) : kOOB, wv[i]);
#pragma unroll
        for (int e = 0; e < N; ++e) wv[i][e] = hw ? wv[i][e] : 1.f;
    }
    float acc[DW ? VPL : 1][N];
#pragma unroll
    for (int i = 0; i < (DW ? VPL : 1); ++i)
#pragma unroll
        for (int e = 0; e < N; ++e) acc[i][e] = 0.f;

    // Software pipeline, one row in flight: the raw 16-byte vectors of the
    // wave's next row are requested before the current row is used (bf16
    // rows stay packed until use, which halves the registers they hold).
    auto load_row = [&](int64_t q, i32x4 (&xq)[VPL], i32x4 (&gq)[VPL]) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int vi = lane + i * kWave;
            const uint32_t off = vi < nvec ? (uint32_t)((q * dim + vi * N) * ES) : kOOB;
            xq[i] = buf_load16(rx, off);
            gq[i] = buf_load16(rg, off);
        }
    };
    i32x4 nx[VPL], ng[VPL];
    if (wave < nr) load_row(wave, nx, ng);
    for (int64_t q = wave; q < nr; q += kRowsPerBlock) {
        i32x4 xq[VPL], gq[VPL];
#pragma unroll
        for (int i = 0; i < VPL; ++i) { xq[i] = nx[i]; gq[i] = ng[i]; }
        if (q + kRowsPerBlock < nr) load_row(q + kRowsPerBlock, nx, ng);  // wave-uniform
        float ss = 0.f, gx = 0.f;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            float xv[N], gv[N];
            BVec<T>::unpack(xq[i], xv);
            BVec<T>::unpack(gq[i], gv);
#pragma unroll
            for (int e = 0; e < N; ++e) {
                ss += xv[e] * xv[e];
                gx += gv[e] * wv[i][e] * xv[e];
            }
        }
        float r;
        if (rstd) {
            r = rstd[r0 + q];
            gx = wave_sum(gx);
        } else {
            ss = wave_sum(ss);
            gx = wave_sum(gx);
            r = 1.0f / sqrtf(ss / (float)dim + eps);
        }
        const float c = r * r * r * gx / (float)dim;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int vi = lane + i * kWave;
            float xv[N], gv[N], o[N];
            BVec<T>::unpack(xq[i], xv);
            BVec<T>::unpack(gq[i], gv);
#pragma unroll
            for (int e = 0; e < N; ++e) o[e] = r * gv[e] * wv[i][e] - xv[e] * c;
            BVec<T>::store(rd, vi < nvec ? (uint32_t)((q * dim + vi * N) * ES) : kOOB, o);
            if constexpr (DW) {
#pragma unroll
                for (int e = 0; e < N; ++e) acc[i][e] += gv[e] * xv[e] * r;
            }
        }
    }
    if constexpr (DW) {
        // Fixed-order combine of the 4 waves' partials through LDS.
        extern __shared__ float lds[];  // [kRowsPerBlock][dim]
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int vi = lane + i * kWave;
            if (vi < nvec)
#pragma unroll
                for (int e = 0; e < N; ++e) lds[wave * dim + vi * N + e] = acc[i][e];
        }
        __syncthreads();
        for (int j = threadIdx.x; j < dim; j += blockDim.x) {
            float s = lds[j];
#pragma unroll
            for (int k = 1; k < kRowsPerBlock; ++k) s += lds[k * dim + j];
            partial[(int64_t)blockIdx.x * dim + j] = s;
        }
    }
}

template <typename T, bool DW>
__global__ __launch_bounds__(256) void rmsnorm_bwd_scalar(int64_t rows, int64_t dim, float eps,
                                                          int64_t chunk, const T* __restrict__ x,
                                                          const T* __restrict__ w,
                                                          const float* __restrict__ rstd,
                                                          const T* __restrict__ dy,
                                                          T* __restrict__ dx,
                                                          float* __restrict__ partial) {
    // Rows of the block's range are walked in order by the whole workgroup:
    // the row sums are combined over the 4 waves through LDS in wave order,
    // and each thread owns columns j = tid, tid+256, ... of the block's dw
    // partial, which it accumulates in place in the workspace.
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * chunk;
    const int64_t r1 = r0 + chunk < rows ? r0 + chunk : rows;
    __shared__ float red[2][kRowsPerBlock];
    float* part = partial + (int64_t)blockIdx.x * dim;
    if constexpr (DW) {
        for (int64_t j = threadIdx.x; j < dim; j += blockDim.x) part[j] = 0.f;
    }
    for (int64_t row = r0; row < r1; ++row) {
        const T* xr = x + row * dim;
        const T* gr = dy + row * dim;
        float ss = 0.f, gx = 0.f;
        for (int64_t j = threadIdx.x; j < dim; j += blockDim.x) {
            float a = Elem<T>::load(xr, j);
            float g = Elem<T>::load(gr, j) * (w ? Elem<T>::load(w, j) : 1.f);
            ss += a * a;
            gx += g * a;
        }
        ss = wave_sum(ss);
        gx = wave_sum(gx);
        if (lane == 0) { red[0][wave] = ss; red[1][wave] = gx; }
        __syncthreads();
        ss = red[0][0]; gx = red[1][0];
#pragma unroll
        for (int k = 1; k < kRowsPerBlock; ++k) { ss += red[0][k]; gx += red[1][k]; }
        __syncthreads();
        const float r = rstd ? rstd[row] : 1.0f / sqrtf(ss / (float)dim + eps);
        const float c = r * r * r * gx / (float)dim;
        for (int64_t j = threadIdx.x; j < dim; j += blockDim.x) {
            float a = Elem<T>::load(xr, j);
            float gy = Elem<T>::load(gr, j);
            float g = gy * (w ? Elem<T>::load(w, j) : 1.f);
            Elem<T>::store(dx + row * dim, j, r * g - a * c);
            if constexpr (DW) part[j] += gy * a * r;
        }
    }
}

// ------------------------------------------------------------- wide rows
// Rows past the one-wave paths (forward: more than 8 vectors per lane, fp32
// past 2048 / bf16 past 4096 columns; backward: more than 4): a
// workgroup of up to 1024 threads per row (forward) or per block of rows
// (backward), vector v of a row held by thread v % blockDim.x, so x and dy
// are still read once. The row sums combine the waves' butterflies in wave
// order through LDS.
constexpr int kWideThreads = 1024;

template <typename T, int VPL>
__global__ __launch_bounds__(kWideThreads) void rmsnorm_fwd_wide(int64_t row0, int dim, float eps,
                                                                 const T* __restrict__ x, const T* __restrict__ w,
                                                                 T* __restrict__ y, float* __restrict__ rstd) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    __shared__ float red[kMaxWaves];
    const int tid = threadIdx.x, nt = blockDim.x;
    const int64_t row = row0 + blockIdx.x;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + row * dim, (int64_t)dim * ES);
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(y + row * dim, (int64_t)dim * ES);
    const bool hw = w != nullptr;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, hw ? (int64_t)dim * ES : 0);
    const int nvec = dim / N;
    // x and w stay packed until use (64 registers at VPL = 8 in bf16)
    i32x4 xq[VPL], wq[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        const uint32_t off = vi < nvec ? (uint32_t)(vi * N * ES) : kOOB;
        xq[i] = buf_load16(rx, off);
        wq[i] = buf_load16(rw, off);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        float v[N];
        BVec<T>::unpack(xq[i], v);
#pragma unroll
        for (int e = 0; e < N; ++e) ss += v[e] * v[e];
    }
    ss = wg_sum(ss, red);
    const float r = 1.0f / sqrtf(ss / (float)dim + eps);
    if (rstd && tid == 0) rstd[row] = r;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        float v[N], wv[N], o[N];
        BVec<T>::unpack(xq[i], v);
        BVec<T>::unpack(wq[i], wv);
#pragma unroll
        for (int e = 0; e < N; ++e) o[e] = v[e] * r * (hw ? wv[e] : 1.f);
        BVec<T>::store(ry, vi < nvec ? (uint32_t)(vi * N * ES) : kOOB, o);
    }
}

// Block b owns rows [b*chunk, min(rows, (b+1)*chunk)) and walks them in
// order with the whole workgroup, the next row's loads issued before the
// current row is used. Each thread owns the columns of its vectors, so its
// dw partial accumulates in registers in row order and is written to
// partial[b][dim] as it is. The two row sums of a row share one LDS round
// (slots alternate between rows, so one barrier per row suffices).
template <typename T, int VPL, bool DW>
__global__ __launch_bounds__(kWideThreads) void rmsnorm_bwd_wide(int64_t rows, int dim, float eps, int64_t chunk,
                                                                 const T* __restrict__ x, const T* __restrict__ w,
                                                                 const float* __restrict__ rstd,
                                                                 const T* __restrict__ dy, T* __restrict__ dx,
                                                                 float* __restrict__ partial) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    __shared__ float red[2][2][kMaxWaves];
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = lane_id(), wave = wave_id(), nw = nt >> 6;
    const int nvec = dim / N;
    const int64_t r0 = (int64_t)blockIdx.x * chunk;
    const int64_t r1 = r0 + chunk < rows ? r0 + chunk : rows;
    const int64_t nr = r1 > r0 ? r1 - r0 : 0;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + r0 * dim, nr * dim * ES);
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(dy + r0 * dim, nr * dim * ES);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(dx + r0 * dim, nr * dim * ES);
    const bool hw = w != nullptr;
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, hw ? (int64_t)dim * ES : 0);
    float wv[VPL][N];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        BVec<T>::load(rw, vi < nvec ? (uint32_t)(vi * N * ES) : kOOB, wv[i]);
#pragma unroll
        for (int e = 0; e < N; ++e) wv[i][e] = hw ? wv[i][e] : 1.f;
    }
    float acc[DW ? VPL : 1][N];
#pragma unroll
    for (int i = 0; i < (DW ? VPL : 1); ++i)
#pragma unroll
        for (int e = 0; e < N; ++e) acc[i][e] = 0.f;
    auto load_row = [&](int64_t q, i32x4 (&xq)[VPL], i32x4 (&gq)[VPL]) {
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int vi = tid + i * nt;
            const uint32_t off = vi < nvec ? (uint32_t)((q * dim + vi * N) * ES) : kOOB;
            xq[i] = buf_load16(rx, off);
            gq[i] = buf_load16(rg, off);
        }
    };
    i32x4 nx[VPL], ng[VPL];
    if (nr > 0) load_row(0, nx, ng);
    for (int64_t q = 0; q < nr; ++q) {
        i32x4 xq[VPL], gq[VPL];
#pragma unroll
        for (int i = 0; i < VPL; ++i) { xq[i] = nx[i]; gq[i] = ng[i]; }
        if (q + 1 < nr) load_row(q + 1, nx, ng);  // workgroup-uniform
        float ss = 0.f, gx = 0.f;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            float xv[N], gv[N];
            BVec<T>::unpack(xq[i], xv);
            BVec<T>::unpack(gq[i], gv);
#pragma unroll
            for (int e = 0; e < N; ++e) {
                ss += xv[e] * xv[e];
                gx += gv[e] * wv[i][e] * xv[e];
            }
        }
        const int slot = (int)(q & 1);
        if (!rstd) ss = wave_sum(ss);
        gx = wave_sum(gx);
        if (lane == 0) { red[slot][0][wave] = ss; red[slot][1][wave] = gx; }
        __syncthreads();
        gx = red[slot][1][0];
        for (int k = 1; k < nw; ++k) gx += red[slot][1][k];
        float r;
        if (rstd) {
            r = rstd[r0 + q];
        } else {
            ss = red[slot][0][0];
            for (int k = 1; k < nw; ++k) ss += red[slot][0][k];
            r = 1.0f / sqrtf(ss / (float)dim + eps);
        }
        const float c = r * r * r * gx / (float)dim;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int vi = tid + i * nt;
            float xv[N], gv[N], o[N];
            BVec<T>::unpack(xq[i], xv);
            BVec<T>::unpack(gq[i], gv);
#pragma unroll
            for (int e = 0; e < N; ++e) o[e] = r * gv[e] * wv[i][e] - xv[e] * c;
            BVec<T>::store(rd, vi < nvec ? (uint32_t)((q * dim + vi * N) * ES) : kOOB, o);
            if constexpr (DW) {
#pragma unroll
                for (int e = 0; e < N; ++e) acc[i][e] += gv[e] * xv[e] * r;
            }
        }
    }
    if constexpr (DW) {
        float* part = partial + (int64_t)blockIdx.x * dim;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int vi = tid + i * nt;
            if (vi < nvec)
#pragma unroll
                for (int e = 0; e < N; ++e) part[vi * N + e] = acc[i][e];
        }
    }
}

// One wave per row up to 8 vectors per lane (4096 bf16 / 2048 fp32 columns).
// At 9-16 vectors per lane the workgroup per row measured faster in the
// forward (bf16 [16384, 5120] 74 -> 55 us, [16384, 8192] 96 -> 82 us).
template <typename T>
bool vec_ok(int64_t dim) {
    return dim % Vec16<T>::N == 0 && dim / Vec16<T>::N <= 8 * kWave;
}

// Vectors per thread of the wide paths: forward up to 8 (x and w packed),
// backward up to 2 (bf16) or 4 (fp32): the backward holds w and the dw
// partial unpacked beside two rows of packed x and dy.
template <typename T>
int wide_fwd_vpl(int64_t dim) {
    if (dim % Vec16<T>::N != 0) return 0;
    const int64_t nvec = dim / Vec16<T>::N;
    return nvec <= 2 * kWideThreads ? 2 : nvec <= 4 * kWideThreads ? 4 : nvec <= 8 * kWideThreads ? 8 : 0;
}
template <typename T>
int wide_bwd_vpl(int64_t dim) {
    if (dim % Vec16<T>::N != 0) return 0;
    const int64_t nvec = dim / Vec16<T>::N;
    const int cap = sizeof(T) == 2 ? 2 : 4;
    for (int v = 1; v <= cap; v *= 2)
        if (nvec <= (int64_t)v * kWideThreads) return v;
    return 0;
}
template <typename T>
int wide_threads(int64_t dim, int vpl) {
    const int64_t per = (dim / Vec16<T>::N + vpl - 1) / vpl;
    return (int)((per + kWave - 1) / kWave * kWave);
}

template <typename T>
int vpl_for(int64_t dim) {
    const int64_t nvec = dim / Vec16<T>::N;
    const int64_t per = (nvec + kWave - 1) / kWave;
    return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
}

template <typename T>
hipError_t fwd_impl(int64_t rows, int64_t dim, float eps, const void* x, const void* w, void* y,
                    float* rstd, hipStream_t stream) {
    const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const T* xp = static_cast<const T*>(x);
    const T* wp = static_cast<const T*>(w);
    T* yp = static_cast<T*>(y);
    const int wvpl = vec_ok<T>(dim) ? 0 : wide_fwd_vpl<T>(dim);
    if (wvpl) {
        const int nt = wide_threads<T>(dim, wvpl);
        const int d = (int)dim;
        const int64_t cap = (((int64_t)1 << 32) - 1) / nt;  // a launch's thread count is 32-bit
        for (int64_t r0 = 0; r0 < rows; r0 += cap) {
            const dim3 g((unsigned)(rows - r0 < cap ? rows - r0 : cap));
            switch (wvpl) {
                case 2: rmsnorm_fwd_wide<T, 2><<<g, nt, 0, stream>>>(r0, d, eps, xp, wp, yp, rstd); break;
                case 4: rmsnorm_fwd_wide<T, 4><<<g, nt, 0, stream>>>(r0, d, eps, xp, wp, yp, rstd); break;
                default: rmsnorm_fwd_wide<T, 8><<<g, nt, 0, stream>>>(r0, d, eps, xp, wp, yp, rstd); break;
            }
        }
    } else if (vec_ok<T>(dim)) {
        const int d = (int)dim;
        switch (vpl_for<T>(dim)) {
            case 1: rmsnorm_fwd_vec<T, 1><<<grid, 256, 0, stream>>>(rows, d, eps, xp, wp, yp, rstd); break;
            case 2: rmsnorm_fwd_vec<T, 2><<<grid, 256, 0, stream>>>(rows, d, eps, xp, wp, yp, rstd); break;
            case 4: rmsnorm_fwd_vec<T, 4><<<grid, 256, 0, stream>>>(rows, d, eps, xp, wp, yp, rstd); break;
            default: rmsnorm_fwd_vec<T, 8><<<grid, 256, 0, stream>>>(rows, d, eps, xp, wp, yp, rstd); break;
        }
    } else {
        rmsnorm_fwd_scalar<T><<<grid, 256, 0, stream>>>(rows, dim, eps, xp, wp, yp, rstd);
    }
    return hipGetLastError();
}

template <typename T, bool DW>
void bwd_vec_launch(int vpl, dim3 grid, size_t lds, hipStream_t s, int64_t rows, int d, float eps,
                    int64_t chunk, const T* x, const T* w, const float* rstd, const T* dy, T* dx,
                    float* part) {
    switch (vpl) {
        case 1: rmsnorm_bwd_vec<T, 1, DW><<<grid, 256, lds, s>>>(rows, d, eps, chunk, x, w, rstd, dy, dx, part); break;
        case 2: rmsnorm_bwd_vec<T, 2, DW><<<grid, 256, lds, s>>>(rows, d, eps, chunk, x, w, rstd, dy, dx, part); break;
        default: rmsnorm_bwd_vec<T, 4, DW><<<grid, 256, lds, s>>>(rows, d, eps, chunk, x, w, rstd, dy, dx, part); break;
    }
}

template <typename T, bool DW>
void bwd_wide_launch(int vpl, dim3 grid, int nt, hipStream_t s, int64_t rows, int d, float eps, int64_t chunk,
                     const T* x, const T* w, const float* rstd, const T* dy, T* dx, float* part) {
    switch (vpl) {
        case 1: rmsnorm_bwd_wide<T, 1, DW><<<grid, nt, 0, s>>>(rows, d, eps, chunk, x, w, rstd, dy, dx, part); break;
        case 2: rmsnorm_bwd_wide<T, 2, DW><<<grid, nt, 0, s>>>(rows, d, eps, chunk, x, w, rstd, dy, dx, part); break;
        default:
            if constexpr (sizeof(T) == 4)
                rmsnorm_bwd_wide<T, 4, DW><<<grid, nt, 0, s>>>(rows, d, eps, chunk, x, w, rstd, dy, dx, part);
            break;
    }
}

template <typename T>
hipError_t bwd_impl(int64_t rows, int64_t dim, float eps, const void* x, const void* w,
                    const float* rstd, const void* dy, void* dx, float* dw, float* partial,
                    hipStream_t stream) {
    const int nb = rmsnorm_bwd_blocks(rows, dim);
    const int64_t chunk = (rows + nb - 1) / nb;
    const dim3 grid((unsigned)nb);
    const T* xp = static_cast<const T*>(x);
    const T* wp = static_cast<const T*>(w);
    const T* gp = static_cast<const T*>(dy);
    T* dxp = static_cast<T*>(dx);
    // One wave per row up to 4 vectors per lane (2048 bf16 / 1024 fp32
    // columns); the workgroup per row block past that (at 5-8 vectors per
    // lane it measured faster: bf16 [16384, 3584] 75.5 -> 68.4 us), to 2048
    // (bf16) or 4096 (fp32) vectors per row; the scalar kernel beyond.
    if (vec_ok<T>(dim) && vpl_for<T>(dim) <= 4 && (!dw || dim * kRowsPerBlock * sizeof(float) <= 64 * 1024)) {
        const int vpl = vpl_for<T>(dim);
        if (dw)
            bwd_vec_launch<T, true>(vpl, grid, dim * kRowsPerBlock * sizeof(float), stream, rows, (int)dim,
                                    eps, chunk, xp, wp, rstd, gp, dxp, partial);
        else
            bwd_vec_launch<T, false>(vpl, grid, 0, stream, rows, (int)dim, eps, chunk, xp, wp, rstd, gp,
                                     dxp, nullptr);
    } else if (const int wvpl = wide_bwd_vpl<T>(dim)) {
        const int nt = wide_threads<T>(dim, wvpl);
        if (dw)
            bwd_wide_launch<T, true>(wvpl, grid, nt, stream, rows, (int)dim, eps, chunk, xp, wp, rstd, gp, dxp,
                                     partial);
        else
            bwd_wide_launch<T, false>(wvpl, grid, nt, stream, rows, (int)dim, eps, chunk, xp, wp, rstd, gp, dxp,
                                      nullptr);
    } else if (dw) {
        rmsnorm_bwd_scalar<T, true><<<grid, 256, 0, stream>>>(rows, dim, eps, chunk, xp, wp, rstd, gp, dxp, partial);
    } else {
        rmsnorm_bwd_scalar<T, false><<<grid, 256, 0, stream>>>(rows, dim, eps, chunk, xp, wp, rstd, gp, dxp, nullptr);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !dw) return e;
    const dim3 sgrid((unsigned)((dim + kSumCols - 1) / kSumCols));
    if (dim % 4 == 0 && (reinterpret_cast<uintptr_t>(partial) & 15) == 0)
        column_sum<true><<<sgrid, 256, 0, stream>>>(nb, dim, partial, dw);
    else
        column_sum<false><<<sgrid, 256, 0, stream>>>(nb, dim, partial, dw);
    return hipGetLastError();
}

}  // namespace

int rmsnorm_bwd_blocks(int64_t rows, int64_t dim) {
    (void)dim;
    // ~2 workgroups per CU of the 256-CU part, at least 8 rows per block.
    int64_t nb = (rows + 7) / 8;
    if (nb > 512) nb = 512;
    if (nb < 1) nb = 1;
    return (int)nb;
}

hipError_t launch_rmsnorm_fwd(int64_t rows, int64_t dim, float eps, int dtype, const void* x,
                              const void* w, void* y, float* rstd, hipStream_t stream) {
    if (dtype == MC_F32) return fwd_impl<float>(rows, dim, eps, x, w, y, rstd, stream);
    return fwd_impl<uint16_t>(rows, dim, eps, x, w, y, rstd, stream);
}

hipError_t launch_rmsnorm_bwd(int64_t rows, int64_t dim, float eps, int dtype, const void* x,
                              const void* w, const float* rstd, const void* dy, void* dx, float* dw,
                              float* partial, hipStream_t stream) {
    if (dtype == MC_F32) return bwd_impl<float>(rows, dim, eps, x, w, rstd, dy, dx, dw, partial, stream);
    return bwd_impl<uint16_t>(rows, dim, eps, x, w, rstd, dy, dx, dw, partial, stream);
}

}  // namespace mc
