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
// reproducible. Rows whose length is not a multiple of the vector width
// use a scalar variant that reads x twice.
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
hipError_t fwd_impl(int64_t rows, int64_t dim, float eps, const void* x, const void* w, void* y,
                    float* rstd, hipStream_t stream) {
    const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const T* xp = static_cast<const T*>(x);
    const T* wp = static_cast<const T*>(w);
    T* yp = static_cast<T*>(y);
    if (vec_ok<T>(dim)) {
        const int d = (int)dim;
        switch (vpl_for<T>(dim)) {
            case 1: rmsnorm_fwd_vec<T, 1><<<grid, 256, 0, stream>>>(rows, d, eps, xp, wp, yp, rstd); break;
            case 2: rmsnorm_fwd_vec<T, 2><<<grid, 256, 0, stream>>>(rows, d, eps, xp, wp, yp, rstd); break;
            case 4: rmsnorm_fwd_vec<T, 4><<<grid, 256, 0, stream>>>(rows, d, eps, xp, wp, yp, rstd); break;
            case 8: rmsnorm_fwd_vec<T, 8><<<grid, 256, 0, stream>>>(rows, d, eps, xp, wp, yp, rstd); break;
            default: rmsnorm_fwd_vec<T, 16><<<grid, 256, 0, stream>>>(rows, d, eps, xp, wp, yp, rstd); break;
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
        case 4: rmsnorm_bwd_vec<T, 4, DW><<<grid, 256, lds, s>>>(rows, d, eps, chunk, x, w, rstd, dy, dx, part); break;
        default: rmsnorm_bwd_vec<T, 8, DW><<<grid, 256, lds, s>>>(rows, d, eps, chunk, x, w, rstd, dy, dx, part); break;
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
    // The backward keeps x, dy, w (and the dw partials) of a row in registers:
    // up to 8 vectors per lane (4096 bf16 / 2048 fp32 columns).
    if (vec_ok<T>(dim) && vpl_for<T>(dim) <= 8 && (!dw || dim * kRowsPerBlock * sizeof(float) <= 64 * 1024)) {
        const int vpl = vpl_for<T>(dim);
        if (dw)
            bwd_vec_launch<T, true>(vpl, grid, dim * kRowsPerBlock * sizeof(float), stream, rows, (int)dim,
                                    eps, chunk, xp, wp, rstd, gp, dxp, partial);
        else
            bwd_vec_launch<T, false>(vpl, grid, 0, stream, rows, (int)dim, eps, chunk, xp, wp, rstd, gp,
                                     dxp, nullptr);
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
