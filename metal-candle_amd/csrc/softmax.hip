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
// computed; the kernel writes exact zeros there. P and dS are written with
// non-temporal stores (whole 1 KB wave rows, not read again here): the
// [8,14,1024,1024] fp32 forward went 139 -> 109 us and the backward 187 ->
// 171 us, and the c4 step ran 0.5% faster (the kernels after the softmax no
// longer write back its lines). Offsets are 64-bit: a
// [4,28,4096,4096] score tensor has 1.9e9 elements. Longer rows (past 8
// vectors per lane) take one workgroup per row with the row in the
// registers of up to 1024 threads, and rows past that (128 KB) two
// streaming passes; rows that are not whole 16-byte vectors take a scalar
// kernel.
#include "common.hpp"
#include "kernels.hpp"

namespace mc {
namespace {

constexpr int kRowsPerBlock = 4;
// The backward vector kernel runs one row (one wave) per workgroup: on the
// causal fp32 scores [8, 14, 1024, 1024] it measured 179 -> 168 us against
// four rows per workgroup, while the forward is faster at four (108 us
// against 115 at one).
constexpr int kBwdRowsPerBlock = 1;
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
__global__ __launch_bounds__(256) void softmax_fwd_vec(int64_t rbase, int64_t rows, int dim, int64_t causal_rows,
                                                       const T* __restrict__ s, T* __restrict__ p) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    const int lane = lane_id();
    const int wave = wave_id();
    const int64_t r0 = rbase + (int64_t)blockIdx.x * kRowsPerBlock;
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
        BVec<T>::store_nt(rp, vi < nvec ? rowoff + (uint32_t)(vi * N * ES) : kOOB, o);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_fwd_scalar(int64_t rbase, int64_t rows, int64_t dim,
                                                          int64_t causal_rows, const T* __restrict__ s,
                                                          T* __restrict__ p) {
    const int lane = lane_id();
    const int64_t row = rbase + (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
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
__global__ __launch_bounds__(64 * kBwdRowsPerBlock) void softmax_bwd_vec(int64_t rbase, int64_t rows, int dim,
                                                                          int64_t causal_rows,
                                                                          const T* __restrict__ p,
                                                                          const T* __restrict__ dp,
                                                                          T* __restrict__ ds) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    const int lane = lane_id();
    const int wave = wave_id();
    const int64_t r0 = rbase + (int64_t)blockIdx.x * kBwdRowsPerBlock;
    const int64_t row = r0 + wave;
    if (row >= rows) return;
    const int64_t nrows = rows - r0 < kBwdRowsPerBlock ? rows - r0 : kBwdRowsPerBlock;
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
        BVec<T>::store_nt(rd, vi < nvec ? rowoff + (uint32_t)(vi * N * ES) : kOOB, o);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void softmax_bwd_scalar(int64_t rbase, int64_t rows, int64_t dim,
                                                          int64_t causal_rows, const T* __restrict__ p,
                                                          const T* __restrict__ dp, T* __restrict__ ds) {
    const int lane = lane_id();
    const int64_t row = rbase + (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
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

// ------------------------------------------------------------- wide rows
// Rows of more than 8 vectors per lane (fp32 past 2048 columns, bf16 past
// 4096): one workgroup of up to 1024 threads per row, vector v of the row
// held by thread v % blockDim.x, VPL vectors per thread, so the row is still
// read once and written once. Max, sum and dot combine the waves'
// butterflies in wave order through LDS. A row of up to 8 x 1024 vectors
// (32768 fp32 / 65536 bf16 columns, 128 KB) fits; one buffer resource per
// row.
constexpr int kWideThreads = 1024;

template <typename T, int VPL>
__global__ __launch_bounds__(kWideThreads) void softmax_fwd_wide(int64_t row0, int dim, int64_t causal_rows,
                                                                 const T* __restrict__ s, T* __restrict__ p) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    __shared__ float red[2][kMaxWaves];
    const int tid = threadIdx.x, nt = blockDim.x;
    const int64_t row = row0 + blockIdx.x;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(s + row * dim, (int64_t)dim * ES);
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(p + row * dim, (int64_t)dim * ES);
    const int nvec = dim / N;
    const int lim = (int)row_limit(row, dim, causal_rows);
    float v[VPL][N];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        const bool ok = vi < nvec && vi * N <= lim;
        BVec<T>::load(rs, ok ? (uint32_t)(vi * N * ES) : kOOB, v[i]);
    }
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            v[i][e] = (vi < nvec && vi * N + e <= lim) ? v[i][e] : -INFINITY;
            m = fmaxf(m, v[i][e]);
        }
    }
    m = wg_max(m, red[0]);
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float ex = fast_exp2((v[i][e] - m) * kLog2e);
            v[i][e] = ex;
            sum += ex;
        }
    sum = wg_sum(sum, red[1]);
    const float inv = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        float o[N];
#pragma unroll
        for (int e = 0; e < N; ++e) o[e] = v[i][e] * inv;
        BVec<T>::store_nt(rp, vi < nvec ? (uint32_t)(vi * N * ES) : kOOB, o);
    }
}

// p and dp stay packed (16-byte raw vectors) until use, which keeps a
// 1024-thread workgroup within its 128 registers per thread at VPL = 8.
template <typename T, int VPL>
__global__ __launch_bounds__(kWideThreads) void softmax_bwd_wide(int64_t row0, int dim, int64_t causal_rows,
                                                                 const T* __restrict__ p, const T* __restrict__ dp,
                                                                 T* __restrict__ ds) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    __shared__ float red[kMaxWaves];
    const int tid = threadIdx.x, nt = blockDim.x;
    const int64_t row = row0 + blockIdx.x;
    const __amdgpu_buffer_rsrc_t rp = make_rsrc(p + row * dim, (int64_t)dim * ES);
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(dp + row * dim, (int64_t)dim * ES);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(ds + row * dim, (int64_t)dim * ES);
    const int nvec = dim / N;
    const int lim = (int)row_limit(row, dim, causal_rows);
    i32x4 pq[VPL], gq[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        const uint32_t off = (vi < nvec && vi * N <= lim) ? (uint32_t)(vi * N * ES) : kOOB;
        pq[i] = buf_load16(rp, off);
        gq[i] = buf_load16(rg, off);
    }
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        float pv[N], gv[N];
        BVec<T>::unpack(pq[i], pv);
        BVec<T>::unpack(gq[i], gv);
#pragma unroll
        for (int e = 0; e < N; ++e) dot += ((vi < nvec && vi * N + e <= lim) ? pv[e] : 0.f) * gv[e];
    }
    dot = wg_sum(dot, red);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        float pv[N], gv[N], o[N];
        BVec<T>::unpack(pq[i], pv);
        BVec<T>::unpack(gq[i], gv);
#pragma unroll
        for (int e = 0; e < N; ++e) o[e] = ((vi < nvec && vi * N + e <= lim) ? pv[e] : 0.f) * (gv[e] - dot);
        BVec<T>::store_nt(rd, vi < nvec ? (uint32_t)(vi * N * ES) : kOOB, o);
    }
}

// ------------------------------------------------------------ stream rows
// Rows past the wide path's 128 KB (vector-aligned): one 1024-thread
// workgroup per row streams the row twice with 16-byte vectors, four in
// flight per thread. Forward: an online (max, sum) per thread (one rescale
// per vector, Milakov & Gimelshein's online normaliser), combined over the
// workgroup, then a second read that writes p. Backward: the dot product,
// then a second read of p and dp that writes ds. Wholly masked vectors are
// not read; 64-bit addressing throughout.
constexpr int kStreamUnroll = 4;

template <typename T>
__global__ __launch_bounds__(kWideThreads) void softmax_fwd_stream(int64_t row0, int64_t dim, int64_t causal_rows,
                                                                   const T* __restrict__ s, T* __restrict__ p) {
    constexpr int N = Vec16<T>::N;
    __shared__ float red[2][kMaxWaves];
    const int64_t tid = threadIdx.x, nt = blockDim.x;
    const int64_t row = row0 + blockIdx.x;
    const T* sr = s + row * dim;
    T* pr = p + row * dim;
    const int64_t nvec = dim / N;
    const int64_t lim = row_limit(row, dim, causal_rows);
    const int64_t nread = lim / N + 1;  // vectors holding an unmasked column
    float m = -INFINITY, sum = 0.f;
    for (int64_t c0 = tid; c0 < nread; c0 += nt * kStreamUnroll) {
        uint4 q[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t c = c0 + u * nt;
            q[u] = load16(sr, c * N, c < nread);
        }
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t c = c0 + u * nt;
            float v[N];
            BVec<T>::unpack(__builtin_bit_cast(i32x4, q[u]), v);
            float vm = -INFINITY;
#pragma unroll
            for (int e = 0; e < N; ++e) {
                v[e] = (c < nread && c * N + e <= lim) ? v[e] : -INFINITY;
                vm = fmaxf(vm, v[e]);
            }
            if (vm > m) {  // rescale the running sum to the new max (never from -inf to -inf)
                sum = m == -INFINITY ? 0.f : sum * fast_exp2((m - vm) * kLog2e);
                m = vm;
            }
            if (m != -INFINITY) {
#pragma unroll
                for (int e = 0; e < N; ++e) sum += fast_exp2((v[e] - m) * kLog2e);
            }
        }
    }
    const float gm = wg_max(m, red[0]);
    const float gs = wg_sum(m == -INFINITY ? 0.f : sum * fast_exp2((m - gm) * kLog2e), red[1]);
    const float inv = 1.0f / gs;
    for (int64_t c0 = tid; c0 < nvec; c0 += nt * kStreamUnroll) {
        uint4 q[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t c = c0 + u * nt;
            q[u] = load16(sr, c * N, c < nread);
        }
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t c = c0 + u * nt;
            if (c >= nvec) break;
            float v[N];
            BVec<T>::unpack(__builtin_bit_cast(i32x4, q[u]), v);
#pragma unroll
            for (int e = 0; e < N; ++e) v[e] = c * N + e <= lim ? fast_exp2((v[e] - gm) * kLog2e) * inv : 0.f;
            Vec16<T>::store(pr + c * N, v);
        }
    }
}

template <typename T>
__global__ __launch_bounds__(kWideThreads) void softmax_bwd_stream(int64_t row0, int64_t dim, int64_t causal_rows,
                                                                   const T* __restrict__ p, const T* __restrict__ dp,
                                                                   T* __restrict__ ds) {
    constexpr int N = Vec16<T>::N;
    __shared__ float red[kMaxWaves];
    const int64_t tid = threadIdx.x, nt = blockDim.x;
    const int64_t row = row0 + blockIdx.x;
    const T* pr = p + row * dim;
    const T* gr = dp + row * dim;
    T* dr = ds + row * dim;
    const int64_t nvec = dim / N;
    const int64_t lim = row_limit(row, dim, causal_rows);
    const int64_t nread = lim / N + 1;
    float dot = 0.f;
    for (int64_t c0 = tid; c0 < nread; c0 += nt * kStreamUnroll) {
        uint4 pq[kStreamUnroll], gq[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t c = c0 + u * nt;
            pq[u] = load16(pr, c * N, c < nread);
            gq[u] = load16(gr, c * N, c < nread);
        }
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t c = c0 + u * nt;
            float pv[N], gv[N];
            BVec<T>::unpack(__builtin_bit_cast(i32x4, pq[u]), pv);
            BVec<T>::unpack(__builtin_bit_cast(i32x4, gq[u]), gv);
#pragma unroll
            for (int e = 0; e < N; ++e) dot += (c * N + e <= lim ? pv[e] : 0.f) * gv[e];
        }
    }
    dot = wg_sum(dot, red);
    for (int64_t c0 = tid; c0 < nvec; c0 += nt * kStreamUnroll) {
        uint4 pq[kStreamUnroll], gq[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t c = c0 + u * nt;
            pq[u] = load16(pr, c * N, c < nread);
            gq[u] = load16(gr, c * N, c < nread);
        }
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const int64_t c = c0 + u * nt;
            if (c >= nvec) break;
            float pv[N], gv[N];
            BVec<T>::unpack(__builtin_bit_cast(i32x4, pq[u]), pv);
            BVec<T>::unpack(__builtin_bit_cast(i32x4, gq[u]), gv);
#pragma unroll
            for (int e = 0; e < N; ++e) pv[e] = c * N + e <= lim ? pv[e] * (gv[e] - dot) : 0.f;
            Vec16<T>::store(dr + c * N, pv);
        }
    }
}

// Row paths by length (rows of 16-byte vectors; ragged rows take the scalar
// kernels): one wave per row up to 8 vectors per lane, a workgroup per row
// up to max_vpl vectors per thread of 1024 threads, else two streaming
// passes. (One wave at 9-16 vectors per lane measured slower than the
// workgroup per row: bf16 [8192, 8192] backward 137 against 61 us, forward
// 48 against 44 us.) The bf16 backward holds at most 4 vectors of p and 4 of dp per
// thread: at 8 it needs more than the 128 registers a 1024-thread workgroup
// leaves each thread.
enum class RowPath { kScalar, kWave, kWide, kStream };

template <typename T>
RowPath row_path(int64_t dim, int max_vpl) {
    if (dim % Vec16<T>::N != 0) return RowPath::kScalar;
    const int64_t nvec = dim / Vec16<T>::N;
    if (nvec <= 8 * kWave) return RowPath::kWave;
    if (nvec <= (int64_t)max_vpl * kWideThreads) return RowPath::kWide;
    return RowPath::kStream;
}

// Vectors per thread and threads per workgroup of the wide path.
struct WideShape {
    int vpl, threads;
};
template <typename T>
WideShape wide_shape(int64_t dim) {
    const int64_t nvec = dim / Vec16<T>::N;
    const int vpl = nvec <= 2 * kWideThreads ? 2 : nvec <= 4 * kWideThreads ? 4 : 8;
    const int64_t per = (nvec + vpl - 1) / vpl;
    return {vpl, (int)((per + kWave - 1) / kWave * kWave)};
}

// Launches over the rows, rows_per_block rows per workgroup of `threads`
// threads, each launch at most 2^32 - 1 threads (a launch's thread count is
// 32-bit) and given its first row.
template <typename F>
void for_row_chunks(int64_t rows, int threads, F&& launch, int rows_per_block = 1) {
    const int64_t cap = (((int64_t)1 << 32) - 1) / threads * rows_per_block;
    for (int64_t r0 = 0; r0 < rows; r0 += cap) {
        const int64_t n = rows - r0 < cap ? rows - r0 : cap;
        launch(r0, dim3((unsigned)((n + rows_per_block - 1) / rows_per_block)));
    }
}

template <typename T>
int vpl_for(int64_t dim) {
    const int64_t nvec = dim / Vec16<T>::N;
    const int64_t per = (nvec + kWave - 1) / kWave;
    return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
}

template <typename T>
hipError_t fwd_impl(int64_t rows, int64_t dim, int64_t causal, const void* s, void* p, hipStream_t st) {
    const T* sp = static_cast<const T*>(s);
    T* pp = static_cast<T*>(p);
    const RowPath path = row_path<T>(dim, 8);
    if (path == RowPath::kWide) {
        const WideShape w = wide_shape<T>(dim);
        const int d = (int)dim;
        for_row_chunks(rows, w.threads, [&](int64_t r0, dim3 g) {
            switch (w.vpl) {
                case 2: softmax_fwd_wide<T, 2><<<g, w.threads, 0, st>>>(r0, d, causal, sp, pp); break;
                case 4: softmax_fwd_wide<T, 4><<<g, w.threads, 0, st>>>(r0, d, causal, sp, pp); break;
                default: softmax_fwd_wide<T, 8><<<g, w.threads, 0, st>>>(r0, d, causal, sp, pp); break;
            }
        });
    } else if (path == RowPath::kStream) {
        for_row_chunks(rows, kWideThreads, [&](int64_t r0, dim3 g) {
            softmax_fwd_stream<T><<<g, kWideThreads, 0, st>>>(r0, dim, causal, sp, pp);
        });
    } else if (path == RowPath::kWave) {
        const int d = (int)dim;
        const int vpl = vpl_for<T>(dim);
        for_row_chunks(rows, 256, [&](int64_t r0, dim3 g) {
            switch (vpl) {
                case 1: softmax_fwd_vec<T, 1><<<g, 256, 0, st>>>(r0, rows, d, causal, sp, pp); break;
                case 2: softmax_fwd_vec<T, 2><<<g, 256, 0, st>>>(r0, rows, d, causal, sp, pp); break;
                case 4: softmax_fwd_vec<T, 4><<<g, 256, 0, st>>>(r0, rows, d, causal, sp, pp); break;
                default: softmax_fwd_vec<T, 8><<<g, 256, 0, st>>>(r0, rows, d, causal, sp, pp); break;
            }
        }, kRowsPerBlock);
    } else {
        for_row_chunks(rows, 256, [&](int64_t r0, dim3 g) {
            softmax_fwd_scalar<T><<<g, 256, 0, st>>>(r0, rows, dim, causal, sp, pp);
        }, kRowsPerBlock);
    }
    return hipGetLastError();
}

template <typename T>
hipError_t bwd_impl(int64_t rows, int64_t dim, int64_t causal, const void* p, const void* dp, void* ds,
                    hipStream_t st) {
    const T* pp = static_cast<const T*>(p);
    const T* gp = static_cast<const T*>(dp);
    T* dsp = static_cast<T*>(ds);
    const RowPath path = row_path<T>(dim, sizeof(T) == 2 ? 4 : 8);
    if (path == RowPath::kWide) {
        const WideShape w = wide_shape<T>(dim);
        const int d = (int)dim;
        for_row_chunks(rows, w.threads, [&](int64_t r0, dim3 g) {
            switch (w.vpl) {
                case 2: softmax_bwd_wide<T, 2><<<g, w.threads, 0, st>>>(r0, d, causal, pp, gp, dsp); break;
                case 4: softmax_bwd_wide<T, 4><<<g, w.threads, 0, st>>>(r0, d, causal, pp, gp, dsp); break;
                default:
                    if constexpr (sizeof(T) == 4)
                        softmax_bwd_wide<T, 8><<<g, w.threads, 0, st>>>(r0, d, causal, pp, gp, dsp);
                    break;
            }
        });
    } else if (path == RowPath::kStream) {
        for_row_chunks(rows, kWideThreads, [&](int64_t r0, dim3 g) {
            softmax_bwd_stream<T><<<g, kWideThreads, 0, st>>>(r0, dim, causal, pp, gp, dsp);
        });
    } else if (path == RowPath::kWave) {
        const int d = (int)dim;
        const int vpl = vpl_for<T>(dim);
        constexpr int nt = 64 * kBwdRowsPerBlock;
        for_row_chunks(rows, nt, [&](int64_t r0, dim3 g) {
            switch (vpl) {
                case 1: softmax_bwd_vec<T, 1><<<g, nt, 0, st>>>(r0, rows, d, causal, pp, gp, dsp); break;
                case 2: softmax_bwd_vec<T, 2><<<g, nt, 0, st>>>(r0, rows, d, causal, pp, gp, dsp); break;
                case 4: softmax_bwd_vec<T, 4><<<g, nt, 0, st>>>(r0, rows, d, causal, pp, gp, dsp); break;
                default: softmax_bwd_vec<T, 8><<<g, nt, 0, st>>>(r0, rows, d, causal, pp, gp, dsp); break;
            }
        }, kBwdRowsPerBlock);
    } else {
        for_row_chunks(rows, 256, [&](int64_t r0, dim3 g) {
            softmax_bwd_scalar<T><<<g, 256, 0, st>>>(r0, rows, dim, causal, pp, gp, dsp);
        }, kRowsPerBlock);
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
