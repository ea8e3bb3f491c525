// Row kernels next to the hot path, gfx950: LayerNorm, log-softmax and the
// cross-entropy loss that feeds the layer's output gradient.
//
// LayerNorm (LayerNormOp, src/backend/custom_ops.rs:826-1079; the CPU path of
// its cpu_fwd and TensorExt::layer_norm, src/backend/tensor.rs:100-109;
// MetalLayerNorm's weight and bias, src/embeddings/metal_bert.rs:30-72):
//   mean = sum(x) / D, var = sum((x - mean)^2) / D (two passes, as cpu_fwd),
//   y = (x - mean) / sqrt(var + eps) * w + b.
// One wave per row with the row held in registers (16-byte vectors), as the
// RMSNorm kernels; the backward reduces dw and db over rows in two
// fixed-order stages. Longer rows take a workgroup per row (forward) or per
// block of rows (backward) with the row still in registers; rows that fit
// neither, or are not whole 16-byte vectors, use a scalar path.
//
// log-softmax (candle_nn::ops::log_softmax as cross_entropy_loss calls it,
// src/training/loss.rs:108): y = (x - max) - log(sum(exp(x - max))).
// Cross entropy (cross_entropy_loss, loss.rs:58-148; label smoothing,
// loss.rs:208-245): per row the log-sum-exp and log p[target]; the mean over
// the rows whose target is not ignore_index, negated; with smoothing s,
// (1 - s) * that + s * (-mean of every log-probability of every row).
// Vocabulary rows are long (10^5 entries), so these use one 256-thread
// workgroup per row with an online (max, sum) per thread, combined in a
// fixed order. The loss is a second, single-workgroup pass over the per-row
// values in row order, so it is bitwise reproducible.
#include "column_sum.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace mc {
namespace {

constexpr int kRowsPerBlock = 4;
constexpr float kNegInf = -__builtin_inff();

// ---------------------------------------------------------- LayerNorm fwd
template <typename T, int VPL>
__global__ __launch_bounds__(256) void layernorm_fwd_vec(int64_t rows, int dim, float eps, const T* __restrict__ x,
                                                         const T* __restrict__ w, const T* __restrict__ b,
                                                         T* __restrict__ y, float* __restrict__ mean_out,
                                                         float* __restrict__ rstd_out) {
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
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w ? (int64_t)dim * ES : 0);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(b, b ? (int64_t)dim * ES : 0);
    const int nvec = dim / N;
    const uint32_t rowoff = (uint32_t)(wave * dim * ES);
    // x, w and b are all requested before the row's two reductions (w and b
    // stay packed until use), so their latency is not paid after them
    float v[VPL][N];
    i32x4 wq[VPL], bq[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
        const uint32_t off = vi < nvec ? (uint32_t)(vi * N * ES) : kOOB;
        BVec<T>::load(rx, off == kOOB ? kOOB : rowoff + off, v[i]);
        wq[i] = buf_load16(rw, off);
        bq[i] = buf_load16(rb, off);
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int e = 0; e < N; ++e) s += v[i][e];
    const float mean = wave_sum(s) / (float)dim;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const bool ok = lane + i * kWave < nvec;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float c = v[i][e] - mean;
            q += ok ? c * c : 0.f;
        }
    }
    const float var = wave_sum(q) / (float)dim;
    const float r = 1.0f / sqrtf(var + eps);
    if (lane == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = r;
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
        const uint32_t off = vi < nvec ? (uint32_t)(vi * N * ES) : kOOB;
        float wv[N], bv[N], o[N];
        BVec<T>::unpack(wq[i], wv);
        BVec<T>::unpack(bq[i], bv);
#pragma unroll
        for (int e = 0; e < N; ++e) {
            float t = (v[i][e] - mean) * r;
            if (w) t = t * wv[e];
            if (b) t = t + bv[e];
            o[e] = t;
        }
        BVec<T>::store(ry, off == kOOB ? kOOB : rowoff + off, o);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void layernorm_fwd_scalar(int64_t rows, int64_t dim, float eps,
                                                            const T* __restrict__ x, const T* __restrict__ w,
                                                            const T* __restrict__ b, T* __restrict__ y,
                                                            float* __restrict__ mean_out,
                                                            float* __restrict__ rstd_out) {
    const int lane = lane_id();
    const int64_t row = (int64_t)blockIdx.x * kRowsPerBlock + (threadIdx.x >> 6);
    if (row >= rows) return;
    const T* xr = x + row * dim;
    float s = 0.f;
    for (int64_t j = lane; j < dim; j += kWave) s += Elem<T>::load(xr, j);
    const float mean = wave_sum(s) / (float)dim;
    float q = 0.f;
    for (int64_t j = lane; j < dim; j += kWave) {
        const float c = Elem<T>::load(xr, j) - mean;
        q += c * c;
    }
    const float r = 1.0f / sqrtf(wave_sum(q) / (float)dim + eps);
    if (lane == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = r;
    }
    for (int64_t j = lane; j < dim; j += kWave) {
        float t = (Elem<T>::load(xr, j) - mean) * r;
        if (w) t = t * Elem<T>::load(w, j);
        if (b) t = t + Elem<T>::load(b, j);
        Elem<T>::store(y + row * dim, j, t);
    }
}

// ---------------------------------------------------------- LayerNorm bwd
// xh = (x - mean) r, g = dy w:  dx = r (g - mean(g) - xh mean(g xh));
// dw = sum_rows dy xh, db = sum_rows dy (per-block partials [nb][dim] each,
// rows of a block in order, waves combined in wave order through LDS).
template <typename T, int VPL, bool DW>
__global__ __launch_bounds__(256) void layernorm_bwd_vec(int64_t rows, int dim, float eps, int64_t chunk,
                                                         const T* __restrict__ x, const T* __restrict__ w,
                                                         const float* __restrict__ mean_in,
                                                         const float* __restrict__ rstd_in,
                                                         const T* __restrict__ dy, T* __restrict__ dx,
                                                         float* __restrict__ part_w, float* __restrict__ part_b) {
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
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w ? (int64_t)dim * ES : 0);
    float wv[VPL][N];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = lane + i * kWave;
        BVec<T>::load(rw, vi < nvec ? (uint32_t)(vi * N * ES) : kOOB, wv[i]);
#pragma unroll
        for (int e = 0; e < N; ++e) wv[i][e] = w ? wv[i][e] : 1.f;
    }
    float aw[DW ? VPL : 1][N], ab[DW ? VPL : 1][N];
#pragma unroll
    for (int i = 0; i < (DW ? VPL : 1); ++i)
#pragma unroll
        for (int e = 0; e < N; ++e) aw[i][e] = ab[i][e] = 0.f;

    // Software pipeline, one row in flight: the raw 16-byte vectors of the
    // wave's next row are requested before the current row is used.
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
        // raw vectors of the current row, converted on use (bf16 rows stay
        // packed, which halves the registers they hold)
        i32x4 xq[VPL], gq[VPL];
#pragma unroll
        for (int i = 0; i < VPL; ++i) { xq[i] = nx[i]; gq[i] = ng[i]; }
        if (q + kRowsPerBlock < nr) load_row(q + kRowsPerBlock, nx, ng);  // wave-uniform
        float mean, r;
        if (mean_in && rstd_in) {
            mean = mean_in[r0 + q];
            r = rstd_in[r0 + q];
        } else {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                float xv[N];
                BVec<T>::unpack(xq[i], xv);
#pragma unroll
                for (int e = 0; e < N; ++e) s += xv[e];
            }
            mean = wave_sum(s) / (float)dim;
            float c2 = 0.f;
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                const bool ok = lane + i * kWave < nvec;
                float xv[N];
                BVec<T>::unpack(xq[i], xv);
#pragma unroll
                for (int e = 0; e < N; ++e) {
                    const float c = xv[e] - mean;
                    c2 += ok ? c * c : 0.f;
                }
            }
            r = 1.0f / sqrtf(wave_sum(c2) / (float)dim + eps);
        }
        float sg = 0.f, sgx = 0.f;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const bool ok = lane + i * kWave < nvec;
            float xv[N], gv[N];
            BVec<T>::unpack(xq[i], xv);
            BVec<T>::unpack(gq[i], gv);
#pragma unroll
            for (int e = 0; e < N; ++e) {
                const float xh = ok ? (xv[e] - mean) * r : 0.f;
                const float g = gv[e] * wv[i][e];
                sg += g;
                sgx += g * xh;
            }
        }
        const float mg = wave_sum(sg) / (float)dim;
        const float mgx = wave_sum(sgx) / (float)dim;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int vi = lane + i * kWave;
            float xv[N], gv[N], o[N];
            BVec<T>::unpack(xq[i], xv);
            BVec<T>::unpack(gq[i], gv);
#pragma unroll
            for (int e = 0; e < N; ++e) {
                const float xh = (xv[e] - mean) * r;
                o[e] = r * (gv[e] * wv[i][e] - mg - xh * mgx);
                if constexpr (DW) {
                    aw[i][e] += gv[e] * xh;
                    ab[i][e] += gv[e];
                }
            }
            BVec<T>::store(rd, vi < nvec ? (uint32_t)((q * dim + vi * N) * ES) : kOOB, o);
        }
    }
    if constexpr (DW) {
        // The two partials pass through one [kRowsPerBlock][dim] LDS buffer in
        // turn (dw, then db), each summed over the waves in wave order.
        extern __shared__ float lds[];
#pragma unroll
        for (int pass = 0; pass < 2; ++pass) {
            if (pass) __syncthreads();  // every wave has read the dw pass
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                const int vi = lane + i * kWave;
                if (vi < nvec)
#pragma unroll
                    for (int e = 0; e < N; ++e) lds[wave * dim + vi * N + e] = pass ? ab[i][e] : aw[i][e];
            }
            __syncthreads();
            float* part = pass ? part_b : part_w;
            for (int j = threadIdx.x; j < dim; j += blockDim.x) {
                float sum = lds[j];
#pragma unroll
                for (int k = 1; k < kRowsPerBlock; ++k) sum += lds[k * dim + j];
                part[(int64_t)blockIdx.x * dim + j] = sum;
            }
        }
    }
}

template <typename T, bool DW>
__global__ __launch_bounds__(256) void layernorm_bwd_scalar(int64_t rows, int64_t dim, float eps, int64_t chunk,
                                                            const T* __restrict__ x, const T* __restrict__ w,
                                                            const float* __restrict__ mean_in,
                                                            const float* __restrict__ rstd_in,
                                                            const T* __restrict__ dy, T* __restrict__ dx,
                                                            float* __restrict__ part_w, float* __restrict__ part_b) {
    // The block walks its rows in order with all 4 waves; row sums are
    // combined over the waves through LDS in wave order; thread t owns
    // columns t, t + 256, ... of the block's partials.
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * chunk;
    const int64_t r1 = r0 + chunk < rows ? r0 + chunk : rows;
    __shared__ float red[3][kRowsPerBlock];
    float* pw = part_w + (int64_t)blockIdx.x * dim;
    float* pb = part_b + (int64_t)blockIdx.x * dim;
    if constexpr (DW) {
        for (int64_t j = threadIdx.x; j < dim; j += blockDim.x) pw[j] = pb[j] = 0.f;
    }
    auto block_sum = [&](float v, int slot) {
        v = wave_sum(v);
        if (lane == 0) red[slot][wave] = v;
        __syncthreads();
        float t = red[slot][0];
#pragma unroll
        for (int k = 1; k < kRowsPerBlock; ++k) t += red[slot][k];
        __syncthreads();
        return t;
    };
    for (int64_t row = r0; row < r1; ++row) {
        const T* xr = x + row * dim;
        const T* gr = dy + row * dim;
        float mean, r;
        if (mean_in && rstd_in) {
            mean = mean_in[row];
            r = rstd_in[row];
        } else {
            float s = 0.f;
            for (int64_t j = threadIdx.x; j < dim; j += blockDim.x) s += Elem<T>::load(xr, j);
            mean = block_sum(s, 0) / (float)dim;
            float c2 = 0.f;
            for (int64_t j = threadIdx.x; j < dim; j += blockDim.x) {
                const float c = Elem<T>::load(xr, j) - mean;
                c2 += c * c;
            }
            r = 1.0f / sqrtf(block_sum(c2, 1) / (float)dim + eps);
        }
        float sg = 0.f, sgx = 0.f;
        for (int64_t j = threadIdx.x; j < dim; j += blockDim.x) {
            const float g = Elem<T>::load(gr, j) * (w ? Elem<T>::load(w, j) : 1.f);
            sg += g;
            sgx += g * (Elem<T>::load(xr, j) - mean) * r;
        }
        const float mg = block_sum(sg, 1) / (float)dim;
        const float mgx = block_sum(sgx, 2) / (float)dim;
        for (int64_t j = threadIdx.x; j < dim; j += blockDim.x) {
            const float gy = Elem<T>::load(gr, j);
            const float g = gy * (w ? Elem<T>::load(w, j) : 1.f);
            const float xh = (Elem<T>::load(xr, j) - mean) * r;
            Elem<T>::store(dx + row * dim, j, r * (g - mg - xh * mgx));
            if constexpr (DW) {
                pw[j] += gy * xh;
                pb[j] += gy;
            }
        }
    }
}

// --------------------------------------------------- row (max, sum) helpers
__device__ __forceinline__ void lse_combine(float& m, float& s, float m2, float s2) {
    const float mn = fmaxf(m, m2);
    if (mn == kNegInf) {  // both empty (all -inf so far)
        s = s + s2;
        m = mn;
        return;
    }
    s = s * __expf(m - mn) + s2 * __expf(m2 - mn);
    m = mn;
}

// Combines the per-thread (max, sum) of a 256-thread workgroup: a butterfly
// over each wave (symmetric, so every lane agrees), then the 4 waves in order.
__device__ __forceinline__ void block_lse(float& m, float& s, float* red) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float m2 = __shfl_xor(m, o, kWave), s2 = __shfl_xor(s, o, kWave);
        lse_combine(m, s, m2, s2);
    }
    const int wave = threadIdx.x >> 6;
    if (lane_id() == 0) {
        red[2 * wave] = m;
        red[2 * wave + 1] = s;
    }
    __syncthreads();
    m = red[0];
    s = red[1];
#pragma unroll
    for (int k = 1; k < 4; ++k) lse_combine(m, s, red[2 * k], red[2 * k + 1]);
    __syncthreads();
}

__device__ __forceinline__ float block_sum256(float v, float* red) {
    v = wave_sum(v);
    if (lane_id() == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const float t = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return t;
}

// Per-thread online (max, sum of exp, sum) over the row; 16-byte vectors when
// the row is vector-aligned, else elements.
template <typename T>
__device__ __forceinline__ void row_stats(const T* __restrict__ xr, int64_t dim, bool vec, float& m, float& s,
                                          float* sumx) {
    constexpr int N = Vec16<T>::N;
    m = kNegInf;
    s = 0.f;
    float sx = 0.f;
    auto add = [&](float v) {
        if (v > m) {
            s = (m == kNegInf ? 0.f : s * __expf(m - v)) + 1.f;
            m = v;
        } else if (v != kNegInf) {
            s += __expf(v - m);
        }
        sx += v;
    };
    if (vec) {
        // per vector: one rescale to the vector's max, then one exp per element
        for (int64_t c = threadIdx.x; c < dim / N; c += 256) {
            float v[N];
            Vec16<T>::load(xr + c * N, v);
            float vm = v[0];
#pragma unroll
            for (int e = 1; e < N; ++e) vm = fmaxf(vm, v[e]);
            if (vm > m) {
                s = m == kNegInf ? 0.f : s * __expf(m - vm);
                m = vm;
            }
            if (m != kNegInf) {
#pragma unroll
                for (int e = 0; e < N; ++e) s += __expf(v[e] - m);
            }
#pragma unroll
            for (int e = 0; e < N; ++e) sx += v[e];
        }
    } else {
        for (int64_t j = threadIdx.x; j < dim; j += 256) add(Elem<T>::load(xr, j));
    }
    if (sx != sx) s = __builtin_nanf("");  // a NaN anywhere in the row makes the row's sum NaN, as in the reference
    if (sumx) *sumx = sx;
}

// ------------------------------------------------------------ log-softmax
template <typename T>
__global__ __launch_bounds__(256) void log_softmax_fwd_k(int64_t dim, bool vec, const T* __restrict__ x,
                                                         T* __restrict__ y) {
    constexpr int N = Vec16<T>::N;
    __shared__ float red[8];
    const T* xr = x + (int64_t)blockIdx.x * dim;
    T* yr = y + (int64_t)blockIdx.x * dim;
    float m, s;
    row_stats<T>(xr, dim, vec, m, s, nullptr);
    block_lse(m, s, red);
    const float ls = __logf(s);
    // (x - max) - log(sum): the two subtractions of candle's log_softmax
    if (vec) {
        for (int64_t c = threadIdx.x; c < dim / N; c += 256) {
            float v[N];
            Vec16<T>::load(xr + c * N, v);
#pragma unroll
            for (int e = 0; e < N; ++e) v[e] = (v[e] - m) - ls;
            Vec16<T>::store(yr + c * N, v);
        }
    } else {
        for (int64_t j = threadIdx.x; j < dim; j += 256) Elem<T>::store(yr, j, (Elem<T>::load(xr, j) - m) - ls);
    }
}

// dx = dy - exp(y) sum(dy)
template <typename T>
__global__ __launch_bounds__(256) void log_softmax_bwd_k(int64_t dim, bool vec, const T* __restrict__ y,
                                                         const T* __restrict__ dy, T* __restrict__ dx) {
    constexpr int N = Vec16<T>::N;
    __shared__ float red[4];
    const int64_t base = (int64_t)blockIdx.x * dim;
    float t = 0.f;
    if (vec) {
        for (int64_t c = threadIdx.x; c < dim / N; c += 256) {
            float g[N];
            Vec16<T>::load(dy + base + c * N, g);
#pragma unroll
            for (int e = 0; e < N; ++e) t += g[e];
        }
    } else {
        for (int64_t j = threadIdx.x; j < dim; j += 256) t += Elem<T>::load(dy + base, j);
    }
    const float sg = block_sum256(t, red);
    if (vec) {
        for (int64_t c = threadIdx.x; c < dim / N; c += 256) {
            float g[N], v[N];
            Vec16<T>::load(dy + base + c * N, g);
            Vec16<T>::load(y + base + c * N, v);
#pragma unroll
            for (int e = 0; e < N; ++e) g[e] = g[e] - __expf(v[e]) * sg;
            Vec16<T>::store(dx + base + c * N, g);
        }
    } else {
        for (int64_t j = threadIdx.x; j < dim; j += 256)
            Elem<T>::store(dx + base, j, Elem<T>::load(dy + base, j) - __expf(Elem<T>::load(y + base, j)) * sg);
    }
}

// ---------------------------------------------------------- cross entropy
// Per row: lse and the row terms of the loss, rowv[row] = {valid * (lse -
// x[t]), sum_j (x_j - lse), valid}. A target outside [0, vocab) that is not
// ignored makes its term NaN (the reference's gather fails on it).
template <typename T>
__global__ __launch_bounds__(256) void xent_rows_k(int64_t vocab, bool vec, const T* __restrict__ logits,
                                                   const uint32_t* __restrict__ targets, int64_t ignore_index,
                                                   float* __restrict__ rowv, float* __restrict__ lse_out) {
    __shared__ float red[8];
    const int64_t row = blockIdx.x;
    const T* xr = logits + row * vocab;
    float m, s, sx;
    row_stats<T>(xr, vocab, vec, m, s, &sx);
    block_lse(m, s, red);
    sx = block_sum256(sx, red);
    if (threadIdx.x == 0) {
        const float lse = m + __logf(s);
        const uint32_t t = targets[row];
        const bool ignored = ignore_index >= 0 && (int64_t)t == ignore_index;
        float nll = 0.f;
        if (!ignored) nll = (int64_t)t < vocab ? lse - Elem<T>::load(xr, t) : __builtin_nanf("");
        rowv[3 * row] = nll;
        rowv[3 * row + 1] = sx - (float)vocab * lse;
        rowv[3 * row + 2] = ignored ? 0.f : 1.f;
        if (lse_out) lse_out[row] = lse;
    }
}

// loss = -(sum log p[t] / count) * (1 - s) + s * (-(sum of all log p) / (rows vocab)),
// sums in row order (each thread a contiguous run of rows, then the threads in order).
__global__ __launch_bounds__(1024) void xent_final_k(int64_t rows, int64_t vocab, float smoothing,
                                                     const float* __restrict__ rowv, float* __restrict__ loss,
                                                     float* __restrict__ count_out) {
    // rowv is [rows][3] = (nll, sum x - V lse, valid): read flat as float4
    // (16 per thread in flight: one round for up to 16384 rows, the whole
    // array being fetched from other XCDs' writes); element f belongs to
    // component f % 3, and for f = 4 v + e that is (v + e) % 3. Fixed-order
    // wave and block sums make the result reproducible.
    constexpr int kT = 1024, kU = 16;
    __shared__ float red[kT / 64][3];
    const int64_t nf = 3 * rows, nv = nf / 4;
    const float4* rv4 = reinterpret_cast<const float4*>(rowv);
    float acc[3] = {0.f, 0.f, 0.f};
    auto add = [&](int64_t f, float x) {
        const int c = (int)(f % 3);
        acc[0] += c == 0 ? x : 0.f;
        acc[1] += c == 1 ? x : 0.f;
        acc[2] += c == 2 ? x : 0.f;
    };
    for (int64_t v0 = threadIdx.x; v0 < nv; v0 += (int64_t)kT * kU) {
        float4 x[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t v = v0 + (int64_t)kT * u;
            x[u] = v < nv ? rv4[v] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t f = 4 * (v0 + (int64_t)kT * u);
            add(f, x[u].x);
            add(f + 1, x[u].y);
            add(f + 2, x[u].z);
            add(f + 3, x[u].w);
        }
    }
    if (threadIdx.x < nf - 4 * nv) add(4 * nv + threadIdx.x, rowv[4 * nv + threadIdx.x]);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float w = wave_sum(acc[c]);
        if (lane_id() == 0) red[threadIdx.x >> 6][c] = w;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float tn = 0.f, ts = 0.f, tc = 0.f;
        for (int w = 0; w < kT / 64; ++w) {
            tn += red[w][0];
            ts += red[w][1];
            tc += red[w][2];
        }
        // mean of -nll over the counted rows; all ignored: 0 / 0 = NaN
        const float nll = tn / tc;
        float l = nll;
        if (smoothing != 0.f) {
            const float smooth = -(ts / ((float)rows * (float)vocab));
            l = nll * (1.0f - smoothing) + smooth * smoothing;
        }
        loss[0] = l;
        if (count_out) count_out[0] = tc;
    }
}

// dlogits = dloss ((1 - s) valid (p - onehot(t)) / count + s (p - 1/V) / rows), p = exp(x - lse)
template <typename T>
__global__ __launch_bounds__(256) void xent_bwd_k(int64_t rows, int64_t vocab, bool vec, float smoothing,
                                                  const T* __restrict__ logits, const uint32_t* __restrict__ targets,
                                                  int64_t ignore_index, const float* __restrict__ stats,
                                                  const float* __restrict__ dloss, T* __restrict__ dlogits) {
    constexpr int N = Vec16<T>::N;
    const int64_t row = blockIdx.x;
    const T* xr = logits + row * vocab;
    T* dr = dlogits + row * vocab;
    const float lse = stats[row];
    const float count = stats[rows];
    const uint32_t t = targets[row];
    const bool valid = !(ignore_index >= 0 && (int64_t)t == ignore_index);
    const float g = dloss[0];
    const float a = valid ? g * (1.0f - smoothing) / count : 0.f;  // weight of (p - onehot)
    const float c = g * smoothing / (float)rows;                    // weight of (p - 1/V)
    const float inv_v = 1.0f / (float)vocab;
    auto grad = [&](float x, int64_t j) {
        const float p = __expf(x - lse);
        return a * (p - (j == (int64_t)t ? 1.f : 0.f)) + c * (p - inv_v);
    };
    if (vec) {
        for (int64_t cc = threadIdx.x; cc < vocab / N; cc += 256) {
            float v[N];
            Vec16<T>::load(xr + cc * N, v);
#pragma unroll
            for (int e = 0; e < N; ++e) v[e] = grad(v[e], cc * N + e);
            Vec16<T>::store(dr + cc * N, v);
        }
    } else {
        for (int64_t j = threadIdx.x; j < vocab; j += 256) Elem<T>::store(dr, j, grad(Elem<T>::load(xr, j), j));
    }
}

// ---------------------------------------------------- LayerNorm, long rows
// Rows past the one-wave paths (more than 8 vectors per lane: fp32 past 2048,
// bf16 past 4096 columns; forward to 32768 / 65536, backward to 8192 / 8192):
// a workgroup of up to 1024 threads per row
// (forward) or per block of rows (backward), vector v of a row held by
// thread v % blockDim.x, so x and dy are still read once. Row sums combine
// the waves' butterflies in wave order through LDS (wg_sum); the backward
// gives each of a row's reduction rounds its own slot array and alternates
// two sets between rows, so one barrier per round suffices.
constexpr int kLnWideThreads = 1024;

template <typename T, int VPL>
__global__ __launch_bounds__(kLnWideThreads) void layernorm_fwd_wide(int64_t row0, int dim, float eps,
                                                                     const T* __restrict__ x, const T* __restrict__ w,
                                                                     const T* __restrict__ b, T* __restrict__ y,
                                                                     float* __restrict__ mean_out,
                                                                     float* __restrict__ rstd_out) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    __shared__ float red[2][kMaxWaves];
    const int tid = threadIdx.x, nt = blockDim.x;
    const int64_t row = row0 + blockIdx.x;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + row * dim, (int64_t)dim * ES);
    const __amdgpu_buffer_rsrc_t ry = make_rsrc(y + row * dim, (int64_t)dim * ES);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w ? (int64_t)dim * ES : 0);
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(b, b ? (int64_t)dim * ES : 0);
    const int nvec = dim / N;
    i32x4 xq[VPL];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        xq[i] = buf_load16(rx, vi < nvec ? (uint32_t)(vi * N * ES) : kOOB);
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        float v[N];
        BVec<T>::unpack(xq[i], v);
#pragma unroll
        for (int e = 0; e < N; ++e) s += v[e];
    }
    const float mean = wg_sum(s, red[0]) / (float)dim;
    float q = 0.f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const bool ok = tid + i * nt < nvec;
        float v[N];
        BVec<T>::unpack(xq[i], v);
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float c = v[e] - mean;
            q += ok ? c * c : 0.f;
        }
    }
    const float r = 1.0f / sqrtf(wg_sum(q, red[1]) / (float)dim + eps);
    if (tid == 0) {
        if (mean_out) mean_out[row] = mean;
        if (rstd_out) rstd_out[row] = r;
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        const uint32_t off = vi < nvec ? (uint32_t)(vi * N * ES) : kOOB;
        float v[N], wv[N], bv[N], o[N];
        BVec<T>::unpack(xq[i], v);
        BVec<T>::load(rw, off, wv);
        BVec<T>::load(rb, off, bv);
#pragma unroll
        for (int e = 0; e < N; ++e) {
            float t = (v[e] - mean) * r;
            if (w) t = t * wv[e];
            if (b) t = t + bv[e];
            o[e] = t;
        }
        BVec<T>::store(ry, off, o);
    }
}

// Block b owns rows [b*chunk, min(rows, (b+1)*chunk)) and walks them in
// order with the whole workgroup, the next row's loads issued before the
// current row is used. Each thread owns the columns of its vectors, so its
// dw / db partials accumulate in registers in row order and are written to
// part_w[b] / part_b[b] as they are.
template <typename T, int VPL, bool DW>
__global__ __launch_bounds__(kLnWideThreads) void layernorm_bwd_wide(int64_t rows, int dim, float eps, int64_t chunk,
                                                                     const T* __restrict__ x, const T* __restrict__ w,
                                                                     const float* __restrict__ mean_in,
                                                                     const float* __restrict__ rstd_in,
                                                                     const T* __restrict__ dy, T* __restrict__ dx,
                                                                     float* __restrict__ part_w,
                                                                     float* __restrict__ part_b) {
    constexpr int N = BVec<T>::N;
    constexpr int ES = (int)sizeof(T);
    __shared__ float red[2][3][2][kMaxWaves];  // [row parity][round][value][wave]
    const int tid = threadIdx.x, nt = blockDim.x;
    const int lane = lane_id(), wave = wave_id(), nw = nt >> 6;
    const int nvec = dim / N;
    const int64_t r0 = (int64_t)blockIdx.x * chunk;
    const int64_t r1 = r0 + chunk < rows ? r0 + chunk : rows;
    const int64_t nr = r1 > r0 ? r1 - r0 : 0;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + r0 * dim, nr * dim * ES);
    const __amdgpu_buffer_rsrc_t rg = make_rsrc(dy + r0 * dim, nr * dim * ES);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(dx + r0 * dim, nr * dim * ES);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(w, w ? (int64_t)dim * ES : 0);
    float wv[VPL][N];
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
        const int vi = tid + i * nt;
        BVec<T>::load(rw, vi < nvec ? (uint32_t)(vi * N * ES) : kOOB, wv[i]);
#pragma unroll
        for (int e = 0; e < N; ++e) wv[i][e] = w ? wv[i][e] : 1.f;
    }
    float aw[DW ? VPL : 1][N], ab[DW ? VPL : 1][N];
#pragma unroll
    for (int i = 0; i < (DW ? VPL : 1); ++i)
#pragma unroll
        for (int e = 0; e < N; ++e) aw[i][e] = ab[i][e] = 0.f;
    // Sum of (u, v) over the workgroup into round k's slots of the row's set.
    auto wg_sum2 = [&](float& u, float& v, float (*slot)[kMaxWaves]) {
        u = wave_sum(u);
        v = wave_sum(v);
        if (lane == 0) { slot[0][wave] = u; slot[1][wave] = v; }
        __syncthreads();
        u = slot[0][0];
        v = slot[1][0];
        for (int k = 1; k < nw; ++k) { u += slot[0][k]; v += slot[1][k]; }
    };
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
        float (*set)[2][kMaxWaves] = red[q & 1];
        float mean, r;
        if (mean_in && rstd_in) {
            mean = mean_in[r0 + q];
            r = rstd_in[r0 + q];
        } else {
            float s = 0.f, unused = 0.f;
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                float xv[N];
                BVec<T>::unpack(xq[i], xv);
#pragma unroll
                for (int e = 0; e < N; ++e) s += xv[e];
            }
            wg_sum2(s, unused, set[0]);
            mean = s / (float)dim;
            float c2 = 0.f;
#pragma unroll
            for (int i = 0; i < VPL; ++i) {
                const bool ok = tid + i * nt < nvec;
                float xv[N];
                BVec<T>::unpack(xq[i], xv);
#pragma unroll
                for (int e = 0; e < N; ++e) {
                    const float c = xv[e] - mean;
                    c2 += ok ? c * c : 0.f;
                }
            }
            wg_sum2(c2, unused, set[1]);
            r = 1.0f / sqrtf(c2 / (float)dim + eps);
        }
        float sg = 0.f, sgx = 0.f;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const bool ok = tid + i * nt < nvec;
            float xv[N], gv[N];
            BVec<T>::unpack(xq[i], xv);
            BVec<T>::unpack(gq[i], gv);
#pragma unroll
            for (int e = 0; e < N; ++e) {
                const float xh = ok ? (xv[e] - mean) * r : 0.f;
                const float g = gv[e] * wv[i][e];
                sg += g;
                sgx += g * xh;
            }
        }
        wg_sum2(sg, sgx, set[2]);
        const float mg = sg / (float)dim;
        const float mgx = sgx / (float)dim;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int vi = tid + i * nt;
            float xv[N], gv[N], o[N];
            BVec<T>::unpack(xq[i], xv);
            BVec<T>::unpack(gq[i], gv);
#pragma unroll
            for (int e = 0; e < N; ++e) {
                const float xh = (xv[e] - mean) * r;
                o[e] = r * (gv[e] * wv[i][e] - mg - xh * mgx);
                if constexpr (DW) {
                    aw[i][e] += gv[e] * xh;
                    ab[i][e] += gv[e];
                }
            }
            BVec<T>::store(rd, vi < nvec ? (uint32_t)((q * dim + vi * N) * ES) : kOOB, o);
        }
    }
    if constexpr (DW) {
        float* pw = part_w + (int64_t)blockIdx.x * dim;
        float* pb = part_b + (int64_t)blockIdx.x * dim;
#pragma unroll
        for (int i = 0; i < VPL; ++i) {
            const int vi = tid + i * nt;
            if (vi < nvec)
#pragma unroll
                for (int e = 0; e < N; ++e) {
                    pw[vi * N + e] = aw[i][e];
                    pb[vi * N + e] = ab[i][e];
                }
        }
    }
}

// Vectors per thread of the LayerNorm wide paths (0: the row does not fit):
// forward up to 8 (x packed; w and b loaded at use), backward up to 2 in
// fp32 and 1 in bf16 (w and both partials held unpacked beside two rows of
// packed x and dy; bf16 at 2 needs more than 128 registers per thread).
template <typename T>
int ln_wide_vpl(int64_t dim, bool bwd) {
    if (dim % Vec16<T>::N != 0) return 0;
    const int64_t nvec = dim / Vec16<T>::N;
    const int cap = bwd ? (sizeof(T) == 2 ? 1 : 2) : 8;
    for (int v = bwd ? 1 : 2; v <= cap; v *= 2)
        if (nvec <= (int64_t)v * kLnWideThreads) return v;
    return 0;
}
template <typename T>
int ln_wide_threads(int64_t dim, int vpl) {
    const int64_t per = (dim / Vec16<T>::N + vpl - 1) / vpl;
    return (int)((per + kWave - 1) / kWave * kWave);
}

template <typename T>
bool ln_vec_ok(int64_t dim) {
    return dim % Vec16<T>::N == 0 && dim / Vec16<T>::N <= 8 * kWave;
}

template <typename T>
int ln_vpl(int64_t dim) {
    const int64_t per = (dim / Vec16<T>::N + kWave - 1) / kWave;
    return per <= 1 ? 1 : per <= 2 ? 2 : per <= 4 ? 4 : 8;
}

template <typename T>
bool row_vec(const void* p, int64_t dim) {
    return dim % Vec16<T>::N == 0 && (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

template <typename T>
hipError_t ln_fwd(int64_t rows, int64_t dim, float eps, const void* x, const void* w, const void* b, void* y,
                  float* mean, float* rstd, hipStream_t st) {
    const dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock));
    const T *xp = static_cast<const T*>(x), *wp = static_cast<const T*>(w), *bp = static_cast<const T*>(b);
    T* yp = static_cast<T*>(y);
    const int wvpl = ln_vec_ok<T>(dim) ? 0 : ln_wide_vpl<T>(dim, false);
    if (wvpl) {
        const int nt = ln_wide_threads<T>(dim, wvpl);
        const int d = (int)dim;
        const int64_t cap = (((int64_t)1 << 32) - 1) / nt;  // a launch's thread count is 32-bit
        for (int64_t r0 = 0; r0 < rows; r0 += cap) {
            const dim3 g((unsigned)(rows - r0 < cap ? rows - r0 : cap));
            switch (wvpl) {
                case 2: layernorm_fwd_wide<T, 2><<<g, nt, 0, st>>>(r0, d, eps, xp, wp, bp, yp, mean, rstd); break;
                case 4: layernorm_fwd_wide<T, 4><<<g, nt, 0, st>>>(r0, d, eps, xp, wp, bp, yp, mean, rstd); break;
                default: layernorm_fwd_wide<T, 8><<<g, nt, 0, st>>>(r0, d, eps, xp, wp, bp, yp, mean, rstd); break;
            }
        }
    } else if (ln_vec_ok<T>(dim)) {
        const int d = (int)dim;
        switch (ln_vpl<T>(dim)) {
            case 1: layernorm_fwd_vec<T, 1><<<grid, 256, 0, st>>>(rows, d, eps, xp, wp, bp, yp, mean, rstd); break;
            case 2: layernorm_fwd_vec<T, 2><<<grid, 256, 0, st>>>(rows, d, eps, xp, wp, bp, yp, mean, rstd); break;
            case 4: layernorm_fwd_vec<T, 4><<<grid, 256, 0, st>>>(rows, d, eps, xp, wp, bp, yp, mean, rstd); break;
            default: layernorm_fwd_vec<T, 8><<<grid, 256, 0, st>>>(rows, d, eps, xp, wp, bp, yp, mean, rstd); break;
        }
    } else {
        layernorm_fwd_scalar<T><<<grid, 256, 0, st>>>(rows, dim, eps, xp, wp, bp, yp, mean, rstd);
    }
    return hipGetLastError();
}

template <typename T, bool DW>
void ln_bwd_vec_launch(int vpl, dim3 grid, size_t lds, hipStream_t st, int64_t rows, int d, float eps,
                       int64_t chunk, const T* x, const T* w, const float* mean, const float* rstd, const T* dy,
                       T* dx, float* pw, float* pb) {
    switch (vpl) {
        case 1: layernorm_bwd_vec<T, 1, DW><<<grid, 256, lds, st>>>(rows, d, eps, chunk, x, w, mean, rstd, dy, dx, pw, pb); break;
        case 2: layernorm_bwd_vec<T, 2, DW><<<grid, 256, lds, st>>>(rows, d, eps, chunk, x, w, mean, rstd, dy, dx, pw, pb); break;
        case 4: layernorm_bwd_vec<T, 4, DW><<<grid, 256, lds, st>>>(rows, d, eps, chunk, x, w, mean, rstd, dy, dx, pw, pb); break;
        default: layernorm_bwd_vec<T, 8, DW><<<grid, 256, lds, st>>>(rows, d, eps, chunk, x, w, mean, rstd, dy, dx, pw, pb); break;
    }
}

template <typename T>
hipError_t ln_bwd(int64_t rows, int64_t dim, float eps, const void* x, const void* w, const float* mean,
                  const float* rstd, const void* dy, void* dx, float* dw, float* db, float* ws, hipStream_t st) {
    const int nb = layernorm_bwd_blocks(rows);
    const int64_t chunk = (rows + nb - 1) / nb;
    const dim3 grid((unsigned)nb);
    const T *xp = static_cast<const T*>(x), *wp = static_cast<const T*>(w), *gp = static_cast<const T*>(dy);
    T* dxp = static_cast<T*>(dx);
    const bool need = dw || db;
    float* pw = need ? ws : nullptr;
    float* pb = need ? ws + (size_t)nb * dim : nullptr;
    const size_t lds = (size_t)kRowsPerBlock * dim * sizeof(float);
    if (ln_vec_ok<T>(dim) && (!need || lds <= 64 * 1024)) {
        const int vpl = ln_vpl<T>(dim);
        if (need) ln_bwd_vec_launch<T, true>(vpl, grid, lds, st, rows, (int)dim, eps, chunk, xp, wp, mean, rstd, gp, dxp, pw, pb);
        else ln_bwd_vec_launch<T, false>(vpl, grid, 0, st, rows, (int)dim, eps, chunk, xp, wp, mean, rstd, gp, dxp, nullptr, nullptr);
    } else if (const int wvpl = ln_wide_vpl<T>(dim, true)) {
        const int nt = ln_wide_threads<T>(dim, wvpl);
        const int d = (int)dim;
        constexpr int kV2 = sizeof(T) == 2 ? 1 : 2;  // bf16 rows stop at one vector per thread
        if (need) {
            if (wvpl == 1) layernorm_bwd_wide<T, 1, true><<<grid, nt, 0, st>>>(rows, d, eps, chunk, xp, wp, mean, rstd, gp, dxp, pw, pb);
            else layernorm_bwd_wide<T, kV2, true><<<grid, nt, 0, st>>>(rows, d, eps, chunk, xp, wp, mean, rstd, gp, dxp, pw, pb);
        } else {
            if (wvpl == 1) layernorm_bwd_wide<T, 1, false><<<grid, nt, 0, st>>>(rows, d, eps, chunk, xp, wp, mean, rstd, gp, dxp, nullptr, nullptr);
            else layernorm_bwd_wide<T, kV2, false><<<grid, nt, 0, st>>>(rows, d, eps, chunk, xp, wp, mean, rstd, gp, dxp, nullptr, nullptr);
        }
    } else if (need) {
        layernorm_bwd_scalar<T, true><<<grid, 256, 0, st>>>(rows, dim, eps, chunk, xp, wp, mean, rstd, gp, dxp, pw, pb);
    } else {
        layernorm_bwd_scalar<T, false><<<grid, 256, 0, st>>>(rows, dim, eps, chunk, xp, wp, mean, rstd, gp, dxp, nullptr,
                                                            nullptr);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !need) return e;
    const dim3 sgrid((unsigned)((dim + kSumCols - 1) / kSumCols));
    const bool v4 = dim % 4 == 0;
    if (dw) {
        if (v4) column_sum<true><<<sgrid, 256, 0, st>>>(nb, dim, pw, dw);
        else column_sum<false><<<sgrid, 256, 0, st>>>(nb, dim, pw, dw);
    }
    if (db) {
        if (v4) column_sum<true><<<sgrid, 256, 0, st>>>(nb, dim, pb, db);
        else column_sum<false><<<sgrid, 256, 0, st>>>(nb, dim, pb, db);
    }
    return hipGetLastError();
}

}  // namespace

int layernorm_bwd_blocks(int64_t rows) {
    int64_t nb = (rows + 7) / 8;
    if (nb > 512) nb = 512;
    if (nb < 1) nb = 1;
    return (int)nb;
}

hipError_t launch_layernorm_fwd(int64_t rows, int64_t dim, float eps, int dtype, const void* x, const void* w,
                                const void* b, void* y, float* mean, float* rstd, hipStream_t stream) {
    if (dtype == MC_F32) return ln_fwd<float>(rows, dim, eps, x, w, b, y, mean, rstd, stream);
    return ln_fwd<uint16_t>(rows, dim, eps, x, w, b, y, mean, rstd, stream);
}

hipError_t launch_layernorm_bwd(int64_t rows, int64_t dim, float eps, int dtype, const void* x, const void* w,
                                const float* mean, const float* rstd, const void* dy, void* dx, float* dw, float* db,
                                float* ws, hipStream_t stream) {
    if (dtype == MC_F32) return ln_bwd<float>(rows, dim, eps, x, w, mean, rstd, dy, dx, dw, db, ws, stream);
    return ln_bwd<uint16_t>(rows, dim, eps, x, w, mean, rstd, dy, dx, dw, db, ws, stream);
}

hipError_t launch_log_softmax_fwd(int64_t rows, int64_t dim, int dtype, const void* x, void* y, hipStream_t stream) {
    const dim3 grid((unsigned)rows);
    if (dtype == MC_F32) {
        const bool v = row_vec<float>(x, dim) && row_vec<float>(y, dim);
        log_softmax_fwd_k<float><<<grid, 256, 0, stream>>>(dim, v, static_cast<const float*>(x), static_cast<float*>(y));
    } else {
        const bool v = row_vec<uint16_t>(x, dim) && row_vec<uint16_t>(y, dim);
        log_softmax_fwd_k<uint16_t><<<grid, 256, 0, stream>>>(dim, v, static_cast<const uint16_t*>(x),
                                                              static_cast<uint16_t*>(y));
    }
    return hipGetLastError();
}

hipError_t launch_log_softmax_bwd(int64_t rows, int64_t dim, int dtype, const void* y, const void* dy, void* dx,
                                  hipStream_t stream) {
    const dim3 grid((unsigned)rows);
    if (dtype == MC_F32) {
        const bool v = row_vec<float>(y, dim) && row_vec<float>(dy, dim) && row_vec<float>(dx, dim);
        log_softmax_bwd_k<float><<<grid, 256, 0, stream>>>(dim, v, static_cast<const float*>(y),
                                                           static_cast<const float*>(dy), static_cast<float*>(dx));
    } else {
        const bool v = row_vec<uint16_t>(y, dim) && row_vec<uint16_t>(dy, dim) && row_vec<uint16_t>(dx, dim);
        log_softmax_bwd_k<uint16_t><<<grid, 256, 0, stream>>>(dim, v, static_cast<const uint16_t*>(y),
                                                              static_cast<const uint16_t*>(dy),
                                                              static_cast<uint16_t*>(dx));
    }
    return hipGetLastError();
}

hipError_t launch_cross_entropy_fwd(const mc_xent_desc& d, const void* logits, const uint32_t* targets, float* loss,
                                    float* stats, float* ws, hipStream_t stream) {
    const dim3 grid((unsigned)d.rows);
    if (d.dtype == MC_F32)
        xent_rows_k<float><<<grid, 256, 0, stream>>>(d.vocab, row_vec<float>(logits, d.vocab),
                                                     static_cast<const float*>(logits), targets, d.ignore_index, ws,
                                                     stats);
    else
        xent_rows_k<uint16_t><<<grid, 256, 0, stream>>>(d.vocab, row_vec<uint16_t>(logits, d.vocab),
                                                        static_cast<const uint16_t*>(logits), targets, d.ignore_index,
                                                        ws, stats);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    xent_final_k<<<1, 1024, 0, stream>>>(d.rows, d.vocab, d.smoothing, ws, loss, stats ? stats + d.rows : nullptr);
    return hipGetLastError();
}

hipError_t launch_cross_entropy_bwd(const mc_xent_desc& d, const void* logits, const uint32_t* targets,
                                    const float* stats, const float* dloss, void* dlogits, hipStream_t stream) {
    const dim3 grid((unsigned)d.rows);
    if (d.dtype == MC_F32)
        xent_bwd_k<float><<<grid, 256, 0, stream>>>(
            d.rows, d.vocab, row_vec<float>(logits, d.vocab) && row_vec<float>(dlogits, d.vocab), d.smoothing,
            static_cast<const float*>(logits), targets, d.ignore_index, stats, dloss, static_cast<float*>(dlogits));
    else
        xent_bwd_k<uint16_t><<<grid, 256, 0, stream>>>(
            d.rows, d.vocab, row_vec<uint16_t>(logits, d.vocab) && row_vec<uint16_t>(dlogits, d.vocab), d.smoothing,
            static_cast<const uint16_t*>(logits), targets, d.ignore_index, stats, dloss,
            static_cast<uint16_t*>(dlogits));
    return hipGetLastError();
}

}  // namespace mc
