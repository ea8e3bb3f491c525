// Low-rank (rank-r) kernels of the LoRA linear, gfx950.
//
// The reference computes the LoRA delta as H = x.A, dropout(H), H.B, *scale
// (src/training/lora.rs:320-339); its Metal kernel fused_lora_forward_tiled
// (src/backend/kernels.metal:108-159) recomputes the whole x.A row for every
// output element. Here the rank-r products are separate HBM-streaming passes:
//
//  rowproj    H = x.A (forward) and G = scale dY.B^T (backward): a reduction
//             over the feature dim per token row. MFMA 16x16x32 bf16 with the
//             bf16 activations as the A operand straight from HBM and the
//             fp32 parameter split into bf16 hi + lo (two MFMAs), so the
//             parameter keeps ~16 mantissa bits. Dropout mask and 1/(1-p) are
//             applied in the epilogue.
//  colreduce  dA = x^T.Gd and dB = scale Hd^T.dY: reductions over tokens.
//             The token dim is the MFMA K dim, but it is the strided dim of
//             x / dY, so each lane loads an 8 x 8 bf16 block (8 rows, 16 B
//             each) and transposes it in registers; the 8 resulting columns
//             feed 8 MFMAs whose 16 column slots are the lanes' 16 column
//             groups. The fp32 Gd^T / Hd^T operand is split hi + lo as above.
//             Tokens are split in a fixed partition; the partials are summed
//             in split order by split_sum (deterministic, no atomics).
//
// fp32 variants (plain FMA) serve act_dtype == MC_F32.
#include "common.hpp"
#include "lora_kernels.hpp"

namespace mc {
namespace {

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

__device__ __forceinline__ void split_hilo8(const float (&v)[8], uint4& hi, uint4& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint16_t h0 = f32_to_bf16(v[2 * q]), h1 = f32_to_bf16(v[2 * q + 1]);
        const float r0 = v[2 * q] - bf16_to_f32(h0), r1 = v[2 * q + 1] - bf16_to_f32(h1);
        h[q] = (uint32_t)h0 | ((uint32_t)h1 << 16);
        l[q] = pack_bf16x2(r0, r1);
    }
    hi = make_uint4(h[0], h[1], h[2], h[3]);
    lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// 8 x 8 transpose of bf16: R[i] holds columns 0..7 of row i (dword q = cols
// 2q, 2q+1); O[e] receives rows 0..7 of column e (dword p = rows 2p, 2p+1).
__device__ __forceinline__ void transpose8x8(const uint4 (&R)[8], uint4 (&O)[8]) {
    uint32_t r[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i) { r[i][0] = R[i].x; r[i][1] = R[i].y; r[i][2] = R[i].z; r[i][3] = R[i].w; }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        uint32_t o[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t a = r[2 * p][e >> 1], b = r[2 * p + 1][e >> 1];
            o[p] = (e & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
        }
        O[e] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// ------------------------------------------------------------------ prep
__global__ __launch_bounds__(256) void prep_bf16(const float* __restrict__ src, int64_t ld_src,
                                                 int64_t valid_rows, int64_t valid_cols, int transpose,
                                                 uint16_t* __restrict__ hi, uint16_t* __restrict__ lo,
                                                 int64_t rows_out, int64_t cols_out) {
    const int64_t n = rows_out * cols_out;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t i = idx / cols_out, j = idx % cols_out;
        float v = 0.f;
        if (i < valid_rows && j < valid_cols) v = transpose ? src[j * ld_src + i] : src[i * ld_src + j];
        const uint16_t h = f32_to_bf16(v);
        hi[idx] = h;
        if (lo) lo[idx] = f32_to_bf16(v - bf16_to_f32(h));
    }
}

// --------------------------------------------------------------- rowproj
// Workgroup: 4 waves, 16 token rows. Wave w takes 32-column steps w, w+4, ...
// (so the 4 waves read 4 adjacent 64-byte pieces of each row at once); their
// accumulators are combined in wave order through LDS.
template <int RC>
__global__ __launch_bounds__(256) void rowproj_bf16(const uint16_t* __restrict__ X, int64_t T, int64_t C,
                                                    const uint16_t* __restrict__ Phi,
                                                    const uint16_t* __restrict__ Plo, int r, float scale,
                                                    const uint8_t* __restrict__ mask, float keep,
                                                    float* __restrict__ out_t, uint16_t* __restrict__ out_ext,
                                                    int rext, float ext_scale) {
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int64_t t0 = (int64_t)blockIdx.x * 16;
    const int64_t trow = t0 + (lane & 15);
    const bool row_ok = trow < T;
    const int kgrp = (lane >> 4) * 8;
    const uint16_t* xrow = X + (row_ok ? trow : 0) * C + kgrp;
    const int64_t nsteps = (C + 31) / 32;

    f32x4 acc[RC];
#pragma unroll
    for (int rc = 0; rc < RC; ++rc) acc[rc] = f32x4{0.f, 0.f, 0.f, 0.f};

    constexpr int U = 4;
    for (int64_t s0 = wave; s0 < nsteps; s0 += 4 * U) {
        uint4 xa[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t s = s0 + 4 * u;
            const int64_t c = s * 32 + kgrp;
            xa[u] = load16(xrow, s * 32, row_ok && s < nsteps && c < C);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t s = s0 + 4 * u;
            if (s < nsteps) {
                const int64_t c = s * 32 + kgrp;
                const bool c_ok = c < C;
#pragma unroll
                for (int rc = 0; rc < RC; ++rc) {
                    const int64_t prow = (int64_t)(rc * 16 + (lane & 15)) * C + c;
                    const uint4 ph = load16(Phi, prow, c_ok);
                    const uint4 pl = load16(Plo, prow, c_ok);
                    acc[rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xa[u]), as_bf16x8(ph), acc[rc], 0, 0, 0);
                    acc[rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xa[u]), as_bf16x8(pl), acc[rc], 0, 0, 0);
                }
            }
        }
    }

    // combine the 4 waves: [wave][rc][q][lane]
    __shared__ float red[4][RC][4][64];
#pragma unroll
    for (int rc = 0; rc < RC; ++rc)
#pragma unroll
        for (int q = 0; q < 4; ++q) red[wave][rc][q][lane] = acc[rc][q];
    __syncthreads();
    // every thread finalises (rc, q) entries: 64*4*RC values over 256 threads
    for (int idx = threadIdx.x; idx < RC * 4 * 64; idx += 256) {
        const int l = idx & 63, q = (idx >> 6) & 3, rc = idx >> 8;
        float v = red[0][rc][q][l];
#pragma unroll
        for (int w = 1; w < 4; ++w) v += red[w][rc][q][l];
        const int j = rc * 16 + (l & 15);
        const int64_t t = t0 + (l >> 4) * 4 + q;
        if (t >= T) continue;
        if (j < r) {
            v *= scale;
            if (mask) v = mask[t * r + j] ? v * keep : 0.f;
            if (out_t) out_t[(int64_t)j * T + t] = v;
            if (out_ext) out_ext[t * rext + j] = f32_to_bf16(v * ext_scale);
        } else if (j < rext && out_ext) {
            out_ext[t * rext + j] = 0;
        }
    }
}

// ------------------------------------------------------------- colreduce
// Workgroup: 4 waves, 128 columns, token range of split blockIdx.y. Wave w
// takes 32-row steps w, w+4, ... of the range. Lane l loads rows
// t0 + 8*(l/16) + 0..7 at columns c0 + 8*(l%16) + 0..7.
template <int RC>
__global__ __launch_bounds__(256) void colreduce_bf16(const uint16_t* __restrict__ X, int64_t T, int64_t C,
                                                      const float* __restrict__ Pt, int r, int64_t chunk,
                                                      float* __restrict__ partial, int64_t part_stride) {
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int64_t c0 = (int64_t)blockIdx.x * 128;
    const int64_t tb = (int64_t)blockIdx.y * chunk;
    const int64_t te = tb + chunk < T ? tb + chunk : T;
    const int64_t col = c0 + 8 * (lane & 15);
    const bool col_ok = col < C;
    const int g8 = 8 * (lane >> 4);
    const bool pt_vec = (T & 3) == 0;

    f32x4 acc[8][RC];
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int rc = 0; rc < RC; ++rc) acc[e][rc] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int64_t t0 = tb + 32 * wave; t0 < te; t0 += 128) {
        uint4 R[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t t = t0 + g8 + i;
            R[i] = load16(X, t * C + col, col_ok && t < te);
        }
        uint4 ahi[RC], alo[RC];
#pragma unroll
        for (int rc = 0; rc < RC; ++rc) {
            const int j = rc * 16 + (lane & 15);
            float v[8];
            const int64_t t = t0 + g8;
            if (j < r && t + 8 <= te && pt_vec) {
                const float4 a = *reinterpret_cast<const float4*>(Pt + (int64_t)j * T + t);
                const float4 b = *reinterpret_cast<const float4*>(Pt + (int64_t)j * T + t + 4);
                v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = (j < r && t + e < te) ? Pt[(int64_t)j * T + t + e] : 0.f;
            }
            split_hilo8(v, ahi[rc], alo[rc]);
        }
        uint4 Bt[8];
        transpose8x8(R, Bt);
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int rc = 0; rc < RC; ++rc) {
                acc[e][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ahi[rc]), as_bf16x8(Bt[e]), acc[e][rc], 0, 0, 0);
                acc[e][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(alo[rc]), as_bf16x8(Bt[e]), acc[e][rc], 0, 0, 0);
            }
    }

    // combine waves in order 0,1,2,3 through one LDS staging buffer
    __shared__ float stage[8 * RC * 4][64];
    for (int w = 1; w < 4; ++w) {
        if (wave == w) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int rc = 0; rc < RC; ++rc)
#pragma unroll
                    for (int q = 0; q < 4; ++q) stage[(e * RC + rc) * 4 + q][lane] = acc[e][rc][q];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int rc = 0; rc < RC; ++rc)
#pragma unroll
                    for (int q = 0; q < 4; ++q) acc[e][rc][q] += stage[(e * RC + rc) * 4 + q][lane];
        }
        __syncthreads();
    }
    if (wave == 0) {
        float* out = partial + (int64_t)blockIdx.y * part_stride;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t c = col + e;
            if (!col_ok) continue;
#pragma unroll
            for (int rc = 0; rc < RC; ++rc)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int j = rc * 16 + (lane >> 4) * 4 + q;
                    out[(int64_t)j * C + c] = acc[e][rc][q];
                }
        }
    }
}

__global__ __launch_bounds__(256) void split_sum(const float* __restrict__ partial, int splits, int r16, int r,
                                                 int64_t C, float scale, int transpose_out,
                                                 float* __restrict__ out) {
    const int64_t n = (int64_t)r * C;
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        const int64_t j = idx / C, c = idx % C;
        float s = 0.f;
        for (int k = 0; k < splits; ++k) s += partial[((int64_t)k * r16 + j) * C + c];
        s *= scale;
        if (transpose_out) out[c * r + j] = s;
        else out[j * C + c] = s;
    }
}

// -------------------------------------------------------- bf16 transpose
// 64 x 64 tiles through LDS: 16-byte row chunks in, 16-byte column chunks
// out (the frozen W of the backward GEMM, read and written once per call).
__global__ __launch_bounds__(256) void transpose_bf16(const uint16_t* __restrict__ in, int64_t rows, int64_t cols,
                                                      uint16_t* __restrict__ out) {
    __shared__ uint16_t tile[64][64 + 2];
    const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
    for (int i = threadIdx.x; i < 512; i += 256) {
        const int r = i >> 3, c = (i & 7) * 8;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (r0 + r < rows && c0 + c < cols) v = *reinterpret_cast<const uint4*>(in + (r0 + r) * cols + c0 + c);
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            tile[r][c + 2 * e] = (uint16_t)w[e];
            tile[r][c + 2 * e + 1] = (uint16_t)(w[e] >> 16);
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 512; i += 256) {
        const int c = i >> 3, r = (i & 7) * 8;  // output row c (input column), 8 input rows r..r+7
        if (c0 + c < cols && r0 + r < rows) {
            uint32_t w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = (uint32_t)tile[r + 2 * e][c] | ((uint32_t)tile[r + 2 * e + 1][c] << 16);
            *reinterpret_cast<uint4*>(out + (c0 + c) * rows + r0 + r) = make_uint4(w[0], w[1], w[2], w[3]);
        }
    }
}

// ------------------------------------------------------------ fp32 path
__global__ __launch_bounds__(256) void rowproj_f32(const float* __restrict__ X, int64_t T, int64_t C,
                                                   const float* __restrict__ P, int transpose_p, int r,
                                                   float scale, const uint8_t* __restrict__ mask, float keep,
                                                   float* __restrict__ out_t, float* __restrict__ out_ext,
                                                   float ext_scale) {
    // one wave per (token row, rank index); lanes split the reduction
    const int lane = lane_id();
    const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (item >= T * r) return;
    const int64_t t = item / r;
    const int j = (int)(item % r);
    const float* xr = X + t * C;
    float s = 0.f;
    for (int64_t c = lane; c < C; c += kWave) s += xr[c] * (transpose_p ? P[c * r + j] : P[(int64_t)j * C + c]);
    s = wave_sum(s);
    if (lane == 0) {
        float v = s * scale;
        if (mask) v = mask[t * r + j] ? v * keep : 0.f;
        if (out_t) out_t[(int64_t)j * T + t] = v;
        if (out_ext) out_ext[t * r + j] = v * ext_scale;
    }
}

__global__ __launch_bounds__(256) void colreduce_f32(const float* __restrict__ X, int64_t T, int64_t C,
                                                     const float* __restrict__ Pt, int r, float scale,
                                                     int transpose_out, float* __restrict__ out) {
    // thread per (j, c), c fastest: X reads are coalesced, Pt reads broadcast
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)r * C) return;
    const int64_t j = idx / C, c = idx % C;
    float s = 0.f;
    for (int64_t t = 0; t < T; ++t) s += Pt[j * T + t] * X[t * C + c];
    s *= scale;
    if (transpose_out) out[c * r + j] = s;
    else out[j * C + c] = s;
}

}  // namespace

hipError_t launch_prep_bf16(const float* src, int64_t ld_src, int64_t valid_rows, int64_t valid_cols,
                            bool transpose, uint16_t* hi, uint16_t* lo, int64_t rows_out,
                            int64_t cols_out, hipStream_t stream) {
    const int64_t n = rows_out * cols_out;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (blocks < 1) blocks = 1;
    prep_bf16<<<dim3((unsigned)blocks), 256, 0, stream>>>(src, ld_src, valid_rows, valid_cols, transpose ? 1 : 0,
                                                          hi, lo, rows_out, cols_out);
    return hipGetLastError();
}

hipError_t launch_rowproj_bf16(const uint16_t* X, int64_t T, int64_t C, const uint16_t* P_hi,
                               const uint16_t* P_lo, int r, float scale, const uint8_t* mask,
                               float keep, float* out_t, uint16_t* out_ext, int rext, float ext_scale,
                               hipStream_t stream) {
    const dim3 grid((unsigned)((T + 15) / 16));
    // P_hi / P_lo hold r16 = 16, 32, 64 or 128 rows (zero past r)
    const int rc = r <= 16 ? 1 : r <= 32 ? 2 : r <= 64 ? 4 : 8;
    switch (rc) {
        case 1: rowproj_bf16<1><<<grid, 256, 0, stream>>>(X, T, C, P_hi, P_lo, r, scale, mask, keep, out_t, out_ext, rext, ext_scale); break;
        case 2: rowproj_bf16<2><<<grid, 256, 0, stream>>>(X, T, C, P_hi, P_lo, r, scale, mask, keep, out_t, out_ext, rext, ext_scale); break;
        case 4: rowproj_bf16<4><<<grid, 256, 0, stream>>>(X, T, C, P_hi, P_lo, r, scale, mask, keep, out_t, out_ext, rext, ext_scale); break;
        default: rowproj_bf16<8><<<grid, 256, 0, stream>>>(X, T, C, P_hi, P_lo, r, scale, mask, keep, out_t, out_ext, rext, ext_scale); break;
    }
    return hipGetLastError();
}

// Column-tile count times splits should give >= ~1024 workgroups, with each
// wave still walking several 32-row steps.
int colreduce_splits(int64_t T, int64_t C) {
    const int64_t ctiles = (C + 127) / 128;
    int64_t s = (1536 + ctiles - 1) / ctiles;
    const int64_t max_s = (T + 511) / 512;  // >= 4 steps per wave
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    return (int)s;
}

hipError_t launch_colreduce_bf16(const uint16_t* X, int64_t T, int64_t C, const float* Pt, int r,
                                 int splits, float* partial, hipStream_t stream) {
    // Rank tiles are processed 32 at a time (accumulators and the LDS combine
    // buffer are sized for two 16-row MFMA tiles); each group re-reads X.
    const int64_t chunk = round_up((T + splits - 1) / splits, 32);
    const dim3 grid((unsigned)((C + 127) / 128), (unsigned)splits);
    const int64_t part_stride = (int64_t)(r <= 16 ? 16 : r <= 32 ? 32 : r <= 64 ? 64 : 128) * C;
    for (int g = 0; g * 32 < r; ++g) {
        const int rs = r - 32 * g < 32 ? r - 32 * g : 32;
        const float* pt = Pt + (int64_t)32 * g * T;
        float* part = partial + (int64_t)32 * g * C;
        if (rs <= 16)
            colreduce_bf16<1><<<grid, 256, 0, stream>>>(X, T, C, pt, rs, chunk, part, part_stride);
        else
            colreduce_bf16<2><<<grid, 256, 0, stream>>>(X, T, C, pt, rs, chunk, part, part_stride);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_split_sum(const float* partial, int splits, int r16, int r, int64_t C, float scale,
                            bool transpose_out, float* out, hipStream_t stream) {
    const int64_t n = (int64_t)r * C;
    int64_t blocks = (n + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    split_sum<<<dim3((unsigned)blocks), 256, 0, stream>>>(partial, splits, r16, r, C, scale,
                                                          transpose_out ? 1 : 0, out);
    return hipGetLastError();
}

hipError_t launch_transpose_bf16(const uint16_t* in, int64_t rows, int64_t cols, uint16_t* out,
                                 hipStream_t stream) {
    transpose_bf16<<<dim3((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64)), 256, 0, stream>>>(in, rows, cols,
                                                                                                      out);
    return hipGetLastError();
}

hipError_t launch_rowproj_f32(const float* X, int64_t T, int64_t C, const float* P, bool transpose_p,
                              int r, float scale, const uint8_t* mask, float keep, float* out_t,
                              float* out_ext, float ext_scale, hipStream_t stream) {
    const int64_t items = T * r;
    rowproj_f32<<<dim3((unsigned)((items + 3) / 4)), 256, 0, stream>>>(X, T, C, P, transpose_p ? 1 : 0, r, scale,
                                                                      mask, keep, out_t, out_ext, ext_scale);
    return hipGetLastError();
}

hipError_t launch_colreduce_f32(const float* X, int64_t T, int64_t C, const float* Pt, int r,
                                float scale, bool transpose_out, float* out, hipStream_t stream) {
    const int64_t n = (int64_t)r * C;
    colreduce_f32<<<dim3((unsigned)((n + 255) / 256)), 256, 0, stream>>>(X, T, C, Pt, r, scale,
                                                                         transpose_out ? 1 : 0, out);
    return hipGetLastError();
}

}  // namespace mc
