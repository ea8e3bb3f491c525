// GEMMs of the LoRA linear, gfx950.
//
// The frozen base projection of the reference is candle_nn::Linear,
// y = x.W^T (+ b) with W stored [out, in] (src/models/transformer.rs:189-192);
// the LoRA delta scale * Hd.B (src/training/lora.rs:336-339) is folded into
// the same GEMM as extra reduction columns:
//
//   forward   y  = [x | s*Hd] . [W | B^T]^T + b     (NT: both operands
//                                                   reduction-contiguous)
//   backward  dX = [dY | Gd] . [W ; A^T]            (NN: W rows are the
//                                                   reduction index)
//
// so one kernel produces the fused result with no separate epilogue pass
// over y / dX. The two reduction segments (main, rank extension) have
// their own base pointers and strides.
//
// bf16 kernel: 256 threads (4 waves as 2 x 2), tile 128 x 128 x 64, each
// wave 64 x 64 as 2 x 2 MFMA 32x32x16 bf16 blocks, fp32 accumulation.
// Operands are staged through LDS (row stride 72 bf16 = 144 B to spread
// banks), double-buffered with one barrier per k-step: global loads of
// step k+1 are issued before the MFMAs of step k. In NN mode the B tile is
// loaded as 8 x 8 blocks and transposed in registers before the LDS write,
// so both LDS tiles are reduction-contiguous and the MFMA reads are the
// same 16-byte ds_read in both modes.
#include "common.hpp"
#include "lora_kernels.hpp"

namespace mc {
namespace {

constexpr int BM = 128, BN = 128, BK = 64, LDK = BK + 8;

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

template <bool NN>
__global__ __launch_bounds__(256, 2) void gemm_bf16_kernel(int64_t M, int64_t N, GemmSeg s0, GemmSeg s1,
                                                           const uint16_t* __restrict__ bias,
                                                           uint16_t* __restrict__ C, int64_t ldc) {
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM * LDK];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN * LDK];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t m0 = (int64_t)blockIdx.y * BM, n0 = (int64_t)blockIdx.x * BN;
    const int nk0 = (int)((s0.k + BK - 1) / BK);
    const int nk = nk0 + (int)((s1.k + BK - 1) / BK);

    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

    uint4 ra[4];
    uint4 rb[NN ? 8 : 4];
    const uint4 zero = make_uint4(0, 0, 0, 0);

    auto load_tile = [&](int kt) {
        const GemmSeg& s = kt < nk0 ? s0 : s1;
        const int64_t kb = (int64_t)(kt < nk0 ? kt : kt - nk0) * BK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int chunk = tid + 256 * i;
            const int row = chunk >> 3, kc = (chunk & 7) * 8;
            const int64_t gm = m0 + row, k = kb + kc;
            ra[i] = (gm < M && k < s.k) ? *reinterpret_cast<const uint4*>(s.a + gm * s.lda + k) : zero;
        }
        if constexpr (!NN) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int chunk = tid + 256 * i;
                const int row = chunk >> 3, kc = (chunk & 7) * 8;
                const int64_t gn = n0 + row, k = kb + kc;
                rb[i] = (gn < N && k < s.k) ? *reinterpret_cast<const uint4*>(s.b + gn * s.ldb + k) : zero;
            }
        } else {
            if (tid < 128) {
                const int kr = (tid >> 4) * 8, nc = (tid & 15) * 8;
                const int64_t gn = n0 + nc;
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    const int64_t k = kb + kr + i;
                    rb[i] = (gn < N && k < s.k) ? *reinterpret_cast<const uint4*>(s.b + k * s.ldb + gn) : zero;
                }
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int chunk = tid + 256 * i;
            const int row = chunk >> 3, kc = (chunk & 7) * 8;
            *reinterpret_cast<uint4*>(&As[buf][row * LDK + kc]) = ra[i];
        }
        if constexpr (!NN) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int chunk = tid + 256 * i;
                const int row = chunk >> 3, kc = (chunk & 7) * 8;
                *reinterpret_cast<uint4*>(&Bs[buf][row * LDK + kc]) = rb[i];
            }
        } else {
            if (tid < 128) {
                const int kr = (tid >> 4) * 8, nc = (tid & 15) * 8;
                uint4 o[8];
                transpose8x8(rb, o);
#pragma unroll
                for (int e = 0; e < 8; ++e) *reinterpret_cast<uint4*>(&Bs[buf][(nc + e) * LDK + kr]) = o[e];
            }
        }
    };

    if (nk > 0) {
        load_tile(0);
        store_tile(0);
    }
    __syncthreads();
    const int frag_row = lane & 31, frag_k = (lane >> 5) * 8;
    for (int kt = 0; kt < nk; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < nk) load_tile(kt + 1);
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            bf16x8 a[2], b[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                a[t] = *reinterpret_cast<const bf16x8*>(&As[buf][(wm * 64 + t * 32 + frag_row) * LDK + ks * 16 + frag_k]);
                b[t] = *reinterpret_cast<const bf16x8*>(&Bs[buf][(wn * 64 + t * 32 + frag_row) * LDK + ks * 16 + frag_k]);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store_tile(buf ^ 1);
        __syncthreads();
    }

    // Epilogue: MFMA 32x32 accumulator q of lane l holds row
    // 8*(q/4) + 4*(l/32) + q%4, column l%32 of the block.
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int64_t gn = n0 + wn * 64 + j * 32 + (lane & 31);
        if (gn >= N) continue;
        const float bv = bias ? bf16_to_f32(bias[gn]) : 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const int64_t gm = m0 + wm * 64 + i * 32 + 8 * (q >> 2) + 4 * (lane >> 5) + (q & 3);
                if (gm < M) C[gm * ldc + gn] = f32_to_bf16(acc[i][j][q] + bv);
            }
    }
}

// ------------------------------------------------------------- fp32 GEMM
// 64 x 64 tile, 16-deep k-steps, 4 x 4 outputs per thread, sequential FMA
// chain over k (fixed order).
template <bool NN>
__global__ __launch_bounds__(256) void gemm_f32_kernel(int64_t M, int64_t N, GemmSegF32 s0, GemmSegF32 s1,
                                                       const float* __restrict__ bias, float* __restrict__ C,
                                                       int64_t ldc) {
    constexpr int TM = 64, TN = 64, TK = 16;
    __shared__ float As[TK][TM + 4];
    __shared__ float Bs[TK][TN + 4];
    const int tid = threadIdx.x;
    const int ty = tid >> 4, tx = tid & 15;
    const int64_t m0 = (int64_t)blockIdx.y * TM, n0 = (int64_t)blockIdx.x * TN;
    const int nk0 = (int)((s0.k + TK - 1) / TK);
    const int nk = nk0 + (int)((s1.k + TK - 1) / TK);
    float acc[4][4] = {};
    for (int kt = 0; kt < nk; ++kt) {
        const GemmSegF32& s = kt < nk0 ? s0 : s1;
        const int64_t kb = (int64_t)(kt < nk0 ? kt : kt - nk0) * TK;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = tid + 256 * i;
            const int m = e >> 4, k = e & 15;
            const int64_t gm = m0 + m, gk = kb + k;
            As[k][m] = (gm < M && gk < s.k) ? s.a[gm * s.lda + gk] : 0.f;
            if constexpr (!NN) {
                const int64_t gn = n0 + m;
                Bs[k][m] = (gn < N && gk < s.k) ? s.b[gn * s.ldb + gk] : 0.f;
            } else {
                const int kk = e >> 6, n = e & 63;
                const int64_t gn = n0 + n, gk2 = kb + kk;
                Bs[kk][n] = (gn < N && gk2 < s.k) ? s.b[gk2 * s.ldb + gn] : 0.f;
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < TK; ++k) {
            float a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) { a[i] = As[k][ty * 4 + i]; b[i] = Bs[k][tx * 4 + i]; }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t gm = m0 + ty * 4 + i;
        if (gm >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t gn = n0 + tx * 4 + j;
            if (gn < N) C[gm * ldc + gn] = acc[i][j] + (bias ? bias[gn] : 0.f);
        }
    }
}

}  // namespace

hipError_t launch_gemm_bf16(bool nn, int64_t M, int64_t N, GemmSeg s0, GemmSeg s1, const uint16_t* bias,
                            uint16_t* c, int64_t ldc, hipStream_t stream) {
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    if (nn) gemm_bf16_kernel<true><<<grid, 256, 0, stream>>>(M, N, s0, s1, bias, c, ldc);
    else gemm_bf16_kernel<false><<<grid, 256, 0, stream>>>(M, N, s0, s1, bias, c, ldc);
    return hipGetLastError();
}

hipError_t launch_gemm_f32(bool nn, int64_t M, int64_t N, GemmSegF32 s0, GemmSegF32 s1, const float* bias,
                           float* c, int64_t ldc, hipStream_t stream) {
    const dim3 grid((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
    if (nn) gemm_f32_kernel<true><<<grid, 256, 0, stream>>>(M, N, s0, s1, bias, c, ldc);
    else gemm_f32_kernel<false><<<grid, 256, 0, stream>>>(M, N, s0, s1, bias, c, ldc);
    return hipGetLastError();
}

}  // namespace mc
