// Attention core of the reference decoder layer, gfx950.
//
// Attention::forward (src/models/transformer.rs:258-283) computes, for every
// batch b and query head h, with the K/V heads repeated by repeat_kv
// (transformer.rs:295-319: query head h reads K/V head h / (H / Hkv)):
//
//     scores = q . k^T / sqrt(d)  (+ attention_mask, broadcast over b, h)
//     p      = softmax_stable(scores)              (src/backend/tensor.rs:91-98)
//     o      = p . v, written [B, S, H * D]        (transpose(1, 2) + reshape)
//
// The [S, S] score matrix never reaches HBM. bf16, D = 64 or 128:
//
//  attn_vt_bf16   V [B, Hkv, S, D] -> V^T [B, Hkv, D, Sp] (Sp = S rounded up to
//                 64, zero padded), keys permuted inside each 16-key group so
//                 that the MFMA operand of P.V is one 16-byte LDS read.
//  attn_fwd_bf16  one workgroup per (b, h, 128 queries), 4 waves of 32 queries.
//                 Per block of 64 keys, K [64, D] and V^T [D, 64] go straight
//                 into LDS (buffer_load ... lds, two stages), and each wave
//                   S^T = K . Q^T       MFMA 32x32x16, Q^T fragments held in
//                                       registers for the whole loop;
//                   online softmax      a lane holds 32 of the 64 scores of
//                                       one query (its partner lane l ^ 32 the
//                                       other 32): one exchange per block for
//                                       the row max;
//                   O^T += V^T . P^T    P^T straight from the S^T accumulators
//                                       (rounded to bf16), V^T from LDS.
//                 Scores are kept in the log2 domain (scale * log2 e folded in)
//                 and exponentiated with exp2. Causal blocks past a wave's last
//                 query are skipped; heavier query blocks are dispatched first.
//                 The output goes through LDS for 16-byte row stores; the
//                 log-sum-exp of every score row is saved for the backward.
//
// Other head dims and fp32: attn_fwd_generic, one wave per query row (lanes
// over the head dim), online softmax in fp32.
#include "common.hpp"
#include "kernels.hpp"

namespace mc {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr float kNegInf = -__builtin_inff();

// Position p of a 16-key group of the transposed V holds key perm16(p): the
// positions 0-3, 4-7, 8-11, 12-15 hold keys 0-3, 8-11, 4-7, 12-15 (bits 2 and
// 3 swapped; the map is its own inverse). This is the order in which a lane
// half of the S^T accumulator holds its keys (rows 8 (j/4) + 4 (l/32) + j%4).
__device__ __forceinline__ int perm16(int p) { return (p & 3) | ((p & 4) << 1) | ((p & 8) >> 1); }

// ------------------------------------------------------------ V^T prepass
// Workgroup: one (b, kv head) and one block of 64 keys; the [64, D] tile is
// staged through LDS (rows padded by 16 bytes) and written as D rows of 64
// permuted key positions. Keys past S are written as zeros.
template <int D>
__global__ __launch_bounds__(256) void attn_vt_bf16(const uint16_t* __restrict__ V, int64_t S, int64_t Sp,
                                                    uint16_t* __restrict__ Vt) {
    constexpr int CPR = D / 8;
    __shared__ __attribute__((aligned(16))) uint16_t tile[64][D + 8];
    const int64_t bh = blockIdx.y;
    const int64_t k0 = (int64_t)blockIdx.x * 64;
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(V + bh * S * D, S * D * 2);
    for (int i = threadIdx.x; i < 64 * CPR; i += 256) {
        const int key = i / CPR, c = i % CPR;
        const uint32_t off = k0 + key < S ? (uint32_t)(((k0 + key) * D + 8 * c) * 2) : kOOB;
        const i32x4 v = buf_load16(rv, off);
        *reinterpret_cast<i32x4*>(&tile[key][8 * c]) = v;
    }
    __syncthreads();
    uint16_t* dst = Vt + bh * D * Sp + k0;
    for (int i = threadIdx.x; i < D * 8; i += 256) {
        const int d = i >> 3, c = i & 7;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int p0 = 8 * c + 2 * e, p1 = p0 + 1;
            const int key0 = (p0 & ~15) | perm16(p0 & 15), key1 = (p1 & ~15) | perm16(p1 & 15);
            w[e] = (uint32_t)tile[key0][d] | ((uint32_t)tile[key1][d] << 16);
        }
        *reinterpret_cast<uint4*>(dst + (int64_t)d * Sp + 8 * c) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// ------------------------------------------------------- flash forward
struct AttnFwdArgs {
    const uint16_t* q;   // [B, H, S, D]
    const uint16_t* k;   // [B, Hkv, S, D]
    const uint16_t* vt;  // [B, Hkv, D, Sp]
    const float* mask;   // [S, S] additive, or null
    uint16_t* o;         // [B, S, H, D]
    float* lse;          // [B, H, S], or null
    int64_t S, Sp;
    int B, H, Hkv, nqb, causal;
    float scale_log2;    // score scale * log2 e
};

template <int D>
__global__ __launch_bounds__(256, 2) void attn_fwd_bf16(AttnFwdArgs a) {
    constexpr int KB = 64;            // keys per block
    constexpr int QB = 128;           // queries per workgroup, 32 per wave
    constexpr int KS = D / 16;        // MFMA k-steps over the head dim
    constexpr int DT = D / 32;        // 32-row tiles of O^T
    constexpr int K_ELEMS = KB * D;   // K tile [64][D], rows of D bf16
    constexpr int STAGE = 2 * KB * D; // K tile, then V^T tile [D][64]
    constexpr int CPR_K = D / 8, RPI_K = 64 / CPR_K;
    constexpr int LOADS_K = KB / RPI_K / 4, LOADS_V = D / 8 / 4;  // DMA per wave per block
    static_assert(LOADS_K >= 1 && LOADS_V >= 1, "tile split over 4 waves");
    __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * STAGE];
    const uint32_t smem_byte = (uint32_t)reinterpret_cast<uintptr_t>(smem);

    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int col = lane & 31, half = lane >> 5;
    const int nbh = a.B * a.H;
    const int qb = a.nqb - 1 - (int)(blockIdx.x / nbh);  // heaviest query blocks first
    const int bh = (int)(blockIdx.x % nbh);
    const int b = bh / a.H, h = bh % a.H;
    const int hk = h / (a.H / a.Hkv);
    const int64_t S = a.S;
    const int64_t q0 = (int64_t)qb * QB;
    const int64_t qw = q0 + 32 * wave;  // first query of this wave
    const int64_t my_q = qw + col;

    // Q^T fragments (B operand of S^T = K.Q^T): query my_q, dims 16 s + 8 half .. +7.
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q + (int64_t)bh * S * D, S * D * 2);
    bf16x8 qf[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        const uint32_t off = my_q < S ? (uint32_t)((my_q * D + 16 * s + 8 * half) * 2) : kOOB;
        qf[s] = __builtin_bit_cast(bf16x8, buf_load16(rq, off));
    }

    const int64_t bhk = (int64_t)b * a.Hkv + hk;
    const i32x4 rk = rsrc_words(a.k + bhk * S * D, S * D * 2);
    const i32x4 rv = rsrc_words(a.vt + bhk * D * a.Sp, (int64_t)D * a.Sp * 2);

    const int nkb_all = (int)((S + KB - 1) / KB);
    int nkb = nkb_all, wkb = nkb_all;  // key blocks of the workgroup / of this wave
    if (a.causal) {
        nkb = min(nkb_all, (int)((min(q0 + QB, S) - 1) / KB) + 1);
        wkb = min(nkb, (int)(min(qw + 31, S - 1) / KB) + 1);
    }
    if (qw >= S) wkb = 0;

    // K rows key0 .. key0+63 into the swizzled [64][D] layout, then V^T rows
    // d = 0 .. D-1 (64 positions each) into [D][64]. Rows of K past S load as
    // zeros (buffer range); V^T is zero padded up to Sp.
    auto issue = [&](int kb, int stage) {
        const uint32_t base = smem_byte + (uint32_t)(stage * STAGE * 2);
        const uint32_t key0 = (uint32_t)kb * KB;
#pragma unroll
        for (int j = 0; j < LOADS_K; ++j) {
            const int blk = wave * LOADS_K + j;
            const int row = blk * RPI_K + lane / CPR_K;
            const uint32_t chunk = (uint32_t)swz<D>(row, lane % CPR_K);
            const uint32_t off = ((key0 + (uint32_t)row) * D + 8u * chunk) * 2u;
            dma16(rk, __builtin_amdgcn_readfirstlane(base + (uint32_t)blk * 1024u), off);
        }
#pragma unroll
        for (int j = 0; j < LOADS_V; ++j) {
            const int blk = wave * LOADS_V + j;
            const int row = blk * 8 + lane / 8;
            const uint32_t chunk = (uint32_t)swz<64>(row, lane % 8);
            const uint32_t off = ((uint32_t)row * (uint32_t)a.Sp + key0 + 8u * chunk) * 2u;
            dma16(rv, __builtin_amdgcn_readfirstlane(base + (uint32_t)(K_ELEMS * 2) + (uint32_t)blk * 1024u), off);
        }
    };

    f32x16 oacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) oacc[t][j] = 0.f;
    float m_run = kNegInf, l_run = 0.f;
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(a.mask, a.mask ? S * S * 4 : 0);

    if (nkb > 0) issue(0, 0);
    for (int kb = 0; kb < nkb; ++kb) {
        wait_vmcnt<0>();
        __syncthreads();
        if (kb + 1 < nkb) issue(kb + 1, (kb + 1) & 1);
        if (kb >= wkb) continue;  // wave-uniform: no query of this wave sees the block
        const uint16_t* sk = smem + (kb & 1) * STAGE;
        const uint16_t* sv = sk + K_ELEMS;

        // S^T tiles t = 0, 1 (keys 32 t .. 32 t + 31) x the wave's 32 queries
        f32x16 sacc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 16; ++j) sacc[t][j] = 0.f;
#pragma unroll
        for (int s = 0; s < KS; ++s)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int row = 32 * t + col;
                const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&sk[row * D + 8 * swz<D>(row, 2 * s + half)]);
                sacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[s], sacc[t], 0, 0, 0);
            }

        // accumulator j of tile t is key key0 + 32 t + 8 (j/4) + 4 half + j%4
        const int64_t key0 = (int64_t)kb * KB;
        float x[2][16];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 16; ++j) x[t][j] = sacc[t][j] * a.scale_log2;
        if (a.mask) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int64_t key = key0 + 32 * t + 8 * (j >> 2) + 4 * half + (j & 3);
                    const uint32_t off = (my_q < S && key < S) ? (uint32_t)((my_q * S + key) * 4) : kOOB;
                    x[t][j] += __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rm, (int)off, 0, 0)) * kLog2e;
                }
        }
        const bool edge = key0 + KB > S || (a.causal && key0 + KB - 1 > qw);
        if (edge) {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int64_t key = key0 + 32 * t + 8 * (j >> 2) + 4 * half + (j & 3);
                    if (key >= S || (a.causal && key > my_q)) x[t][j] = kNegInf;
                }
        }

        // online softmax over this block's 64 keys (32 here, 32 in lane ^ 32)
        float mx = x[0][0];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 16; ++j) mx = fmaxf(mx, x[t][j]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
        const float m_new = fmaxf(m_run, mx);
        const float m_use = m_new == kNegInf ? 0.f : m_new;  // a row with no key yet keeps p = 0
        const float alpha = exp2f(m_run - m_use);
        m_run = m_new;
        float ps = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                x[t][j] = exp2f(x[t][j] - m_use);
                ps += x[t][j];
            }
        l_run = l_run * alpha + ps;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
            for (int j = 0; j < 16; ++j) oacc[t][j] *= alpha;

        // P^T fragments: k-step (t, kk) takes accumulators 8 kk .. 8 kk + 7 of
        // tile t, i.e. keys 32 t + 16 kk + perm16(8 half + e), e = 0..7.
        bf16x8 pf[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int e = 0; e < 8; ++e) pf[t][kk][e] = static_cast<__bf16>(x[t][8 * kk + e]);

        // O^T (d x query) += V^T . P^T; V^T positions 16 (2t + kk) + 8 half .. +7
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int row = 32 * dt + col;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const int chunk = 4 * t + 2 * kk + half;
                    const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&sv[row * KB + 8 * swz<64>(row, chunk)]);
                    oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[t][kk], oacc[dt], 0, 0, 0);
                }
        }
    }

    // normalise; l = 0 (every key masked) gives 0/0 = NaN, as softmax of an
    // all -inf row does in the reference
    const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
    const float inv = 1.f / l_tot;
    if (a.lse && half == 0 && my_q < S) a.lse[(int64_t)bh * S + my_q] = (m_run + __log2f(l_tot)) * kLn2;

    // O^T accumulator j of tile dt is dim 32 dt + 8 (j/4) + 4 half + j%4 of
    // query my_q: through a per-wave LDS patch [32 queries][D + 8] to 16-byte
    // row stores.
    __syncthreads();
    constexpr int PROW = D + 8;
    uint16_t* patch = smem + wave * 32 * PROW;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const int d = 32 * dt + 8 * jq + 4 * half;
            const uint32_t lo = pack_bf16x2(oacc[dt][4 * jq] * inv, oacc[dt][4 * jq + 1] * inv);
            const uint32_t hi = pack_bf16x2(oacc[dt][4 * jq + 2] * inv, oacc[dt][4 * jq + 3] * inv);
            *reinterpret_cast<uint2*>(&patch[col * PROW + d]) = make_uint2(lo, hi);
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's patch is written
    constexpr int CPRO = D / 8;
    const int64_t ld = (int64_t)a.H * D;
    uint16_t* obase = a.o + ((int64_t)b * S * a.H + h) * D;
#pragma unroll
    for (int it = 0; it < 32 * CPRO / 64; ++it) {
        const int i = it * 64 + lane;
        const int r = i / CPRO, c = i % CPRO;
        if (qw + r < S) {
            const uint4 v = *reinterpret_cast<const uint4*>(&patch[r * PROW + 8 * c]);
            *reinterpret_cast<uint4*>(obase + (qw + r) * ld + 8 * c) = v;
        }
    }
}

// ----------------------------------------------------- generic forward
// One wave per (b, h, query); lane l holds dims l, l + 64, l + 128, l + 192.
template <typename T>
__global__ __launch_bounds__(256) void attn_fwd_generic(const T* __restrict__ q, const T* __restrict__ k,
                                                        const T* __restrict__ v, const float* __restrict__ mask,
                                                        T* __restrict__ o, float* __restrict__ lse, int B, int H,
                                                        int Hkv, int64_t S, int D, float scale, int causal) {
    const int lane = lane_id();
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= (int64_t)B * H * S) return;
    const int64_t bh = row / S, qi = row % S;
    const int b = (int)(bh / H), h = (int)(bh % H);
    const int64_t bhk = (int64_t)b * Hkv + h / (H / Hkv);
    float qv[4], acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        qv[i] = d < D ? Elem<T>::load(q, (bh * S + qi) * D + d) : 0.f;
        acc[i] = 0.f;
    }
    float m = kNegInf, l = 0.f;
    const int64_t kend = causal ? qi + 1 : S;
    for (int64_t key = 0; key < kend; ++key) {
        const int64_t kr = (bhk * S + key) * D;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = lane + 64 * i;
            if (d < D) s += qv[i] * Elem<T>::load(k, kr + d);
        }
        s = wave_sum(s) * scale;
        if (mask) s += mask[qi * S + key];
        const float m_new = fmaxf(m, s);
        const float m_use = m_new == kNegInf ? 0.f : m_new;
        const float alpha = __expf(m - m_use), p = __expf(s - m_use);
        l = l * alpha + p;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int d = lane + 64 * i;
            acc[i] = acc[i] * alpha + (d < D ? p * Elem<T>::load(v, kr + d) : 0.f);
        }
        m = m_new;
    }
    const float inv = 1.f / l;
    const int64_t orow = ((int64_t)b * S + qi) * H + h;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int d = lane + 64 * i;
        if (d < D) Elem<T>::store(o, orow * D + d, acc[i] * inv);
    }
    if (lse && lane == 0) lse[bh * S + qi] = m + __logf(l);
}

}  // namespace

AttnWs attention_fwd_ws(const mc_attn_desc& d) {
    AttnWs w{};
    if (attention_uses_mfma(d)) {
        const int64_t Sp = (d.seq + 63) / 64 * 64;
        w.vt = 0;
        w.total = (size_t)d.batch * d.kv_heads * d.head_dim * Sp * 2;
    }
    return w;
}

bool attention_uses_mfma(const mc_attn_desc& d) {
    return d.dtype == MC_BF16 && (d.head_dim == 64 || d.head_dim == 128);
}

hipError_t launch_attention_fwd(const mc_attn_desc& d, const void* q, const void* k, const void* v,
                                const float* mask, void* o, float* lse, void* ws, hipStream_t stream) {
    const int B = (int)d.batch, H = d.heads, Hkv = d.kv_heads, D = d.head_dim;
    const int64_t S = d.seq;
    if (attention_uses_mfma(d)) {
        const int64_t Sp = (S + 63) / 64 * 64;
        uint16_t* vt = static_cast<uint16_t*>(ws);
        AttnFwdArgs a;
        a.q = static_cast<const uint16_t*>(q);
        a.k = static_cast<const uint16_t*>(k);
        a.vt = vt;
        a.mask = mask;
        a.o = static_cast<uint16_t*>(o);
        a.lse = lse;
        a.S = S;
        a.Sp = Sp;
        a.B = B; a.H = H; a.Hkv = Hkv;
        a.nqb = (int)((S + 127) / 128);
        a.causal = d.causal ? 1 : 0;
        a.scale_log2 = d.scale * kLog2e;
        const dim3 gvt((unsigned)(Sp / 64), (unsigned)(B * Hkv));
        const dim3 grid((unsigned)((int64_t)a.nqb * B * H));
        if (D == 64) {
            attn_vt_bf16<64><<<gvt, 256, 0, stream>>>(static_cast<const uint16_t*>(v), S, Sp, vt);
            attn_fwd_bf16<64><<<grid, 256, 0, stream>>>(a);
        } else {
            attn_vt_bf16<128><<<gvt, 256, 0, stream>>>(static_cast<const uint16_t*>(v), S, Sp, vt);
            attn_fwd_bf16<128><<<grid, 256, 0, stream>>>(a);
        }
        return hipGetLastError();
    }
    const dim3 grid((unsigned)(((int64_t)B * H * S + 3) / 4));
    if (d.dtype == MC_F32)
        attn_fwd_generic<float><<<grid, 256, 0, stream>>>(static_cast<const float*>(q), static_cast<const float*>(k),
                                                          static_cast<const float*>(v), mask, static_cast<float*>(o),
                                                          lse, B, H, Hkv, S, D, d.scale, d.causal);
    else
        attn_fwd_generic<uint16_t><<<grid, 256, 0, stream>>>(
            static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), mask,
            static_cast<uint16_t*>(o), lse, B, H, Hkv, S, D, d.scale, d.causal);
    return hipGetLastError();
}

}  // namespace mc
