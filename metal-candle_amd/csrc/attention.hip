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
#include <algorithm>
#include <type_traits>

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
// Growth of a row's score max (log2 units) that the forward absorbs before it
// moves its softmax reference point and rescales O.
constexpr float kMaxSlack = 8.f;

// 64-bit integer min / max. (The device min / max templates instantiated at
// int64_t were lowered through double-precision min / max and conversions.)
__device__ __forceinline__ int64_t min64(int64_t x, int64_t y) { return x < y ? x : y; }
__device__ __forceinline__ int64_t max64(int64_t x, int64_t y) { return x > y ? x : y; }

// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008, kSchedDsRead = 0x100;

// max(v of lane l, v of lane l ^ 32) without LDS. v_permlane32_swap swaps
// lanes 32-63 of its first register with lanes 0-31 of its second; with v in
// both, every lane then holds v of lanes l & 31 and (l & 31) + 32.
__device__ __forceinline__ float half_pair_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Position of a workgroup among the B * H (batch, head) workgroups of its
// query-block round. Workgroups are dispatched round-robin over the 8 XCDs
// (id mod 8); when the round is a multiple of 8 long, each XCD takes a
// contiguous run of (b, h), so the heads that share a K / V head share that
// XCD's L2. The rounds, heaviest query blocks first, keep their order.
__device__ __forceinline__ int xcd_head_order(int j, int nbh) {
    return (nbh & 7) ? j : (j & 7) * (nbh >> 3) + (j >> 3);
}

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

// RAW: no additive mask and a positive scale, so the scores can stay
// unscaled until the exponent (see the online softmax below).
template <int D, bool RAW>
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
    const int bh = xcd_head_order((int)(blockIdx.x % nbh), nbh);
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
        // K fragments one k-step ahead of their MFMAs, so each pair's LDS
        // latency runs under the previous pair's MFMAs
        bf16x8 kf[2][2];
        auto kread = [&](int s, int slot) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int row = 32 * t + col;
                kf[slot][t] = *reinterpret_cast<const bf16x8*>(&sk[row * D + 8 * swz<D>(row, 2 * s + half)]);
            }
        };
        kread(0, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            if (s + 1 < KS) {
                kread(s + 1, (s + 1) & 1);
                __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
            }
#pragma unroll
            for (int t = 0; t < 2; ++t)
                sacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[s & 1][t], qf[s], sacc[t], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
        }

        // accumulator j of tile t is key key0 + 32 t + 8 (j/4) + 4 half + j%4.
        // RAW: the scores stay unscaled, the max is taken over the raw
        // products and scaled once, and the scale goes into the exponent's
        // fma (one fma per score instead of a multiply and a subtract).
        // Otherwise x holds scale * log2 e * s (+ mask) and cx = 1.
        const int64_t key0 = (int64_t)kb * KB;
        float x[2][16];
        const float cx = RAW ? a.scale_log2 : 1.f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 16; ++j) x[t][j] = RAW ? sacc[t][j] : sacc[t][j] * a.scale_log2;
        if (!RAW && a.mask) {
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
            // key offsets in the block (32 t + 8 (j/4) + 4 half + j%4) against
            // the first offset past S and, causal, this lane's query offset;
            // the lane's 4 half moves to the bounds, so each test compares a
            // constant
            const int lim = (int)min64(S - key0, KB) - 4 * half;
            const int qrel = (a.causal ? (int)max64(min64(my_q - key0, KB), -1) : KB) - 4 * half;
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int ko = 32 * t + 8 * (j >> 2) + (j & 3);
                    if (ko >= lim || ko > qrel) x[t][j] = kNegInf;
                }
        }

        // online softmax over this block's 64 keys (32 here, 32 in lane ^ 32)
        float mx = x[0][0];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 16; ++j) mx = fmaxf(mx, x[t][j]);
        mx = half_pair_max(mx) * cx;  // cx > 0: -inf stays -inf
        // The reference point m_run moves only when the block's max exceeds
        // it by more than kMaxSlack (log2 units; first block: any finite max).
        // Below that, p = 2^(x - m_run) stays under 2^kMaxSlack, which fp32 sums
        // and bf16 P carry at full relative precision, and O and l keep one
        // common reference, so the result is the same softmax; what it saves
        // is the O rescale of every block whose max moved a little, which for
        // 32 queries per wave was nearly every block.
        float alpha = 1.f;
        if (mx > m_run + kMaxSlack) {
            alpha = exp2_hw(m_run - mx);  // m_run = -inf: 0 (O and l are 0 then)
            m_run = mx;
        }
        const float m_use = m_run == kNegInf ? 0.f : m_run;  // a row with no key yet keeps p = 0
        float ps = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                x[t][j] = exp2_hw(__builtin_fmaf(x[t][j], cx, -m_use));
                ps += x[t][j];
            }
        l_run = l_run * alpha + ps;
        // rescale O only when some lane's running max moved (alpha = 1
        // elsewhere, so skipping the multiply changes nothing)
        if (__any(alpha != 1.f)) {
#pragma unroll
            for (int t = 0; t < DT; ++t)
#pragma unroll
                for (int j = 0; j < 16; ++j) oacc[t][j] *= alpha;
        }

        // P^T fragments: k-step (t, kk) takes accumulators 8 kk .. 8 kk + 7 of
        // tile t, i.e. keys 32 t + 16 kk + perm16(8 half + e), e = 0..7.
        bf16x8 pf[2][2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) pf[t][kk] = pack_bf16x8(&x[t][8 * kk]);

        // O^T (d x query) += V^T . P^T; V^T positions 16 (2t + kk) + 8 half .. +7.
        // Step v = 2 dt + t multiplies two fragments (kk = 0, 1), read one
        // step ahead of their MFMAs.
        bf16x8 vf[2][2];
        auto vread = [&](int v, int slot) {
            const int row = 32 * (v >> 1) + col, t = v & 1;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
                vf[slot][kk] = *reinterpret_cast<const bf16x8*>(&sv[row * KB + 8 * swz<64>(row, 4 * t + 2 * kk + half)]);
        };
        vread(0, 0);
        __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
        for (int v = 0; v < 2 * DT; ++v) {
            if (v + 1 < 2 * DT) {
                vread(v + 1, (v + 1) & 1);
                __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
            }
            const int dt = v >> 1, t = v & 1;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
                oacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[v & 1][kk], pf[t][kk], oacc[dt], 0, 0, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
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

// ================================================================ backward
// Gradients of the forward (candle autograd of transformer.rs:264-278; the
// reference has no kernel): with P = softmax(scores), dO the output gradient
// [B, S, H, D], Delta_i = sum_d dO_id O_id and lse_i the forward's
// log-sum-exp,
//   P_ij = exp(scale q_i.k_j + mask_ij - lse_i)      (recomputed)
//   dP_ij = dO_i . v_j,   dS_ij = P_ij (dP_ij - Delta_i)
//   dV_j = sum_i P_ij dO_i,   dK_j = scale sum_i dS_ij q_i,   dQ_i = scale sum_j dS_ij k_j
// and dK / dV of a K/V head sum over the H / Hkv query heads that read it.
// Every sum runs in a fixed order: results are bitwise reproducible.
//
// bf16, D = 64 or 128:
//  attn_bwd_prep_bf16  per (b, h, 64 queries): Delta and lse * log2 e, both
//                      into one [2][64] fp32 block per query block.
//  attn_bwd_dkdv_bf16  one workgroup per (b, K/V head, group of query heads,
//                      128 keys), 4 waves of 32 keys; for each query head of
//                      the group, per block of 64 queries (Q, dO and the
//                      lse/Delta block through LDS, two stages):
//                        S = Q.K^T, dP = dO.V^T    (lane = key: K, V held in
//                                                   registers as B operands)
//                        dV^T += dO^T.P,  dK^T += Q^T.dS   (P, dS straight from
//                                                   the accumulators as the
//                                                   B operand; dO^T, Q^T by
//                                                   transposed LDS reads of
//                                                   the dO, Q tiles)
//                      dK, dV accumulate over the group's heads: written
//                      directly when one group holds all H / Hkv heads of a
//                      K/V head, else as fp32 partials per group summed by
//                      attn_bwd_sum; dS^T (bf16, key rows) stored for the
//                      dQ pass.
//  attn_bwd_dq_ds_bf16 one workgroup per (b, h, 128 queries):
//                        dQ^T += K^T.dS^T         (both operands by transposed
//                                                   LDS reads of the K and
//                                                   stored dS^T tiles)
//  attn_bwd_dq_bf16    the same without a stored dS^T (S * ldst * 2 bytes of a
//                      head past 2^31), shaped as the forward:
//                        S^T = K.Q^T, dP^T = V.dO^T (lane = query: Q, dO held
//                                                   in registers)
//                        dQ^T += K^T.dS^T         (K^T by transposed LDS
//                                                   reads of the K tile)
struct AttnBwdArgs {
    const uint16_t* q;     // [B, H, S, D]
    const uint16_t* k;     // [B, Hkv, S, D]
    const uint16_t* v;     // [B, Hkv, S, D]
    const uint16_t* dout;  // [B, S, H, D]
    const float* mask;     // [S, S] or null
    const float* lsd;      // [B, H, Sp / 64, 2, 64]: lse * log2 e, Delta
    uint16_t* dq;          // [B, H, S, D]
    uint16_t* dk;          // [B, Hkv, S, D] (H == Hkv)
    uint16_t* dv;
    float* dk_part;        // [B, H, S, D] fp32 (H > Hkv)
    float* dv_part;
    uint16_t* dst;         // [B, H, S, ldst]: dS^T (key rows, query columns) for the dQ pass, or null
    int64_t ldst;
    int ngroups;           // query-head groups per K/V head in the dK/dV kernel (H / Hkv / ngroups heads each)
    int64_t dq_blocks;     // the dQ pass's own workgroups; blocks past them sum the groups' partials
    int64_t sum_n8;        // 8-element units of one of dk / dv (B Hkv S D / 8)
    int64_t S, Sp;
    int B, H, Hkv, causal, nblk;
    float scale, scale_log2;
};

// Position of 16-byte chunk c of row r in the backward's [64][D] LDS tiles.
// Two read patterns must be bank-conflict free (64 banks x 4 B): row reads
// (16 consecutive rows of one chunk per 16 lanes) need the row's low bits to
// permute the chunk; the transposed reads (4 consecutive rows x 4
// consecutive chunks per 32 lanes) need the row's two lowest bits on the
// chunk's bits 2-3. Swapping the row's bit pairs 0-1 and 2-3 into the XOR
// mask serves both (D = 128: 16 chunks per 256-byte row; D = 64: 8 chunks,
// two rows per 256 bytes). The row-major swizzle of the forward (swz) put
// two (row, chunk) pairs of each transposed read on one bank group.
template <int D>
__device__ __forceinline__ int aswz(int r, int c) {
    static_assert(D == 64 || D == 128, "head dims with an MFMA backward");
    if constexpr (D == 128) return c ^ (((r & 3) << 2) | ((r >> 2) & 3));
    else return c ^ ((((r >> 1) & 1) << 2) | ((r >> 2) & 3));
}

// [ROWS][D] tile into the swizzled LDS layout from rows row0 .. row0+ROWS-1
// of a buffer with row stride ld (elements); rows past the buffer load zeros.
// Each of the 4 waves issues LOADS of the tile's 1 KB DMA pieces.
template <int D, int ROWS = 64>
__device__ __forceinline__ void dma_rows(i32x4 r, uint32_t lds_byte, uint32_t row0, uint32_t ld, int wave,
                                         int lane) {
    constexpr int CPR = D / 8, RPI = 64 / CPR, LOADS = ROWS / RPI / 4;
    static_assert(LOADS >= 1 && LOADS * RPI * 4 == ROWS, "whole 1 KB pieces per wave");
#pragma unroll
    for (int j = 0; j < LOADS; ++j) {
        const int blk = wave * LOADS + j;
        const int row = blk * RPI + lane / CPR;
        const uint32_t chunk = (uint32_t)aswz<D>(row, lane % CPR);
        const uint32_t off = ((row0 + (uint32_t)row) * ld + 8u * chunk) * 2u;
        dma16(r, __builtin_amdgcn_readfirstlane(lds_byte + (uint32_t)blk * 1024u), off);
    }
}

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i % 4
// of the 8-byte pieces addressed by the group's lanes i / 4, 4 + i / 4,
// 8 + i / 4 and 12 + i / 4 (in that order).
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
__device__ __forceinline__ s16x4 ds_read_tr16(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
}

// MFMA 32x32x16 fragments from a swizzled [rows][D] tile, addressed by
// per-lane byte offsets computed once per kernel. Inside a tile the swizzle
// depends only on a row's low four bits, so the lane's offset is the same for
// every 32-row (row fragments) or 16-row (transposed fragments) step of the
// tile, and the step enters as a constant that folds into the LDS
// instruction's offset field; the kernels hold a handful of offsets rather
// than one address per fragment read.
//
// Row fragment (the A or B operand from rows of the tile): lane l reads row
// 32 k + l % 32, 16-byte chunk c.
template <int D>
__device__ __forceinline__ uint32_t rows_off(int lane, int c) {
    const int col = lane & 31;
    return (uint32_t)((col * D + 8 * aswz<D>(col, c)) * 2);
}
// Transposed fragment (operand of M^T for a row-major tile M): lane l gets
// column dcol + l % 32 of M and the 8 rows 16 k + 4 (l / 32) +
// {0, 1, 2, 3, 8, 9, 10, 11}, the order in which a lane half of an S (or S^T)
// accumulator holds its rows (8 (j/4) + 4 half + j%4). Two transposed reads
// of 4 rows each (h = 0, 1): lane i of 16-lane group g addresses row
// 16 k + 4 (g / 2) + i / 4 + 8 h, columns dcol + 16 (g % 2) + 4 (i % 4) .. +3.
template <int D>
__device__ __forceinline__ uint32_t tr_off(int lane, int dcol, int h) {
    const int i = lane & 15, g = lane >> 4;
    const int r = 4 * (g >> 1) + (i >> 2) + 8 * h;
    const int c = (dcol >> 3) + 2 * (g & 1) + ((i & 3) >> 1);
    return (uint32_t)((r * D + 8 * aswz<D>(r, c) + 4 * (i & 1)) * 2);
}
__device__ __forceinline__ bf16x8 frag_at(const uint16_t* t, uint32_t byte_off) {
    return *reinterpret_cast<const bf16x8*>(reinterpret_cast<const char*>(t) + byte_off);
}
__device__ __forceinline__ bf16x8 frag_tr_at(const uint16_t* t, uint32_t off_lo, uint32_t off_hi) {
    const char* b = reinterpret_cast<const char*>(t);
    const s16x4 v8[2] = {ds_read_tr16(reinterpret_cast<const uint16_t*>(b + off_lo)),
                         ds_read_tr16(reinterpret_cast<const uint16_t*>(b + off_hi))};
    return __builtin_bit_cast(bf16x8, v8);
}

// Rows of a wave's transposed accumulators (acc[dt] element j = dim
// 32 dt + 8 (j/4) + 4 half + j%4 of row `col`) through a per-wave LDS patch
// to 16-byte stores of rows row0 + r (r < 32, row0 + r < nrows) of dst
// (row stride ld elements). OutT: uint16_t (bf16) or float.
template <int D, typename OutT>
__device__ __forceinline__ void store_rows(const f32x16 (&acc)[D / 32], float scale, void* patch_mem, OutT* dst,
                                           int64_t ld, int64_t row0, int64_t nrows, int lane) {
    constexpr int EPC = 16 / sizeof(OutT);    // elements per 16-byte chunk
    constexpr int PROW = D + 16 / sizeof(OutT);  // padded patch row (elements)
    constexpr int CPR = D / EPC;
    OutT* patch = static_cast<OutT*>(patch_mem);
    const int col = lane & 31, half = lane >> 5;
#pragma unroll
    for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
            const int d = 32 * dt + 8 * jq + 4 * half;
            if constexpr (sizeof(OutT) == 2) {
                const uint32_t lo = pack_bf16x2(acc[dt][4 * jq] * scale, acc[dt][4 * jq + 1] * scale);
                const uint32_t hi = pack_bf16x2(acc[dt][4 * jq + 2] * scale, acc[dt][4 * jq + 3] * scale);
                *reinterpret_cast<uint2*>(&patch[col * PROW + d]) = make_uint2(lo, hi);
            } else {
                *reinterpret_cast<float4*>(&patch[col * PROW + d]) =
                    make_float4(acc[dt][4 * jq] * scale, acc[dt][4 * jq + 1] * scale, acc[dt][4 * jq + 2] * scale,
                                acc[dt][4 * jq + 3] * scale);
            }
        }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave's patch is written
#pragma unroll
    for (int it = 0; it < 32 * CPR / 64; ++it) {
        const int i = it * 64 + lane;
        const int r = i / CPR, c = i % CPR;
        if (row0 + r < nrows) {
            const uint4 v = *reinterpret_cast<const uint4*>(&patch[r * PROW + EPC * c]);
            *reinterpret_cast<uint4*>(dst + (row0 + r) * ld + EPC * c) = v;
        }
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // patch reads done before it is rewritten
}

// --------------------------------------------------------- backward prep
// Per (b, h, 64 queries): Delta = rowsum(dO * O) and lse * log2 e into one
// [2][64] fp32 block (4 threads per query row, D / 4 dims each).
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_prep_bf16(const uint16_t* __restrict__ o,
                                                          const uint16_t* __restrict__ dout,
                                                          const float* __restrict__ lse, int H, int64_t S,
                                                          int64_t Sp, float* __restrict__ lsd) {
    constexpr int CPR = D / 8;
    const int64_t bh = blockIdx.y;
    const int64_t b = bh / H, h = bh % H;
    const int64_t q0 = (int64_t)blockIdx.x * 64;
    const int64_t ldo = (int64_t)H * D;
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(o + (b * S * H + h) * D, (S * H - h) * D * 2);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(dout + (b * S * H + h) * D, (S * H - h) * D * 2);
    // Each wave takes 16 rows. One load instruction covers RPI whole rows:
    // lane l reads chunk l % CPR of row l / CPR, so the wave's 64 lanes read
    // contiguous 16-byte chunks; the CPR lanes of a row then add their parts.
    constexpr int RPI = 64 / CPR, NI = 16 / RPI;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int ch = lane % CPR, rsub = lane / CPR;
    float acc[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int row = wave * 16 + i * RPI + rsub;
        const uint32_t off = q0 + row < S ? (uint32_t)(((q0 + row) * ldo + 8 * ch) * 2) : kOOB;
        float x[8], g[8];
        BVec<uint16_t>::unpack(buf_load16(ro, off), x);
        BVec<uint16_t>::unpack(buf_load16(rd, off), g);
        acc[i] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[i] += x[e] * g[e];
    }
#pragma unroll
    for (int i = 0; i < NI; ++i)
#pragma unroll
        for (int m = 1; m < CPR; m <<= 1) acc[i] += __shfl_xor(acc[i], m, kWave);
    if (ch == 0) {
        float* blk = lsd + (bh * (Sp / 64) + blockIdx.x) * 128;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int row = wave * 16 + i * RPI + rsub;
            const bool ok = q0 + row < S;
            // padded queries: lse = +inf makes their P exactly 0
            blk[row] = ok ? lse[bh * S + q0 + row] * kLog2e : __builtin_inff();
            blk[64 + row] = ok ? acc[i] : 0.f;
        }
    }
}

// ------------------------------------------------------------ dK and dV
template <int D>
__global__ __launch_bounds__(256, 1) void attn_bwd_dkdv_bf16(AttnBwdArgs a) {
    constexpr int KS = D / 16, DT = D / 32;
    constexpr int TILE = 64 * D;                 // one [64][D] or [D][64] tile
    constexpr int STAGE = 2 * TILE + 512;        // Q, dO, lse/Delta (1 KB)
    constexpr int KV = 2 * 128 * D;              // the workgroup's K and V rows, [128][D] each, after the stages
    // the epilogue reuses the stages as per-wave patches of 32 rows x (D + 8)
    // uint16 x 2 (fp32 partials with 16-byte row padding); allocate the larger
    constexpr int PATCH = 4 * 32 * (D + 8) * 2;
    constexpr int SMEM = 2 * STAGE + KV > PATCH ? 2 * STAGE + KV : PATCH;
    __shared__ __attribute__((aligned(1024))) uint16_t smem[SMEM];
    const uint32_t smem_byte = (uint32_t)reinterpret_cast<uintptr_t>(smem);
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int col = lane & 31, half = lane >> 5;
    const int ng = a.ngroups;
    const int nwg = a.B * a.Hkv * ng;
    const int kb = (int)(blockIdx.x / nwg);      // key block 0 sees the most queries: dispatched first
    const int grp = (int)(blockIdx.x % nwg) % ng;
    const int64_t bhk = (int64_t)(blockIdx.x % nwg) / ng;  // b * Hkv + K/V head
    const int b = (int)(bhk / a.Hkv);
    const int rep = a.H / a.Hkv, hpg = rep / ng;
    const int h0 = (int)(bhk % a.Hkv) * rep + grp * hpg;  // the group's first query head
    const int64_t S = a.S;
    const int64_t key0 = (int64_t)kb * 128;
    const int64_t kw = key0 + 32 * wave;         // first key of this wave
    const int64_t my_key = kw + col;
    uint32_t roff[KS], troff[DT][2];
#pragma unroll
    for (int s = 0; s < KS; ++s) roff[s] = rows_off<D>(lane, 2 * s + half);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int h = 0; h < 2; ++h) troff[dt][h] = tr_off<D>(lane, 32 * dt, h);

    // K and V rows of the workgroup's 128 keys (B operands of S = Q.K^T and
    // dP = dO.V^T) stay in LDS for the whole query loop; held as register
    // fragments they pushed the kernel past 256 VGPRs into AGPR spills.
    // Keys past S load as zeros.
    const i32x4 rk = rsrc_words(a.k + bhk * S * D, S * D * 2);
    const i32x4 rv = rsrc_words(a.v + bhk * S * D, S * D * 2);
    const uint16_t* sk = smem + 2 * STAGE;
    const uint16_t* sv = sk + 128 * D;
    const uint16_t* skw = sk + 32 * wave * D;  // this wave's 32 keys
    const uint16_t* svw = sv + 32 * wave * D;
    {
        const uint32_t kv_byte = smem_byte + (uint32_t)(2 * STAGE * 2);
        dma_rows<D>(rk, kv_byte, (uint32_t)key0, D, wave, lane);
        dma_rows<D>(rk, kv_byte + 64 * D * 2, (uint32_t)key0 + 64, D, wave, lane);
        dma_rows<D>(rv, kv_byte + 128 * D * 2, (uint32_t)key0, D, wave, lane);
        dma_rows<D>(rv, kv_byte + 192 * D * 2, (uint32_t)key0 + 64, D, wave, lane);
    }

    const __amdgpu_buffer_rsrc_t rm = make_rsrc(a.mask, a.mask ? S * S * 4 : 0);

    const int nqb = (int)((S + 63) / 64);
    const int qstart = a.causal ? (int)(key0 / 64) : 0;  // earlier query blocks see none of these keys
    const int nq = nqb - qstart;                          // query blocks per head
    const int nit = hpg * nq;                             // (head, query block) steps, head-major

    // step it: query head h0 + it / nq, query block qstart + it % nq
    auto issue = [&](int it, int stage) {
        const int h = h0 + it / nq, qb = qstart + it % nq;
        const int64_t bh = (int64_t)b * a.H + h;
        const i32x4 rq = rsrc_words(a.q + bh * S * D, S * D * 2);
        const i32x4 rdo = rsrc_words(a.dout + ((int64_t)b * S * a.H + h) * D, (S * a.H - h) * D * 2);
        const i32x4 rl = rsrc_words(a.lsd + bh * (a.Sp / 64) * 128, (a.Sp / 64) * 128 * 4);
        const uint32_t base = smem_byte + (uint32_t)(stage * STAGE * 2);
        const uint32_t q0 = (uint32_t)qb * 64;
        dma_rows<D>(rq, base, q0, D, wave, lane);
        dma_rows<D>(rdo, base + TILE * 2, q0, (uint32_t)(a.H * D), wave, lane);
        if (wave == 0)  // the [2][64] fp32 lse/Delta block (512 B; lanes 32-63 fall outside and write zeros)
            dma16(rl, __builtin_amdgcn_readfirstlane(base + 2 * TILE * 2),
                  lane < 32 ? (uint32_t)(qb * 512 + lane * 16) : kOOB);
    };

    f32x16 dvacc[DT], dkacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) dvacc[t][j] = dkacc[t][j] = 0.f;

    if (nit > 0) issue(0, 0);
    // The wave's K and V fragments (B operands of S and dP) are the same for
    // every block: read from LDS once, then held in AGPRs (an empty asm with
    // AGPR operands puts them there; MFMAs read their A / B operands from
    // either file). This file is compiled with the MFMAs' accumulators in
    // VGPRs (-amdgpu-mfma-vgpr-form), so the score arithmetic reads S and dP
    // where the MFMAs leave them, and the VGPRs the fragments would take hold
    // the dV / dK accumulators.
    wait_vmcnt<0>();
    __syncthreads();
    bf16x8 kf[KS], vf[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) {
        kf[s] = frag_at(skw, roff[s]);
        vf[s] = frag_at(svw, roff[s]);
        asm volatile("" : "+a"(kf[s]), "+a"(vf[s]));
    }
    for (int it = 0; it < nit; ++it) {
        wait_vmcnt<0>();
        __syncthreads();
        if (it + 1 < nit) issue(it + 1, (it + 1) & 1);
        const int qb = qstart + it % nq;
        const __amdgpu_buffer_rsrc_t rds =
            make_rsrc(a.dst ? a.dst + ((int64_t)b * a.H + h0 + it / nq) * S * a.ldst : nullptr,
                      a.dst ? S * a.ldst * 2 : 0);
        // Every wave runs every block: in a block before the wave's first key
        // (causal) every P is masked to 0, and a wave past S computes rows
        // that are never stored. Skipping those blocks made the accumulators
        // take a VGPR round trip on every iteration.
        const uint16_t* sq = smem + (it & 1) * STAGE;
        const uint16_t* sdo = sq + TILE;
        const float* sl = reinterpret_cast<const float*>(sq + 2 * TILE);
        const int64_t q0 = (int64_t)qb * 64;

        // accumulator j of tile t: query q0 + 32 t + 8 (j/4) + 4 half + j%4, key my_key
        // P and dS of query tile t; MASK adds the additive mask, EDGE applies
        // the causal test (key offset from q0 against the query offset)
        auto scores = [&](auto mask_tag, auto edge_tag, auto t_tag, const f32x16& sacc, const f32x16& dpacc,
                          bf16x8 (&pb)[2], bf16x8 (&db)[2]) {
            constexpr bool MASK = decltype(mask_tag)::value, EDGE = decltype(edge_tag)::value;
            constexpr int t = decltype(t_tag)::value;
            // the lane's 4 half moves to the key side, so each causal test
            // compares a constant
            const int kq = (int)(my_key - q0) - 4 * half;
            float p[16], ds[16];
#pragma unroll
            for (int jq = 0; jq < 4; ++jq) {
                const int qi = 32 * t + 8 * jq + 4 * half;  // first of 4 consecutive queries
                const float4 l2 = *reinterpret_cast<const float4*>(&sl[qi]);
                const float4 dl = *reinterpret_cast<const float4*>(&sl[64 + qi]);
                const float lv[4] = {l2.x, l2.y, l2.z, l2.w}, dv4[4] = {dl.x, dl.y, dl.z, dl.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int j = 4 * jq + e;
                    // exponent s * scale * log2 e - lse * log2 e, as one fma
                    // where there is no mask term
                    float x;
                    if constexpr (MASK) {
                        const int64_t qq = q0 + qi + e;
                        const uint32_t off = (qq < S && my_key < S) ? (uint32_t)((qq * S + my_key) * 4) : kOOB;
                        x = sacc[j] * a.scale_log2 +
                            __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rm, (int)off, 0, 0)) * kLog2e - lv[e];
                    } else {
                        x = __builtin_fmaf(sacc[j], a.scale_log2, -lv[e]);
                    }
                    if constexpr (EDGE) {
                        if ((!MASK || a.causal) && kq > 32 * t + 8 * jq + e) x = kNegInf;
                    }
                    p[j] = exp2_hw(x);
                    ds[j] = p[j] * (dpacc[j] - dv4[e]);
                }
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                pb[kk] = pack_bf16x8(&p[8 * kk]);
                db[kk] = pack_bf16x8(&ds[8 * kk]);
            }
        };
        // one 32-query tile at a time: S = Q.K^T and dP = dO.V^T, its P and
        // dS, then its share of dV^T (d x key) += dO^T . P and
        // dK^T += Q^T . dS, with dO^T and Q^T by transposed reads of the dO,
        // Q tiles in the accumulators' query order. With both tiles' S and dP
        // live at once the kernel needed more than 256 VGPRs and copied the
        // dV / dK accumulators between AGPRs and VGPRs every block.
        auto tile = [&](auto t_tag) {
            constexpr int t = decltype(t_tag)::value;
            f32x16 sacc, dpacc;
#pragma unroll
            for (int j = 0; j < 16; ++j) sacc[j] = dpacc[j] = 0.f;
            // Q and dO fragments one k-chunk ahead of their MFMAs, so each
            // pair's LDS latency runs under the previous pair's MFMAs
            bf16x8 qf[2], df[2];
            qf[0] = frag_at(sq + 32 * t * D, roff[0]);
            df[0] = frag_at(sdo + 32 * t * D, roff[0]);
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                if (s + 1 < KS) {
                    qf[(s + 1) & 1] = frag_at(sq + 32 * t * D, roff[s + 1]);
                    df[(s + 1) & 1] = frag_at(sdo + 32 * t * D, roff[s + 1]);
                    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
                }
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[s & 1], kf[s], sacc, 0, 0, 0);
                dpacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(df[s & 1], vf[s], dpacc, 0, 0, 0);
                __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
            }
            bf16x8 pb[2], db[2];
            if (a.mask) scores(std::true_type{}, std::true_type{}, t_tag, sacc, dpacc, pb, db);
            else if (a.causal && q0 < kw + 31) scores(std::false_type{}, std::true_type{}, t_tag, sacc, dpacc, pb, db);
            else scores(std::false_type{}, std::false_type{}, t_tag, sacc, dpacc, pb, db);
            if (a.dst) {
                // dS^T for the dQ pass: elements 4 hh .. 4 hh + 3 of db[kk] are
                // queries q0 + 32 t + 16 kk + 8 hh + 4 half + 0..3 of this
                // lane's key, 8 contiguous bytes of its dS^T row; keys past S
                // fall outside the buffer range and are dropped
#pragma unroll
                for (int kk = 0; kk < 2; ++kk) {
                    const uint4 w4 = __builtin_bit_cast(uint4, db[kk]);
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int64_t qq = q0 + 32 * t + 16 * kk + 8 * hh + 4 * half;
                        const u32x2 v2 = {hh ? w4.z : w4.x, hh ? w4.w : w4.y};
                        __builtin_amdgcn_raw_buffer_store_b64(v2, rds, (int)(uint32_t)((my_key * a.ldst + qq) * 2), 0, 0);
                    }
                }
            }
            // dO^T and Q^T fragments (two transposed reads each) one step
            // ahead of their MFMAs; step u = 2 dt + kk
            bf16x8 ot[2], qt[2];
            auto tr_frags = [&](int u, int slot) {
                const int dt = u >> 1, r0 = (32 * t + 16 * (u & 1)) * D;
                ot[slot] = frag_tr_at(sdo + r0, troff[dt][0], troff[dt][1]);
                qt[slot] = frag_tr_at(sq + r0, troff[dt][0], troff[dt][1]);
            };
            tr_frags(0, 0);
            __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
#pragma unroll
            for (int u = 0; u < 2 * DT; ++u) {
                if (u + 1 < 2 * DT) {
                    tr_frags(u + 1, (u + 1) & 1);
                    __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
                }
                const int dt = u >> 1, kk = u & 1;
                dvacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ot[u & 1], pb[kk], dvacc[dt], 0, 0, 0);
                dkacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qt[u & 1], db[kk], dkacc[dt], 0, 0, 0);
                __builtin_amdgcn_sched_group_barrier(kSchedMfma, 2, 0);
            }
        };
        tile(std::integral_constant<int, 0>{});
        tile(std::integral_constant<int, 1>{});
    }

    wait_vmcnt<0>();  // every DMA has landed (also when the loop ran no block)
    __syncthreads();
    static_assert(32 * (D + 4) * 4 <= 32 * (D + 8) * 2 * 2, "fp32 patch rows fit a wave's share");
    void* patch = smem + wave * 32 * (D + 8) * 2;  // 32 rows of up to D + 4 floats per wave
    if (ng == 1) {
        store_rows<D, uint16_t>(dvacc, 1.f, patch, a.dv + bhk * S * D, D, kw, S, lane);
        store_rows<D, uint16_t>(dkacc, a.scale, patch, a.dk + bhk * S * D, D, kw, S, lane);
    } else {
        const int64_t pg = (bhk * ng + grp) * S * D;  // this group's partial
        store_rows<D, float>(dvacc, 1.f, patch, a.dv_part + pg, D, kw, S, lane);
        store_rows<D, float>(dkacc, a.scale, patch, a.dk_part + pg, D, kw, S, lane);
    }
}

// dk / dv [B, Hkv, S, D] = sum over the rep query-head groups of each K/V
// head of the fp32 partials, in group order; 8 elements per thread.
__device__ __forceinline__ void bwd_sum_range(const float* __restrict__ dk_part, const float* __restrict__ dv_part,
                                              uint16_t* __restrict__ dk, uint16_t* __restrict__ dv, int rep,
                                              int64_t per_head, int64_t n8, int64_t first, int64_t stride) {
    for (int64_t i = first; i < 2 * n8; i += stride) {
        const bool second = i >= n8;
        const int64_t e = (second ? i - n8 : i) * 8;  // element of [B, Hkv, S, D]
        const int64_t bhk = e / per_head, off = e % per_head;
        const float* src = (second ? dv_part : dk_part) + bhk * rep * per_head + off;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int r = 0; r < rep; ++r) {
            const float4 x0 = *reinterpret_cast<const float4*>(src + r * per_head);
            const float4 x1 = *reinterpret_cast<const float4*>(src + r * per_head + 4);
            acc[0] += x0.x; acc[1] += x0.y; acc[2] += x0.z; acc[3] += x0.w;
            acc[4] += x1.x; acc[5] += x1.y; acc[6] += x1.z; acc[7] += x1.w;
        }
        uint16_t* dst = (second ? dv : dk) + e;
        *reinterpret_cast<uint4*>(dst) = make_uint4(pack_bf16x2(acc[0], acc[1]), pack_bf16x2(acc[2], acc[3]),
                                                    pack_bf16x2(acc[4], acc[5]), pack_bf16x2(acc[6], acc[7]));
    }
}
__global__ __launch_bounds__(256) void attn_bwd_sum(const float* __restrict__ dk_part,
                                                    const float* __restrict__ dv_part, uint16_t* __restrict__ dk,
                                                    uint16_t* __restrict__ dv, int rep, int64_t per_head,
                                                    int64_t n8) {
    bwd_sum_range(dk_part, dv_part, dk, dv, rep, per_head, n8, (int64_t)blockIdx.x * blockDim.x + threadIdx.x,
                  (int64_t)gridDim.x * blockDim.x);
}

// ------------------------------------------------------------------- dQ
template <int D>
__global__ __launch_bounds__(256, 1) void attn_bwd_dq_bf16(AttnBwdArgs a) {
    constexpr int KB = 64, QB = 128, KS = D / 16, DT = D / 32;
    constexpr int TILE = 64 * D;
    constexpr int STAGE = 2 * TILE;  // K, V [64][D]
    constexpr int QDO = 2 * QB * D;  // the workgroup's Q and dO rows, [128][D] each, after the stages
    __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * STAGE + QDO];
    static_assert(4 * 32 * (D + 8) <= 2 * STAGE, "the epilogue's bf16 patches fit in the stages");
    const uint32_t smem_byte = (uint32_t)reinterpret_cast<uintptr_t>(smem);
    const int tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    const int col = lane & 31, half = lane >> 5;
    const int nbh = a.B * a.H;
    const int nqb = (int)((a.S + QB - 1) / QB);
    const int qb = nqb - 1 - (int)(blockIdx.x / nbh);  // heaviest query blocks first
    const int bh = xcd_head_order((int)(blockIdx.x % nbh), nbh);
    const int b = bh / a.H, h = bh % a.H;
    const int64_t bhk = (int64_t)b * a.Hkv + h / (a.H / a.Hkv);
    const int64_t S = a.S;
    const int64_t q0 = (int64_t)qb * QB;
    const int64_t qw = q0 + 32 * wave;
    const int64_t my_q = qw + col;

    uint32_t roff[KS], troff[DT][2];
#pragma unroll
    for (int s = 0; s < KS; ++s) roff[s] = rows_off<D>(lane, 2 * s + half);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int h = 0; h < 2; ++h) troff[dt][h] = tr_off<D>(lane, 32 * dt, h);

    // Q and dO rows of the workgroup's 128 queries (B operands of
    // S^T = K.Q^T and dP^T = V.dO^T) stay in LDS for the whole key loop
    // (held as register fragments they crowded the VGPRs). Queries past S
    // load as zeros.
    const i32x4 rq = rsrc_words(a.q + (int64_t)bh * S * D, S * D * 2);
    const i32x4 rdo = rsrc_words(a.dout + ((int64_t)b * S * a.H + h) * D, (S * a.H - h) * D * 2);
    const uint16_t* sqw = smem + 2 * STAGE + 32 * wave * D;  // this wave's 32 queries
    const uint16_t* sdow = sqw + QB * D;
    {
        const uint32_t qd_byte = smem_byte + (uint32_t)(2 * STAGE * 2);
        dma_rows<D>(rq, qd_byte, (uint32_t)q0, D, wave, lane);
        dma_rows<D>(rq, qd_byte + 64 * D * 2, (uint32_t)q0 + 64, D, wave, lane);
        dma_rows<D>(rdo, qd_byte + QB * D * 2, (uint32_t)q0, (uint32_t)(a.H * D), wave, lane);
        dma_rows<D>(rdo, qd_byte + (QB + 64) * D * 2, (uint32_t)q0 + 64, (uint32_t)(a.H * D), wave, lane);
    }
    float lse2 = __builtin_inff(), delta = 0.f;
    if (my_q < S) {
        const float* blk = a.lsd + ((int64_t)bh * (a.Sp / 64) + my_q / 64) * 128;
        lse2 = blk[my_q % 64];
        delta = blk[64 + my_q % 64];
    }

    const i32x4 rk = rsrc_words(a.k + bhk * S * D, S * D * 2);
    const i32x4 rv = rsrc_words(a.v + bhk * S * D, S * D * 2);
    const __amdgpu_buffer_rsrc_t rm = make_rsrc(a.mask, a.mask ? S * S * 4 : 0);

    const int nkb_all = (int)((S + KB - 1) / KB);
    int nkb = nkb_all;
    if (a.causal) nkb = min(nkb_all, (int)((min(q0 + QB, S) - 1) / KB) + 1);

    auto issue = [&](int kb, int stage) {
        const uint32_t base = smem_byte + (uint32_t)(stage * STAGE * 2);
        const uint32_t key0 = (uint32_t)kb * KB;
        dma_rows<D>(rk, base, key0, D, wave, lane);
        dma_rows<D>(rv, base + TILE * 2, key0, D, wave, lane);
    };

    f32x16 dqacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) dqacc[t][j] = 0.f;

    if (nkb > 0) issue(0, 0);
    for (int kb = 0; kb < nkb; ++kb) {
        wait_vmcnt<0>();
        __syncthreads();
        if (kb + 1 < nkb) issue(kb + 1, (kb + 1) & 1);
        // Every wave runs every block: keys after all of a wave's queries
        // (causal) or queries past S give dS = 0. Skipping those blocks made
        // the accumulators take a VGPR round trip on every iteration.
        const uint16_t* sk = smem + (kb & 1) * STAGE;
        const uint16_t* sv = sk + TILE;
        const int64_t key0 = (int64_t)kb * KB;

        // accumulator j of tile t: key key0 + 32 t + 8 (j/4) + 4 half + j%4, query my_q
        // dS of key tile t; MASK adds the additive mask, EDGE drops keys past
        // S and (causal) keys after this lane's query, as offsets in the block
        auto scores = [&](auto mask_tag, auto edge_tag, auto t_tag, const f32x16& sacc, const f32x16& dpacc,
                          bf16x8 (&db)[2]) {
            constexpr bool MASK = decltype(mask_tag)::value, EDGE = decltype(edge_tag)::value;
            constexpr int t = decltype(t_tag)::value;
            const int lim = (int)min64(S - key0, KB);
            const int qrel = a.causal ? (int)max64(min64(my_q - key0, KB), -1) : KB;
            float ds[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int ko = 32 * t + 8 * (j >> 2) + 4 * half + (j & 3);
                float x;
                if constexpr (MASK) {
                    const int64_t key = key0 + ko;
                    const uint32_t off = (my_q < S && key < S) ? (uint32_t)((my_q * S + key) * 4) : kOOB;
                    x = sacc[j] * a.scale_log2 +
                        __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rm, (int)off, 0, 0)) * kLog2e - lse2;
                } else {
                    x = __builtin_fmaf(sacc[j], a.scale_log2, -lse2);
                }
                if constexpr (EDGE) {
                    if (ko >= lim || ko > qrel) x = kNegInf;
                }
                ds[j] = exp2_hw(x) * (dpacc[j] - delta);
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) db[kk] = pack_bf16x8(&ds[8 * kk]);
        };
        // one 32-key tile at a time: S^T = K.Q^T and dP^T = V.dO^T, its dS,
        // then its share of dQ^T (d x query) += K^T . dS^T, with K^T by
        // transposed reads of the K tile in the accumulators' key order
        auto tile = [&](auto t_tag) {
            constexpr int t = decltype(t_tag)::value;
            f32x16 sacc, dpacc;
#pragma unroll
            for (int j = 0; j < 16; ++j) sacc[j] = dpacc[j] = 0.f;
#pragma unroll
            for (int s = 0; s < KS; ++s) {
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_at(sk + 32 * t * D, roff[s]), frag_at(sqw, roff[s]),
                                                              sacc, 0, 0, 0);
                dpacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_at(sv + 32 * t * D, roff[s]),
                                                               frag_at(sdow, roff[s]), dpacc, 0, 0, 0);
            }
            bf16x8 db[2];
            if (a.mask) scores(std::true_type{}, std::true_type{}, t_tag, sacc, dpacc, db);
            else if (key0 + KB > S || (a.causal && key0 + KB - 1 > qw))
                scores(std::false_type{}, std::true_type{}, t_tag, sacc, dpacc, db);
            else scores(std::false_type{}, std::false_type{}, t_tag, sacc, dpacc, db);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                for (int kk = 0; kk < 2; ++kk)
                    dqacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        frag_tr_at(sk + (32 * t + 16 * kk) * D, troff[dt][0], troff[dt][1]), db[kk], dqacc[dt], 0, 0,
                        0);
        };
        tile(std::integral_constant<int, 0>{});
        tile(std::integral_constant<int, 1>{});
    }

    wait_vmcnt<0>();  // every DMA has landed (also when the loop ran no block)
    __syncthreads();
    store_rows<D, uint16_t>(dqacc, a.scale, smem + wave * 32 * (D + 8), a.dq + (int64_t)bh * S * D, D, qw, S, lane);
}

// dQ from the stored dS^T (written by attn_bwd_dkdv_bf16): one workgroup
// per (b, h, 128 queries), 4 waves of 32 queries. Per block of 64 keys (up
// to the diagonal when causal) the K tile [64][D] and the dS^T tile
// [64 keys][128 queries] go into LDS (two stages, the backward's swizzled
// layout); dQ^T (d x query) += K^T . dS^T takes both operands by transposed
// reads in the same key order, so nothing is recomputed: no S, no dP, no
// score arithmetic or mask (dS already holds them). Keys past S load as
// zeros from both buffers; dS^T columns of queries past S are never stored.
template <int D>
__global__ __launch_bounds__(256, 2) void attn_bwd_dq_ds_bf16(AttnBwdArgs a) {
    if ((int64_t)blockIdx.x >= a.dq_blocks) {
        // the groups' dK / dV partial sums (independent of dQ), as blocks
        // dispatched after the dQ blocks so that they fill the pass's tail
        const int64_t sb = (int64_t)blockIdx.x - a.dq_blocks, nsb = (int64_t)gridDim.x - a.dq_blocks;
        bwd_sum_range(a.dk_part, a.dv_part, a.dk, a.dv, a.ngroups, a.S * D, a.sum_n8, sb * 256 + threadIdx.x,
                      nsb * 256);
        return;
    }
    constexpr int KB = 64, QB = 128, DT = D / 32;
    constexpr int KT = 64 * D, DSTILE = 64 * QB;  // K tile, dS^T tile (elements)
    constexpr int STAGE = KT + DSTILE;
    __shared__ __attribute__((aligned(1024))) uint16_t smem[2 * STAGE];
    static_assert(4 * 32 * (D + 8) <= 2 * STAGE, "the epilogue's bf16 patches fit in the stages");
    const uint32_t smem_byte = (uint32_t)reinterpret_cast<uintptr_t>(smem);
    const int lane = threadIdx.x & 63, wave = wave_id();
    const int nbh = a.B * a.H;
    const int nqb = (int)((a.S + QB - 1) / QB);
    const int qb = nqb - 1 - (int)(blockIdx.x / nbh);  // heaviest query blocks first
    const int bh = xcd_head_order((int)(blockIdx.x % nbh), nbh);
    const int b = bh / a.H, h = bh % a.H;
    const int64_t bhk = (int64_t)b * a.Hkv + h / (a.H / a.Hkv);
    const int64_t S = a.S;
    const int64_t q0 = (int64_t)qb * QB;
    const int64_t qw = q0 + 32 * wave;

    uint32_t tk[DT][2], td[2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) tk[dt][hh] = tr_off<D>(lane, 32 * dt, hh);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) td[hh] = tr_off<QB>(lane, 32 * wave, hh);

    const i32x4 rk = rsrc_words(a.k + bhk * S * D, S * D * 2);
    // dS^T rows of this head from column q0: rows past S fall outside
    const i32x4 rds = rsrc_words(a.dst + (int64_t)bh * S * a.ldst + q0, (S * a.ldst - q0) * 2);

    const int nkb_all = (int)((S + KB - 1) / KB);
    int nkb = nkb_all;
    if (a.causal) nkb = min(nkb_all, (int)((min(q0 + QB, S) - 1) / KB) + 1);

    auto issue = [&](int kb, int stage) {
        const uint32_t base = smem_byte + (uint32_t)(stage * STAGE * 2);
        const uint32_t key0 = (uint32_t)kb * KB;
        dma_rows<D>(rk, base, key0, D, wave, lane);
        dma_rows<QB>(rds, base + KT * 2, key0, (uint32_t)a.ldst, wave, lane);
    };

    f32x16 dqacc[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int j = 0; j < 16; ++j) dqacc[t][j] = 0.f;

    if (nkb > 0) issue(0, 0);
    for (int kb = 0; kb < nkb; ++kb) {
        wait_vmcnt<0>();
        __syncthreads();
        if (kb + 1 < nkb) issue(kb + 1, (kb + 1) & 1);
        const uint16_t* sk = smem + (kb & 1) * STAGE;
        const uint16_t* sds = sk + KT;
#pragma unroll
        for (int kc = 0; kc < KB / 16; ++kc) {
            const bf16x8 bfr = frag_tr_at(sds + 16 * kc * QB, td[0], td[1]);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
                dqacc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(frag_tr_at(sk + 16 * kc * D, tk[dt][0], tk[dt][1]),
                                                                   bfr, dqacc[dt], 0, 0, 0);
        }
    }

    wait_vmcnt<0>();  // every DMA has landed (also when the loop ran no block)
    __syncthreads();
    store_rows<D, uint16_t>(dqacc, a.scale, smem + wave * 32 * (D + 8), a.dq + (int64_t)bh * S * D, D, qw, S, lane);
}

// ------------------------------------------------------ generic backward
// One wave per row; lanes over the head dim (dims l, l + 64, l + 128, l + 192).
template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_delta_generic(const T* __restrict__ o, const T* __restrict__ dout,
                                                              float* __restrict__ delta, int B, int H, int64_t S,
                                                              int D) {
    const int lane = lane_id();
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (b, h, i)
    if (row >= (int64_t)B * H * S) return;
    const int64_t bh = row / S, i = row % S, b = bh / H, h = bh % H;
    const int64_t base = ((b * S + i) * H + h) * D;
    float acc = 0.f;
    for (int d = lane; d < D; d += 64) acc += Elem<T>::load(o, base + d) * Elem<T>::load(dout, base + d);
    acc = wave_sum(acc);
    if (lane == 0) delta[row] = acc;
}

template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_dq_generic(const T* __restrict__ q, const T* __restrict__ k,
                                                           const T* __restrict__ v, const float* __restrict__ mask,
                                                           const float* __restrict__ lse,
                                                           const float* __restrict__ delta,
                                                           const T* __restrict__ dout, T* __restrict__ dq, int B,
                                                           int H, int Hkv, int64_t S, int D, float scale,
                                                           int causal) {
    const int lane = lane_id();
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= (int64_t)B * H * S) return;
    const int64_t bh = row / S, i = row % S;
    const int b = (int)(bh / H), h = (int)(bh % H);
    const int64_t bhk = (int64_t)b * Hkv + h / (H / Hkv);
    float qv[4], gv[4], acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int d = lane + 64 * u;
        qv[u] = d < D ? Elem<T>::load(q, (bh * S + i) * D + d) : 0.f;
        gv[u] = d < D ? Elem<T>::load(dout, (((int64_t)b * S + i) * H + h) * D + d) : 0.f;
        acc[u] = 0.f;
    }
    const float li = lse[row], di = delta[row];
    const int64_t kend = causal ? i + 1 : S;
    for (int64_t j = 0; j < kend; ++j) {
        const int64_t kr = (bhk * S + j) * D;
        float s = 0.f, dp = 0.f;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int d = lane + 64 * u;
            if (d < D) {
                s += qv[u] * Elem<T>::load(k, kr + d);
                dp += gv[u] * Elem<T>::load(v, kr + d);
            }
        }
        s = wave_sum(s) * scale;
        dp = wave_sum(dp);
        if (mask) s += mask[i * S + j];
        const float ds = __expf(s - li) * (dp - di);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int d = lane + 64 * u;
            if (d < D) acc[u] += ds * Elem<T>::load(k, kr + d);
        }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int d = lane + 64 * u;
        if (d < D) Elem<T>::store(dq, (bh * S + i) * D + d, acc[u] * scale);
    }
}

template <typename T>
__global__ __launch_bounds__(256) void attn_bwd_dkdv_generic(const T* __restrict__ q, const T* __restrict__ k,
                                                             const T* __restrict__ v,
                                                             const float* __restrict__ mask,
                                                             const float* __restrict__ lse,
                                                             const float* __restrict__ delta,
                                                             const T* __restrict__ dout, T* __restrict__ dk,
                                                             T* __restrict__ dv, int B, int H, int Hkv, int64_t S,
                                                             int D, float scale, int causal) {
    const int lane = lane_id();
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (b, hk, j)
    if (row >= (int64_t)B * Hkv * S) return;
    const int64_t bhk = row / S, j = row % S;
    const int b = (int)(bhk / Hkv), hk = (int)(bhk % Hkv);
    const int rep = H / Hkv;
    float kv[4], vv[4], gk[4], gvv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int d = lane + 64 * u;
        kv[u] = d < D ? Elem<T>::load(k, row * D + d) : 0.f;
        vv[u] = d < D ? Elem<T>::load(v, row * D + d) : 0.f;
        gk[u] = gvv[u] = 0.f;
    }
    for (int h = hk * rep; h < (hk + 1) * rep; ++h) {
        const int64_t bh = (int64_t)b * H + h;
        for (int64_t i = causal ? j : 0; i < S; ++i) {
            const int64_t qr = (bh * S + i) * D, gr = (((int64_t)b * S + i) * H + h) * D;
            float s = 0.f, dp = 0.f;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int d = lane + 64 * u;
                if (d < D) {
                    s += Elem<T>::load(q, qr + d) * kv[u];
                    dp += Elem<T>::load(dout, gr + d) * vv[u];
                }
            }
            s = wave_sum(s) * scale;
            dp = wave_sum(dp);
            if (mask) s += mask[i * S + j];
            const float p = __expf(s - lse[bh * S + i]);
            const float ds = p * (dp - delta[bh * S + i]);
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int d = lane + 64 * u;
                if (d < D) {
                    gk[u] += ds * Elem<T>::load(q, qr + d);
                    gvv[u] += p * Elem<T>::load(dout, gr + d);
                }
            }
        }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const int d = lane + 64 * u;
        if (d < D) {
            Elem<T>::store(dk, row * D + d, gk[u] * scale);
            Elem<T>::store(dv, row * D + d, gvv[u]);
        }
    }
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
        const bool raw = mask == nullptr && a.scale_log2 > 0.f;
        if (D == 64) {
            attn_vt_bf16<64><<<gvt, 256, 0, stream>>>(static_cast<const uint16_t*>(v), S, Sp, vt);
            if (raw) attn_fwd_bf16<64, true><<<grid, 256, 0, stream>>>(a);
            else attn_fwd_bf16<64, false><<<grid, 256, 0, stream>>>(a);
        } else {
            attn_vt_bf16<128><<<gvt, 256, 0, stream>>>(static_cast<const uint16_t*>(v), S, Sp, vt);
            if (raw) attn_fwd_bf16<128, true><<<grid, 256, 0, stream>>>(a);
            else attn_fwd_bf16<128, false><<<grid, 256, 0, stream>>>(a);
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

namespace {
size_t align256(size_t n) { return (n + 255) / 256 * 256; }
}  // namespace

// The MFMA backward's dQ pass reads dS^T stored by the dK/dV kernel (bf16
// [B, H, S, ldst], ldst = S rounded up to 128) when a head's dS^T rows fit
// 32-bit buffer offsets; beyond that (S > ~32k) it recomputes S and dP.
int64_t dst_ld(int64_t S) { return (S + 127) / 128 * 128; }
bool attention_dq_from_ds(const mc_attn_desc& d) {
    return attention_uses_mfma(d) && (int64_t)d.seq * dst_ld(d.seq) * 2 < ((int64_t)1 << 31);
}

// Query heads per dK/dV workgroup: the largest divisor g of H / Hkv whose
// heaviest workgroup (g heads x every query block, key block 0) does no more
// 64-query block steps than the average share of 256 CUs, so that the
// heaviest-first dispatch still balances. Each group's heads accumulate in
// the workgroup's registers; one group per K/V head leaves no partials to
// sum. A function of the shape only (not of the device), so the sums'
// order, and the results, do not depend on where the call runs.
int attn_dkdv_groups(const mc_attn_desc& d) {
    const int rep = d.heads / d.kv_heads;
    const int64_t nqb = (d.seq + 63) / 64, nkb = (d.seq + 127) / 128;
    int64_t steps = 0;  // 64-query block steps of one (b, h) over all key blocks
    for (int64_t kb = 0; kb < nkb; ++kb) steps += d.causal ? std::max<int64_t>(nqb - 2 * kb, 0) : nqb;
    const double avg = (double)steps * d.batch * d.heads / 256.0;
    for (int g = rep; g > 1; --g)
        if (rep % g == 0 && (double)g * nqb <= avg) return rep / g;
    return rep;
}

AttnBwdWs attention_bwd_ws(const mc_attn_desc& d) {
    AttnBwdWs w{};
    const size_t B = (size_t)d.batch, H = (size_t)d.heads, Hkv = (size_t)d.kv_heads, D = (size_t)d.head_dim;
    const size_t S = (size_t)d.seq;
    size_t off = 0;
    if (attention_uses_mfma(d)) {
        const size_t Sp = (S + 63) / 64 * 64;
        w.lsd = off;  off += align256(B * H * (Sp / 64) * 128 * 4);
        const size_t ng = (size_t)attn_dkdv_groups(d);
        if (ng > 1) {
            w.dk_part = off;  off += align256(B * Hkv * ng * S * D * 4);
            w.dv_part = off;  off += align256(B * Hkv * ng * S * D * 4);
        }
        w.dst = off;
        if (attention_dq_from_ds(d)) off += align256(B * H * S * (size_t)dst_ld(d.seq) * 2);
    } else {
        w.lsd = off;  off += align256(B * H * S * 4);  // Delta
    }
    w.total = off;
    return w;
}

hipError_t launch_attention_bwd(const mc_attn_desc& d, const void* q, const void* k, const void* v,
                                const float* mask, const void* o, const float* lse, const void* dout, void* dq,
                                void* dk, void* dv, void* ws, hipStream_t stream) {
    const int B = (int)d.batch, H = d.heads, Hkv = d.kv_heads, D = d.head_dim;
    const int64_t S = d.seq;
    const AttnBwdWs w = attention_bwd_ws(d);
    char* base = static_cast<char*>(ws);
    if (attention_uses_mfma(d)) {
        const int64_t Sp = (S + 63) / 64 * 64;
        AttnBwdArgs a;
        a.q = static_cast<const uint16_t*>(q);
        a.k = static_cast<const uint16_t*>(k);
        a.v = static_cast<const uint16_t*>(v);
        a.dout = static_cast<const uint16_t*>(dout);
        a.mask = mask;
        a.lsd = reinterpret_cast<const float*>(base + w.lsd);
        a.dq = static_cast<uint16_t*>(dq);
        a.dk = static_cast<uint16_t*>(dk);
        a.dv = static_cast<uint16_t*>(dv);
        a.ngroups = attn_dkdv_groups(d);
        a.dk_part = a.ngroups > 1 ? reinterpret_cast<float*>(base + w.dk_part) : nullptr;
        a.dv_part = a.ngroups > 1 ? reinterpret_cast<float*>(base + w.dv_part) : nullptr;
        const bool from_ds = attention_dq_from_ds(d);
        a.dst = from_ds ? reinterpret_cast<uint16_t*>(base + w.dst) : nullptr;
        a.ldst = dst_ld(S);
        a.S = S;
        a.Sp = Sp;
        a.B = B; a.H = H; a.Hkv = Hkv;
        a.causal = d.causal ? 1 : 0;
        a.nblk = (int)((S + 127) / 128);
        a.dq_blocks = (int64_t)a.nblk * B * H;
        a.sum_n8 = (int64_t)B * Hkv * S * D / 8;
        a.scale = d.scale;
        a.scale_log2 = d.scale * kLog2e;
        const dim3 gprep((unsigned)(Sp / 64), (unsigned)(B * H));
        const dim3 grid((unsigned)((int64_t)a.nblk * B * H));
        const dim3 gkv((unsigned)((int64_t)a.nblk * B * Hkv * a.ngroups));
        float* lsd = reinterpret_cast<float*>(base + w.lsd);
        const uint16_t* o16 = static_cast<const uint16_t*>(o);
        const uint16_t* do16 = static_cast<const uint16_t*>(dout);
        if (D == 64) {
            attn_bwd_prep_bf16<64><<<gprep, 256, 0, stream>>>(o16, do16, lse, H, S, Sp, lsd);
            attn_bwd_dkdv_bf16<64><<<gkv, 256, 0, stream>>>(a);
        } else {
            attn_bwd_prep_bf16<128><<<gprep, 256, 0, stream>>>(o16, do16, lse, H, S, Sp, lsd);
            attn_bwd_dkdv_bf16<128><<<gkv, 256, 0, stream>>>(a);
        }
        const int64_t n8 = a.sum_n8;
        if (a.ngroups > 1 && !from_ds) {
            const int64_t blocks = std::min<int64_t>((2 * n8 + 255) / 256, 4096);
            attn_bwd_sum<<<dim3((unsigned)blocks), 256, 0, stream>>>(a.dk_part, a.dv_part, a.dk, a.dv, a.ngroups,
                                                                     S * D, n8);
        }
        if (from_ds) {
            // with partials, the dQ launch also sums them: 512 more blocks
            // (a round of its two-per-CU slots), dispatched after the dQ blocks
            const int64_t nsum = a.ngroups > 1 ? std::min<int64_t>((2 * n8 + 255) / 256, 512) : 0;
            const dim3 gds((unsigned)(a.dq_blocks + nsum));
            if (D == 64) attn_bwd_dq_ds_bf16<64><<<gds, 256, 0, stream>>>(a);
            else attn_bwd_dq_ds_bf16<128><<<gds, 256, 0, stream>>>(a);
        } else {
            if (D == 64) attn_bwd_dq_bf16<64><<<grid, 256, 0, stream>>>(a);
            else attn_bwd_dq_bf16<128><<<grid, 256, 0, stream>>>(a);
        }
        return hipGetLastError();
    }
    float* delta = reinterpret_cast<float*>(base + w.lsd);
    const dim3 gq((unsigned)(((int64_t)B * H * S + 3) / 4));
    const dim3 gk((unsigned)(((int64_t)B * Hkv * S + 3) / 4));
    if (d.dtype == MC_F32) {
        const float *qf = static_cast<const float*>(q), *kf = static_cast<const float*>(k),
                    *vf = static_cast<const float*>(v), *of = static_cast<const float*>(o),
                    *gf = static_cast<const float*>(dout);
        attn_bwd_delta_generic<float><<<gq, 256, 0, stream>>>(of, gf, delta, B, H, S, D);
        attn_bwd_dq_generic<float><<<gq, 256, 0, stream>>>(qf, kf, vf, mask, lse, delta, gf,
                                                           static_cast<float*>(dq), B, H, Hkv, S, D, d.scale,
                                                           d.causal);
        attn_bwd_dkdv_generic<float><<<gk, 256, 0, stream>>>(qf, kf, vf, mask, lse, delta, gf,
                                                             static_cast<float*>(dk), static_cast<float*>(dv), B, H,
                                                             Hkv, S, D, d.scale, d.causal);
    } else {
        const uint16_t *qh = static_cast<const uint16_t*>(q), *kh = static_cast<const uint16_t*>(k),
                       *vh = static_cast<const uint16_t*>(v), *oh = static_cast<const uint16_t*>(o),
                       *gh = static_cast<const uint16_t*>(dout);
        attn_bwd_delta_generic<uint16_t><<<gq, 256, 0, stream>>>(oh, gh, delta, B, H, S, D);
        attn_bwd_dq_generic<uint16_t><<<gq, 256, 0, stream>>>(qh, kh, vh, mask, lse, delta, gh,
                                                              static_cast<uint16_t*>(dq), B, H, Hkv, S, D, d.scale,
                                                              d.causal);
        attn_bwd_dkdv_generic<uint16_t><<<gk, 256, 0, stream>>>(qh, kh, vh, mask, lse, delta, gh,
                                                                static_cast<uint16_t*>(dk),
                                                                static_cast<uint16_t*>(dv), B, H, Hkv, S, D, d.scale,
                                                                d.causal);
    }
    return hipGetLastError();
}

}  // namespace mc
