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
//  rowsplit   the same products for passes of up to 64 ranks as a skinny
//             GEMM through LDS: 256-row workgroups share each parameter
//             stage, columns split over workgroups, partials finished (sum in
//             split order, scale, mask, both output layouts) by dy_finish.
//  colreduce  dA = x^T.Gd and dB = scale Hd^T.dY: reductions over tokens.
//             The token dim is the MFMA K dim, but it is the strided dim of
//             x / dY, so each lane loads an 8 x 8 bf16 block (8 rows, 16 B
//             each) and transposes it in registers; the 8 resulting columns
//             feed 8 MFMAs whose 16 column slots are the lanes' 16 column
//             groups. The fp32 Gd^T / Hd^T operand is split hi + lo as above.
//             Tokens are split in a fixed partition; the partials are summed
//             in split order by split_sum (deterministic, no atomics).
//  All bf16 kernels load through buffer resources whose range checks zero
//  the out-of-range rows and columns, so their loops have no branches and
//  issue every load of an unrolled block before its MFMAs.
//
// fp32 variants (plain FMA) serve act_dtype == MC_F32.
#include <algorithm>

#include "common.hpp"
#include "lora_kernels.hpp"

namespace mc {
namespace {

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// Instruction classes of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008, kSchedVmemRead = 0x020;

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
// Up to kPrepJobs operand-preparation jobs in one launch: element idx of the
// launch belongs to the job whose range [start[j], start[j + 1]) holds it.
__device__ __forceinline__ void prep_one(const PrepJob& j, int64_t idx) {
    const int64_t i = idx / j.cols_out, c = idx % j.cols_out;
    float v = 0.f;
    if (i < j.valid_rows && c < j.valid_cols) v = j.transpose ? j.src[c * j.ld_src + i] : j.src[i * j.ld_src + c];
    const uint16_t h = f32_to_bf16(v);
    const int64_t o = j.frag_rc ? rowproj_frag_index(j.frag_rc, j.frag_row0 + i, c) : i * j.ld_out + c;
    j.hi[o] = h;
    if (j.lo) j.lo[o] = f32_to_bf16(v - bf16_to_f32(h));
}

// Eight consecutive output columns 8 g' .. +7 of one output row (g' the
// group within the row): one division per eight elements and 16-byte stores
// of hi and lo. Used when every job of a batch has cols_out and ld_out
// multiples of 8 and 16-byte aligned outputs (prep_vec8).
__device__ __forceinline__ void prep_one8(const PrepJob& j, int64_t g) {
    const int64_t cg = j.cols_out >> 3;
    const int64_t i = g / cg, c0 = (g - i * cg) * 8;
    const bool row_ok = i < j.valid_rows;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int64_t c = c0 + e;
        const bool ok = row_ok && c < j.valid_cols;
        const float x = j.src[ok ? (j.transpose ? c * j.ld_src + i : i * j.ld_src + c) : 0];  // an in-range address
        v[e] = ok ? x : 0.f;
    }
    uint4 hi, lo;
    split_hilo8(v, hi, lo);
    const int64_t o = j.frag_rc ? rowproj_frag_index(j.frag_rc, j.frag_row0 + i, c0) : i * j.ld_out + c0;
    *reinterpret_cast<uint4*>(j.hi + o) = hi;
    if (j.lo) *reinterpret_cast<uint4*>(j.lo + o) = lo;
}

bool prep_vec8(const PrepJob& j) {
    // prep_one8 reads src[0] for the zero elements: src must exist; in
    // fragment order eight columns from a multiple of 8 are 16 contiguous bytes
    return j.src && j.cols_out % 8 == 0 && (j.frag_rc || j.ld_out % 8 == 0) &&
           reinterpret_cast<uintptr_t>(j.hi) % 16 == 0 && reinterpret_cast<uintptr_t>(j.lo) % 16 == 0;
}

struct PrepBatch {
    PrepJob job[kPrepJobs];
    int64_t start[kPrepJobs + 1];  // in elements, or in 8-element groups (vec8)
    int njobs;
};

template <bool VEC8>
__global__ __launch_bounds__(256) void prep_bf16(PrepBatch b) {
    const int64_t n = b.start[b.njobs];
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        int j = 0;
        while (j + 1 < b.njobs && idx >= b.start[j + 1]) ++j;
        if constexpr (VEC8) prep_one8(b.job[j], idx - b.start[j]);
        else prep_one(b.job[j], idx - b.start[j]);
    }
}

// --------------------------------------------------------------- rowproj
// Workgroup: NW waves, 16 RT token rows (RT MFMA row tiles). Wave w takes the
// 64-column steps w, w+NW, ...; in a step, lane l (row l % 16 of each row
// tile, group g = l / 16) takes the 16 contiguous columns 64 s + 16 g .. +15
// of x and of the parameter rows and feeds them to two MFMA 16x16x32 as
// k-chunks (columns 0-7, then 8-15 of its 16): the k order inside a step is
// permuted identically for x and P, so the sum over columns is unchanged.
// The parameter fragments are shared by the RT row tiles. x is loaded in
// whole 128-byte lines (8 rows per load) one step ahead and reaches the
// MFMA layout through a per-wave LDS tile; at c4 the MFMA layout loaded
// straight from memory (16 rows x 64 bytes per load) took the operand passes
// 19.2 us against 16.8. Buffer range checks zero rows past T and columns
// past C (no branches). The NW waves' partial sums are combined in wave order
// through LDS.
// Arguments of one row projection. With PF32 the parameter is read as fp32
// P [prows][C] (rows past prows load as zeros) and split into bf16 hi + lo in
// registers; otherwise it comes prepared as bf16 P_hi / P_lo [16 RC][C] in
// fragment order (rowproj_frag_index), so that each of its loads reads 1 KB
// of contiguous lines: read as [16 RC][C] rows, every load touched 16 rows
// of 64 bytes, and at c4 the parameter loads took 3.8-7.8 us of the 17-24 us
// row projections (a copy without them ran that much faster).
// The r ranks of a pass may belong to several projections of the same x
// (rp ranks each, projection p = j / rp): rank j then takes projection p's
// mask row and goes to its out_t rows and to columns p rext_p .. of the
// extension operand (row stride ext_ld), whose pad columns rp .. rext_p-1 are
// written as zeros.
struct RowprojArgs {
    const uint16_t* X;
    int64_t T, C;
    const uint16_t* Phi;
    const uint16_t* Plo;
    const float* Pf;
    int prows;
    int r;
    int rp;
    float scale;
    const uint8_t* mask[kMaxProj];
    int64_t mask_ld;  // elements between the mask rows of consecutive tokens
    float keep;
    float* out_t[kMaxProj];
    uint16_t* out_ext;
    int rext_p;
    int ext_ld;
    float ext_scale;
};

template <int RC, int RT, int U, bool PF32, int NW>
__device__ __forceinline__ void rowproj_body(const RowprojArgs& A, int64_t blk) {
    static_assert(U == 1, "one step per iteration, the next step's x in flight");
    const uint16_t* __restrict__ X = A.X;
    const int64_t T = A.T, C = A.C;
    const int r = A.r, rp = A.rp, rext_p = A.rext_p, ext_ld = A.ext_ld;
    const float scale = A.scale, keep = A.keep, ext_scale = A.ext_scale;
    uint16_t* __restrict__ out_ext = A.out_ext;
    constexpr int ROWS = 16 * RT;
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int64_t t0 = blk * ROWS;
    const int64_t nrows = T - t0 < ROWS ? T - t0 : ROWS;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(X + t0 * C, nrows * C * 2);
    const int64_t pbytes = (int64_t)16 * RC * ((C + 63) / 64 * 64) * 2;  // fragment-order operand
    const __amdgpu_buffer_rsrc_t rhi = make_rsrc(PF32 ? (const void*)A.Pf : (const void*)A.Phi,
                                                 PF32 ? (int64_t)A.prows * C * 4 : pbytes);
    const __amdgpu_buffer_rsrc_t rlo = make_rsrc(A.Plo, PF32 ? 0 : pbytes);
    const int row = lane & 15, grp = lane >> 4;
    const int64_t nsteps = (C + 63) / 64;

    f32x4 acc[RT][RC];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int rc = 0; rc < RC; ++rc) acc[rt][rc] = f32x4{0.f, 0.f, 0.f, 0.f};

    // x goes through a per-wave LDS tile: each load covers 8 rows x 128
    // bytes (whole lines) instead of the MFMA layout's 16 rows x 64 bytes;
    // chunk c of tile row rr sits in slot c ^ ((rr >> 1) & 7). The next
    // step's x is loaded while this step's is used. The tile shares its
    // memory with the wave-combine buffer below.
    constexpr int XST_BYTES = NW * RT * 16 * 128;
    constexpr int RED_BYTES = NW * RT * RC * 4 * 64 * 4;
    __shared__ __attribute__((aligned(16))) char lds_buf[XST_BYTES > RED_BYTES ? XST_BYTES : RED_BYTES];
    uint4 (*xst)[16][8] = reinterpret_cast<uint4 (*)[16][8]>(lds_buf) + wave * RT;
    const int nsw = nsteps > wave ? (int)((nsteps - wave + NW - 1) / NW) : 0;  // this wave's steps
    const int xr = lane >> 3, xc8 = lane & 7;
    i32x4 xa[RT][2], xb[RT][2];
    auto load_x = [&](int64_t st, i32x4 (&v)[RT][2]) {
        const int64_t col = st * 64 + 8 * xc8;
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int hp = 0; hp < 2; ++hp)
                v[rt][hp] = buf_load16(rx, col < C ? (uint32_t)(((int64_t)(rt * 16 + 8 * hp + xr) * C + col) * 2) : kOOB);
    };
    if (nsw > 0) load_x(wave, xa);
    for (int i = 0; i < nsw; ++i) {
        const int64_t st = wave + (int64_t)NW * i;
        const int64_t c = st * 64 + grp * 16;
        i32x4 ph[RC][2], pl[RC][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const bool ok = c + 8 * h < C;
#pragma unroll
            for (int rc = 0; rc < RC; ++rc) {
                if constexpr (PF32) {
                    const uint32_t off = ok ? (uint32_t)(((int64_t)(rc * 16 + row) * C + c + 8 * h) * 4) : kOOB;
                    const i32x4 a = buf_load16(rhi, off), b = buf_load16(rhi, ok ? off + 16 : kOOB);
                    float v[8], rem[8];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[e] = __int_as_float(a[e]);
                        v[4 + e] = __int_as_float(b[e]);
                    }
                    const bf16x8 hi = pack_bf16x8(v);
#pragma unroll
                    for (int e = 0; e < 8; ++e) rem[e] = v[e] - static_cast<float>(hi[e]);
                    ph[rc][h] = __builtin_bit_cast(i32x4, hi);
                    pl[rc][h] = __builtin_bit_cast(i32x4, pack_bf16x8(rem));
                } else {
                    const uint32_t off = ok ? (uint32_t)((((st * RC + rc) * 2 + h) * 64 + lane) * 16) : kOOB;
                    ph[rc][h] = buf_load16(rhi, off);
                    pl[rc][h] = buf_load16(rlo, off);
                }
            }
        }
        if (i + 1 < nsw) load_x(st + NW, xb);  // wave-uniform
        // this step's x: whole-line registers -> LDS -> MFMA layout (a
        // wave's LDS operations complete in order)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int hp = 0; hp < 2; ++hp) {
                const int rr = 8 * hp + xr;
                xst[rt][rr][xc8 ^ ((rr >> 1) & 7)] = __builtin_bit_cast(uint4, xa[rt][hp]);
            }
        i32x4 xv[RT][2];
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int h = 0; h < 2; ++h) xv[rt][h] = __builtin_bit_cast(i32x4, xst[rt][row][(2 * grp + h) ^ ((row >> 1) & 7)]);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int rc = 0; rc < RC; ++rc) {
                    const bf16x8 xq = __builtin_bit_cast(bf16x8, xv[rt][h]);
                    acc[rt][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        xq, __builtin_bit_cast(bf16x8, ph[rc][h]), acc[rt][rc], 0, 0, 0);
                    acc[rt][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        xq, __builtin_bit_cast(bf16x8, pl[rc][h]), acc[rt][rc], 0, 0, 0);
                }
#pragma unroll
        for (int rt = 0; rt < RT; ++rt)
#pragma unroll
            for (int hp = 0; hp < 2; ++hp) xa[rt][hp] = xb[rt][hp];
    }
    __syncthreads();  // every wave is done with its x tile before the buffer is reused

    // combine the NW waves: [wave][rt][rc][q][lane]; accumulator q of lane l
    // is token 4 (l / 16) + q of its row tile, rank index l % 16.
    float (*red)[RT][RC][4][64] = reinterpret_cast<float (*)[RT][RC][4][64]>(lds_buf);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int rc = 0; rc < RC; ++rc)
#pragma unroll
            for (int q = 0; q < 4; ++q) red[wave][rt][rc][q][lane] = acc[rt][rc][q];
    __syncthreads();
    // A thread finishes 4 consecutive tokens of one rank (accumulators
    // q = 0..3 of a lane), so each out_t row segment goes out as one 16-byte
    // store. With one value per thread (4-byte out_t pieces over 16 rows) the
    // r48 row projection at c4 took 17.5 us against 16.5, the operand passes
    // 20.0 us against 19.3. Staging the extension rows through LDS for 16-byte
    // stores as well measured no faster.
    for (int idx = threadIdx.x; idx < RT * RC * 64; idx += 64 * NW) {
        const int l = idx & 63, rc = (idx >> 6) % RC, rt = (idx >> 6) / RC;
        const int j = rc * 16 + (l & 15);
        const int64_t tq = t0 + rt * 16 + (l >> 4) * 4;  // tokens tq .. tq + 3
        if (tq >= T || j >= r) continue;
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[q] = red[0][rt][rc][q][l];
#pragma unroll
            for (int w = 1; w < NW; ++w) v[q] += red[w][rt][rc][q][l];
        }
        const int p = j / rp, jj = j - p * rp;
        const uint8_t* mask = p == 0 ? A.mask[0] : p == 1 ? A.mask[1] : p == 2 ? A.mask[2] : A.mask[3];
        float* out_t = p == 0 ? A.out_t[0] : p == 1 ? A.out_t[1] : p == 2 ? A.out_t[2] : A.out_t[3];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v[q] *= scale;
            if (mask && tq + q < T) v[q] = mask[(tq + q) * A.mask_ld + jj] ? v[q] * keep : 0.f;
        }
        if (out_t) {
            float* o = out_t + (int64_t)jj * T + tq;
            if (tq + 3 < T && (reinterpret_cast<uintptr_t>(o) & 15) == 0) {
                *reinterpret_cast<float4*>(o) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (tq + q < T) o[q] = v[q];
            }
        }
        if (out_ext) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (tq + q >= T) break;
                uint16_t* e = out_ext + (tq + q) * ext_ld + p * rext_p;
                e[jj] = f32_to_bf16(v[q] * ext_scale);
                if (jj == rp - 1)
                    for (int z = rp; z < rext_p; ++z) e[z] = 0;
            }
        }
    }
}

// Eight waves per workgroup: at c4 (1536 columns, 24 steps) the 48- and
// 32-rank passes ran 20.6 -> 18.0 and 15.9 -> 14.5 us against four waves.
constexpr int kRowprojWaves = 8;
template <int RC, int RT, int U>
__global__ __launch_bounds__(64 * kRowprojWaves) void rowproj_bf16(RowprojArgs A) {
    rowproj_body<RC, RT, U, false, kRowprojWaves>(A, blockIdx.x);
}

// ------------------------------------------------------------- colreduce
// Up to two column-reduction jobs in one launch (blocks [0, nblk0) job 0).
// Workgroup: 4 waves, 128 columns, the token range of one split. Wave w takes
// 32-row steps w, w+4, ... of the range; lane l loads rows t0 + 8 (l/16) + i
// (i < 8) at columns c0 + 8 (l%16) .. +7 (256 contiguous bytes per row and
// wave), transposes the 8 x 8 block in registers and feeds the 8 columns to
// 8 MFMAs whose 16 output columns are the lanes' 16 column groups. Loads of
// U steps are issued ahead of their MFMAs; buffer range checks zero rows
// past the split and columns past C.
struct ColJobDev {
    const uint16_t* X;
    int64_t C;
    const float* Pt;
    int r;
    int64_t chunk;
    float* partial;
    int64_t part_stride;
    int ctiles;
    int splits;  // every split writes its partial (splits past T write zeros)
};
struct ColBatch {
    ColJobDev job[kColJobs];
    int start[kColJobs + 1];  // first workgroup of each job
    int njobs;
};

// Two waves per SIMD (256 registers per lane at most): at 64 ranks the
// kernel otherwise took 142 VGPRs + 128 AGPRs, one wave per SIMD, and
// streamed at 2.4 TB/s; with the bound it fits in 236 VGPRs, no spills.
template <int RC, int U, bool PTV>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void colreduce_bf16(int64_t T, ColBatch cb) {
    int ji = 0;
    while (ji + 1 < cb.njobs && (int)blockIdx.x >= cb.start[ji + 1]) ++ji;  // wave-uniform
    const ColJobDev& J = cb.job[ji];
    const int b = (int)blockIdx.x - cb.start[ji];
    const uint16_t* X = J.X;
    const int64_t C = J.C;
    const float* Pt = J.Pt;
    const int r = J.r;
    const int64_t chunk = J.chunk;
    const int ctiles = J.ctiles;
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int64_t c0 = (int64_t)(b % ctiles) * 128;
    const int64_t tb = (int64_t)(b / ctiles) * chunk;
    const int64_t te = tb + chunk < T ? tb + chunk : T;
    const int64_t col = c0 + 8 * (lane & 15);
    const bool col_ok = col < C;
    const int g8 = 8 * (lane >> 4);
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(X + tb * C, (te - tb) * C * 2);
    // Pt through one resource per 16-rank tile: a tile's offsets stay below
    // 16 T 4 bytes (< 2^30 for T < 2^24); rows past r fall outside
    __amdgpu_buffer_rsrc_t rp[RC];
#pragma unroll
    for (int rc = 0; rc < RC; ++rc) {
        const int rows = r - rc * 16 < 16 ? (r - rc * 16 > 0 ? r - rc * 16 : 0) : 16;
        rp[rc] = make_rsrc(Pt + (int64_t)rc * 16 * T, (int64_t)rows * T * 4);
    }

    f32x4 acc[8][RC];
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int rc = 0; rc < RC; ++rc) acc[e][rc] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int64_t s0 = tb + 32 * wave; s0 < te; s0 += 128 * U) {
        uint4 R[U][8];
        float pv[U][RC][8];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t t0 = s0 + 128 * u;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int64_t t = t0 + g8 + i - tb;
                const i32x4 v = buf_load16(rx, col_ok ? (uint32_t)((t * C + col) * 2) : kOOB);
                R[u][i] = __builtin_bit_cast(uint4, v);
            }
#pragma unroll
            for (int rc = 0; rc < RC; ++rc) {
                const int jl = lane & 15;  // rank within the tile
                const int64_t t = t0 + g8;
                if constexpr (PTV) {  // T % 4 == 0: 16-byte aligned rows of Pt
                    const uint32_t off = (uint32_t)(((int64_t)jl * T + t) * 4);
                    const i32x4 a = buf_load16(rp[rc], off), bq = buf_load16(rp[rc], off + 16);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        pv[u][rc][e] = __int_as_float(a[e]);
                        pv[u][rc][4 + e] = __int_as_float(bq[e]);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        pv[u][rc][e] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                            rp[rc], (int)(((int64_t)jl * T + t + e) * 4), 0, 0));
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            uint4 ahi[RC], alo[RC];
#pragma unroll
            for (int rc = 0; rc < RC; ++rc) {
                // tokens past the range: x is zero there, and Pt is zeroed so
                // that a non-finite value of another token cannot leak in
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = (s0 + 128 * u + g8 + e < te) ? pv[u][rc][e] : 0.f;
                split_hilo8(v, ahi[rc], alo[rc]);
            }
            uint4 Bt[8];
            transpose8x8(R[u], Bt);
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int rc = 0; rc < RC; ++rc) {
                    acc[e][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ahi[rc]), as_bf16x8(Bt[e]), acc[e][rc], 0, 0, 0);
                    acc[e][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(alo[rc]), as_bf16x8(Bt[e]), acc[e][rc], 0, 0, 0);
                }
        }
        // every load of the block first (see rowproj_bf16)
        __builtin_amdgcn_sched_group_barrier(kSchedVmemRead, U * (8 + (PTV ? 2 : 8) * RC), 0);
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
    if (wave == 0 && col_ok) {
        float* out = J.partial + (int64_t)(b / ctiles) * J.part_stride;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t c = col + e;
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

// ------------------------------------------------------------- colsplit
// The column reduction of a group of up to 64 ranks with the token-side
// operand given as bf16 hi / lo planes [rows][T] (Gd^T or Hd^T split once,
// so the loop does no fp32 splitting). Workgroup: 4 waves over 512 columns
// (wave w: columns c0 + 128 w .. +127) and the token range of one split,
// walked in 32-token stages; each stage of x (32 rows x 512 columns, plain
// row-major rows of 1 KB) and of both planes (64 rank rows x 32 tokens, the
// GEMM kernels' swizzled layout) goes into LDS with buffer_load ... lds, in
// a ring of three stages (two in flight while one is multiplied), so a CU
// keeps 80 KB of loads outstanding. Lane l reads rows 8 (l/16) + i (i < 8)
// of its wave's columns 8 (l%16) .. +7 from LDS, transposes the 8 x 8 block
// in registers and feeds colreduce_bf16's MFMAs; the planes' fragments are
// shared by the four waves. Rows past the split and columns past C load as
// zeros (buffer range checks), and so do plane tokens past the split (whole
// 8-token chunks: T % 8 == 0 and splits of whole stages).
struct ColsplitJobDev {
    const uint16_t* X;
    int64_t C;
    const uint16_t* Phi;
    const uint16_t* Plo;
    int r;
    int64_t chunk;
    float* partial;
    int64_t part_stride;
    int ctiles;
    int splits;  // every split writes its partial (splits past T write zeros)
};
struct ColsplitBatch {
    ColsplitJobDev job[kColJobs];
    int start[kColJobs + 1];  // first workgroup of each job
    int njobs;
};

template <int RC>
__global__ __launch_bounds__(256) void colsplit_bf16(int64_t T, ColsplitBatch cb) {
    constexpr int TOK = 32, BCOLS = 512;
    constexpr int XB = TOK * BCOLS * 2, PB = 64 * TOK * 2, SB = XB + 2 * PB;
    constexpr int NL = (XB + 2 * PB) / 1024 / 4;  // loads per wave per stage
    __shared__ __attribute__((aligned(1024))) char smem[3 * SB];
    const uint32_t sbyte = (uint32_t)reinterpret_cast<uintptr_t>(smem);
    int ji = 0;
    while (ji + 1 < cb.njobs && (int)blockIdx.x >= cb.start[ji + 1]) ++ji;  // wave-uniform
    // the job's fields into registers before any LDS traffic (a scalar
    // load's wait also waits for the LDS reads)
    const ColsplitJobDev J = cb.job[ji];
    const int b = (int)blockIdx.x - cb.start[ji];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t C = J.C;
    const int64_t cb0 = (int64_t)(b % J.ctiles) * BCOLS;
    const int64_t split = b / J.ctiles;
    const int64_t tb = split * J.chunk;
    const int64_t te = tb + J.chunk < T ? tb + J.chunk : T;
    const int nst = te > tb ? (int)((te - tb + TOK - 1) / TOK) : 0;
    const i32x4 rx = rsrc_words(J.X + tb * C, (te - tb) * C * 2);
    const i32x4 rh = rsrc_words(J.Phi, (int64_t)J.r * T * 2);
    const i32x4 rl = rsrc_words(J.Plo, (int64_t)J.r * T * 2);
    // x: DMA k of wave w moves tile row 8 w + k (1 KB), lane l its chunk l
    const bool xc_ok = cb0 + 8 * lane < C;
    auto issue = [&](int st) {
        const uint32_t base = sbyte + (uint32_t)((st % 3) * SB);
        const int64_t t0 = tb + (int64_t)st * TOK;
#pragma unroll
        for (int k = 0; k < XB / 1024 / 4; ++k) {
            const int row = wave * (XB / 1024 / 4) + k;
            const uint32_t off = xc_ok ? (uint32_t)(((t0 - tb + row) * C + cb0 + 8 * lane) * 2) : kOOB;
            dma16(rx, __builtin_amdgcn_readfirstlane(base + (uint32_t)row * 1024u), off);
        }
        dma_tile<64, 256, TOK>(rh, base + XB, (uint32_t)T, (uint32_t)t0, (uint32_t)te, tid);
        dma_tile<64, 256, TOK>(rl, base + XB + PB, (uint32_t)T, (uint32_t)t0, (uint32_t)te, tid);
    };

    f32x4 acc[8][RC];
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int rc = 0; rc < RC; ++rc) acc[e][rc] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int g8 = 8 * (lane >> 4);
    const int psw = ((lane & 15) / (128 / TOK)) % (TOK / 8);  // swizzle term of plane rows rc 16 + l % 16

    if (nst > 0) issue(0);
    if (nst > 1) issue(1);
    for (int st = 0; st < nst; ++st) {
        if (st + 1 < nst) wait_vmcnt<NL>();  // stage st + 1 may stay in flight
        else wait_vmcnt<0>();
        __syncthreads();  // stage st visible to every wave; stage st - 1 free
        if (st + 2 < nst) issue(st + 2);
        const char* sx = smem + (st % 3) * SB;
        const char* sp = sx + XB;
        uint4 R[8];
#pragma unroll
        for (int i = 0; i < 8; ++i)
            R[i] = *reinterpret_cast<const uint4*>(sx + (g8 + i) * (BCOLS * 2) + (wave * 16 + (lane & 15)) * 16);
        bf16x8 ahi[RC], alo[RC];
#pragma unroll
        for (int rc = 0; rc < RC; ++rc) {
            const int off = (rc * 16 + (lane & 15)) * (TOK * 2) + (((lane >> 4) ^ psw) * 16);
            ahi[rc] = *reinterpret_cast<const bf16x8*>(sp + off);
            alo[rc] = *reinterpret_cast<const bf16x8*>(sp + PB + off);
        }
        uint4 Bt[8];
        transpose8x8(R, Bt);
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int rc = 0; rc < RC; ++rc) {
                acc[e][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi[rc], as_bf16x8(Bt[e]), acc[e][rc], 0, 0, 0);
                acc[e][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo[rc], as_bf16x8(Bt[e]), acc[e][rc], 0, 0, 0);
            }
    }

    // accumulator q of lane l, MFMA e: rank rc 16 + 4 (l/16) + q, column
    // 8 (l%16) + e of the wave's 128
    const int64_t col = cb0 + 128 * wave + 8 * (lane & 15);
    if (col < C) {
        float* out = J.partial + split * J.part_stride;
#pragma unroll
        for (int rc = 0; rc < RC; ++rc)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int j = rc * 16 + (lane >> 4) * 4 + q;
                if (j >= J.r) continue;
#pragma unroll
                for (int e = 0; e < 8; e += 4)
                    *reinterpret_cast<float4*>(out + (int64_t)j * C + col + e) =
                        make_float4(acc[e][rc][q], acc[e + 1][rc][q], acc[e + 2][rc][q], acc[e + 3][rc][q]);
            }
    }
}

// out = scale * sum_s partial[s][j][c] (s ascending) for up to two jobs
// (threads [0, n0) job 0). Splits are unrolled by 8 so that their loads are
// in flight together; the adds stay in split order.
__device__ __forceinline__ void split_sum_one(const SumJob& J, int64_t idx) {
    const int r = J.r;
    const int64_t j = idx / J.C, c = idx % J.C;
    const float* p = J.partial + j * J.C + c;
    const int64_t stride = J.part_stride;
    float s = 0.f;
    int k = 0;
    for (; k + 8 <= J.splits; k += 8) {
        float v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = p[(int64_t)(k + u) * stride];
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; k < J.splits; ++k) s += p[(int64_t)k * stride];
    s *= J.scale;
    if (J.transpose_out) J.out[c * r + j] = s;
    else J.out[j * J.C + c] = s;
}

// Four consecutive columns of one row (C % 4 == 0, 16-byte aligned
// partials and, for the untransposed output, out): the 16-byte loads of
// eight splits are issued together (splits past the job's read zeros through
// an empty buffer range), and each column's adds stay in split order, so the
// sums equal split_sum_one's.
__device__ __forceinline__ void split_sum_four(const SumJob& J, int64_t g) {
    const int64_t cq = J.C >> 2;
    const int64_t j = g / cq, c0 = (g - j * cq) * 4;
    const uint32_t off = (uint32_t)((j * J.C + c0) * 4);
    const int64_t split_bytes = J.part_stride * 4;
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < J.splits; k0 += 8) {
        f32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const __amdgpu_buffer_rsrc_t rs =
                make_rsrc(J.partial + (int64_t)(k0 + u) * J.part_stride, k0 + u < J.splits ? split_bytes : 0);
            v[u] = __builtin_bit_cast(f32x4, buf_load16(rs, off));
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) s += v[u];
    }
    s *= J.scale;
    if (J.transpose_out) {
#pragma unroll
        for (int e = 0; e < 4; ++e) J.out[(c0 + e) * J.r + j] = s[e];
    } else {
        *reinterpret_cast<f32x4*>(J.out + j * J.C + c0) = s;
    }
}

struct SumBatch {
    SumJob job[kSumJobs];
    int64_t start[kSumJobs + 1];  // in elements, or in 4-column groups (vec4)
    int njobs;
};

template <bool VEC4>
__global__ __launch_bounds__(256) void split_sum(SumBatch sb) {
    const int64_t n = sb.start[sb.njobs];
    for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
         idx += (int64_t)gridDim.x * blockDim.x) {
        int j = 0;
        while (j + 1 < sb.njobs && idx >= sb.start[j + 1]) ++j;
        if constexpr (VEC4) split_sum_four(sb.job[j], idx - sb.start[j]);
        else split_sum_one(sb.job[j], idx - sb.start[j]);
    }
}

// --------------------------------------------------------- fused dY pass
// Workgroup: 4 waves over one column group (wave w: columns c0 + 128 w ..
// +127) and the token range of one split; the waves walk the range together
// in 32-row steps, the next step's loads issued before the current step is
// used. In a step lane l holds rows 8 (l/16) + i (i < 8) at columns
// 8 (l%16) .. +7 of its wave's 128 (colreduce_bf16's blocks) and
//  - dB: transposes the 8 x 8 block in registers for colreduce's MFMAs
//    (Hd^T split hi + lo as the A operand), accumulating over the split;
//    each wave owns its columns, so there is no cross-wave combine;
//  - G: writes the block to its wave's LDS tile [32 rows][128 columns]
//    (16-byte chunks XOR-swizzled by row, conflict-free both ways), reads it
//    back as MFMA 16x16x32 A fragments (row l%16, 8 columns) against the
//    B rows (split hi + lo, in registers for the wave's columns); the four
//    waves' sums for the step's 32 rows are added in wave order through a
//    double-buffered LDS exchange (one barrier per step) and written to
//    gpart[group][t][0..r).
struct DyJobDev {
    const uint16_t* dY;
    int64_t N;
    const float* B;
    const float* Pt;
    float* partB;
    float* gpart;
    int64_t chunk;
    int64_t part_stride;
    int groups;
};
struct DyBatch {
    DyJobDev job[kMaxProj];
    int start[kMaxProj + 1];
    int njobs;
    int r;
};

template <int RC, bool PTV>
__global__ __launch_bounds__(256) void dy_pass_bf16(int64_t T, DyBatch db) {
    int ji = 0;
    while (ji + 1 < db.njobs && (int)blockIdx.x >= db.start[ji + 1]) ++ji;  // wave-uniform
    const DyJobDev& J = db.job[ji];
    const int b = (int)blockIdx.x - db.start[ji];
    const int r = db.r;
    const int64_t N = J.N;
    const int lane = lane_id();
    const int wave = threadIdx.x >> 6;
    const int grp = b % J.groups;
    const int64_t split = b / J.groups;
    const int64_t cw0 = (int64_t)grp * kDyCols + 128 * wave;
    const int64_t tb = split * J.chunk;
    const int64_t te = tb + J.chunk < T ? tb + J.chunk : T;
    const int64_t col = cw0 + 8 * (lane & 15);
    const bool col_ok = col < N;
    const int g8 = 8 * (lane >> 4);
    const bool do_b = J.partB != nullptr, do_g = J.gpart != nullptr;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(J.dY + tb * N, (te - tb) * N * 2);
    // Hd^T through one resource per 16-rank tile (offsets below 16 T 4 bytes)
    __amdgpu_buffer_rsrc_t rp[RC];
#pragma unroll
    for (int rc = 0; rc < RC; ++rc) {
        const int rows = r - rc * 16 < 16 ? (r - rc * 16 > 0 ? r - rc * 16 : 0) : 16;
        rp[rc] = make_rsrc(J.Pt + (int64_t)rc * 16 * T, do_b ? (int64_t)rows * T * 4 : 0);
    }
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(J.B, do_g ? (int64_t)r * N * 4 : 0);

    // G's B operand of k-chunk kc (32 columns): lane l holds B[16 rc + l%16]
    // [cw0 + 32 kc + 8 (l/16) .. +7], split hi + lo; ranks past r and
    // columns past N load as zeros
    uint4 bh[4][RC], bl[4][RC];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc)
#pragma unroll
        for (int rc = 0; rc < RC; ++rc) {
            const int j = rc * 16 + (lane & 15);
            const int64_t c = cw0 + 32 * kc + 8 * (lane >> 4);
            const bool ok = j < r && c < N;
            const uint32_t off = ok ? (uint32_t)(((int64_t)j * N + c) * 4) : kOOB;
            const i32x4 a = buf_load16(rb, off), q = buf_load16(rb, ok ? off + 16 : kOOB);
            float v[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[e] = __int_as_float(a[e]);
                v[4 + e] = __int_as_float(q[e]);
            }
            split_hilo8(v, bh[kc][rc], bl[kc][rc]);
        }

    f32x4 acc[8][RC];
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
        for (int rc = 0; rc < RC; ++rc) acc[e][rc] = f32x4{0.f, 0.f, 0.f, 0.f};

    __shared__ uint4 gtile[4][32 * 16];            // per wave: [32 rows][16 chunks]
    __shared__ float gx[2][4][2][RC][4][64];       // [buffer][wave][row tile][rc][q][lane]
    uint4* tile = gtile[wave];

    auto load_step = [&](int64_t t0, uint4 (&R)[8], float (&pv)[RC][8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t t = t0 + g8 + i - tb;
            R[i] = __builtin_bit_cast(uint4, buf_load16(rx, col_ok ? (uint32_t)((t * N + col) * 2) : kOOB));
        }
        if (do_b) {
#pragma unroll
            for (int rc = 0; rc < RC; ++rc) {
                const int jl = lane & 15;
                const int64_t t = t0 + g8;
                if constexpr (PTV) {
                    const uint32_t off = (uint32_t)(((int64_t)jl * T + t) * 4);
                    const i32x4 a = buf_load16(rp[rc], off), q = buf_load16(rp[rc], off + 16);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        pv[rc][e] = __int_as_float(a[e]);
                        pv[rc][4 + e] = __int_as_float(q[e]);
                    }
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        pv[rc][e] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                            rp[rc], (int)(((int64_t)jl * T + t + e) * 4), 0, 0));
                }
            }
        }
    };

    uint4 R[8];
    float pv[RC][8];
    if (tb < te) load_step(tb, R, pv);
    int buf = 0;
    for (int64_t t0 = tb; t0 < te; t0 += 32, buf ^= 1) {
        uint4 cR[8];
        float cp[RC][8];
#pragma unroll
        for (int i = 0; i < 8; ++i) cR[i] = R[i];
#pragma unroll
        for (int rc = 0; rc < RC; ++rc)
#pragma unroll
            for (int e = 0; e < 8; ++e) cp[rc][e] = pv[rc][e];
        if (t0 + 32 < te) load_step(t0 + 32, R, pv);  // uniform
        if (do_b) {
            uint4 ahi[RC], alo[RC];
#pragma unroll
            for (int rc = 0; rc < RC; ++rc) {
                // tokens past the range: dY is zero there, and Hd^T is zeroed
                // so that a non-finite value of another token cannot leak in
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = (t0 + g8 + e < te) ? cp[rc][e] : 0.f;
                split_hilo8(v, ahi[rc], alo[rc]);
            }
            uint4 Bt[8];
            transpose8x8(cR, Bt);
#pragma unroll
            for (int e = 0; e < 8; ++e)
#pragma unroll
                for (int rc = 0; rc < RC; ++rc) {
                    acc[e][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ahi[rc]), as_bf16x8(Bt[e]), acc[e][rc], 0, 0, 0);
                    acc[e][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(alo[rc]), as_bf16x8(Bt[e]), acc[e][rc], 0, 0, 0);
                }
        }
        if (do_g) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int row = g8 + i;
                tile[row * 16 + ((lane & 15) ^ (row & 15))] = cR[i];
            }
            // a wave's DS operations complete in order: the reads below see
            // the writes above
            f32x4 ag[2][RC];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int rc = 0; rc < RC; ++rc) ag[rt][rc] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int kc = 0; kc < 4; ++kc) {
                    const int row = rt * 16 + (lane & 15);
                    const uint4 a = tile[row * 16 + ((4 * kc + (lane >> 4)) ^ (row & 15))];
#pragma unroll
                    for (int rc = 0; rc < RC; ++rc) {
                        ag[rt][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(bh[kc][rc]), ag[rt][rc], 0, 0, 0);
                        ag[rt][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(bl[kc][rc]), ag[rt][rc], 0, 0, 0);
                    }
                }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
#pragma unroll
                for (int rc = 0; rc < RC; ++rc)
#pragma unroll
                    for (int q = 0; q < 4; ++q) gx[buf][wave][rt][rc][q][lane] = ag[rt][rc][q];
            __syncthreads();
            for (int idx = threadIdx.x; idx < 2 * RC * 4 * 64; idx += 256) {
                const int l = idx & 63, q = (idx >> 6) & 3, rc = (idx >> 8) % RC, rt = (idx >> 8) / RC;
                const float v = gx[buf][0][rt][rc][q][l] + gx[buf][1][rt][rc][q][l] + gx[buf][2][rt][rc][q][l] +
                                gx[buf][3][rt][rc][q][l];
                const int64_t t = t0 + rt * 16 + 4 * (l >> 4) + q;
                const int j = rc * 16 + (l & 15);
                if (t < te && j < r) J.gpart[((int64_t)grp * T + t) * r + j] = v;
            }
        }
    }
    if (do_b && col_ok) {
        float* out = J.partB + split * J.part_stride;
#pragma unroll
        for (int e = 0; e < 8; ++e)
#pragma unroll
            for (int rc = 0; rc < RC; ++rc)
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int j = rc * 16 + (lane >> 4) * 4 + q;
                    out[(int64_t)j * N + col + e] = acc[e][rc][q];
                }
    }
}

// Finishing of rank-r partials, one workgroup per 64 tokens of one job: the
// groups' (splits') partials are summed in group order, scaled and masked;
// the result goes to gd_ext row-wise and, through LDS, to gd_t [r][T] in
// 64-token row segments. A thread takes up to four quads (four consecutive
// ranks of one token) and issues the loads of four groups for all of them
// before adding (buffer loads: quads and groups past the end read zeros), so
// each thread keeps 16 loads in flight. VEC: ld is a multiple of 4 and a quad
// is one 16-byte load; otherwise four 4-byte loads, ranks past r zeroed.
// Blocks past the jobs' run the PrepJobs (grid-stride).
struct DyFinishBatch {
    DyFinishJob job[kMaxProj];
    PrepJob prep[kPrepJobs];
    int njobs, npreps;
    int64_t prep_start[kPrepJobs + 1];  // in elements, or in 8-element groups (prep_vec8)
    int prep8;
    int blocks_per_job;
    int r, rext, ext_ld;
    float scale, keep, ext_scale;
};

template <bool VEC>
__global__ __launch_bounds__(256) void dy_finish(int64_t T, DyFinishBatch fb) {
    const int b = (int)blockIdx.x;
    const int jobs_blocks = fb.njobs * fb.blocks_per_job;
    if (b >= jobs_blocks) {
        const int64_t n = fb.prep_start[fb.npreps];
        const int64_t nb = (int64_t)gridDim.x - jobs_blocks;
        for (int64_t idx = (int64_t)(b - jobs_blocks) * 256 + threadIdx.x; idx < n; idx += nb * 256) {
            int j = 0;
            while (j + 1 < fb.npreps && idx >= fb.prep_start[j + 1]) ++j;
            if (fb.prep8) prep_one8(fb.prep[j], idx - fb.prep_start[j]);
            else prep_one(fb.prep[j], idx - fb.prep_start[j]);
        }
        return;
    }
    const DyFinishJob J = fb.job[b / fb.blocks_per_job];
    const int64_t t0 = (int64_t)(b % fb.blocks_per_job) * 64;
    const int r = fb.r, nq = (r + 3) / 4;
    const int64_t ld = J.ld > 0 ? J.ld : r, mask_ld = J.mask_ld > 0 ? J.mask_ld : r;
    const int64_t split_bytes = T * ld * 4;
    __shared__ float tt[kFinishMaxRank][65];  // [rank][token] for the transposed store
    uint32_t off[4];
    bool valid[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int item = threadIdx.x + 256 * i, tl = item / nq, q = item % nq;
        valid[i] = item < 64 * nq && t0 + tl < T;
        off[i] = valid[i] ? (uint32_t)(((t0 + tl) * ld + 4 * q) * 4) : kOOB;
    }
    f32x4 v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int g0 = 0; g0 < J.groups; g0 += 4) {
        __amdgpu_buffer_rsrc_t rs[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            rs[k] = make_rsrc(J.gpart + (int64_t)(g0 + k) * T * ld, g0 + k < J.groups ? split_bytes : 0);
        f32x4 u[4][4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (VEC) {
                    u[k][i] = __builtin_bit_cast(f32x4, buf_load16(rs[k], off[i]));
                } else {
                    const int q = (int)((threadIdx.x + 256 * i) % nq);
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        u[k][i][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                                    rs[k], 4 * q + e < r ? off[i] + 4 * e : kOOB, 0, 0));
                }
            }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] += u[k][i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int item = threadIdx.x + 256 * i, tl = item / nq, q = item % nq;
        if (item >= 64 * nq) break;
        const int64_t t = t0 + tl;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = 4 * q + e;
            if (j >= r) break;
            float x = valid[i] ? v[i][e] * fb.scale : 0.f;
            if (valid[i]) {
                if (J.mask) x = J.mask[t * mask_ld + j] ? x * fb.keep : 0.f;
                if (J.gd_ext) {
                    uint16_t* eo = J.gd_ext + t * fb.ext_ld;
                    eo[j] = f32_to_bf16(x * fb.ext_scale);
                    if (j == r - 1)
                        for (int z = r; z < fb.rext; ++z) eo[z] = 0;
                }
            }
            tt[j][tl] = x;
        }
    }
    if (!J.gd_t && !J.gd_hi) return;  // uniform
    __syncthreads();
    if (J.gd_t)
        for (int idx = threadIdx.x; idx < 64 * r; idx += 256) {
            const int j = idx / 64, tl = idx % 64;
            if (t0 + tl < T) J.gd_t[(int64_t)j * T + t0 + tl] = tt[j][tl];
        }
    if (J.gd_hi)  // two tokens per thread: 4-byte stores of each plane
        for (int idx = threadIdx.x; idx < 32 * r; idx += 256) {
            const int j = idx / 32, tl = 2 * (idx % 32);
            const int64_t t = t0 + tl;
            const float a = tt[j][tl], c = tt[j][tl + 1];
            const uint16_t ha = f32_to_bf16(a), hc = f32_to_bf16(c);
            const uint16_t la = f32_to_bf16(a - bf16_to_f32(ha)), lc = f32_to_bf16(c - bf16_to_f32(hc));
            if (t + 1 < T && (T & 1) == 0) {
                *reinterpret_cast<uint32_t*>(J.gd_hi + (int64_t)j * T + t) = (uint32_t)ha | ((uint32_t)hc << 16);
                *reinterpret_cast<uint32_t*>(J.gd_lo + (int64_t)j * T + t) = (uint32_t)la | ((uint32_t)lc << 16);
            } else {
                if (t < T) {
                    J.gd_hi[(int64_t)j * T + t] = ha;
                    J.gd_lo[(int64_t)j * T + t] = la;
                }
                if (t + 1 < T) {
                    J.gd_hi[(int64_t)j * T + t + 1] = hc;
                    J.gd_lo[(int64_t)j * T + t + 1] = lc;
                }
            }
        }
}

// ------------------------------------------------- split row projection
// The rank-r row projection of a pass of up to 64 ranks as a skinny GEMM
// through LDS. Workgroup: 4 waves, BM = 64 RT token rows (wave w owns row
// tiles w RT .. w RT + RT - 1 of 16 rows) and one column split
// [c_begin, c_end) of one job. Every BK-column stage of x (BM rows) and of
// the parameter (64 rank rows: bf16 hi and lo planes, or one fp32 plane of
// the same size) goes from HBM / L2 into LDS with buffer_load ... lds, whole
// 128-byte lines per lane group, in the XOR-swizzled row layout of the GEMM
// kernels; a ring of three stages keeps two in flight while one is
// multiplied. The four waves read the same parameter fragments from LDS, so
// the parameter is fetched once per BM rows (once per 64 rows when each wave
// loads its own, as rowproj_bf16 does). MFMA 16x16x32 with the parameter as
// the A operand (rank rows) and x as the B operand (token columns):
// accumulator q of lane l is rank 4 (l / 16) + q, token l % 16 of its tile,
// so each lane stores four consecutive ranks of one token (16 bytes) of the
// split's partials part[s][t][16 RC]. Rows past T and columns past the split
// load as zeros through the buffer range checks.
struct RowsplitJobDev {
    const uint16_t* X;
    int64_t C;
    const void* P0;      // bf16 P_hi, or fp32 P
    const uint16_t* P1;  // bf16 P_lo (unused for fp32)
    int64_t pbytes;      // bytes of P0 (rows past them load as zeros)
    float* part;
    int splits;
    int64_t cps;  // columns per split, a multiple of BK
};
struct RowsplitBatch {
    RowsplitJobDev job[kMaxProj];
    int64_t start[kMaxProj + 1];  // first tile of each job (job-major order)
    int njobs;
    int interleave;  // jobs share X, C and splits: tile l is job l % njobs
    int64_t T;
};

template <int RT, int RC, int BK, bool PF32>
__global__ __launch_bounds__(256) void rowsplit_bf16(RowsplitBatch b) {
    constexpr int BM = 64 * RT;
    constexpr int XB = BM * BK * 2;        // x stage bytes
    constexpr int PB = 64 * BK * 2;        // one bf16 parameter plane; fp32 fills both
    constexpr int SB = XB + 2 * PB;        // stage bytes
    constexpr int PBK = PF32 ? 2 * BK : BK;  // parameter row length in bf16 units
    constexpr int NL = (XB + 2 * PB) / 1024 / 4;  // loads per wave per stage
    constexpr int KS = BK / 32;            // MFMA k-substeps per stage
    constexpr int LD = 16 * RC;            // partial row length
    static_assert(BK == 32 || BK == 64, "stage width");
    __shared__ __attribute__((aligned(1024))) char smem[3 * SB];
    const uint32_t smem_byte = (uint32_t)reinterpret_cast<uintptr_t>(smem);

    // logical tile: each XCD (workgroup id % 8) owns a contiguous range, so
    // the jobs of one (row block, split) that interleave shares x through
    // one L2
    const int total = (int)gridDim.x, pid = (int)blockIdx.x;
    const int per = total / 8, rem = total % 8, xcd = pid % 8;
    const int64_t l = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + pid / 8;
    int j = 0;
    int64_t u = 0;
    if (b.interleave) {
        j = (int)(l % b.njobs);
        u = l / b.njobs;
    } else {
        while (j + 1 < b.njobs && l >= b.start[j + 1]) ++j;
        u = l - b.start[j];
    }
    // every field of the job into registers before any LDS traffic (a
    // scalar load's wait also waits for the LDS reads)
    const RowsplitJobDev J = b.job[j];
    const int64_t T = b.T;
    const int64_t rb = u / J.splits, s = u % J.splits;
    const int64_t t0 = rb * BM;
    const int64_t nrows = T - t0 < BM ? T - t0 : BM;
    const int64_t c_begin = s * J.cps;
    const int64_t c_end = c_begin + J.cps < J.C ? c_begin + J.cps : J.C;
    const int nst = c_end > c_begin ? (int)((c_end - c_begin + BK - 1) / BK) : 0;
    const i32x4 rx = rsrc_words(J.X + t0 * J.C, nrows * J.C * 2);
    const i32x4 rp0 = rsrc_words(J.P0, J.pbytes);
    const i32x4 rp1 = rsrc_words(PF32 ? J.P0 : (const void*)J.P1, PF32 ? 0 : J.pbytes);
    const uint32_t ldx = (uint32_t)J.C, ldp = (uint32_t)(PF32 ? 2 * J.C : J.C);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    auto issue = [&](int st) {
        const uint32_t base = smem_byte + (uint32_t)((st % 3) * SB);
        const uint32_t kb = (uint32_t)(c_begin + (int64_t)st * BK), ke = (uint32_t)c_end;
        dma_tile<BM, 256, BK>(rx, base, ldx, kb, ke, tid);
        if constexpr (PF32) {
            dma_tile<64, 256, PBK>(rp0, base + XB, ldp, 2 * kb, 2 * ke, tid);
        } else {
            dma_tile<64, 256, BK>(rp0, base + XB, ldp, kb, ke, tid);
            dma_tile<64, 256, BK>(rp1, base + XB + PB, ldp, kb, ke, tid);
        }
    };

    f32x4 acc[RT][RC];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int rc = 0; rc < RC; ++rc) acc[rt][rc] = f32x4{0.f, 0.f, 0.f, 0.f};

    // fragment rows of a lane differ by multiples of 16, so the swizzle term
    // depends on the lane only
    const int fr = lane & 15, kc = lane >> 4;
    const int swx = (fr / (128 / BK)) % (BK / 8);
    const int swp = (fr / (128 / PBK)) % (PBK / 8);

    if (nst > 0) issue(0);
    if (nst > 1) issue(1);
    for (int st = 0; st < nst; ++st) {
        if (st + 1 < nst) wait_vmcnt<NL>();  // stage st + 1 may stay in flight
        else wait_vmcnt<0>();
        __syncthreads();  // stage st visible to every wave; stage st - 1 free
        if (st + 2 < nst) issue(st + 2);
        const char* sx = smem + (st % 3) * SB;
        const char* sp = sx + XB;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            const int chunk = 4 * ks + kc;
            bf16x8 xf[RT], ph[RC], pl[RC];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                const int row = (wave * RT + rt) * 16 + fr;
                xf[rt] = *reinterpret_cast<const bf16x8*>(sx + row * (BK * 2) + ((chunk ^ swx) * 16));
            }
#pragma unroll
            for (int rc = 0; rc < RC; ++rc) {
                const int prow = rc * 16 + fr;
                if constexpr (PF32) {
                    const char* pr = sp + prow * (PBK * 2);
                    const f32x4 a = *reinterpret_cast<const f32x4*>(pr + (((2 * chunk) ^ swp) * 16));
                    const f32x4 c = *reinterpret_cast<const f32x4*>(pr + (((2 * chunk + 1) ^ swp) * 16));
                    float v[8], rem8[8];
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        v[e] = a[e];
                        v[4 + e] = c[e];
                    }
                    ph[rc] = pack_bf16x8(v);
#pragma unroll
                    for (int e = 0; e < 8; ++e) rem8[e] = v[e] - static_cast<float>(ph[rc][e]);
                    pl[rc] = pack_bf16x8(rem8);
                } else {
                    const int off = prow * (BK * 2) + ((chunk ^ swx) * 16);
                    ph[rc] = *reinterpret_cast<const bf16x8*>(sp + off);
                    pl[rc] = *reinterpret_cast<const bf16x8*>(sp + PB + off);
                }
            }
#pragma unroll
            for (int rt = 0; rt < RT; ++rt)
#pragma unroll
                for (int rc = 0; rc < RC; ++rc) {
                    acc[rt][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ph[rc], xf[rt], acc[rt][rc], 0, 0, 0);
                    acc[rt][rc] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pl[rc], xf[rt], acc[rt][rc], 0, 0, 0);
                }
        }
    }

    // partials: lane l of tile (rt, rc) holds ranks rc 16 + 4 (l / 16) + q of
    // token (wave RT + rt) 16 + l % 16; rows past T fall outside the range
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(J.part + ((int64_t)s * T + t0) * LD, nrows * LD * 4);
#pragma unroll
    for (int rt = 0; rt < RT; ++rt)
#pragma unroll
        for (int rc = 0; rc < RC; ++rc) {
            const int t = (wave * RT + rt) * 16 + fr;
            const i32x4 q = __builtin_bit_cast(i32x4, acc[rt][rc]);
            __builtin_amdgcn_raw_buffer_store_b128(q, ro, (int)((t * LD + rc * 16 + 4 * kc) * 4), 0, 0);
        }
}

// -------------------------------------------------------- bf16 transpose
// 64 x 64 tiles through LDS: 16-byte row chunks in, 16-byte column chunks
// out (the frozen W of the backward GEMM, read and written once per call).
__device__ __forceinline__ void transpose_tile(const uint16_t* __restrict__ in, int64_t rows, int64_t cols,
                                               uint16_t* __restrict__ out, int64_t tile_r, int64_t tile_c) {
    __shared__ uint16_t tile[64][64 + 2];
    const int64_t r0 = tile_r * 64, c0 = tile_c * 64;
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

// A whole matrix: workgroup b transposes tile (b / tiles_c, b % tiles_c).
__global__ __launch_bounds__(256) void transpose_bf16_k(const uint16_t* __restrict__ in, int64_t rows, int64_t cols,
                                                        uint16_t* __restrict__ out, int64_t tiles_c) {
    transpose_tile(in, rows, cols, out, (int64_t)blockIdx.x / tiles_c, (int64_t)blockIdx.x % tiles_c);
}

// ------------------------------------------- backward operands, one launch
// The inputs of the backward GEMM and the rank-r pass of each dY, as block
// roles of one launch (none reads another's output), for every projection
// o < nproj of a call:
//   row projection  G_o = s dY_o.B_o^T (B_o read as fp32), masked
//   A extension     A_o -> the bf16 extension operand of the dX GEMM
//   transpose       W_o [N_o][K] -> W_o^T [K][N_o] (64 x 64 tiles)
// Workgroup b finds its role and projection from the prefix table `start`:
// entry k nproj + o begins role k (0: row projection, 1: A extension,
// 2: transpose) of projection o. Every projection's row-projection blocks
// come first: they are the long-running ones, and dispatched behind the
// thousands of short transpose blocks they would run as a tail.
struct OperandsBatch {
    RowprojArgs rp[kMaxProj];
    PrepJob prep[kMaxProj];
    const uint16_t* w[kMaxProj];
    uint16_t* wt[kMaxProj];
    int64_t wrows[kMaxProj], wcols[kMaxProj], tcols[kMaxProj];
    int64_t start[3 * kMaxProj + 1];
    int nproj;
};

template <int RC, int RT>
__global__ __launch_bounds__(256) void lora_bwd_operands(OperandsBatch ob) {
    const int64_t b = blockIdx.x;
    int role = 0;
    while (role + 1 < 3 * ob.nproj && b >= ob.start[role + 1]) ++role;  // wave-uniform
    const int kind = role / ob.nproj, o = role % ob.nproj;
    const int64_t lb = b - ob.start[role];
    const int64_t nblk = ob.start[role + 1] - ob.start[role];
    if (kind == 0) {
        rowproj_body<RC, RT, 1, true, 4>(ob.rp[o], lb);
    } else if (kind == 1) {
        const PrepJob& ja = ob.prep[o];
        const int64_t n = ja.rows_out * ja.cols_out;
        for (int64_t idx = lb * 256 + threadIdx.x; idx < n; idx += nblk * 256) prep_one(ja, idx);
    } else {
        transpose_tile(ob.w[o], ob.wrows[o], ob.wcols[o], ob.wt[o], lb / ob.tcols[o], lb % ob.tcols[o]);
    }
}

// ------------------------------------------------------------ fp32 path
// fp32 row projection: one workgroup per token t, ranks in chunks of 8. The
// 256 threads take columns c = tid, tid + 256, ... of x's row (read once per
// chunk, coalesced) and accumulate the chunk's 8 products per column in
// column order; the 8 sums are reduced over each wave by butterfly and over
// the 4 waves in wave order through LDS.
__global__ __launch_bounds__(256) void rowproj_f32(const float* __restrict__ X, int64_t T, int64_t C,
                                                   const float* __restrict__ P, int transpose_p, int r,
                                                   float scale, const uint8_t* __restrict__ mask, float keep,
                                                   float* __restrict__ out_t, float* __restrict__ out_ext,
                                                   float ext_scale) {
    const int64_t t = blockIdx.x;
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const float* xr = X + t * C;
    __shared__ float red[4][8];
    for (int j0 = 0; j0 < r; j0 += 8) {
        const int nj = r - j0 < 8 ? r - j0 : 8;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int64_t c = threadIdx.x; c < C; c += 256) {
            const float xv = xr[c];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                if (j < nj) acc[j] += xv * (transpose_p ? P[c * r + j0 + j] : P[(int64_t)(j0 + j) * C + c]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = wave_sum(acc[j]);
            if (lane == 0) red[wave][j] = v;
        }
        __syncthreads();
        if (threadIdx.x < nj) {
            const int j = j0 + (int)threadIdx.x;
            float v = red[0][threadIdx.x] + red[1][threadIdx.x] + red[2][threadIdx.x] + red[3][threadIdx.x];
            v *= scale;
            if (mask) v = mask[t * r + j] ? v * keep : 0.f;
            if (out_t) out_t[(int64_t)j * T + t] = v;
            if (out_ext) out_ext[t * r + j] = v * ext_scale;
        }
        __syncthreads();
    }
}
// fp32 column reduction out[j][c] = scale * sum_t Pt[j][t] X[t][c] (or out
// [c][j] with transpose_out): a workgroup owns 16 columns and a chunk of 8
// ranks; its 256 threads are 4 column quads x 64 token slices, slice s
// summing t = s, s + 64, ... in order (one 16-byte load of x per token when
// C % 4 == 0, the 8 Pt values broadcast); the 64 slice sums are added in
// slice order in two LDS stages (8 runs of 8, then the runs).
// One or two reductions (dA over x and dB over dY) in one launch: blocks
// [0, nblk0) take job 0, the rest job 1.
struct ColF32Job {
    const float* X;
    int64_t C;
    const float* Pt;
    float scale;
    int transpose_out;
    float* out;
    int64_t ctiles;
};
__global__ __launch_bounds__(256) void colreduce_f32(int64_t T, int r, ColF32Job ja, ColF32Job jb, int64_t nblk0) {
    const bool second = (int64_t)blockIdx.x >= nblk0;  // workgroup-uniform
    const ColF32Job& J = second ? jb : ja;
    const int64_t b = (int64_t)blockIdx.x - (second ? nblk0 : 0);
    const float* __restrict__ X = J.X;
    const float* __restrict__ Pt = J.Pt;
    const int64_t C = J.C, ctiles = J.ctiles;
    const int64_t c0 = (b % ctiles) * 16;
    const int j0 = (int)(b / ctiles) * 8;
    const int nj = r - j0 < 8 ? r - j0 : 8;
    const int cq = threadIdx.x & 3, sl = threadIdx.x >> 2;
    const int64_t c = c0 + 4 * cq;
    const bool vec = (C & 3) == 0 && c + 3 < C;
    float acc[8][4];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[j][e] = 0.f;
    for (int64_t t = sl; t < T; t += 64) {
        float xv[4];
        if (vec) {
            const float4 q = *reinterpret_cast<const float4*>(X + t * C + c);
            xv[0] = q.x; xv[1] = q.y; xv[2] = q.z; xv[3] = q.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[e] = c + e < C ? X[t * C + c + e] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float pv = j < nj ? Pt[(int64_t)(j0 + j) * T + t] : 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[j][e] += pv * xv[e];
        }
    }
    __shared__ float red[64][8][17];  // [slice][rank][column]
    __shared__ float red2[8][8][17];  // [run][rank][column]
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[sl][j][4 * cq + e] = acc[j][e];
    __syncthreads();
    {
        // thread -> (run, rank, 2 columns): 8 x 8 x 8 = 512 sums over 2 passes
        for (int i = threadIdx.x; i < 8 * 8 * 16; i += 256) {
            const int col = i & 15, j = (i >> 4) & 7, run = i >> 7;
            float v = red[8 * run][j][col];
#pragma unroll
            for (int k = 1; k < 8; ++k) v += red[8 * run + k][j][col];
            red2[run][j][col] = v;
        }
    }
    __syncthreads();
    if (threadIdx.x < 8 * 16) {
        const int col = threadIdx.x & 15, j = threadIdx.x >> 4;
        float v = red2[0][j][col];
#pragma unroll
        for (int k = 1; k < 8; ++k) v += red2[k][j][col];
        const int64_t cc = c0 + col;
        if (j < nj && cc < C) {
            v *= J.scale;
            if (J.transpose_out) J.out[cc * r + j0 + j] = v;
            else J.out[(int64_t)(j0 + j) * C + cc] = v;
        }
    }
}

}  // namespace

hipError_t launch_prep_bf16(const PrepJob* jobs, int n, hipStream_t stream) {
    PrepBatch b{};
    int k = 0;
    bool vec8 = true;
    for (int i = 0; i < n; ++i) {
        if (!jobs[i].hi) continue;
        if (k == kPrepJobs) return hipErrorInvalidValue;
        b.job[k] = jobs[i];
        if (b.job[k].ld_out == 0) b.job[k].ld_out = b.job[k].cols_out;
        vec8 = vec8 && prep_vec8(b.job[k]);
        ++k;
    }
    b.njobs = k;
    for (int i = 0; i < k; ++i)
        b.start[i + 1] = b.start[i] + b.job[i].rows_out * b.job[i].cols_out / (vec8 ? 8 : 1);
    const int64_t total = b.start[k];
    if (total == 0) return hipSuccess;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (vec8) prep_bf16<true><<<dim3((unsigned)blocks), 256, 0, stream>>>(b);
    else prep_bf16<false><<<dim3((unsigned)blocks), 256, 0, stream>>>(b);
    return hipGetLastError();
}

hipError_t launch_prep_bf16(const PrepJob& j0, const PrepJob& j1, hipStream_t stream) {
    const PrepJob jobs[2] = {j0, j1};
    return launch_prep_bf16(jobs, 2, stream);
}

namespace {
RowprojArgs rowproj_args(const RowprojCall& c) {
    RowprojArgs A{};
    A.X = c.X; A.T = c.T; A.C = c.C;
    A.Phi = c.P_hi; A.Plo = c.P_lo; A.Pf = c.P_f32; A.prows = c.r;
    A.r = c.r; A.rp = c.rp > 0 ? c.rp : c.r;
    A.scale = c.scale; A.keep = c.keep;
    for (int p = 0; p < kMaxProj; ++p) { A.mask[p] = c.mask[p]; A.out_t[p] = c.out_t[p]; }
    A.mask_ld = c.mask_ld > 0 ? c.mask_ld : A.rp;
    A.out_ext = c.out_ext; A.rext_p = c.rext_p; A.ext_ld = c.ext_ld; A.ext_scale = c.ext_scale;
    return A;
}
}  // namespace

hipError_t launch_rowproj_bf16(const RowprojCall& c, hipStream_t stream) {
    // 64 token rows per workgroup: four MFMA row tiles share each parameter
    // fragment (measured at the c4 shapes, loading the fragments costs as
    // much per byte as streaming x, so the rows per fragment set the speed;
    // 16 or 32 rows per workgroup ran at 2.7 / 3.6 TB/s, 64 at 4.9 TB/s for
    // x [16384, 8960]). More than 64 ranks keep 32 rows (register budget).
    // P_hi / P_lo hold 16 rowproj_rc(r) rows (zero past r) in fragment order.
    const dim3 g64((unsigned)((c.T + 63) / 64)), g32((unsigned)((c.T + 31) / 32));
    const RowprojArgs A = rowproj_args(c);
    switch (rowproj_rc(c.r)) {
        case 1: rowproj_bf16<1, 4, 1><<<g64, 64 * kRowprojWaves, 0, stream>>>(A); break;
        case 2: rowproj_bf16<2, 4, 1><<<g64, 64 * kRowprojWaves, 0, stream>>>(A); break;
        case 3: rowproj_bf16<3, 4, 1><<<g64, 64 * kRowprojWaves, 0, stream>>>(A); break;
        case 4: rowproj_bf16<4, 4, 1><<<g64, 64 * kRowprojWaves, 0, stream>>>(A); break;
        default: rowproj_bf16<8, 2, 1><<<g32, 64 * kRowprojWaves, 0, stream>>>(A); break;
    }
    return hipGetLastError();
}

hipError_t launch_transpose_bf16(const void* in, int64_t rows, int64_t cols, void* out, hipStream_t stream) {
    const int64_t tiles_c = (cols + 63) / 64, tiles = tiles_c * ((rows + 63) / 64);
    if (tiles == 0) return hipSuccess;
    transpose_bf16_k<<<dim3((unsigned)tiles), 256, 0, stream>>>(static_cast<const uint16_t*>(in), rows, cols,
                                                                static_cast<uint16_t*>(out), tiles_c);
    return hipGetLastError();
}

hipError_t launch_lora_bwd_operands(const OperandsCall* calls, int n, int64_t T, int64_t K, int r, float scale,
                                    float keep, int rext_p, int ext_ld, hipStream_t stream) {
    // row projection blocks as launch_rowproj_bf16 chooses them for one
    // projection's r ranks; B rows past r load as zeros
    if (n < 1 || n > kMaxProj) return hipErrorInvalidValue;
    const int rc = rowproj_rc(r);
    const int rows_per_block = rc == 8 ? 32 : 64;
    OperandsBatch ob{};
    ob.nproj = n;
    int64_t at = 0;
    for (int o = 0; o < n; ++o) {
        const OperandsCall& c = calls[o];
        RowprojCall rc_call{};
        rc_call.X = c.dY; rc_call.T = T; rc_call.C = c.N; rc_call.P_f32 = c.B; rc_call.r = r; rc_call.rp = r;
        rc_call.scale = scale; rc_call.mask[0] = c.mask; rc_call.mask_ld = c.mask_ld; rc_call.keep = keep;
        rc_call.out_t[0] = c.gd_t;
        rc_call.out_ext = c.gd_ext; rc_call.rext_p = rext_p; rc_call.ext_ld = ext_ld; rc_call.ext_scale = 1.0f;
        ob.rp[o] = rowproj_args(rc_call);
        ob.prep[o] = c.a_ext;
        if (ob.prep[o].ld_out == 0) ob.prep[o].ld_out = ob.prep[o].cols_out;
        ob.w[o] = c.W;
        ob.wt[o] = c.Wt;
        ob.wrows[o] = c.N;  // W is [N][K]
        ob.wcols[o] = K;
        ob.tcols[o] = (K + 63) / 64;
    }
    for (int kind = 0; kind < 3; ++kind)
        for (int o = 0; o < n; ++o) {
            const OperandsCall& c = calls[o];
            int64_t nb = 0;
            if (kind == 0) nb = (c.gd_t || c.gd_ext) ? (T + rows_per_block - 1) / rows_per_block : 0;
            if (kind == 1) nb = c.a_ext.hi ? std::min<int64_t>((c.a_ext.rows_out * c.a_ext.cols_out + 255) / 256, 64) : 0;
            if (kind == 2) nb = c.Wt ? ob.tcols[o] * ((c.N + 63) / 64) : 0;
            ob.start[kind * n + o] = at;
            at += nb;
        }
    ob.start[3 * n] = at;
    if (at == 0) return hipSuccess;
    const dim3 grid((unsigned)at);
    switch (rc) {
        case 1: lora_bwd_operands<1, 4><<<grid, 256, 0, stream>>>(ob); break;
        case 2: lora_bwd_operands<2, 4><<<grid, 256, 0, stream>>>(ob); break;
        case 3: lora_bwd_operands<3, 4><<<grid, 256, 0, stream>>>(ob); break;
        case 4: lora_bwd_operands<4, 4><<<grid, 256, 0, stream>>>(ob); break;
        default: lora_bwd_operands<8, 2><<<grid, 256, 0, stream>>>(ob); break;
    }
    return hipGetLastError();
}

// Column-tile count times splits at most 512 workgroups per job, with each
// wave walking at least eight 32-row steps (c4 medians: a cap of T / 1024
// splits ran the low-rank kernels 1% faster than T / 512, T / 256 and
// T / 2048 ran slower). The kernel holds three workgroups per CU at r <= 32,
// so c4's down dA (70 column tiles x 7 splits) and dB (12 x 16) share one
// round of 768; at ~1536 per job (16 splits for the dA) the launch took 1.7
// rounds, measured 0.538 -> 0.535 ms of low-rank time per step. A split's rows of X are one
// buffer resource with 32-bit offsets, so a split never spans 2^31 bytes:
// that bound wins over the step count (wide X, e.g. a vocabulary-sized dY).
int colreduce_splits(int64_t T, int64_t C) {
    const int64_t ctiles = (C + 127) / 128;
    int64_t s = 512 / ctiles;
    const int64_t max_s = (T + 1023) / 1024;  // >= 8 steps per wave
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    const int64_t rows_cap = (int64_t)0x7fffffff / (2 * C) / 32 * 32;  // chunks are multiples of 32 rows
    const int64_t min_s = rows_cap > 0 ? (T + rows_cap - 1) / rows_cap : T;
    if (s < min_s) s = min_s;
    return (int)s;
}

hipError_t launch_colreduce_bf16(int64_t T, const ColJob* jobs, int n, hipStream_t stream) {
    // Ranks are processed in groups of up to 64 (four 16-row MFMA tiles of
    // accumulators); each group reads X once, so r <= 64 takes one pass. The
    // groups are binned by their rank tiles (16, 32, 48 or 64 rows), one
    // launch per kColJobs groups of a bin; a full bin is launched before
    // more groups are queued (a rank of 8192 has 128 groups). Every group
    // writes its own partial rows, so the launch order does not matter.
    constexpr int GS = 64, CAP = 8 * kColJobs;
    ColJobDev bins[4][CAP];
    int nb[4] = {0, 0, 0, 0};
    const bool ptv = (T & 3) == 0;
    auto flush = [&](int bin) -> hipError_t {
        for (int first = 0; first < nb[bin]; first += kColJobs) {
            ColBatch cb{};
            cb.njobs = std::min(kColJobs, nb[bin] - first);
            for (int k = 0; k < cb.njobs; ++k) {
                cb.job[k] = bins[bin][first + k];
                cb.start[k + 1] = cb.start[k] + cb.job[k].ctiles * cb.job[k].splits;
            }
            const dim3 grid((unsigned)cb.start[cb.njobs]);
            if (bin == 0) {
                if (ptv) colreduce_bf16<1, 2, true><<<grid, 256, 0, stream>>>(T, cb);
                else colreduce_bf16<1, 2, false><<<grid, 256, 0, stream>>>(T, cb);
            } else if (bin == 1) {
                if (ptv) colreduce_bf16<2, 1, true><<<grid, 256, 0, stream>>>(T, cb);
                else colreduce_bf16<2, 1, false><<<grid, 256, 0, stream>>>(T, cb);
            } else if (bin == 2) {
                if (ptv) colreduce_bf16<3, 1, true><<<grid, 256, 0, stream>>>(T, cb);
                else colreduce_bf16<3, 1, false><<<grid, 256, 0, stream>>>(T, cb);
            } else {
                if (ptv) colreduce_bf16<4, 1, true><<<grid, 256, 0, stream>>>(T, cb);
                else colreduce_bf16<4, 1, false><<<grid, 256, 0, stream>>>(T, cb);
            }
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        nb[bin] = 0;
        return hipSuccess;
    };
    for (int i = 0; i < n; ++i) {
        const ColJob& J = jobs[i];
        if (!J.X) continue;
        const int64_t stride = (int64_t)colreduce_rows(J.r) * J.C;
        for (int g = 0; g * GS < J.r; ++g) {
            const int rs = J.r - GS * g < GS ? J.r - GS * g : GS;
            const int bin = rs <= 16 ? 0 : rs <= 32 ? 1 : rs <= 48 ? 2 : 3;
            if (nb[bin] == CAP) {
                const hipError_t e = flush(bin);
                if (e != hipSuccess) return e;
            }
            bins[bin][nb[bin]++] = ColJobDev{J.X, J.C, J.Pt + (int64_t)GS * g * T, rs,
                                             round_up((T + J.splits - 1) / J.splits, 32),
                                             J.partial + (int64_t)GS * g * J.C, stride, (int)((J.C + 127) / 128),
                                             J.splits};
        }
    }
    for (int bin = 0; bin < 4; ++bin) {
        const hipError_t e = flush(bin);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Splits of a colsplit job: about one round of 256 workgroups over the
// job's 512-column tiles (c5: 37 tiles x 6 splits for 18944 columns, 7 x 36
// for 3584, which measured fastest among 1-3 rounds), each split at least
// 256 tokens.
int colsplit_splits(int64_t T, int64_t C) {
    const int64_t ctiles = (C + 511) / 512;
    int64_t s = 256 / ctiles;
    const int64_t max_s = T / 256;
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    return (int)s;
}

hipError_t launch_colsplit_bf16(int64_t T, const ColsplitJob* jobs, int n, hipStream_t stream) {
    // Ranks in groups of up to 64 (four 16-row MFMA tiles of accumulators),
    // each group one pass over X, binned by its rank tiles; one launch per
    // kColJobs groups of a bin, a full bin launched before more are queued.
    if (T % 8 != 0) return hipErrorInvalidValue;
    constexpr int GS = 64, CAP = 8 * kColJobs;
    ColsplitJobDev bins[4][CAP];
    int nb[4] = {0, 0, 0, 0};
    auto flush = [&](int bin) -> hipError_t {
        for (int first = 0; first < nb[bin]; first += kColJobs) {
            ColsplitBatch cb{};
            cb.njobs = std::min(kColJobs, nb[bin] - first);
            for (int k = 0; k < cb.njobs; ++k) {
                cb.job[k] = bins[bin][first + k];
                cb.start[k + 1] = cb.start[k] + cb.job[k].ctiles * cb.job[k].splits;
            }
            const dim3 grid((unsigned)cb.start[cb.njobs]);
            switch (bin) {
                case 0: colsplit_bf16<1><<<grid, 256, 0, stream>>>(T, cb); break;
                case 1: colsplit_bf16<2><<<grid, 256, 0, stream>>>(T, cb); break;
                case 2: colsplit_bf16<3><<<grid, 256, 0, stream>>>(T, cb); break;
                default: colsplit_bf16<4><<<grid, 256, 0, stream>>>(T, cb); break;
            }
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        nb[bin] = 0;
        return hipSuccess;
    };
    for (int i = 0; i < n; ++i) {
        const ColsplitJob& J = jobs[i];
        if (!J.X) continue;
        if (J.splits < 1 || J.C % 8 != 0 || J.C >= ((int64_t)1 << 22)) return hipErrorInvalidValue;
        const int64_t stride = (int64_t)colreduce_rows(J.r) * J.C;
        for (int g = 0; g * GS < J.r; ++g) {
            const int rs = J.r - GS * g < GS ? J.r - GS * g : GS;
            const int bin = rs <= 16 ? 0 : rs <= 32 ? 1 : rs <= 48 ? 2 : 3;
            if (nb[bin] == CAP) {
                const hipError_t e = flush(bin);
                if (e != hipSuccess) return e;
            }
            bins[bin][nb[bin]++] = ColsplitJobDev{J.X, J.C, J.P_hi + (int64_t)GS * g * T, J.P_lo + (int64_t)GS * g * T,
                                                  rs, round_up((T + J.splits - 1) / J.splits, 32),
                                                  J.partial + (int64_t)GS * g * J.C, stride, (int)((J.C + 511) / 512),
                                                  J.splits};
        }
    }
    for (int bin = 0; bin < 4; ++bin) {
        const hipError_t e = flush(bin);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_split_sum(const SumJob* jobs, int n, hipStream_t stream) {
    // one launch per kSumJobs jobs with an output
    int first = 0, valid = 0;
    for (int i = 0; i < n; ++i) {
        if (!jobs[i].out) continue;
        if (++valid > kSumJobs) {
            const hipError_t e = launch_split_sum(jobs + first, i - first, stream);
            if (e != hipSuccess) return e;
            first = i;
            valid = 1;
        }
    }
    n -= first;
    jobs += first;
    SumBatch sb{};
    int k = 0;
    bool vec4 = true;
    for (int i = 0; i < n; ++i) {
        if (!jobs[i].out) continue;
        const SumJob& J = jobs[i];
        // a split's partial is one buffer resource with 32-bit offsets
        vec4 = vec4 && J.C % 4 == 0 && J.part_stride % 4 == 0 && J.part_stride * 4 < ((int64_t)1 << 31) &&
               reinterpret_cast<uintptr_t>(J.partial) % 16 == 0 &&
               (J.transpose_out || reinterpret_cast<uintptr_t>(J.out) % 16 == 0);
        sb.job[k++] = J;
    }
    sb.njobs = k;
    for (int i = 0; i < k; ++i) sb.start[i + 1] = sb.start[i] + (int64_t)sb.job[i].r * sb.job[i].C / (vec4 ? 4 : 1);
    const int64_t total = sb.start[k];
    if (total == 0) return hipSuccess;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 4096) blocks = 4096;
    if (vec4) split_sum<true><<<dim3((unsigned)blocks), 256, 0, stream>>>(sb);
    else split_sum<false><<<dim3((unsigned)blocks), 256, 0, stream>>>(sb);
    return hipGetLastError();
}

// Splits of the fused dY pass: at most 256 workgroups per job over its
// column groups and splits, each split at least eight 32-row steps, and no
// split's rows of dY spanning 2^31 bytes (32-bit buffer offsets). The
// kernel holds two workgroups per CU at r <= 16 (one at r <= 32), so the
// grouped gate / up launch (two jobs) runs in one round of the 256 CUs.
// The earlier ~512 per job (c4: 2 x 18 groups x 29 splits = 1044
// workgroups) ran two full rounds and a third of 20 workgroups; the
// one-round split measured 0.559 -> 0.541 ms of low-rank time per c4 step
// (~256 per job; ~512 per job exactly filling two rounds: 0.549).
int dy_splits(int64_t T, int64_t N) {
    const int64_t groups = dy_groups(N);
    int64_t s = 256 / groups;
    const int64_t max_s = (T + 255) / 256;
    if (s > max_s) s = max_s;
    if (s < 1) s = 1;
    const int64_t rows_cap = (int64_t)0x7fffffff / (2 * N) / 32 * 32;
    const int64_t min_s = rows_cap > 0 ? (T + rows_cap - 1) / rows_cap : T;
    if (s < min_s) s = min_s;
    return (int)s;
}

hipError_t launch_dy_pass(int64_t T, int r, const DyJob* jobs, int n, hipStream_t stream) {
    DyBatch db{};
    db.r = r;
    int k = 0;
    for (int i = 0; i < n; ++i) {
        const DyJob& J = jobs[i];
        if (!J.dY || (!J.partB && !J.gpart)) continue;
        if (k == kMaxProj) return hipErrorInvalidValue;
        const int splits = dy_splits(T, J.N);
        DyJobDev d{J.dY, J.N, J.B, J.Pt, J.partB, J.gpart, round_up((T + splits - 1) / splits, 32),
                   (int64_t)colreduce_rows(r) * J.N, dy_groups(J.N)};
        // the chunk is rounded to whole steps: splits past T write zero partials
        db.job[k] = d;
        db.start[k + 1] = db.start[k] + d.groups * splits;
        ++k;
    }
    db.njobs = k;
    if (k == 0) return hipSuccess;
    const dim3 grid((unsigned)db.start[k]);
    const bool ptv = (T & 3) == 0;
    if (r <= 16) {
        if (ptv) dy_pass_bf16<1, true><<<grid, 256, 0, stream>>>(T, db);
        else dy_pass_bf16<1, false><<<grid, 256, 0, stream>>>(T, db);
    } else {
        if (ptv) dy_pass_bf16<2, true><<<grid, 256, 0, stream>>>(T, db);
        else dy_pass_bf16<2, false><<<grid, 256, 0, stream>>>(T, db);
    }
    return hipGetLastError();
}

hipError_t launch_dy_finish(int64_t T, int r, float scale, float keep, int rext, int ext_ld, float ext_scale,
                            const DyFinishJob* jobs, int n, const PrepJob* preps, int npreps, hipStream_t stream) {
    if (r < 1 || r > kFinishMaxRank) return hipErrorInvalidValue;
    DyFinishBatch fb{};
    fb.r = r; fb.rext = rext; fb.ext_ld = ext_ld; fb.scale = scale; fb.keep = keep; fb.ext_scale = ext_scale;
    fb.blocks_per_job = (int)((T + 63) / 64);
    for (int i = 0; i < n; ++i) {
        if (!(jobs[i].gpart && (jobs[i].gd_t || jobs[i].gd_ext || jobs[i].gd_hi))) continue;
        if (fb.njobs == kMaxProj) return hipErrorInvalidValue;
        fb.job[fb.njobs++] = jobs[i];
    }
    bool vec8 = true;
    for (int i = 0; i < npreps; ++i) {
        if (!preps[i].hi) continue;
        if (fb.npreps == kPrepJobs) return hipErrorInvalidValue;
        PrepJob p = preps[i];
        if (p.ld_out == 0) p.ld_out = p.cols_out;
        vec8 = vec8 && prep_vec8(p);
        fb.prep[fb.npreps++] = p;
    }
    fb.prep8 = vec8 ? 1 : 0;
    for (int i = 0; i < fb.npreps; ++i)
        fb.prep_start[i + 1] = fb.prep_start[i] + fb.prep[i].rows_out * fb.prep[i].cols_out / (vec8 ? 8 : 1);
    const int64_t prep_n = fb.prep_start[fb.npreps];
    const int64_t prep_blocks = prep_n > 0 ? std::min<int64_t>((prep_n + 255) / 256, 1024) : 0;
    const int64_t blocks = (int64_t)fb.njobs * fb.blocks_per_job + prep_blocks;
    if (blocks == 0) return hipSuccess;
    for (int i = 0; i < fb.njobs; ++i)  // one split of a job is one buffer resource
        if (T * (fb.job[i].ld > 0 ? fb.job[i].ld : r) * 4 >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    bool vec = true;
    for (int i = 0; i < fb.njobs; ++i) {
        const int64_t ld = fb.job[i].ld > 0 ? fb.job[i].ld : r;
        vec = vec && ld % 4 == 0 && reinterpret_cast<uintptr_t>(fb.job[i].gpart) % 16 == 0;
    }
    if (vec) dy_finish<true><<<dim3((unsigned)blocks), 256, 0, stream>>>(T, fb);
    else dy_finish<false><<<dim3((unsigned)blocks), 256, 0, stream>>>(T, fb);
    return hipGetLastError();
}

// Splits of a rowsplit job of C columns: the smallest count whose row blocks
// x splits fill whole rounds of 256 CUs (or three rounds), with at least
// kRowsplitMinCols columns per split (each split adds a T x 16 ceil(r / 16)
// partial that is written and read back). The count depends on T and C
// only, so every job over the same x splits alike. Measured on the c5 shapes
// (T = 16384: 64 row blocks, 4 splits): one 64-rank pass of 3584 or 18944
// columns ran fastest at 4 splits, and the three q / k / v passes together
// as well (2 and 3 splits were slower, 8 no faster).
int rowsplit_splits(int64_t T, int64_t C) {
    const int64_t rb = (T + kRowsplitRows - 1) / kRowsplitRows;
    const int64_t max_s = C / kRowsplitMinCols > 1 ? C / kRowsplitMinCols : 1;
    int64_t s = 1;
    while (s < max_s) {
        const int64_t w = rb * s;
        if (w >= 768 || (w >= 256 && w % 256 == 0)) break;
        ++s;
    }
    return (int)s;
}

namespace {
template <int RC>
hipError_t rowsplit_go(const RowsplitBatch& b, bool pf32, int64_t tiles, hipStream_t stream) {
    // bf16 parameter: 64-column stages (144 KB of LDS, one workgroup per
    // CU); fp32 parameter: 32-column stages (72 KB, two per CU), which
    // measured faster for each
    const dim3 grid((unsigned)tiles);
    if (pf32) rowsplit_bf16<4, RC, 32, true><<<grid, 256, 0, stream>>>(b);
    else rowsplit_bf16<4, RC, 64, false><<<grid, 256, 0, stream>>>(b);
    return hipGetLastError();
}
}  // namespace

hipError_t launch_rowsplit(int64_t T, int r, const RowsplitJob* jobs, int n, hipStream_t stream) {
    if (n < 1 || n > kMaxProj || r < 1 || r > kRowsplitRanks) return hipErrorInvalidValue;
    const bool pf32 = jobs[0].P_f32 != nullptr;
    const int BK = pf32 ? 32 : 64;
    RowsplitBatch b{};
    b.njobs = n;
    b.T = T;
    b.interleave = 1;
    const int64_t rblocks = (T + kRowsplitRows - 1) / kRowsplitRows;
    int64_t tiles = 0;
    for (int i = 0; i < n; ++i) {
        const RowsplitJob& s = jobs[i];
        // x rows of a workgroup are one buffer resource with 32-bit offsets
        if ((s.P_f32 != nullptr) != pf32 || s.splits < 1 || s.C < 1 || s.C % 8 != 0 || s.C >= ((int64_t)1 << 22))
            return hipErrorInvalidValue;
        RowsplitJobDev& d = b.job[i];
        d.X = s.X; d.C = s.C;
        d.P0 = pf32 ? (const void*)s.P_f32 : (const void*)s.P_hi;
        d.P1 = s.P_lo;
        d.pbytes = (int64_t)s.prows * s.C * (pf32 ? 4 : 2);
        d.part = s.part;
        d.splits = s.splits;
        d.cps = ((s.C + s.splits - 1) / s.splits + BK - 1) / BK * BK;
        b.start[i] = tiles;
        tiles += rblocks * s.splits;
        if (s.X != jobs[0].X || s.C != jobs[0].C || s.splits != jobs[0].splits) b.interleave = 0;
    }
    b.start[n] = tiles;
    if (tiles == 0) return hipSuccess;
    switch ((r + 15) / 16) {
        case 1: return rowsplit_go<1>(b, pf32, tiles, stream);
        case 2: return rowsplit_go<2>(b, pf32, tiles, stream);
        case 3: return rowsplit_go<3>(b, pf32, tiles, stream);
        default: return rowsplit_go<4>(b, pf32, tiles, stream);
    }
}

hipError_t launch_rowproj_f32(const float* X, int64_t T, int64_t C, const float* P, bool transpose_p,
                              int r, float scale, const uint8_t* mask, float keep, float* out_t,
                              float* out_ext, float ext_scale, hipStream_t stream) {
    if (T >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    rowproj_f32<<<dim3((unsigned)T), 256, 0, stream>>>(X, T, C, P, transpose_p ? 1 : 0, r, scale, mask, keep, out_t,
                                                       out_ext, ext_scale);
    return hipGetLastError();
}

hipError_t launch_colreduce_f32(const ColF32Call* calls, int n, int64_t T, int r, hipStream_t stream) {
    if (n < 1 || n > 2) return hipErrorInvalidValue;
    ColF32Job j[2]{};
    int64_t nblk[2] = {0, 0};
    for (int i = 0; i < n; ++i) {
        const ColF32Call& c = calls[i];
        j[i] = ColF32Job{c.X, c.C, c.Pt, c.scale, c.transpose_out ? 1 : 0, c.out, (c.C + 15) / 16};
        nblk[i] = j[i].ctiles * ((r + 7) / 8);
    }
    if (nblk[0] + nblk[1] >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    if (nblk[0] + nblk[1] == 0) return hipSuccess;
    colreduce_f32<<<dim3((unsigned)(nblk[0] + nblk[1])), 256, 0, stream>>>(T, r, j[0], n > 1 ? j[1] : j[0], nblk[0]);
    return hipGetLastError();
}

}  // namespace mc
