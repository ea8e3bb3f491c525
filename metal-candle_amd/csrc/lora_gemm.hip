// GEMMs of the LoRA linear, gfx950.
//
// The frozen base projection of the reference is candle_nn::Linear,
// y = x.W^T (+ b) with W stored [out, in] (src/models/transformer.rs:189-192);
// the LoRA delta scale * Hd.B (src/training/lora.rs:336-339) is folded into
// the same GEMM as extra reduction columns:
//
//   forward   y  = [x | s*Hd] . [W | B^T]^T + b
//   backward  dX = [dY | Gd] . [W^T | A]^T      (W^T transposed once per call)
//
// so both are "NT" products C = A0.B0^T + A1.B1^T with every operand stored
// reduction-contiguous, and one kernel produces the fused result.
//
// bf16 kernel: a workgroup computes a BM x BN tile with (BM/WM) x (BN/WN)
// waves, each a WM x WN block of MFMA 32x32x16 bf16 tiles with fp32
// accumulators. The tiles are chosen per shape (choose_gemm_plan): 256 x 256,
// 256 x 192 or 256 x 128 with 8 waves and one workgroup per CU for the
// large layer products, 128 x 128 with 4 waves where there are too few large
// tiles to fill the 256 CUs; or 256 x 256 tiles over most columns and a
// narrower shape over the rest in one launch (gemm_bf16_split), so that the
// widest tile fills whole rounds of CUs.
//  - Operands go straight from HBM/L2 into LDS with buffer_load ... lds
//    (no VGPR staging, no ds_write), bounds handled by the buffer descriptor
//    (out-of-range chunks load as zeros).
//  - LDS rows are XOR-swizzled 16-byte chunks, so both the loads and the
//    MFMA fragment reads are bank-conflict free without padding.
//  - k-steps of 64 through two LDS stages (the loads of k-step k+1 run
//    while k-step k is multiplied) or a ring of three; MFMA fragments are
//    double-buffered across the substeps.
//  - Workgroup ids are remapped per XCD and grouped by 4 tile-rows for L2
//    reuse (tile_of).
//  - The epilogue goes through a per-wave LDS patch so C is written as whole
//    128-byte lines with non-temporal 16-byte stores, the bias added on the way.
#include <atomic>
#include <type_traits>
#include <cmath>

#include "common.hpp"
#include "lora_kernels.hpp"

namespace mc {
namespace {


// One output block: C[M][N] = sum over the reduction segments of
// A_s . B_s^T (+ bias), the segments' k-tiles taken in segment order.
struct GemmArgs {
    int64_t M, N;
    GemmSeg seg[kGemmMaxSeg];
    int nseg;
    const uint16_t* bias;
    uint16_t* c;
    int64_t ldc;
    int tiles_m, tiles_n, group_m;
};

// Logical tile of a workgroup. Workgroups are dispatched round-robin over the
// 8 XCDs (id % 8), each with its own L2: ids are remapped so every XCD owns a
// contiguous range of logical tiles, and logical tiles run down groups of
// group_m tile-rows before moving along N, so the workgroups resident on one
// XCD share A row-panels and B column-panels in that XCD's L2.
__device__ __forceinline__ void tile_of(int pid, int tiles_m, int tiles_n, int group_m, int& tm, int& tn) {
    const int total = tiles_m * tiles_n;
    const int per = total / 8, rem = total % 8;
    const int x = pid % 8, j = pid / 8;
    const int l = (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + j;
    const int in_group = group_m * tiles_n;
    const int g = l / in_group;
    const int first_m = g * group_m;
    const int gm = min(tiles_m - first_m, group_m);
    const int r = l - g * in_group;
    tm = first_m + r % gm;
    tn = r / gm;
}

// dma_tile for a full k-tile of rows with a fixed row stride: each lane's
// VGPR offset (row * ld + swizzled chunk, in bytes) is precomputed once per
// kernel (tile_offsets) and the k-tile's start kb * 2 goes in soffset, so a
// load costs no vector arithmetic. Rows past the resource's range still load
// zeros (their VGPR offset alone is past num_records).
template <int ROWS, int NT, int BK>
struct TileOffsets {
    static constexpr int CPR = BK / 8, RPI = 64 / CPR;
    static constexpr int PER_WAVE = ROWS / RPI / (NT / 64);
    uint32_t v[PER_WAVE];
    __device__ __forceinline__ void init(uint32_t ld, int tid) {
        const int wave = tid >> 6, lane = tid & 63;
#pragma unroll
        for (int j = 0; j < PER_WAVE; ++j) {
            const int row = (wave * PER_WAVE + j) * RPI + lane / CPR;
            v[j] = ((uint32_t)row * ld + 8u * (uint32_t)swz<BK>(row, lane % CPR)) * 2u;
        }
    }
};
template <int ROWS, int NT, int BK, int PARTS>
__device__ __forceinline__ void dma_tile_full(i32x4 r, uint32_t lds_wave, const TileOffsets<ROWS, NT, BK>& o,
                                              uint32_t kb, int part) {
    constexpr int PER_WAVE = TileOffsets<ROWS, NT, BK>::PER_WAVE;
#pragma unroll
    for (int j = 0; j < PER_WAVE; ++j) {
        if (j % PARTS != part) continue;
        dma16_s(r, lds_wave + (uint32_t)j * 1024u, o.v[j], kb * 2u);
    }
}

template <int N>
__device__ __forceinline__ void wait_tiles(int remaining) {
    // vmcnt may keep `remaining` later tiles (N loads each) in flight
    switch (remaining) {
        case 0: wait_vmcnt<0>(); break;
        case 1: wait_vmcnt<N>(); break;
        case 2: wait_vmcnt<2 * N>(); break;
        default: wait_vmcnt<3 * N>(); break;
    }
}

// Epilogue shared by the GEMM kernels (the stage buffers are free once the
// main loop has finished and a barrier has passed). Pairs of 32 x 32
// accumulator blocks, a 32 x 64 block whose rows are 128 bytes of bf16 (whole
// cache lines), go through a per-wave 8 KB LDS patch: accumulator q of lane l
// is row 8 (q / 4) + 4 (l / 32) + q % 4, column l % 32 of its block; the patch
// is read back as lane l -> row 8 s + l / 8 (s < 4), columns 8 (l % 8) .. +7,
// so 8 lanes store one whole line with one 16-byte store each, with the bias
// added. An odd last block (64 x 96 wave tiles) uses half the lanes. Rows
// past M and columns past N are dropped by the buffer bounds / column check.
//
// The stores are non-temporal (nt): C is not read again by this kernel, and
// whole-line streaming stores leave no dirty lines in L2 for the next kernels
// to write back. Measured on the c4 step against the previous epilogue
// (32-byte pieces of rows per store, write-back policy): GEMM 2.80 -> 2.71 ms,
// the low-rank kernels that follow the GEMMs 0.65 -> 0.61 ms, the step
// 4.02 -> 3.88 ms; the same whole-line stores without nt gave 2.75 / 3.96 ms.
// (nt on the 32-byte pieces had been much slower: each piece went to memory
// as a partial line.)
template <int TM, int TN, int WM, int WN>
__device__ __forceinline__ void store_c(const f32x16 (&acc)[TM][TN], uint16_t* smem, const GemmArgs& g, int64_t m0,
                                        int64_t n0, int wm, int wn) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int frag_row = lane & 31;
    float* patch = reinterpret_cast<float*>(smem) + wave * 2048;  // [32][64] fp32
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(g.c + m0 * g.ldc, (g.M - m0) * g.ldc * 2);
    const __amdgpu_buffer_rsrc_t rbias = make_rsrc(g.bias, g.bias ? g.N * 2 : 0);
    const int lrow = lane >> 3, lcol = (lane & 7) * 8;
    constexpr int NP = (TN + 1) / 2;
    i32x4 bq[NP];
#pragma unroll
    for (int jp = 0; jp < NP; ++jp) {
        const int64_t n = n0 + wn * WN + jp * 64 + lcol;
        const bool ok = n < g.N && (2 * jp + 1 < TN || lcol < 32);
        bq[jp] = __builtin_amdgcn_raw_buffer_load_b128(rbias, (int)(ok ? n * 2 : kOOB), 0, 0);
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int jp = 0; jp < NP; ++jp) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int j = 2 * jp + h;
                if (j >= TN) break;
#pragma unroll
                for (int q = 0; q < 16; ++q)
                    patch[(8 * (q >> 2) + 4 * (lane >> 5) + (q & 3)) * 64 + 32 * h + frag_row] = acc[i][j][q];
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): patch written (same wave)
            const bool half = 2 * jp + 1 >= TN;   // odd last block: columns 0..31 only
            const int64_t n = n0 + wn * WN + jp * 64 + lcol;
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                const int prow = 8 * st + lrow;
                const float4 a = *reinterpret_cast<const float4*>(&patch[prow * 64 + lcol]);
                const float4 b = *reinterpret_cast<const float4*>(&patch[prow * 64 + lcol + 4]);
                const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t bb = (uint32_t)bq[jp][e];
                    w[e] = pack_bf16x2(v[2 * e] + bf16_lo(bb), v[2 * e + 1] + bf16_hi(bb));
                }
                const i32x4 out = {(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
                const uint32_t row = (uint32_t)(wm * WM + i * 32 + prow);
                const bool ok = n < g.N && (!half || lcol < 32);
                const uint32_t off = ok ? (row * (uint32_t)g.ldc + (uint32_t)n) * 2u : kOOB;
                __builtin_amdgcn_raw_buffer_store_b128(out, rc, (int)off, 0, kStoreNT);
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // patch reads done before it is rewritten
        }
}

// LDS elements (bf16) of one tile configuration's stage buffers.
template <int BM, int BN, int BK, int STAGES>
constexpr int kTileSmem = STAGES * (BM + BN) * BK;

// One BM x BN output tile (tm, tn) of g: the whole k loop and the epilogue,
// with the stage buffers at smem (kTileSmem elements, 1 KB aligned).
// MULTI: more than two reduction segments (the cursor form below).
template <int BM, int BN, int WM, int WN, int BK, int STAGES, bool MULTI>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, int tm, int tn, uint16_t* smem) {
    constexpr int NWN = BN / WN;
    constexpr int NT = (BM / WM) * NWN * 64;
    constexpr int TM = WM / 32, TN = WN / 32;
    constexpr int KS = BK / 16;                          // MFMA k-substeps per tile
    constexpr int CPR = BK / 8;                          // 16-byte chunks per LDS row
    constexpr int STAGE = (BM + BN) * BK;                // bf16 elements per stage (A tile, then B tile)
    constexpr int LOADS = (BM + BN) / (512 / BK) / (NT / 64);  // loads per wave per tile
    static_assert(STAGES >= 2 && STAGES <= 5 && (STAGES - 2) * LOADS < 64 && KS % 2 == 0, "pipeline depth");
    static_assert(NT / 64 * 8192 <= STAGES * STAGE * 2, "epilogue staging fits in the stage buffers");

    const uint32_t smem_byte = (uint32_t)reinterpret_cast<uintptr_t>(smem);

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / NWN, wn = wave % NWN;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    // Tile count and the last tile's substeps with data (the last tile
    // belongs to the last non-empty segment), read from the segment table
    // here, before any LDS traffic: a scalar load's wait also waits for LDS.
    int nk = 0;
    int64_t klast = 0;
    for (int s = 0; s < (MULTI ? g.nseg : 2); ++s) {
        const int64_t ks = g.seg[s].k;
        nk += (int)((ks + BK - 1) / BK);
        if (ks > 0) klast = ks - (ks - 1) / BK * BK;
    }
    const int nks_last = klast >= BK ? KS : (int)((klast + 15) / 16);

    // Loads of tile kt into a stage, in KS parts. With two stages and 8
    // waves, only waves 0-3 (one per SIMD) issue them: a wave waits while its
    // DMA instructions issue, and the SIMD's other wave keeps the MFMA pipe
    // busy meanwhile (measured +2-5% on the 2-stage tiles; the 3-stage ring,
    // whose loads are spread over every substep, was 3% slower this way).
    constexpr int DMA_NT = (STAGES == 2 && NT == 512) ? 256 : NT;
    // Two segments (every single projection: the base product, then the
    // rank-r columns) are set up once at the start: buffer resources over the
    // workgroup's rows of A and B (rows past M / N fall outside num_records
    // and load as zero) and the lanes' DMA offsets of segment 0. More
    // segments (a group's dX) go through a cursor that is moved once per tile:
    // at a segment's first tile it sets up that segment's resources and
    // offsets. Full k-tiles of the current (or first) segment load through the
    // precomputed lane offsets; a ragged tile, and in the two-segment form the
    // second segment, take the general path, which zeroes chunks at k >= the
    // segment's length.
    TileOffsets<BM, DMA_NT, BK> offa;
    TileOffsets<BN, DMA_NT, BK> offb;
    const uint32_t lds_wave_a = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)((uint32_t)(tid >> 6) * (uint32_t)TileOffsets<BM, DMA_NT, BK>::PER_WAVE * 1024u));
    const uint32_t lds_wave_b = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)((uint32_t)(tid >> 6) * (uint32_t)TileOffsets<BN, DMA_NT, BK>::PER_WAVE * 1024u));
    // two-segment form: every scalar of the two segments is read into a value
    // here (selecting between fields of the argument struct in the loop
    // compiles to a scalar load from a selected address, and its lgkmcnt wait
    // stalls on the fragment reads in flight)
    const uint32_t k0 = (uint32_t)g.seg[0].k, k1 = (uint32_t)g.seg[1].k;
    const uint32_t lda0 = (uint32_t)g.seg[0].lda, lda1 = (uint32_t)g.seg[1].lda;
    const uint32_t ldb0 = (uint32_t)g.seg[0].ldb, ldb1 = (uint32_t)g.seg[1].ldb;
    const int nk0 = MULTI ? 0 : (int)((k0 + BK - 1) / BK);
    const int nfull0 = MULTI ? 0 : (int)(k0 / BK);
    i32x4 ra0 = {0, 0, 0, 0}, rb0 = {0, 0, 0, 0}, ra1 = {0, 0, 0, 0}, rb1 = {0, 0, 0, 0};
    if constexpr (!MULTI) {
        ra0 = rsrc_words(g.seg[0].a + m0 * lda0, (g.M - m0) * lda0 * 2);
        rb0 = rsrc_words(g.seg[0].b + n0 * ldb0, (g.N - n0) * ldb0 * 2);
        ra1 = rsrc_words(g.seg[1].a + m0 * lda1, (g.M - m0) * lda1 * 2);
        rb1 = rsrc_words(g.seg[1].b + n0 * ldb1, (g.N - n0) * ldb1 * 2);
        offa.init(lda0, tid);
        offb.init(ldb0, tid);
    }
    // cursor form
    int cur = -1, cur_begin = 0, cur_end = 0, cur_full = 0;
    uint32_t cur_lda = 0, cur_ldb = 0, cur_k = 0;
    i32x4 ra = {0, 0, 0, 0}, rb = {0, 0, 0, 0};
    // Moves the cursor to the segment of tile kt. It is called once per tile,
    // before the tile's first load part and at a point where no LDS reads are
    // in flight (right after a barrier or before the first tile): the scalar
    // loads of the segment table wait on lgkmcnt, the counter the fragment
    // reads also use.
    auto advance = [&](int kt) {
        if constexpr (MULTI) {
            while (kt >= cur_end) {  // wave-uniform: the first tile of the next non-empty segment
                ++cur;
                const GemmSeg& sg = g.seg[cur];
                cur_begin = cur_end;
                cur_end = cur_begin + (int)((sg.k + BK - 1) / BK);
                cur_full = (int)(sg.k / BK);
                cur_lda = (uint32_t)sg.lda;
                cur_ldb = (uint32_t)sg.ldb;
                cur_k = (uint32_t)sg.k;
                if (cur_end > cur_begin) {
                    ra = rsrc_words(sg.a + m0 * sg.lda, (g.M - m0) * sg.lda * 2);
                    rb = rsrc_words(sg.b + n0 * sg.ldb, (g.N - n0) * sg.ldb * 2);
                    offa.init(cur_lda, tid);
                    offb.init(cur_ldb, tid);
                }
            }
        }
    };
    auto issue = [&](int kt, int stage, int part) {
        const uint32_t base = smem_byte + (uint32_t)(stage * STAGE * 2);
        if (!(DMA_NT == NT || tid < DMA_NT)) return;  // wave-uniform
        if constexpr (MULTI) {
            const int local = kt - cur_begin;
            const uint32_t kb = (uint32_t)local * BK;
            if (local < cur_full) {
                dma_tile_full<BM, DMA_NT, BK, KS>(ra, base + lds_wave_a, offa, kb, part);
                dma_tile_full<BN, DMA_NT, BK, KS>(rb, base + BM * BK * 2 + lds_wave_b, offb, kb, part);
            } else {
                dma_tile<BM, DMA_NT, BK, KS>(ra, base, cur_lda, kb, cur_k, tid, part);
                dma_tile<BN, DMA_NT, BK, KS>(rb, base + BM * BK * 2, cur_ldb, kb, cur_k, tid, part);
            }
        } else {
            const bool second = kt >= nk0;
            const uint32_t kb = (uint32_t)(second ? kt - nk0 : kt) * BK;
            const uint32_t ks = second ? k1 : k0;
            if (kt < nfull0) {
                dma_tile_full<BM, DMA_NT, BK, KS>(ra0, base + lds_wave_a, offa, kb, part);
                dma_tile_full<BN, DMA_NT, BK, KS>(rb0, base + BM * BK * 2 + lds_wave_b, offb, kb, part);
            } else {
                dma_tile<BM, DMA_NT, BK, KS>(second ? ra1 : ra0, base, second ? lda1 : lda0, kb, ks, tid, part);
                dma_tile<BN, DMA_NT, BK, KS>(second ? rb1 : rb0, base + BM * BK * 2, second ? ldb1 : ldb0, kb, ks,
                                             tid, part);
            }
        }
    };

    f32x16 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[i][j][q] = 0.f;

    // MFMA 32x32x16 fragments: lane l supplies row l % 32 and k-chunk
    // 2 ks + l / 32 of the tile. The fragment rows of a lane differ by
    // multiples of 32, so the swizzle term is the same for all of them: the
    // slot is (2 ks + l / 32) ^ sw with a per-lane sw, and the row offsets are
    // immediates of the ds_read.
    const int frag_row = lane & 31;
    const int sw = (frag_row / (128 / BK)) % CPR;
    const int a_row0 = (wm * WM + frag_row) * BK;
    const int b_row0 = BM * BK + (wn * WN + frag_row) * BK;
    bf16x8 fa[2][TM], fb[2][TN];
    auto load_frags = [&](const uint16_t* st, int ks, int slot) {
        const int col = 8 * ((2 * ks + (lane >> 5)) ^ sw);
#pragma unroll
        for (int t = 0; t < TM; ++t)
            fa[slot][t] = *reinterpret_cast<const bf16x8*>(&st[a_row0 + t * 32 * BK + col]);
#pragma unroll
        for (int t = 0; t < TN; ++t)
            fb[slot][t] = *reinterpret_cast<const bf16x8*>(&st[b_row0 + t * 32 * BK + col]);
    };

    auto mfma_substep = [&](int cur) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[cur][i], fb[cur][j], acc[i][j], 0, 0, 0);
    };
    // The last k-tile, after which nothing is issued: its loads were the last
    // ones, so it waits for all of them. Only its substeps that hold data are
    // multiplied: with the rank-r segment last, a rank of 16 fills one of the
    // four (the rest are range-checked zeros in both operands, whose products
    // add exactly nothing).
    auto last_tile = [&](int kt) {
        wait_vmcnt<0>();
        __syncthreads();
        const uint16_t* st = smem + (kt % STAGES) * STAGE;
        const int nks = nks_last;
        load_frags(st, 0, 0);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
            if (ks >= nks) break;
            const int cur = ks & 1;
            if (ks + 1 < KS && ks + 1 < nks) load_frags(st, ks + 1, cur ^ 1);
            mfma_substep(cur);
        }
    };
    auto issue_all = [&](int t) {
        advance(t);
#pragma unroll
        for (int p = 0; p < KS; ++p) issue(t, t % STAGES, p);
    };
    if constexpr (STAGES == 2) {
        // Two stages: each tile starts with every wave waiting for its own
        // loads of the tile and a barrier (all loads visible, every wave done
        // with the previous tile); the next tile's loads then go out into the
        // other stage, front-loaded so that they have most of the tile to
        // land: half of them before the first MFMA substep, a quarter after
        // each of the first two substeps (issuing a part after every substep
        // left the last part only one substep to land before the wait).
        static_assert(KS == 4, "the two-stage schedule assumes four substeps per tile");
        if (nk > 0) issue_all(0);
        for (int kt = 0; kt + 1 < nk; ++kt) {
            wait_vmcnt<0>();
            __syncthreads();
            const uint16_t* st = smem + (kt & 1) * STAGE;
            advance(kt + 1);
            issue(kt + 1, (kt + 1) & 1, 0);
            issue(kt + 1, (kt + 1) & 1, 1);
            load_frags(st, 0, 0);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int cur = ks & 1;
                if (ks + 1 < KS) load_frags(st, ks + 1, cur ^ 1);
                mfma_substep(cur);
                if (ks < 2) issue(kt + 1, (kt + 1) & 1, ks + 2);
            }
        }
        if (nk > 0) last_tile(nk - 1);
    } else {
        // Ring of STAGES stages: tiles 0 .. STAGES-2 are issued up front;
        // tile kt waits for its own loads (later tiles stay in flight), a
        // barrier publishes it to every wave and frees stage (kt-1) % STAGES
        // (every wave has finished tile kt-1), into which the loads of tile
        // kt+STAGES-1 go, one part after each MFMA substep.
#pragma unroll
        for (int s0 = 0; s0 < STAGES - 1; ++s0)
            if (s0 < nk) issue_all(s0);
        for (int kt = 0; kt + 1 < nk; ++kt) {
            const int ahead = nk - 1 - kt;  // tiles after kt already issued, at most STAGES-2
            wait_tiles<LOADS>(ahead < STAGES - 2 ? ahead : STAGES - 2);
            __syncthreads();
            const uint16_t* st = smem + (kt % STAGES) * STAGE;
            const int nt = kt + STAGES - 1;
            if (nt < nk) advance(nt);
            load_frags(st, 0, 0);
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
                const int cur = ks & 1;
                if (ks + 1 < KS) load_frags(st, ks + 1, cur ^ 1);
                mfma_substep(cur);
                if (nt < nk) issue(nt, nt % STAGES, ks);
            }
        }
        if (nk > 0) last_tile(nk - 1);
    }

    __syncthreads();
    store_c<TM, TN, WM, WN>(acc, smem, g, m0, n0, wm, wn);
}

template <int BM, int BN, int WM, int WN, int BK, int STAGES, bool MULTI>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64, 1)
__attribute__((amdgpu_waves_per_eu(1, 2))) void gemm_bf16_kernel(GemmArgs g) {
    __shared__ __attribute__((aligned(1024))) uint16_t smem[kTileSmem<BM, BN, BK, STAGES>];
    int tm, tn;
    tile_of(blockIdx.x, g.tiles_m, g.tiles_n, g.group_m, tm, tn);
    gemm_tile<BM, BN, WM, WN, BK, STAGES, MULTI>(g, tm, tn, smem);
}

// Two tile shapes in one launch: workgroups [0, wgs1) compute g1's tiles
// (columns [0, n1) of the output), the rest g2's tiles (columns [n1, N)).
// Workgroups are dispatched in id order, so the second shape fills the CUs
// the first shape's last round leaves idle. Both shapes use 8 waves.
template <int BM1, int BN1, int WM1, int WN1, int S1, int BM2, int BN2, int WM2, int WN2, int S2, bool MULTI>
__global__ __launch_bounds__(512, 1) __attribute__((amdgpu_waves_per_eu(1, 2))) void gemm_bf16_split(GemmArgs g1,
                                                                                                     GemmArgs g2,
                                                                                                     int wgs1) {
    static_assert((BM1 / WM1) * (BN1 / WN1) == 8 && (BM2 / WM2) * (BN2 / WN2) == 8, "8 waves");
    constexpr int SM1 = kTileSmem<BM1, BN1, 64, S1>, SM2 = kTileSmem<BM2, BN2, 64, S2>;
    __shared__ __attribute__((aligned(1024))) uint16_t smem[SM1 > SM2 ? SM1 : SM2];
    int tm, tn;
    if ((int)blockIdx.x < wgs1) {
        tile_of(blockIdx.x, g1.tiles_m, g1.tiles_n, g1.group_m, tm, tn);
        gemm_tile<BM1, BN1, WM1, WN1, 64, S1, MULTI>(g1, tm, tn, smem);
    } else {
        tile_of((int)blockIdx.x - wgs1, g2.tiles_m, g2.tiles_n, g2.group_m, tm, tn);
        gemm_tile<BM2, BN2, WM2, WN2, 64, S2, MULTI>(g2, tm, tn, smem);
    }
}

// Output blocks that share the rows of their first A operand (projections of
// one input): up to kGemmMaxOut blocks, each with its own reduction segments,
// bias and C, as one grid of one tile shape. Tile columns run through the
// blocks in order (block o owns columns [col_start[o], col_start[o + 1]) of
// the grid); tile_of orders them as for one wide product, so a tile-row
// group walks the columns of every block.
struct GemmMulti {
    GemmArgs out[kGemmMaxOut];
    int nout;
    int col_start[kGemmMaxOut + 1];
    int tiles_m, tiles_n, group_m;
};

template <int BM, int BN, int WM, int WN, int BK, int STAGES>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64, 1)
__attribute__((amdgpu_waves_per_eu(1, 2))) void gemm_bf16_multi(GemmMulti m) {
    __shared__ __attribute__((aligned(1024))) uint16_t smem[kTileSmem<BM, BN, BK, STAGES>];
    int tm, tn;
    tile_of(blockIdx.x, m.tiles_m, m.tiles_n, m.group_m, tm, tn);
    int o = 0;
    while (o + 1 < m.nout && tn >= m.col_start[o + 1]) ++o;  // wave-uniform
    gemm_tile<BM, BN, WM, WN, BK, STAGES, false>(m.out[o], tm, tn - m.col_start[o], smem);
}

// ------------------------------------------------------------- fp32 GEMM
// C[M][N] = sum over two segments of A_s . B_s (+ bias), fp32 throughout, on
// the fp32 matrix cores (v_mfma_f32_32x32x2_f32). A_s is [M][k] row-major;
// B_s is [N][k] (NT: both reduction-contiguous) or [k][N] (NN), chosen per
// segment, so the rank-r factors are read in their stored layouts (B [r][N]
// in the forward, A [K][r] in the backward) without transposed copies.
//
// A workgroup owns one 32 x 32 tile of C; its 4 waves split each segment's
// chunks of 8 k into 4 contiguous ranges (wave w takes the w-th), each wave
// accumulating a whole 32 x 32 partial; the 4 partials are added in wave
// order through LDS. Small products (the reference's fp32 shapes, 512 x 768
// x 768) thus get a workgroup per 32 x 32 tile and a quarter of the
// reduction per SIMD. A wave moves its row-major operands a group of four
// chunks (32 k) at a time through a private LDS tile: the global loads give
// each 8 lanes one whole 128-byte row segment, and the MFMA layout comes back
// by one 16-byte LDS read per operand and chunk. (Loading the MFMA layout
// straight from memory touched 32 rows per load instruction, 32 bytes of
// each: the c1 forward product took 29.6 us, 19.5 us staged.)
//
// In a chunk at k0, lane l (row / column l % 32 of its tile, half h = l / 32)
// holds k = k0 + 4 h + p (p < 4) of its row of A and its column of B, and
// MFMA p multiplies that pair: MFMA p sums k0 + p (half 0) and k0 + 4 + p
// (half 1), so the chunk's 8 products are all added, in a fixed order. Rows
// past M, columns past N and k past a segment's length load as zeros.
struct F32Seg {
    const float* a;
    const float* b;
    int64_t lda, ldb, k;
    int nch;  // chunks of 8
};

// 4 consecutive k of row `row` of a row-major [rows][ld] operand (zeros past
// the rows and past k_len): one 16-byte load when the 4 lie inside k_len and
// rows are 16-byte aligned, else 4 checked scalar loads.
__device__ __forceinline__ void f32_load4(const float* base, int64_t rows, int64_t ld, int64_t row, int64_t k,
                                          int64_t k_len, bool vec, float (&v)[4]) {
    if (row < rows && k + 3 < k_len && vec) {
        const float4 q = *reinterpret_cast<const float4*>(base + row * ld + k);
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
#pragma unroll
        for (int p = 0; p < 4; ++p) v[p] = (row < rows && k + p < k_len) ? base[row * ld + k + p] : 0.f;
    }
}

// BUF: every operand's tile rows (and an NN operand's k rows) fit 32-bit
// byte offsets, so the loads go through buffer resources whose range checks
// zero the rows past M / N, and no load branches; otherwise per-element
// checked loads (f32_load4).
template <bool NN0, bool NN1, bool BUF>
__global__ __launch_bounds__(256) void gemm_f32_mfma(int64_t M, int64_t N, F32Seg s0, F32Seg s1,
                                                     const float* __restrict__ bias, float* __restrict__ C,
                                                     int64_t ldc, int tiles_n) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rc = lane & 31, h = lane >> 5;
    const int64_t m0 = (int64_t)(blockIdx.x / tiles_n) * 32, n0 = (int64_t)(blockIdx.x % tiles_n) * 32;
    f32x16 acc;
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.f;
    // Per-wave staging of one group (4 chunks = 32 k) of the row-major
    // operands: [32 rows][32 k + 4] floats each (the pad staggers the rows'
    // banks). Global -> registers with whole 128-byte row segments per 8
    // lanes (lane l: row l / 8 + 8 i, k 4 (l % 8) .. +3), registers -> LDS,
    // then the MFMA layout back by one 16-byte read per operand and chunk.
    __shared__ float stage[4][2][32][36];
    float (*sa)[36] = stage[wave][0];
    float (*sb)[36] = stage[wave][1];
    const int lr = lane >> 3, lk = 4 * (lane & 7);
    auto run = [&](const F32Seg& s, auto nn_tag) {
        constexpr bool NN = decltype(nn_tag)::value;
        const int q = (s.nch + 3) / 4;
        const int c_begin = wave * q, c_end = min(s.nch, c_begin + q);
        if (c_begin >= c_end) return;  // wave-uniform
        const int64_t kend = (int64_t)c_end * 8;
        const int64_t klim = s.k < kend ? s.k : kend;  // this wave's k range ends here
        const bool va = ((s.lda & 3) == 0) && ((reinterpret_cast<uintptr_t>(s.a) & 15) == 0);
        const bool vb = !NN && ((s.ldb & 3) == 0) && ((reinterpret_cast<uintptr_t>(s.b) & 15) == 0);
        // Buffer resources (BUF) over the tile's rows of each operand, ending
        // at the last row's k-th element (nothing past the operand is read);
        // an NN operand's over its k rows from column n0.
        auto tile_bytes = [&](int64_t rows_left, int64_t ld) {
            const int64_t rows = rows_left < 32 ? rows_left : 32;
            return rows <= 0 ? (int64_t)0 : ((rows - 1) * ld + s.k) * 4;
        };
        const __amdgpu_buffer_rsrc_t rsa = make_rsrc(s.a + m0 * s.lda, BUF ? tile_bytes(M - m0, s.lda) : 0);
        const __amdgpu_buffer_rsrc_t rsb =
            make_rsrc(NN ? s.b + n0 : s.b + n0 * s.ldb,
                      !BUF ? 0 : NN ? (s.k - 1) * s.ldb * 4 + (N - n0) * 4 : tile_bytes(N - n0, s.ldb));
        // rows [row0, row0 + 32) of a row-major [rows][ld] operand (its
        // resource r when BUF), k from k0: zeros past rows and klim
        auto load_rows = [&](__amdgpu_buffer_rsrc_t r, const float* base, int64_t rows, int64_t ld, int64_t row0,
                             int64_t k0, bool vec, float (&v)[4][4]) {
            if constexpr (BUF) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f32x4 q = __builtin_bit_cast(f32x4, buf_load16(r, (uint32_t)(((8 * i + lr) * ld + k0 + lk) * 4)));
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[i][e] = k0 + lk + e < klim ? q[e] : 0.f;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) f32_load4(base, rows, ld, row0 + 8 * i + lr, k0 + lk, klim, vec, v[i]);
            }
        };
        auto store_rows = [&](float (*st)[36], const float (&v)[4][4]) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<float4*>(&st[8 * i + lr][lk]) = make_float4(v[i][0], v[i][1], v[i][2], v[i][3]);
        };
        // NN: B [k][N] read straight into the MFMA layout (lanes rc of a k
        // row are consecutive columns), one group ahead in registers
        auto load_nn = [&](int c, float (&v)[4][4]) {
            const int64_t n = n0 + rc;
#pragma unroll
            for (int u = 0; u < 4; ++u)
#pragma unroll
                for (int p = 0; p < 4; ++p) {
                    const int64_t k = (int64_t)(c + u) * 8 + 4 * h + p;
                    v[u][p] = (n < N && k < klim) ? s.b[k * s.ldb + n] : 0.f;
                }
        };
        // BUF and NN: the group's 32 k rows x 32 columns of B, whole 128-byte
        // row segments per 8 lanes like the row-major operands, staged as
        // [k][n] and read back one k row (32 consecutive columns) at a time
        auto load_nn_rows = [&](int64_t k0, float (&v)[4][4]) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t k = k0 + 8 * i + lr;
                const f32x4 q = __builtin_bit_cast(f32x4, buf_load16(rsb, (uint32_t)((k * s.ldb + lk) * 4)));
#pragma unroll
                for (int e = 0; e < 4; ++e) v[i][e] = (k < klim && n0 + lk + e < N) ? q[e] : 0.f;
            }
        };
        constexpr bool NN_LDS = NN && BUF;
        float ra[4][4], rb[4][4], nb[4][4];
        load_rows(rsa, s.a, M, s.lda, m0, (int64_t)c_begin * 8, va, ra);
        if constexpr (!NN) load_rows(rsb, s.b, N, s.ldb, n0, (int64_t)c_begin * 8, vb, rb);
        else if constexpr (NN_LDS) load_nn_rows((int64_t)c_begin * 8, rb);
        else load_nn(c_begin, rb);
        for (int c = c_begin; c < c_end; c += 4) {
            store_rows(sa, ra);
            if constexpr (!NN || NN_LDS) store_rows(sb, rb);
            else {
#pragma unroll
                for (int u = 0; u < 4; ++u)
#pragma unroll
                    for (int p = 0; p < 4; ++p) nb[u][p] = rb[u][p];
            }
            if (c + 4 < c_end) {  // the next group's loads run under this group's MFMAs
                load_rows(rsa, s.a, M, s.lda, m0, (int64_t)(c + 4) * 8, va, ra);
                if constexpr (!NN) load_rows(rsb, s.b, N, s.ldb, n0, (int64_t)(c + 4) * 8, vb, rb);
                else if constexpr (NN_LDS) load_nn_rows((int64_t)(c + 4) * 8, rb);
                else load_nn(c + 4, rb);
            }
            // a wave's LDS operations complete in order: the reads below
            // see the writes above, and the next group's writes come after
            // these reads
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int kk = 8 * u + 4 * h;
                const float4 a4 = *reinterpret_cast<const float4*>(&sa[rc][kk]);
                float bq[4];
                if constexpr (!NN) {
                    const float4 b4 = *reinterpret_cast<const float4*>(&sb[rc][kk]);
                    bq[0] = b4.x; bq[1] = b4.y; bq[2] = b4.z; bq[3] = b4.w;
                } else if constexpr (NN_LDS) {
#pragma unroll
                    for (int p = 0; p < 4; ++p) bq[p] = sb[kk + p][rc];
                } else {
#pragma unroll
                    for (int p = 0; p < 4; ++p) bq[p] = nb[u][p];
                }
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.x, bq[0], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.y, bq[1], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.z, bq[2], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4.w, bq[3], acc, 0, 0, 0);
            }
        }
    };
    run(s0, std::integral_constant<bool, NN0>{});
    run(s1, std::integral_constant<bool, NN1>{});
    __shared__ float red[3][16][64];
    if (wave > 0)
#pragma unroll
        for (int q = 0; q < 16; ++q) red[wave - 1][q][lane] = acc[q];
    __syncthreads();
    if (wave != 0) return;
    const int64_t n = n0 + rc;
    const float bv = (bias && n < N) ? bias[n] : 0.f;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const float v = acc[q] + red[0][q][lane] + red[1][q][lane] + red[2][q][lane];
        const int64_t m = m0 + 8 * (q >> 2) + 4 * h + (q & 3);
        if (m < M && n < N) C[m * ldc + n] = v + bv;
    }
}

}  // namespace

// GEMM args of columns [n0, n0 + n) of an output with BN-wide tiles (B rows,
// bias and C offset to the first column).
static GemmArgs col_range(int64_t M, int64_t n0, int64_t n, const GemmSeg* segs, int nseg, const uint16_t* bias,
                          uint16_t* c, int64_t ldc, int bm, int bn, int group_m) {
    GemmArgs g{};
    g.M = M; g.N = n;
    g.nseg = nseg;
    for (int i = 0; i < nseg; ++i) {
        g.seg[i] = segs[i];
        if (g.seg[i].b) g.seg[i].b += n0 * segs[i].ldb;
    }
    g.bias = bias ? bias + n0 : nullptr; g.c = c + n0; g.ldc = ldc;
    g.tiles_m = (int)((M + bm - 1) / bm);
    g.tiles_n = (int)((n + bn - 1) / bn);
    g.group_m = group_m;
    return g;
}

template <int BM, int BN, int WM, int WN, int BK, int STAGES>
hipError_t launch_cfg(int64_t M, int64_t N, const GemmSeg* segs, int nseg, const uint16_t* bias, uint16_t* c,
                      int64_t ldc, hipStream_t stream, int group_m) {
    const GemmArgs g = col_range(M, 0, N, segs, nseg, bias, c, ldc, BM, BN, group_m);
    constexpr int NT = (BM / WM) * (BN / WN) * 64;
    const dim3 grid((unsigned)(g.tiles_m * g.tiles_n));
    if (nseg > 2) gemm_bf16_kernel<BM, BN, WM, WN, BK, STAGES, true><<<grid, NT, 0, stream>>>(g);
    else gemm_bf16_kernel<BM, BN, WM, WN, BK, STAGES, false><<<grid, NT, 0, stream>>>(g);
    return hipGetLastError();
}

template <int BM1, int BN1, int WM1, int WN1, int S1, int BM2, int BN2, int WM2, int WN2, int S2>
hipError_t launch_split(int64_t M, int64_t N, int64_t n1, const GemmSeg* segs, int nseg, const uint16_t* bias,
                        uint16_t* c, int64_t ldc, hipStream_t stream, int group_m) {
    const GemmArgs g1 = col_range(M, 0, n1, segs, nseg, bias, c, ldc, BM1, BN1, group_m);
    const GemmArgs g2 = col_range(M, n1, N - n1, segs, nseg, bias, c, ldc, BM2, BN2, group_m);
    const int wgs1 = g1.tiles_m * g1.tiles_n;
    const dim3 grid((unsigned)(wgs1 + g2.tiles_m * g2.tiles_n));
    if (nseg > 2)
        gemm_bf16_split<BM1, BN1, WM1, WN1, S1, BM2, BN2, WM2, WN2, S2, true><<<grid, 512, 0, stream>>>(g1, g2, wgs1);
    else
        gemm_bf16_split<BM1, BN1, WM1, WN1, S1, BM2, BN2, WM2, WN2, S2, false><<<grid, 512, 0, stream>>>(g1, g2, wgs1);
    return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int BK, int STAGES>
hipError_t launch_multi(int64_t M, const GemmOut* outs, int nout, hipStream_t stream, int group_m) {
    GemmMulti m{};
    m.nout = nout;
    m.col_start[0] = 0;
    for (int o = 0; o < nout; ++o) {
        m.out[o] = col_range(M, 0, outs[o].N, outs[o].seg, outs[o].nseg, outs[o].bias, outs[o].c, outs[o].ldc, BM, BN,
                             group_m);
        m.col_start[o + 1] = m.col_start[o] + m.out[o].tiles_n;
    }
    m.tiles_m = (int)((M + BM - 1) / BM);
    m.tiles_n = m.col_start[nout];
    m.group_m = group_m;
    constexpr int NT = (BM / WM) * (BN / WN) * 64;
    gemm_bf16_multi<BM, BN, WM, WN, BK, STAGES><<<dim3((unsigned)(m.tiles_m * m.tiles_n)), NT, 0, stream>>>(m);
    return hipGetLastError();
}

namespace {
// Compute units of the current device (the number of workgroups one round
// of the 1-workgroup-per-CU tiles runs at once), cached per device.
int cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cache[dev].store(v, std::memory_order_relaxed);
    return v;
}

// Per-tile speed relative to 256 x 256 (the fastest per FLOP), from
// full-round medians on MI355X at the Qwen2.5 layer shapes: 256 x 192 runs
// at 0.85-0.89 of its rate; the 256 x 128 ring at 0.81 (K ~ 1.5k), 0.85
// (K ~ 3.5k) and 0.88 (K = 8960); 128 x 128 (4 waves) serves small grids.
double tile_speed(GemmTile t, int64_t K) {
    switch (t) {
        case GemmTile::k256x256: return 1.0;
        case GemmTile::k256x192: return K >= 4096 ? 0.85 : 0.87;
        case GemmTile::k256x128: return K >= 6144 ? 0.88 : K >= 2048 ? 0.85 : 0.81;
        default: return 0.8;
    }
}

void tile_dims(GemmTile t, int& bm, int& bn) {
    bm = t == GemmTile::k128x128 ? 128 : 256;
    bn = t == GemmTile::k256x256 ? 256 : t == GemmTile::k256x192 ? 192 : 128;
}

// Estimated time of n1 tiles of duration t1 followed by n2 tiles of
// duration t2, dispatched in order onto `cus` CUs one workgroup each: whole
// rounds of the first shape, then the rest of the work spread over every CU
// in steps of t2 (a started first-shape tile still takes t1).
double list_time(int64_t n1, double t1, int64_t n2, double t2, int cus) {
    const int64_t r1 = n1 / cus, q1 = n1 % cus;
    double t = (double)r1 * t1;
    if (q1 == 0 && n2 == 0) return t;
    if (n2 == 0) return t + t1;
    const double rest = (double)q1 * t1 + (double)n2 * t2;
    double tail = std::ceil(rest / ((double)cus * t2)) * t2;
    if (q1 > 0 && tail < t1) tail = t1;
    return t + tail;
}

}  // namespace

// Estimated time of a plan (units of one 256 x 256 tile at full speed).
double plan_time(int64_t M, int64_t N, int64_t K, const GemmPlan& p, int cus) {
    int bm, bn;
    if (p.n1 >= N) {
        tile_dims(p.main, bm, bn);
        const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        return list_time(tiles, (double)bm * bn / tile_speed(p.main, K), 0, 0.0, cus);
    }
    tile_dims(p.tail, bm, bn);
    const int64_t tm = (M + 255) / 256;
    const int64_t n2 = tm * ((N - p.n1 + bn - 1) / bn);
    return list_time(tm * (p.n1 / 256), 65536.0, n2, (double)bm * bn / tile_speed(p.tail, K), cus);
}

double plan_time_multi(int64_t M, const int64_t* Ns, int nout, int64_t K, GemmTile t, int cus) {
    int bm, bn;
    tile_dims(t, bm, bn);
    int64_t cols = 0;
    for (int o = 0; o < nout; ++o) cols += (Ns[o] + bn - 1) / bn;
    return list_time(((M + bm - 1) / bm) * cols, (double)bm * bn / tile_speed(t, K), 0, 0.0, cus);
}

GemmPlan choose_gemm_plan(int64_t M, int64_t N, int64_t K, int cus) {
    // One tile shape over all of N, or 256 x 256 tiles over the first n1 =
    // 256 j columns and a narrower shape over the rest, whichever list_time
    // estimates fastest. The split lets the wide tile fill whole rounds
    // (e.g. N = 1536 at M = 16384: 256 tiles of 256 x 256 + 256 of 256 x 128
    // instead of 384 tiles of 256 x 256 on 256 CUs).
    const GemmTile singles[] = {GemmTile::k256x256, GemmTile::k256x192, GemmTile::k256x128, GemmTile::k128x128};
    GemmPlan best{GemmTile::k128x128, GemmTile::k128x128, N};
    double best_t = 1e300;
    for (GemmTile t : singles) {
        int bm, bn;
        tile_dims(t, bm, bn);
        const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        const double e = list_time(tiles, (double)bm * bn / tile_speed(t, K), 0, 0.0, cus);
        if (e < best_t) { best_t = e; best = GemmPlan{t, t, N}; }
    }
    const int64_t tm = (M + 255) / 256;
    const double t1 = 65536.0;
    const int64_t jmax = N / 256;
    for (int64_t j = jmax; j >= 1 && j >= jmax - 8; --j) {
        const int64_t n1 = 256 * j;
        if (n1 >= N) continue;
        for (GemmTile t : {GemmTile::k256x192, GemmTile::k256x128}) {
            int bm, bn;
            tile_dims(t, bm, bn);
            const int64_t n2 = tm * ((N - n1 + bn - 1) / bn);
            const double e = list_time(tm * j, t1, n2, (double)bm * bn / tile_speed(t, K), cus);
            if (e < best_t) { best_t = e; best = GemmPlan{GemmTile::k256x256, t, n1}; }
        }
    }
    return best;
}

hipError_t launch_gemm_bf16(int64_t M, int64_t N, const GemmSeg* segs, int nseg, const uint16_t* bias, uint16_t* c,
                            int64_t ldc, hipStream_t stream) {
    int64_t K = 0;
    for (int i = 0; i < nseg; ++i) K += segs[i].k;
    const GemmPlan p = choose_gemm_plan(M, N, K, cu_count());
    if (p.n1 < N) {  // 256 x 256 over [0, n1), the tail shape over [n1, N)
        if (p.tail == GemmTile::k256x192)
            return launch_split<256, 256, 128, 64, 2, 256, 192, 64, 96, 2>(M, N, p.n1, segs, nseg, bias, c, ldc,
                                                                            stream, 4);
        return launch_split<256, 256, 128, 64, 2, 256, 128, 64, 64, 3>(M, N, p.n1, segs, nseg, bias, c, ldc, stream,
                                                                        4);
    }
    switch (p.main) {
        case GemmTile::k256x256:  // 8 waves of 128 x 64, k-steps of 64, 2 stages (128 KB LDS)
            return launch_cfg<256, 256, 128, 64, 64, 2>(M, N, segs, nseg, bias, c, ldc, stream, 4);
        case GemmTile::k256x192:  // 8 waves of 64 x 96, 2 stages (112 KB LDS)
            return launch_cfg<256, 192, 64, 96, 64, 2>(M, N, segs, nseg, bias, c, ldc, stream, 4);
        case GemmTile::k256x128:  // 8 waves of 64 x 64, 3 stages (144 KB LDS)
            return launch_cfg<256, 128, 64, 64, 64, 3>(M, N, segs, nseg, bias, c, ldc, stream, 4);
        default:                  // 4 waves of 64 x 64, 3 stages (96 KB LDS)
            return launch_cfg<128, 128, 64, 64, 64, 3>(M, N, segs, nseg, bias, c, ldc, stream, 4);
    }
}

hipError_t launch_gemm_bf16(int64_t M, int64_t N, GemmSeg s0, GemmSeg s1, const uint16_t* bias, uint16_t* c,
                            int64_t ldc, hipStream_t stream) {
    const GemmSeg segs[2] = {s0, s1};
    return launch_gemm_bf16(M, N, segs, 2, bias, c, ldc, stream);
}

GemmTile choose_multi_tile(int64_t M, const int64_t* Ns, int nout, int64_t K, int cus) {
    // one tile shape over every block's columns, by the same list-schedule
    // estimate as choose_gemm_plan's single shapes
    const GemmTile singles[] = {GemmTile::k256x256, GemmTile::k256x192, GemmTile::k256x128, GemmTile::k128x128};
    GemmTile best = GemmTile::k128x128;
    double best_t = 1e300;
    for (GemmTile t : singles) {
        int bm, bn;
        tile_dims(t, bm, bn);
        int64_t cols = 0;
        for (int o = 0; o < nout; ++o) cols += (Ns[o] + bn - 1) / bn;
        const int64_t tiles = ((M + bm - 1) / bm) * cols;
        const double e = list_time(tiles, (double)bm * bn / tile_speed(t, K), 0, 0.0, cus);
        if (e < best_t) { best_t = e; best = t; }
    }
    return best;
}

bool gemm_bf16_multi_one_launch(int64_t M, const GemmOut* outs, int nout) {
    // One launch over every block's columns with one tile shape, or one
    // launch per block with its own plan (a split plan can fill the CUs'
    // last round with narrower tiles), whichever the estimate says is faster.
    // A single block always takes its own plan.
    if (nout <= 1) return false;
    int64_t Ns[kGemmMaxOut];
    int64_t K = 0;
    for (int o = 0; o < nout; ++o) Ns[o] = outs[o].N;
    for (int i = 0; i < outs[0].nseg; ++i) K += outs[0].seg[i].k;
    const int cus = cu_count();
    const GemmTile t = choose_multi_tile(M, Ns, nout, K, cus);
    double sep = 0.0;
    for (int o = 0; o < nout; ++o) sep += plan_time(M, Ns[o], K, choose_gemm_plan(M, Ns[o], K, cus), cus);
    return !(sep < plan_time_multi(M, Ns, nout, K, t, cus));
}

hipError_t launch_gemm_bf16_multi(int64_t M, const GemmOut* outs, int nout, hipStream_t stream) {
    if (!gemm_bf16_multi_one_launch(M, outs, nout)) {
        for (int o = 0; o < nout; ++o) {
            const hipError_t e = launch_gemm_bf16(M, outs[o].N, outs[o].seg, outs[o].nseg, outs[o].bias, outs[o].c,
                                                  outs[o].ldc, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    int64_t Ns[kGemmMaxOut];
    int64_t K = 0;
    for (int o = 0; o < nout; ++o) Ns[o] = outs[o].N;
    for (int i = 0; i < outs[0].nseg; ++i) K += outs[0].seg[i].k;
    const GemmTile t = choose_multi_tile(M, Ns, nout, K, cu_count());
    switch (t) {
        case GemmTile::k256x256: return launch_multi<256, 256, 128, 64, 64, 2>(M, outs, nout, stream, 4);
        case GemmTile::k256x192: return launch_multi<256, 192, 64, 96, 64, 2>(M, outs, nout, stream, 4);
        case GemmTile::k256x128: return launch_multi<256, 128, 64, 64, 64, 3>(M, outs, nout, stream, 4);
        default: return launch_multi<128, 128, 64, 64, 64, 3>(M, outs, nout, stream, 4);
    }
}

hipError_t launch_gemm_f32(bool nn, bool nn1, int64_t M, int64_t N, GemmSegF32 s0, GemmSegF32 s1, const float* bias,
                           float* c, int64_t ldc, hipStream_t stream) {
    const int64_t tiles_m = (M + 31) / 32, tiles_n = (N + 31) / 32;
    if (tiles_m * tiles_n >= ((int64_t)1 << 31) || tiles_n >= ((int64_t)1 << 31)) return hipErrorInvalidValue;
    auto seg = [](const GemmSegF32& g) {
        return F32Seg{g.a, g.b, g.lda, g.ldb, g.k, (int)((g.k + 7) / 8)};
    };
    const dim3 grid((unsigned)(tiles_m * tiles_n));
    const F32Seg a = seg(s0), b = seg(s1);
    const int tn = (int)tiles_n;
    // 32-bit buffer offsets: 32 rows of each row-major operand, every k row
    // of an NN operand
    constexpr int64_t kLim = ((int64_t)1 << 31) - 64;
    auto fits = [&](const GemmSegF32& g, bool g_nn) {
        return 32 * g.lda * 4 < kLim && (g_nn ? (g.k + 1) * g.ldb * 4 < kLim : 32 * g.ldb * 4 < kLim);
    };
    const bool buf = fits(s0, nn) && fits(s1, nn1);
    auto go = [&](auto nn_tag, auto nn1_tag) {
        constexpr bool A = decltype(nn_tag)::value, B = decltype(nn1_tag)::value;
        if (buf) gemm_f32_mfma<A, B, true><<<grid, 256, 0, stream>>>(M, N, a, b, bias, c, ldc, tn);
        else gemm_f32_mfma<A, B, false><<<grid, 256, 0, stream>>>(M, N, a, b, bias, c, ldc, tn);
    };
    if (nn && nn1) go(std::true_type{}, std::true_type{});
    else if (nn) go(std::true_type{}, std::false_type{});
    else if (nn1) go(std::false_type{}, std::true_type{});
    else go(std::false_type{}, std::false_type{});
    return hipGetLastError();
}

}  // namespace mc
