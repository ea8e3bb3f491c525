// Internal launch wrappers of the LoRA kernels (lora_lowrank.hip,
// lora_gemm.hip), orchestrated by lora.hip. Shapes are validated by abi.cpp.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mc {

inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// Projections of one input in a grouped call, and job-table sizes of the
// batched launches.
constexpr int kMaxProj = 4;
constexpr int kPrepJobs = 8;
constexpr int kColJobs = 8;
constexpr int kSumJobs = 8;

// 16-row rank tiles of a row-projection pass over r ranks; a pass holds at
// most kRowprojMaxRanks (more ranks take several passes over the input).
constexpr int kRowprojMaxRanks = 128;
inline int rowproj_rc(int r) { return r <= 16 ? 1 : r <= 32 ? 2 : r <= 48 ? 3 : r <= 64 ? 4 : 8; }
// Rows of the split-T partials of a column reduction over r ranks: ranks go
// in groups of 64, each taking 16, 32, 48 or 64 accumulator rows.
inline int colreduce_rows(int r) { return r <= 16 ? 16 : r <= 32 ? 32 : r <= 48 ? 48 : (int)round_up(r, 64); }

// ------------------------------------------------------ operand preparation
// One job: out[i][j] (bf16, rows_out x cols_out, ld = cols_out) = src element
// (transpose ? src[j*ld_src + i] : src[i*ld_src + j]) for i < valid_rows,
// j < valid_cols, else 0. With lo != nullptr the fp32 value v is split as
// hi = bf16(v), lo = bf16(v - hi). A job with hi == nullptr is skipped.
// ld_out is the row stride of hi / lo (0: cols_out).
// frag_rc > 0 writes the row projection's parameter operand in fragment
// order instead (rowproj_frag_index: rows i of the job are rows
// frag_row0 + i of a 16 frag_rc-row operand; ld_out is unused).
struct PrepJob {
    const float* src;
    int64_t ld_src, valid_rows, valid_cols;
    bool transpose;
    uint16_t* hi;
    uint16_t* lo;
    int64_t rows_out, cols_out;
    int64_t ld_out;
    int frag_rc;
    int64_t frag_row0;
};

// Fragment order of the row projection's bf16 parameter operand P
// [16 RC][C]: element (j, c) at
//   ((((c / 64) RC + j / 16) 2 + (c / 8) % 2) 64 + 16 ((c % 64) / 16) + j % 16) 8 + c % 8,
// i.e. per 64-column step, 16-rank tile and 8-column half, the 16 bytes each
// of the 64 lanes loads, lane after lane (1 KB per load instruction). The
// operand spans round_up(C, 64) columns.
__host__ __device__ inline int64_t rowproj_frag_index(int RC, int64_t j, int64_t c) {
    const int64_t lane = 16 * ((c & 63) >> 4) + (j & 15);
    return (((((c >> 6) * RC + (j >> 4)) * 2 + ((c >> 3) & 1)) * 64 + lane) << 3) + (c & 7);
}

// Up to kPrepJobs jobs in one launch.
hipError_t launch_prep_bf16(const PrepJob* jobs, int n, hipStream_t stream);
hipError_t launch_prep_bf16(const PrepJob& j0, const PrepJob& j1, hipStream_t stream);

// ------------------------------------------------------- row projection
// For t < T, j < r:  v = scale * sum_c X[t][c] * P[j][c]   (P = P_hi + P_lo)
//                    v = mask ? (mask[t*r+j] ? v*keep : 0) : v
//   out_t[j*T + t] = v                       (fp32, may be null)
//   out_ext[t*rext + j] = bf16(ext_scale*v)  (j < r; zero for r <= j < rext; may be null)
// X bf16 [T][C] (C % 8 == 0), P_hi / P_lo bf16 [16 rowproj_rc(r)][C] in
// fragment order (rowproj_frag_index), rows past r zero.
// A pass over one X whose r ranks may be those of several projections
// (rp ranks each): rank j belongs to projection p = j / rp and uses its mask
// [T][rp] and out_t [rp][T] (entries may be null), and goes to column
// p rext_p + j % rp of out_ext (row stride ext_ld; the pad columns up to
// (p + 1) rext_p are zeroed). With P_f32 set the parameter is read as fp32
// [r][C] and split hi / lo in registers instead of P_hi / P_lo.
// mask_ld is the mask's row stride (0: rp); a pass over ranks j0 .. of a
// projection of more ranks passes its mask columns as mask + j0 with
// mask_ld = the projection's rank.
struct RowprojCall {
    const uint16_t* X;
    int64_t T, C;
    const uint16_t* P_hi;
    const uint16_t* P_lo;
    const float* P_f32;
    int r, rp;
    float scale;
    const uint8_t* mask[kMaxProj];
    int64_t mask_ld;
    float keep;
    float* out_t[kMaxProj];
    uint16_t* out_ext;
    int rext_p, ext_ld;
    float ext_scale;
};
hipError_t launch_rowproj_bf16(const RowprojCall& c, hipStream_t stream);

// The backward's operand pass for up to kMaxProj projections in one launch:
// per projection the row projection of dY with the fp32 B [r][N] read
// directly (G = scale dY.B^T, masked, into gd_t [r][T] and the columns of
// gd_ext), the bf16 A extension operand (job a_ext, skipped when a_ext.hi is
// null) and W [N][K] -> Wt [K][N] (skipped when Wt is null).
struct OperandsCall {
    const uint16_t* dY;
    int64_t N;
    const float* B;
    const uint8_t* mask;
    int64_t mask_ld;  // 0: the pass's ranks
    float* gd_t;
    uint16_t* gd_ext;
    PrepJob a_ext;
    const uint16_t* W;
    uint16_t* Wt;
};
hipError_t launch_lora_bwd_operands(const OperandsCall* calls, int n, int64_t T, int64_t K, int r, float scale,
                                    float keep, int rext_p, int ext_ld, hipStream_t stream);

// ------------------------------------------------- column reduction (split T)
// One job: partial[s][j][c] = sum_{t in split s} Pt[j*T + t] * X[t][c] for
// j < r, c < C, in the split partition of `splits` chunks; partial rows are
// colreduce_rows(r) apart per split. X bf16 [T][C] (C % 8 == 0), Pt fp32
// [r][T]. A job with X == nullptr is skipped; the jobs' 64-rank groups run in
// one launch per rank-tile size.
struct ColJob {
    const uint16_t* X;
    int64_t C;
    const float* Pt;
    int r;
    int splits;
    float* partial;
};
int colreduce_splits(int64_t T, int64_t C);
hipError_t launch_colreduce_bf16(int64_t T, const ColJob* jobs, int n, hipStream_t stream);
// The same column reductions with the token-side operand as bf16 hi / lo
// planes [r][T] (P_hi + P_lo = Pt to ~16 mantissa bits, split once by the
// producer) through an LDS ring shared by 512-column workgroups; T % 8 == 0.
// Partials in ColJob's layout: [splits][colreduce_rows(r)][C].
struct ColsplitJob {
    const uint16_t* X;
    int64_t C;
    const uint16_t* P_hi;
    const uint16_t* P_lo;
    int r;
    int splits;
    float* partial;
};
int colsplit_splits(int64_t T, int64_t C);
hipError_t launch_colsplit_bf16(int64_t T, const ColsplitJob* jobs, int n, hipStream_t stream);
// ------------------------------------------------ fused dY pass (r <= 32)
// One read of a projection's dY [T][N] gives both rank-r products of the
// backward that reduce it:
//   dB partials  partB[s][j][c] = sum_{t in split s} Pt[j][t] dY[t][c]
//                (the layout of ColJob's partials: colreduce_rows(r) rows
//                per split, summed by split_sum)
//   G partials   gpart[g][t][j] = sum_{c in column group g} dY[t][c] B[j][c]
//                (groups of kDyCols columns, summed in group order by
//                launch_dy_finish)
// Pt fp32 [r][T] (the forward's Hd^T), B fp32 [r][N]; partB or gpart may be
// null (that product is skipped; Pt is then not read).
constexpr int kDyCols = 512;
constexpr int kDyMaxRank = 32;
inline int dy_groups(int64_t N) { return (int)((N + kDyCols - 1) / kDyCols); }
int dy_splits(int64_t T, int64_t N);  // the split count of launch_dy_pass for this shape
struct DyJob {
    const uint16_t* dY;
    int64_t N;
    const float* B;
    const float* Pt;
    float* partB;
    float* gpart;
};
hipError_t launch_dy_pass(int64_t T, int r, const DyJob* jobs, int n, hipStream_t stream);
// Finishing of rank-r partials (r <= kFinishMaxRank): v = scale * sum_g
// gpart[g][t][j] per projection (partials of token t at gpart + g T ld +
// t ld, ld = r when 0), then the dropout of the rank-r hidden (mask rows of
// mask_ld elements, or null; keep = 1/(1-p)): v^T -> gd_t fp32 [r][T] and /
// or bf16 hi / lo planes gd_hi, gd_lo [r][T] (each may be null) and
// ext_scale v -> gd_ext bf16 columns 0..r-1 of rows of ext_ld elements,
// columns r..rext-1 zeroed (may be null); up to kPrepJobs PrepJobs (operand
// preparation) run in the same launch. It finishes both the fused dY pass's
// G and the split row projection's H / G.
constexpr int kFinishMaxRank = 64;
struct DyFinishJob {
    const float* gpart;
    int groups;
    const uint8_t* mask;
    float* gd_t;
    uint16_t* gd_ext;
    int64_t ld = 0;
    int64_t mask_ld = 0;
    uint16_t* gd_hi = nullptr;  // v^T as bf16 hi / lo planes [r][T] (both or neither)
    uint16_t* gd_lo = nullptr;
};
hipError_t launch_dy_finish(int64_t T, int r, float scale, float keep, int rext, int ext_ld, float ext_scale,
                            const DyFinishJob* jobs, int n, const PrepJob* preps, int npreps, hipStream_t stream);

// ------------------------------------------------- split row projection
// The row projection of a pass of up to 64 ranks (r) as a skinny GEMM: each
// workgroup streams kRowsplitRows token rows of X [T][C] and the parameter
// through LDS for one column split, so the parameter is fetched once per
// kRowsplitRows rows. Job i writes part[s][t][16 ceil(r / 16)] (fp32) for its
// splits s < splits, finished by launch_dy_finish (groups = splits, ld =
// 16 ceil(r / 16)). The parameter is bf16 hi / lo [prows][C] (P_hi, P_lo) or
// fp32 [prows][C] (P_f32, split into hi / lo in registers; every job of a
// launch the same kind); rows past prows and past r contribute zeros. Jobs
// with the same X, C and splits run their tiles interleaved, so the reads of
// one x block by several parameters meet in one L2.
struct RowsplitJob {
    const uint16_t* X;
    int64_t C;
    const uint16_t* P_hi;
    const uint16_t* P_lo;
    const float* P_f32;
    int prows;
    float* part;
    int splits;
};
constexpr int kRowsplitRanks = 64;
constexpr int kRowsplitRows = 256;
constexpr int kRowsplitMinCols = 256;
inline int rowsplit_ld(int r) { return 16 * ((r + 15) / 16); }
// splits of a job of C columns (C % 8 == 0)
int rowsplit_splits(int64_t T, int64_t C);
hipError_t launch_rowsplit(int64_t T, int r, const RowsplitJob* jobs, int n, hipStream_t stream);

// One job: out = scale * sum_s partial[s][j][c] (s ascending) for j < r,
// c < C, written to out[c*r + j] when transpose_out (dA [K][r]) else
// out[j*C + c] (dB [r][N]); part_stride = colreduce_rows * C. A job with
// out == nullptr is skipped; up to kSumJobs jobs run in one launch.
struct SumJob {
    const float* partial;
    int splits;
    int64_t C;
    int64_t part_stride;
    int r;
    float scale;
    bool transpose_out;
    float* out;
};
hipError_t launch_split_sum(const SumJob* jobs, int n, hipStream_t stream);

// -------------------------------------------------------------- GEMM bf16
// C[M][N] = sum over up to kGemmMaxSeg reduction segments of A_s . B_s^T
// (+ bias[n]), bf16 out, the segments' products accumulated in segment
// order. A_s bf16 [M][k_s] (row stride lda_s), B_s bf16 [N][k_s] (row stride
// ldb_s). Row strides and k_s are multiples of 8; k_s may be 0.
constexpr int kGemmMaxSeg = 5;
constexpr int kGemmMaxOut = 4;
struct GemmSeg {
    const uint16_t* a;
    int64_t lda;
    const uint16_t* b;
    int64_t ldb;
    int64_t k;
};
hipError_t launch_gemm_bf16(int64_t M, int64_t N, const GemmSeg* segs, int nseg, const uint16_t* bias, uint16_t* c,
                            int64_t ldc, hipStream_t stream);
hipError_t launch_gemm_bf16(int64_t M, int64_t N, GemmSeg s0, GemmSeg s1, const uint16_t* bias, uint16_t* c,
                            int64_t ldc, hipStream_t stream);
// Up to kGemmMaxOut output blocks of M rows in one launch (projections of
// one input): block o is C_o[M][N_o] = sum over its segments of
// A_s . B_s^T (+ bias_o); all blocks use one tile shape.
struct GemmOut {
    int64_t N;
    GemmSeg seg[2];
    int nseg;
    const uint16_t* bias;
    uint16_t* c;
    int64_t ldc;
};
hipError_t launch_gemm_bf16_multi(int64_t M, const GemmOut* outs, int nout, hipStream_t stream);
// Whether launch_gemm_bf16_multi runs the blocks as one launch (else one
// launch per block, in block order).
bool gemm_bf16_multi_one_launch(int64_t M, const GemmOut* outs, int nout);
// Workgroup tiles of the bf16 GEMM for an M x N output with reduction length
// K on `cus` compute units: `main` over columns [0, n1), `tail` over [n1, N)
// (n1 == N: one tile shape; otherwise main is 256 x 256).
enum class GemmTile { k256x256, k256x192, k256x128, k128x128 };
struct GemmPlan {
    GemmTile main, tail;
    int64_t n1;
};
GemmPlan choose_gemm_plan(int64_t M, int64_t N, int64_t K, int cus);

// ------------------------------------------------------------- fp32 path
// Same contracts as above with fp32 storage and plain FMA arithmetic; used
// for act_dtype == MC_F32 (the fp32 parity configuration).
struct GemmSegF32 {
    const float* a;
    int64_t lda;
    const float* b;
    int64_t ldb;
    int64_t k;
};
// nn / nn1: segment 0 / 1's B stored [k][N] (else [N][k]).
hipError_t launch_gemm_f32(bool nn, bool nn1, int64_t M, int64_t N, GemmSegF32 s0, GemmSegF32 s1,
                           const float* bias, float* c, int64_t ldc, hipStream_t stream);
// v[t][j] = scale * sum_c X[t][c] * (transpose_p ? P[c*r + j] : P[j*C + c]),
// masked as in launch_rowproj_bf16; out_t [r][T]; out_ext [T][r] = ext_scale*v.
hipError_t launch_rowproj_f32(const float* X, int64_t T, int64_t C, const float* P, bool transpose_p,
                              int r, float scale, const uint8_t* mask, float keep, float* out_t,
                              float* out_ext, float ext_scale, hipStream_t stream);
// out = scale * sum_t Pt[j*T + t] * X[t][c]; layout as launch_split_sum.
// One or two such reductions over the same T and r in one launch.
struct ColF32Call {
    const float* X;
    int64_t C;
    const float* Pt;
    float scale;
    bool transpose_out;
    float* out;
};
hipError_t launch_colreduce_f32(const ColF32Call* calls, int n, int64_t T, int r, hipStream_t stream);

}  // namespace mc
