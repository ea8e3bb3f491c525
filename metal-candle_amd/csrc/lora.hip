// LoRA linear forward / backward: workspace layout and launch sequence.
//
// Forward (bf16 activations), reference order lora.rs:320-339 plus the base
// candle Linear (transformer.rs:189-192), three launches:
//   1. A^T -> bf16 hi/lo, B^T -> bf16 ext operand          (one prep launch)
//   2. Hd = dropout(x.A) -> h_save (fp32 [r][T]) and s*Hd (bf16 ext operand)
//   3. y = [x | s*Hd] . [W | B^T]^T + b                    (one MFMA GEMM)
// Backward (W frozen; candle autograd of the same composite):
//   1. G = s dY.B^T, Gd = dropout'(G) -> Gd^T fp32, Gd bf16 (B read as
//      fp32, split hi/lo in registers), with A -> bf16 ext operand and
//      W -> W^T in the same launch
//   2. dX = [dY | Gd] . [W^T | A]^T                         (one MFMA GEMM)
//   3. dA = x^T.Gd and dB = s Hd^T.dY: split-T column reductions (one
//      launch) and their fixed-order split sums (one launch)
// The fp32 path runs the same sequence with fp32 operands and FMA kernels.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"
#include "lora_kernels.hpp"
#include "profile.hpp"

namespace mc {
namespace {

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct Dims {
    int64_t T, K, N;
    int r, r16, rext;
    bool bf16;
};

Dims dims_of(const mc_lora_desc& d) {
    Dims m;
    m.T = d.tokens;
    m.K = d.in_features;
    m.N = d.out_features;
    m.r = d.rank;
    m.r16 = 16 * rowproj_rc(d.rank);  // rank rows of the row projection's parameter operand
    m.rext = (int)round_up(d.rank, 8);
    m.bf16 = d.act_dtype == MC_BF16;
    return m;
}

// Algorithmic work of one GEMM launch: FLOPs of the base product (the rank
// columns when there is no base), bytes of one read of each operand and one
// write of the output.
prof::Scope gemm_scope(hipStream_t st, int64_t M, int64_t N, int64_t kbase, int64_t kext, int r, int es) {
    const double k = (double)(kbase > 0 ? kbase : r);
    return prof::Scope(prof::kGemm, st, 2.0 * M * N * k,
                       (double)es * ((double)(M + N) * (double)(kbase + kext) + (double)M * N));
}

// rowproj / colreduce: one read of X (T x C, act dtype), the rank-r side in fp32.
prof::Scope lowrank_scope(hipStream_t st, int64_t T, int64_t C, int r, int es) {
    return prof::Scope(prof::kLowRank, st, 2.0 * T * C * r, (double)T * C * es + 4.0 * T * r);
}

#define MC_TRY(expr)                          \
    do {                                      \
        hipError_t e_ = (expr);               \
        if (e_ != hipSuccess) return e_;      \
    } while (0)

// Projections of one row-projection pass of a grouped forward: whole
// projections, at most 64 ranks together (the 64-row workgroups of the row
// projection; more ranks take the 32-row form, which loads each parameter
// fragment for half as many token rows), at least one.
int proj_per_pass(int r) { return r >= 64 ? 1 : 64 / r < kMaxProj ? 64 / r : kMaxProj; }

PrepJob prep_job(const float* src, int64_t ld_src, int64_t valid_rows, int64_t valid_cols, bool transpose,
                 uint16_t* hi, uint16_t* lo, int64_t rows_out, int64_t cols_out, int64_t ld_out = 0) {
    PrepJob j{};
    j.src = src; j.ld_src = ld_src; j.valid_rows = valid_rows; j.valid_cols = valid_cols; j.transpose = transpose;
    j.hi = hi; j.lo = lo; j.rows_out = rows_out; j.cols_out = cols_out; j.ld_out = ld_out;
    return j;
}

hipError_t prep_all(const PrepJob* jobs, int n, hipStream_t st) {
    for (int first = 0; first < n; first += kPrepJobs)
        MC_TRY(launch_prep_bf16(jobs + first, n - first < kPrepJobs ? n - first : kPrepJobs, st));
    return hipSuccess;
}

// The backward reads each dY_g once for both rank-r products (launch_dy_pass)
// when that pass has the parallelism to stream at full rate: ranks <= 32 and
// every dY_g of at least 2^26 elements (e.g. the c4 gate / up [16384, 8960]:
// >= 512 workgroups of 512 columns x >= 256 rows). Smaller products run the
// row projection and the column reduction as two passes, which measured
// faster there (c3, and c4's N = 1536 projections).
bool dy_fused(const Dims& m, const int64_t* N, int count) {
    if (m.r > kDyMaxRank) return false;
    for (int g = 0; g < count; ++g)
        if (N[g] * m.T < ((int64_t)1 << 26)) return false;
    return true;
}

// The split row projection (launch_rowsplit: 256-row workgroups sharing the
// parameter through LDS, column splits finished by launch_dy_finish) takes
// the rank-r passes of projections of 33-64 ranks, and in the forward also
// those of at least 4096 columns: measured at the c4 / c5 shapes it ran the
// 64-rank passes 2-2.5x faster than rowproj_bf16 / lora_bwd_operands and the
// 8960-column one 14% faster, while a pass of 32 ranks or fewer over 1536
// columns gained little once its finishing launch is counted. The choice
// depends on the projection's rank and the shared K only, never on the
// group, so a grouped call computes the same sums as single calls.
// Its finishing launch addresses one split's T x 16 ceil(ranks / 16) fp32
// partial (at most 64 ranks per pass) through one buffer resource with
// 32-bit offsets, so token counts whose 64-rank partial reaches 2^31 bytes
// (T >= 2^23) take the unsplit kernels instead.
bool rowsplit_tokens_fit(const Dims& m) { return m.T * (int64_t)kRowsplitRanks * 4 < ((int64_t)1 << 31); }
bool fwd_rowsplit(const Dims& m) {
    return m.r <= kRowsplitRanks && (m.r > 32 || m.K >= 4096) && rowsplit_tokens_fit(m);
}
bool bwd_rowsplit(const Dims& m, const int64_t* N, int count) {
    return m.r > 32 && m.r <= kRowsplitRanks && !dy_fused(m, N, count) && rowsplit_tokens_fit(m);
}
// With it, dA and dB take the column reduction over bf16 hi / lo planes of
// Gd^T (written by the finishing launch) and Hd^T (h_save split by a prep
// job), when T % 8 == 0: at 64 ranks it measured 22% faster than the fp32
// operand path, whose per-step operand split is the kernel's bottleneck.
bool bwd_colsplit(const Dims& m, const int64_t* N, int count) { return bwd_rowsplit(m, N, count) && m.T % 8 == 0; }

// bf16 projections whose K or N is not a multiple of 8 (rows not made of
// 16-byte chunks) run on copies zero-padded to multiples of 8: a padded
// feature adds exact zeros to every product, so y, dX, dA and dB are the
// padded results' leading rows / columns.
bool bf16_padded(const mc_lora_desc& d) {
    return d.act_dtype == MC_BF16 && (d.in_features % 8 != 0 || d.out_features % 8 != 0);
}
mc_lora_desc padded_desc(const mc_lora_desc& d) {
    mc_lora_desc p = d;
    p.in_features = round_up(d.in_features, 8);
    p.out_features = round_up(d.out_features, 8);
    return p;
}
// Row-band copies: a workgroup copies bands of whole rows, each row as
// `chunks` chunks of V elements. A row of at most 256 chunks takes `chunks`
// threads and a band holds 256 / chunks rows; a longer row takes the whole
// workgroup, its threads striding over the chunks. Each thread divides once,
// at the start, and the bands are walked grid-stride.
struct Band {
    int chunks, rows_per_band, row_in_band, chunk0, chunk_step;
    __device__ Band(int64_t nchunks) : chunks((int)nchunks) {
        const int t = (int)threadIdx.x;
        if (chunks <= 256) {
            rows_per_band = 256 / chunks;
            row_in_band = t / chunks;
            chunk0 = t - row_in_band * chunks;
            chunk_step = chunks;
        } else {
            rows_per_band = 1;
            row_in_band = 0;
            chunk0 = t;
            chunk_step = 256;
        }
    }
};
template <typename T, int V>
struct alignas(V * sizeof(T)) VecOf {
    T e[V];
};
// dst [rows_p][cols_p] = src [rows][cols] (row-major), zero elsewhere. With
// cols_p % V == 0 (and dst 16-byte aligned: workspace buffers are 256-byte
// aligned) each chunk is one 16-byte store; src rows of an odd width are
// read element by element.
template <typename T, int V>
__global__ __launch_bounds__(256) void pad_copy(const T* __restrict__ src, int64_t rows, int64_t cols,
                                                T* __restrict__ dst, int64_t rows_p, int64_t cols_p) {
    const Band b(cols_p / V);
    if (b.row_in_band >= b.rows_per_band) return;
    for (int64_t r = (int64_t)blockIdx.x * b.rows_per_band + b.row_in_band; r < rows_p;
         r += (int64_t)gridDim.x * b.rows_per_band) {
        for (int c = b.chunk0; c < b.chunks; c += b.chunk_step) {
            VecOf<T, V> v;
#pragma unroll
            for (int j = 0; j < V; ++j) {
                const int64_t col = (int64_t)c * V + j;
                v.e[j] = r < rows && col < cols ? src[r * cols + col] : T(0);
            }
            *reinterpret_cast<VecOf<T, V>*>(dst + r * cols_p + (int64_t)c * V) = v;
        }
    }
}
// dst [rows][cols] = the leading block of src [.][cols_p], element by element
// (dst rows of an odd width are not 16-byte chunks)
template <typename T>
__global__ __launch_bounds__(256) void unpad_copy(const T* __restrict__ src, int64_t cols_p, T* __restrict__ dst,
                                                  int64_t rows, int64_t cols) {
    const Band b(cols);
    if (b.row_in_band >= b.rows_per_band) return;
    for (int64_t r = (int64_t)blockIdx.x * b.rows_per_band + b.row_in_band; r < rows;
         r += (int64_t)gridDim.x * b.rows_per_band)
        for (int c = b.chunk0; c < b.chunks; c += b.chunk_step) dst[r * cols + c] = src[r * cols_p + c];
}
unsigned band_blocks(int64_t rows, int64_t chunks) {
    const int64_t rpb = chunks <= 256 ? 256 / std::max<int64_t>(chunks, 1) : 1;
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>((rows + rpb - 1) / rpb, 8192));
}
template <typename T>
hipError_t pad(const void* src, int64_t rows, int64_t cols, void* dst, int64_t rows_p, int64_t cols_p,
               hipStream_t st) {
    constexpr int V = 16 / (int)sizeof(T);
    const bool vec = cols_p % V == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0;
    if (vec)
        pad_copy<T, V><<<band_blocks(rows_p, cols_p / V), 256, 0, st>>>(static_cast<const T*>(src), rows, cols,
                                                                        static_cast<T*>(dst), rows_p, cols_p);
    else
        pad_copy<T, 1><<<band_blocks(rows_p, cols_p), 256, 0, st>>>(static_cast<const T*>(src), rows, cols,
                                                                    static_cast<T*>(dst), rows_p, cols_p);
    return hipGetLastError();
}
template <typename T>
hipError_t unpad(const void* src, int64_t cols_p, void* dst, int64_t rows, int64_t cols, hipStream_t st) {
    unpad_copy<T><<<band_blocks(rows, cols), 256, 0, st>>>(static_cast<const T*>(src), cols_p, static_cast<T*>(dst),
                                                           rows, cols);
    return hipGetLastError();
}
// Buffers of a padded call after the inner call's workspace (byte offsets):
// x [T][Kp], W [Np][Kp], bias [Np] (bf16), A [Kp][r], B [r][Np] (fp32), then
// the forward's y [T][Np], or the backward's dY [T][Np], dX [T][Kp] (bf16),
// dA [Kp][r], dB [r][Np] (fp32).
struct PadWs {
    size_t x, w, bias, a, b, y, dy, dx, da, db, total;
};
PadWs pad_ws(const mc_lora_desc& d, size_t inner, bool bwd) {
    const size_t T = (size_t)d.tokens, r = (size_t)d.rank;
    const size_t Kp = (size_t)round_up(d.in_features, 8), Np = (size_t)round_up(d.out_features, 8);
    PadWs w{};
    size_t off = align256(inner);
    w.x = off;    off += align256(T * Kp * 2);
    w.w = off;    off += align256(Np * Kp * 2);
    w.bias = off; off += align256(Np * 2);
    w.a = off;    off += align256(Kp * r * 4);
    w.b = off;    off += align256(r * Np * 4);
    if (!bwd) {
        w.y = off;  off += align256(T * Np * 2);
    } else {
        w.dy = off; off += align256(T * Np * 2);
        w.dx = off; off += align256(T * Kp * 2);
        w.da = off; off += align256(Kp * r * 4);
        w.db = off; off += align256(r * Np * 4);
    }
    w.total = off;
    return w;
}

}  // namespace

LoraFwdWs lora_fwd_ws(const mc_lora_desc& d) {
    if (bf16_padded(d)) {
        LoraFwdWs w{};
        w.total = pad_ws(d, lora_fwd_ws(padded_desc(d)).total, false).total;
        return w;
    }
    const Dims m = dims_of(d);
    LoraFwdWs w{};
    size_t off = 0;
    if (m.bf16) {  // the bf16 forward runs as a grouped forward of one projection
        const int64_t N = m.N;
        off = lora_group_fwd_ws(d, &N, 1).total;
    } else {
        w.hs_ext = off;  off += align256((size_t)m.T * m.r * 4);
    }
    w.hd_t = 0;
    w.total = off;
    return w;
}

LoraBwdWs lora_bwd_ws(const mc_lora_desc& d) {
    if (bf16_padded(d)) {
        LoraBwdWs w{};
        w.total = pad_ws(d, lora_bwd_ws(padded_desc(d)).total, true).total;
        return w;
    }
    const Dims m = dims_of(d);
    LoraBwdWs w{};
    size_t off = 0;
    if (m.bf16) {  // the bf16 backward runs as a grouped backward of one projection
        const int64_t N = m.N;
        const LoraGroupBwdWs g = lora_group_bwd_ws(d, &N, 1);
        w.wt = g.wt[0]; w.at_ext = g.at_ext; w.gd_ext = g.gd_ext; w.gd_t = g.gd_t;
        w.part_a = g.part_a; w.part_b = g.part_b[0];
        off = g.total;
    } else {
        w.gd_ext = off; off += align256((size_t)m.T * m.r * 4);
        w.gd_t = off;   off += align256((size_t)m.r * m.T * 4);
    }
    w.total = off;
    return w;
}

LoraGroupFwdWs lora_group_fwd_ws(const mc_lora_desc& d, const int64_t* N, int count) {
    const Dims m = dims_of(d);
    LoraGroupFwdWs w{};
    size_t off = 0;
    const int ppp = proj_per_pass(m.r);
    for (int p0 = 0, pass = 0; p0 < count; p0 += ppp, ++pass) {
        const int np = count - p0 < ppp ? count - p0 : ppp;
        w.at_hilo[pass] = off;  // hi then lo, row-major [16 rc][K] or in fragment order over round_up(K, 64)
        off += align256((size_t)2 * 16 * rowproj_rc(np * m.r) * round_up(m.K, 64) * 2);
    }
    for (int g = 0; g < count; ++g) {
        w.bt_ext[g] = off;
        off += align256((size_t)N[g] * m.rext * 2);
    }
    w.hs_ext = off; off += align256((size_t)m.T * count * m.rext * 2);
    w.part = off;
    if (fwd_rowsplit(m)) {
        const int npass = (count + ppp - 1) / ppp;
        const int ld = rowsplit_ld((count < ppp ? count : ppp) * m.r);
        off += align256((size_t)npass * rowsplit_splits(m.T, m.K) * m.T * ld * 4);
    }
    w.total = off;
    return w;
}

LoraGroupBwdWs lora_group_bwd_ws(const mc_lora_desc& d, const int64_t* N, int count, const bool* need_wt) {
    const Dims m = dims_of(d);
    LoraGroupBwdWs w{};
    size_t off = 0;
    for (int g = 0; g < count; ++g) {
        w.wt[g] = off;
        if (!need_wt || need_wt[g]) off += align256((size_t)m.K * N[g] * 2);
    }
    w.at_ext = off; off += align256((size_t)m.K * count * m.rext * 2);
    w.gd_ext = off; off += align256((size_t)m.T * count * m.rext * 2);
    w.gd_t = off;   off += align256((size_t)count * m.r * m.T * 4);  // or its bf16 hi / lo planes
    const bool cs = bwd_colsplit(m, N, count);
    w.hd_hilo = off;
    if (cs) off += align256((size_t)count * m.r * m.T * 4);
    w.part_a = off;
    off += align256((size_t)(cs ? colsplit_splits(m.T, m.K) : colreduce_splits(m.T, m.K)) *
                    colreduce_rows(count * m.r) * m.K * 4);
    const bool fused = dy_fused(m, N, count);
    for (int g = 0; g < count; ++g) {
        w.part_b[g] = off;
        const int sb = fused ? dy_splits(m.T, N[g]) : cs ? colsplit_splits(m.T, N[g]) : colreduce_splits(m.T, N[g]);
        off += align256((size_t)sb * colreduce_rows(m.r) * N[g] * 4);
    }
    const bool split = bwd_rowsplit(m, N, count);
    for (int g = 0; g < count; ++g) {
        w.gpart[g] = off;
        if (fused) off += align256((size_t)dy_groups(N[g]) * m.T * m.r * 4);
        if (split) off += align256((size_t)rowsplit_splits(m.T, N[g]) * m.T * rowsplit_ld(m.r) * 4);
    }
    w.total = off;
    return w;
}

hipError_t launch_lora_fwd(const mc_lora_desc& d, const void* x, const void* W, const void* bias,
                           const float* A, const float* B, const uint8_t* mask, void* y,
                           float* h_save, void* ws, hipStream_t st) {
    if (bf16_padded(d)) {
        const mc_lora_desc dp = padded_desc(d);
        const int64_t T = d.tokens, K = d.in_features, N = d.out_features, r = d.rank;
        const int64_t Kp = dp.in_features, Np = dp.out_features;
        const PadWs p = pad_ws(d, lora_fwd_ws(dp).total, false);
        char* base = static_cast<char*>(ws);
        MC_TRY(pad<uint16_t>(x, T, K, base + p.x, T, Kp, st));
        if (W) MC_TRY(pad<uint16_t>(W, N, K, base + p.w, Np, Kp, st));
        if (bias) MC_TRY(pad<uint16_t>(bias, 1, N, base + p.bias, 1, Np, st));
        MC_TRY(pad<float>(A, K, r, base + p.a, Kp, r, st));
        MC_TRY(pad<float>(B, r, N, base + p.b, r, Np, st));
        MC_TRY(launch_lora_fwd(dp, base + p.x, W ? base + p.w : nullptr, bias ? base + p.bias : nullptr,
                               reinterpret_cast<const float*>(base + p.a), reinterpret_cast<const float*>(base + p.b),
                               mask, base + p.y, h_save, ws, st));
        return unpad<uint16_t>(base + p.y, Np, y, T, N, st);
    }
    const Dims m = dims_of(d);
    const LoraFwdWs w = lora_fwd_ws(d);
    char* base = static_cast<char*>(ws);
    const float keep = mask ? 1.0f / (1.0f - d.dropout_p) : 1.0f;
    const int64_t kbase = W ? m.K : 0;
    if (m.bf16) {
        // one projection of the grouped forward (the same prep, row projection
        // and GEMM launches as a group of one)
        const LoraProj p{m.N, W, bias, A, B, mask};
        void* const ys[1] = {y};
        float* const hs[1] = {h_save};
        return launch_lora_group_fwd(d, x, &p, 1, ys, hs, ws, st);
    }
    float* hs = reinterpret_cast<float*>(base + w.hs_ext);
    const float* xf = static_cast<const float*>(x);
    {
        auto sc = lowrank_scope(st, m.T, m.K, m.r, 4);
        MC_TRY(launch_rowproj_f32(xf, m.T, m.K, A, true, m.r, 1.0f, mask, keep, h_save, hs, d.scale, st));
    }
    // y = x.W^T (+ b) + (s Hd).B: W [N][K] is read NT, B [r][N] as stored (NN)
    GemmSegF32 s0{xf, m.K, static_cast<const float*>(W), m.K, kbase};
    GemmSegF32 s1{hs, m.r, B, m.N, m.r};
    auto sc = gemm_scope(st, m.T, m.N, kbase, m.r, m.r, 4);
    return launch_gemm_f32(false, true, m.T, m.N, s0, s1, static_cast<const float*>(bias), static_cast<float*>(y),
                           m.N, st);
}

hipError_t launch_lora_bwd(const mc_lora_desc& d, const void* x, const void* W, const float* A,
                           const float* B, const uint8_t* mask, const float* h_save,
                           const void* dY, void* dX, float* dA, float* dB, void* ws,
                           hipStream_t st) {
    if (bf16_padded(d)) {
        const mc_lora_desc dp = padded_desc(d);
        const int64_t T = d.tokens, K = d.in_features, N = d.out_features, r = d.rank;
        const int64_t Kp = dp.in_features, Np = dp.out_features;
        const PadWs p = pad_ws(d, lora_bwd_ws(dp).total, true);
        char* base = static_cast<char*>(ws);
        if (x) MC_TRY(pad<uint16_t>(x, T, K, base + p.x, T, Kp, st));
        if (W) MC_TRY(pad<uint16_t>(W, N, K, base + p.w, Np, Kp, st));
        MC_TRY(pad<float>(A, K, r, base + p.a, Kp, r, st));
        MC_TRY(pad<float>(B, r, N, base + p.b, r, Np, st));
        MC_TRY(pad<uint16_t>(dY, T, N, base + p.dy, T, Np, st));
        MC_TRY(launch_lora_bwd(dp, x ? base + p.x : nullptr, W ? base + p.w : nullptr,
                               reinterpret_cast<const float*>(base + p.a), reinterpret_cast<const float*>(base + p.b),
                               mask, h_save, base + p.dy, dX ? base + p.dx : nullptr,
                               dA ? reinterpret_cast<float*>(base + p.da) : nullptr,
                               dB ? reinterpret_cast<float*>(base + p.db) : nullptr, ws, st));
        if (dX) MC_TRY(unpad<uint16_t>(base + p.dx, Kp, dX, T, K, st));
        if (dA) MC_TRY(unpad<float>(base + p.da, r, dA, K, r, st));
        if (dB) MC_TRY(unpad<float>(base + p.db, Np, dB, r, N, st));
        return hipSuccess;
    }
    const Dims m = dims_of(d);
    const float keep = mask ? 1.0f / (1.0f - d.dropout_p) : 1.0f;
    if (m.bf16) {
        // one projection of the grouped backward, with its own dX
        const LoraProj p{m.N, W, nullptr, A, B, mask};
        return launch_lora_group_bwd(d, x, &p, 1, &h_save, &dY, dX, &dA, &dB, ws, st);
    }
    const LoraBwdWs w = lora_bwd_ws(d);
    char* base = static_cast<char*>(ws);
    const bool need_g = dX || dA;
    const int64_t kbase = W ? m.N : 0;
    const float* dyf = static_cast<const float*>(dY);
    float* gd = reinterpret_cast<float*>(base + w.gd_ext);
    float* gdt = reinterpret_cast<float*>(base + w.gd_t);
    if (need_g) {
        auto sc = lowrank_scope(st, m.T, m.N, m.r, 4);
        MC_TRY(launch_rowproj_f32(dyf, m.T, m.N, B, false, m.r, d.scale, mask, keep, gdt, gd, 1.0f, st));
    }
    if (dX) {
        // dX = dY.W + Gd.A^T: W [N][K] is read as [k][K] (NN), A [K][r] as [K][k] (NT)
        GemmSegF32 s0{dyf, m.N, static_cast<const float*>(W), m.K, kbase};
        GemmSegF32 s1{gd, m.r, A, m.r, m.r};
        auto sc = gemm_scope(st, m.T, m.K, kbase, m.r, m.r, 4);
        MC_TRY(launch_gemm_f32(true, false, m.T, m.K, s0, s1, nullptr, static_cast<float*>(dX), m.K, st));
    }
    // dA = x^T.Gd and dB = s Hd^T.dY in one launch (one timed scope)
    ColF32Call cc[2];
    int nc = 0;
    if (dA) cc[nc++] = ColF32Call{static_cast<const float*>(x), m.K, gdt, 1.0f, true, dA};
    if (dB) cc[nc++] = ColF32Call{dyf, m.N, h_save, d.scale, false, dB};
    if (nc > 0) {
        auto sc = prof::Scope(prof::kLowRank, st, 2.0 * m.T * m.r * ((dA ? m.K : 0) + (dB ? m.N : 0)),
                              4.0 * m.T * ((dA ? m.K + m.r : 0) + (dB ? m.N + m.r : 0)));
        MC_TRY(launch_colreduce_f32(cc, nc, m.T, m.r, st));
    }
    return hipSuccess;
}

hipError_t launch_lora_group_fwd(const mc_lora_desc& d, const void* x, const LoraProj* proj, int count,
                                 void* const* y, float* const* h_save, void* ws, hipStream_t st) {
    // bf16 only. Per pass of up to proj_per_pass projections: one prep launch
    // (A^T hi / lo of the pass's projections; the B^T extension operands ride
    // with the first pass) and one row projection that reads x once for all
    // of their ranks; then one multi-output GEMM over every projection.
    const Dims m = dims_of(d);
    int64_t Ns[kMaxProj];
    for (int g = 0; g < count; ++g) Ns[g] = proj[g].N;
    const LoraGroupFwdWs w = lora_group_fwd_ws(d, Ns, count);
    char* base = static_cast<char*>(ws);
    const uint16_t* xb = static_cast<const uint16_t*>(x);
    uint16_t* hs = reinterpret_cast<uint16_t*>(base + w.hs_ext);
    const int ext_ld = count * m.rext;
    const int ppp = proj_per_pass(m.r);
    {
        int64_t sumN = 0;
        for (int g = 0; g < count; ++g) sumN += Ns[g];
        auto sc = prof::Scope(prof::kLowRank, st, 2.0 * m.T * m.K * m.r * count,
                              2.0 * m.T * m.K + 6.0 * m.T * m.r * count + 12.0 * m.r * (m.K + sumN / count) * count);
        const bool split = fwd_rowsplit(m);
        if (split) {
            // One prep launch for every pass (A^T hi / lo, B^T extension
            // operands), one split row projection whose passes share x (run
            // interleaved), one finishing launch: H of each projection from
            // its pass's partials -> h_save and the s Hd extension columns.
            const int npass = (count + ppp - 1) / ppp;
            const int rmax = (count < ppp ? count : ppp) * m.r;
            const int ld = rowsplit_ld(rmax);
            const int S = rowsplit_splits(m.T, m.K);
            float* part = reinterpret_cast<float*>(base + w.part);
            PrepJob jobs[3 * kMaxProj];
            RowsplitJob rj[kMaxProj];
            DyFinishJob fin[kMaxProj];
            int nj = 0;
            for (int p0 = 0, pass = 0; p0 < count; p0 += ppp, ++pass) {
                const int np = count - p0 < ppp ? count - p0 : ppp;
                const int rpass = np * m.r, r16 = 16 * rowproj_rc(rpass);
                uint16_t* at_hi = reinterpret_cast<uint16_t*>(base + w.at_hilo[pass]);
                uint16_t* at_lo = at_hi + (size_t)r16 * m.K;
                for (int i = 0; i < np; ++i)  // A_g^T hi / lo as rows [i r, (i + 1) r) of the pass's operand
                    jobs[nj++] = prep_job(proj[p0 + i].A, m.r, m.r, m.K, true, at_hi + (size_t)i * m.r * m.K,
                                          at_lo + (size_t)i * m.r * m.K, m.r, m.K);
                if (r16 > rpass)  // zero rows past the pass's ranks
                    jobs[nj++] = prep_job(proj[p0].A, 0, 0, 0, false, at_hi + (size_t)rpass * m.K,
                                          at_lo + (size_t)rpass * m.K, r16 - rpass, m.K);
                float* pp = part + (size_t)pass * S * m.T * ld;
                rj[pass] = RowsplitJob{xb, m.K, at_hi, at_lo, nullptr, r16, pp, S};
                for (int i = 0; i < np; ++i) {
                    const int g = p0 + i;
                    fin[g] = DyFinishJob{pp + (size_t)i * m.r, S, proj[g].mask, h_save ? h_save[g] : nullptr,
                                         hs + (size_t)g * m.rext, ld, m.r};
                }
            }
            for (int g = 0; g < count; ++g)  // B_g^T, zero-padded to rext columns
                jobs[nj++] = prep_job(proj[g].B, Ns[g], Ns[g], m.r, true, reinterpret_cast<uint16_t*>(base + w.bt_ext[g]),
                                      nullptr, Ns[g], m.rext);
            MC_TRY(prep_all(jobs, nj, st));
            MC_TRY(launch_rowsplit(m.T, rmax, rj, npass, st));
            MC_TRY(launch_dy_finish(m.T, m.r, 1.0f, proj[0].mask ? 1.0f / (1.0f - d.dropout_p) : 1.0f, m.rext, ext_ld,
                                    d.scale, fin, count, nullptr, 0, st));
        }
        for (int p0 = 0, pass = 0; p0 < count && !split; p0 += ppp, ++pass) {
            const int np = count - p0 < ppp ? count - p0 : ppp;
            // A pass holds whole projections; a projection of more than
            // kRowprojMaxRanks ranks (alone in its pass) takes its ranks in
            // chunks [j0, j0 + rc), one pass over x each.
            for (int j0 = 0; j0 < m.r; j0 += kRowprojMaxRanks) {
                const int rc = np > 1 || m.r <= kRowprojMaxRanks ? m.r : std::min(kRowprojMaxRanks, m.r - j0);
                const bool last = j0 + rc == m.r;
                const int rpass = np * rc, RC = rowproj_rc(rpass), r16 = 16 * RC;
                uint16_t* at_hi = reinterpret_cast<uint16_t*>(base + w.at_hilo[pass]);
                uint16_t* at_lo = at_hi + (size_t)r16 * round_up(m.K, 64);
                PrepJob jobs[2 * kMaxProj + 1];
                int nj = 0;
                // the operand in the row projection's fragment order: A_g^T hi / lo
                // (ranks j0 ..) as rows [i rc, (i + 1) rc), zero rows past the pass's ranks
                for (int i = 0; i < np; ++i) {
                    jobs[nj] = prep_job(proj[p0 + i].A + j0, m.r, rc, m.K, true, at_hi, at_lo, rc, m.K);
                    jobs[nj].frag_rc = RC;
                    jobs[nj++].frag_row0 = (int64_t)i * rc;
                }
                if (r16 > rpass) {
                    jobs[nj] = prep_job(proj[p0].A, 0, 0, 0, false, at_hi, at_lo, r16 - rpass, m.K);
                    jobs[nj].frag_rc = RC;
                    jobs[nj++].frag_row0 = rpass;
                }
                if (pass == 0 && j0 == 0)
                    for (int g = 0; g < count; ++g)  // B_g^T, zero-padded to rext columns
                        jobs[nj++] = prep_job(proj[g].B, Ns[g], Ns[g], m.r, true,
                                              reinterpret_cast<uint16_t*>(base + w.bt_ext[g]), nullptr, Ns[g], m.rext);
                MC_TRY(prep_all(jobs, nj, st));
                RowprojCall c{};
                c.X = xb; c.T = m.T; c.C = m.K; c.P_hi = at_hi; c.P_lo = at_lo; c.r = rpass; c.rp = rc;
                c.scale = 1.0f; c.keep = proj[p0].mask ? 1.0f / (1.0f - d.dropout_p) : 1.0f;
                c.mask_ld = m.r;
                for (int i = 0; i < np; ++i) {
                    c.mask[i] = proj[p0 + i].mask ? proj[p0 + i].mask + j0 : nullptr;
                    c.out_t[i] = h_save && h_save[p0 + i] ? h_save[p0 + i] + (size_t)j0 * m.T : nullptr;
                }
                // projection p0 + i's columns start at i rext (+ j0); the last
                // chunk zeroes the pad columns up to rext
                c.out_ext = hs + (size_t)p0 * m.rext + j0;
                c.rext_p = last ? rc + (m.rext - m.r) : rc;
                c.ext_ld = ext_ld; c.ext_scale = d.scale;
                MC_TRY(launch_rowproj_bf16(c, st));
                if (last) break;
            }
        }
    }
    GemmOut outs[kMaxProj];
    double flops[kMaxProj], bytes[kMaxProj];
    for (int g = 0; g < count; ++g) {
        const int64_t kbase = proj[g].W ? m.K : 0;
        outs[g].N = Ns[g];
        outs[g].seg[0] = GemmSeg{xb, m.K, static_cast<const uint16_t*>(proj[g].W), m.K, kbase};
        outs[g].seg[1] = GemmSeg{hs + (size_t)g * m.rext, ext_ld, reinterpret_cast<const uint16_t*>(base + w.bt_ext[g]),
                                 m.rext, m.rext};
        outs[g].nseg = 2;
        outs[g].bias = static_cast<const uint16_t*>(proj[g].bias);
        outs[g].c = static_cast<uint16_t*>(y[g]);
        outs[g].ldc = Ns[g];
        flops[g] = 2.0 * m.T * Ns[g] * (kbase > 0 ? kbase : m.r);
        bytes[g] = 2.0 * (Ns[g] * (double)(kbase + m.rext) + (double)m.T * Ns[g] + (double)m.T * m.rext);
    }
    if (gemm_bf16_multi_one_launch(m.T, outs, count)) {
        double f = 0, b = 2.0 * m.T * m.K;  // x, read once by the whole grid
        for (int g = 0; g < count; ++g) { f += flops[g]; b += bytes[g]; }
        auto sc = prof::Scope(prof::kGemm, st, f, b);
        return launch_gemm_bf16_multi(m.T, outs, count, st);
    }
    for (int g = 0; g < count; ++g) {  // one launch (and one timed scope) per projection
        auto sc = prof::Scope(prof::kGemm, st, flops[g], bytes[g] + 2.0 * m.T * m.K);
        MC_TRY(launch_gemm_bf16(m.T, Ns[g], outs[g].seg, outs[g].nseg, outs[g].bias, outs[g].c, outs[g].ldc, st));
    }
    return hipSuccess;
}

hipError_t launch_lora_group_bwd(const mc_lora_desc& d, const void* x, const LoraProj* proj, int count,
                                 const float* const* h_save, const void* const* dY, void* dX, float* const* dA,
                                 float* const* dB, void* ws, hipStream_t st) {
    // bf16 only. One operand launch for every projection (G_g = s dY_g.B_g^T,
    // the A_g extension columns, W_g -> W_g^T), one dX GEMM whose reduction
    // runs over [dY_0 | .. | dY_{G-1} | Gd_0 .. Gd_{G-1}] (the sum of the
    // projections' input gradients), one column-reduction launch per rank-tile
    // size (dA of every projection from one pass over x; dB_g over dY_g) and
    // one fixed-order split-sum launch.
    const Dims m = dims_of(d);
    int64_t Ns[kMaxProj];
    bool need_wt[kMaxProj];
    for (int g = 0; g < count; ++g) {
        Ns[g] = proj[g].N;
        need_wt[g] = proj[g].W && !proj[g].Wt;
    }
    const LoraGroupBwdWs w = lora_group_bwd_ws(d, Ns, count, need_wt);
    char* base = static_cast<char*>(ws);
    const float keep = proj[0].mask ? 1.0f / (1.0f - d.dropout_p) : 1.0f;
    bool any_dA = false, any_dB = false;
    for (int g = 0; g < count; ++g) {
        any_dA = any_dA || (dA && dA[g]);
        any_dB = any_dB || (dB && dB[g]);
    }
    const bool need_g = dX || any_dA;
    const int ext_ld = count * m.rext;
    const int rtot = count * m.r;
    uint16_t* at = reinterpret_cast<uint16_t*>(base + w.at_ext);
    uint16_t* gd = reinterpret_cast<uint16_t*>(base + w.gd_ext);
    float* gdt = reinterpret_cast<float*>(base + w.gd_t);
    // the column-split path: Gd^T as bf16 hi / lo planes [G r][T] in the
    // Gd^T region, Hd_g^T planes [r][T] per projection from h_save
    const bool cs = bwd_colsplit(m, Ns, count);
    uint16_t* gd_hi = reinterpret_cast<uint16_t*>(base + w.gd_t);
    uint16_t* gd_lo = gd_hi + (size_t)count * m.r * m.T;
    uint16_t* hd_hi = reinterpret_cast<uint16_t*>(base + w.hd_hilo);
    uint16_t* hd_lo = hd_hi + (size_t)count * m.r * m.T;
    auto hd_preps = [&](PrepJob* out) {
        int n = 0;
        for (int g = 0; g < count; ++g)
            if (dB && dB[g])
                out[n++] = prep_job(h_save[g], m.T, m.r, m.T, false, hd_hi + (size_t)g * m.r * m.T,
                                    hd_lo + (size_t)g * m.r * m.T, m.r, m.T);
        return n;
    };
    if (dy_fused(m, Ns, count)) {
        // One read of each dY_g for both of its rank-r products (G_g and the
        // dB_g partials), the G partials finished into Gd (with the A
        // extension operands), then the dX GEMM, dA from one pass over x,
        // and the fixed-order split sums.
        if (need_g || any_dB) {
            DyJob jobs[kMaxProj];
            DyFinishJob fin[kMaxProj];
            PrepJob preps[kMaxProj];
            double bytes = 0, flops = 0;
            for (int g = 0; g < count; ++g) {
                const bool wb = dB && dB[g];
                jobs[g] = DyJob{static_cast<const uint16_t*>(dY[g]), Ns[g], proj[g].B, wb ? h_save[g] : nullptr,
                                wb ? reinterpret_cast<float*>(base + w.part_b[g]) : nullptr,
                                need_g ? reinterpret_cast<float*>(base + w.gpart[g]) : nullptr};
                fin[g] = DyFinishJob{reinterpret_cast<const float*>(base + w.gpart[g]), dy_groups(Ns[g]), proj[g].mask,
                                     any_dA ? gdt + (size_t)g * m.r * m.T : nullptr,
                                     dX ? gd + (size_t)g * m.rext : nullptr};
                preps[g] = dX ? prep_job(proj[g].A, m.r, m.K, m.r, false, at + (size_t)g * m.rext, nullptr, m.K, m.rext,
                                         ext_ld)
                              : PrepJob{};
                // algorithmic: dY_g read once, B_g read, Hd_g read (for dB),
                // Gd_g written (fp32 and bf16), A_g read
                bytes += 2.0 * m.T * Ns[g] + 4.0 * m.r * Ns[g] + (wb ? 4.0 * m.T * m.r : 0.0) +
                         (need_g ? 6.0 * m.T * m.r : 0.0) + (dX ? 6.0 * m.r * m.K : 0.0);
                flops += 2.0 * m.T * Ns[g] * m.r * ((need_g ? 1 : 0) + (wb ? 1 : 0));
            }
            auto sc = prof::Scope(prof::kLowRank, st, flops, bytes);
            MC_TRY(launch_dy_pass(m.T, m.r, jobs, count, st));
            if (need_g)
                MC_TRY(launch_dy_finish(m.T, m.r, d.scale, keep, m.rext, ext_ld, 1.0f, fin, count, preps, count, st));
        }
        if (any_dA || any_dB) {
            // dA_g = x^T.Gd_g for every g from one pass over x (all ranks),
            // then the fixed-order split sums of dA and dB
            SumJob sj[2 * kMaxProj];
            int ns = 0;
            const int sa = colreduce_splits(m.T, m.K);
            float* pa = reinterpret_cast<float*>(base + w.part_a);
            auto sc = prof::Scope(prof::kLowRank, st, any_dA ? 2.0 * m.T * m.K * rtot : 0.0,
                                  any_dA ? 2.0 * m.T * m.K + 4.0 * m.T * rtot : 0.0);
            if (any_dA) {
                const ColJob cj{static_cast<const uint16_t*>(x), m.K, gdt, rtot, sa, pa};
                MC_TRY(launch_colreduce_bf16(m.T, &cj, 1, st));
                for (int g = 0; g < count; ++g)
                    if (dA[g])
                        sj[ns++] = SumJob{pa + (size_t)g * m.r * m.K, sa, m.K, (int64_t)colreduce_rows(rtot) * m.K, m.r,
                                          1.0f, true, dA[g]};
            }
            for (int g = 0; g < count; ++g)
                if (dB && dB[g])
                    sj[ns++] = SumJob{reinterpret_cast<float*>(base + w.part_b[g]), dy_splits(m.T, Ns[g]), Ns[g],
                                      (int64_t)colreduce_rows(m.r) * Ns[g], m.r, d.scale, false, dB[g]};
            MC_TRY(launch_split_sum(sj, ns, st));
        }
        if (dX) {
            for (int g = 0; g < count; ++g)
                if (need_wt[g])  // W^T into the workspace (none when the caller holds it)
                    MC_TRY(launch_transpose_bf16(proj[g].W, Ns[g], m.K, base + w.wt[g], st));
            GemmSeg segs[kGemmMaxSeg];
            int nseg = 0;
            int64_t kbase = 0;
            for (int g = 0; g < count; ++g)
                if (proj[g].W) {
                    const uint16_t* wt = proj[g].Wt ? static_cast<const uint16_t*>(proj[g].Wt)
                                                    : reinterpret_cast<const uint16_t*>(base + w.wt[g]);
                    segs[nseg++] = GemmSeg{static_cast<const uint16_t*>(dY[g]), Ns[g], wt, Ns[g], Ns[g]};
                    kbase += Ns[g];
                }
            segs[nseg++] = GemmSeg{gd, ext_ld, at, ext_ld, ext_ld};
            auto sc = gemm_scope(st, m.T, m.K, kbase, ext_ld, rtot, 2);
            MC_TRY(launch_gemm_bf16(m.T, m.K, segs, nseg, nullptr, static_cast<uint16_t*>(dX), m.K, st));
        }
        return hipSuccess;
    }
    if (need_g) {
        double bytes = 0, flops = 0;
        for (int g = 0; g < count; ++g) {
            // algorithmic: dY_g read, G_g written (fp32 and bf16), B_g and A_g read;
            // the W^T copy is workspace traffic, not counted
            bytes += 2.0 * m.T * Ns[g] + 6.0 * m.T * m.r + 4.0 * m.r * Ns[g] + (dX ? 6.0 * m.r * m.K : 0.0);
            flops += 2.0 * m.T * Ns[g] * m.r;
        }
        auto sc = prof::Scope(prof::kLowRank, st, flops, bytes);
        const bool split = bwd_rowsplit(m, Ns, count);
        if (split) {
            // G_g = s dY_g.B_g^T for every g in one split launch (B_g read as
            // fp32), finished with the mask into Gd^T (fp32, or the bf16 hi /
            // lo planes of the column split) and Gd, together with the A
            // extension operands and the Hd^T planes; W^T (when the caller
            // holds none) by the transpose kernel
            const int ld = rowsplit_ld(m.r);
            RowsplitJob rj[kMaxProj];
            DyFinishJob fin[kMaxProj];
            PrepJob preps[2 * kMaxProj];
            int np = 0;
            for (int g = 0; g < count; ++g) {
                const int S = rowsplit_splits(m.T, Ns[g]);
                float* pp = reinterpret_cast<float*>(base + w.gpart[g]);
                rj[g] = RowsplitJob{static_cast<const uint16_t*>(dY[g]), Ns[g], nullptr, nullptr, proj[g].B, m.r, pp, S};
                fin[g] = DyFinishJob{pp, S, proj[g].mask, any_dA && !cs ? gdt + (size_t)g * m.r * m.T : nullptr,
                                     dX ? gd + (size_t)g * m.rext : nullptr, ld, m.r};
                if (any_dA && cs) {
                    fin[g].gd_hi = gd_hi + (size_t)g * m.r * m.T;
                    fin[g].gd_lo = gd_lo + (size_t)g * m.r * m.T;
                }
                if (dX)
                    preps[np++] = prep_job(proj[g].A, m.r, m.K, m.r, false, at + (size_t)g * m.rext, nullptr, m.K,
                                           m.rext, ext_ld);
            }
            if (cs) np += hd_preps(preps + np);
            MC_TRY(launch_rowsplit(m.T, m.r, rj, count, st));
            MC_TRY(launch_dy_finish(m.T, m.r, d.scale, keep, m.rext, ext_ld, 1.0f, fin, count, preps, np, st));
            if (dX)
                for (int g = 0; g < count; ++g)
                    if (need_wt[g]) MC_TRY(launch_transpose_bf16(proj[g].W, Ns[g], m.K, base + w.wt[g], st));
        }
        // ranks in chunks of at most kRowprojMaxRanks (one pass over dY each);
        // the A extension and the W transposes ride with the first
        for (int j0 = 0; j0 < m.r && !split; j0 += kRowprojMaxRanks) {
            const int rc = std::min(kRowprojMaxRanks, m.r - j0);
            const bool first = j0 == 0, last = j0 + rc == m.r;
            OperandsCall calls[kMaxProj];
            for (int g = 0; g < count; ++g) {
                const bool tw = dX && need_wt[g] && first;  // W^T into the workspace (none when the caller holds it)
                calls[g] = OperandsCall{static_cast<const uint16_t*>(dY[g]), Ns[g], proj[g].B + (size_t)j0 * Ns[g],
                                        proj[g].mask ? proj[g].mask + j0 : nullptr, (int64_t)m.r,
                                        any_dA ? gdt + (size_t)g * m.r * m.T + (size_t)j0 * m.T : nullptr,
                                        dX ? gd + (size_t)g * m.rext + j0 : nullptr,
                                        dX && first ? prep_job(proj[g].A, m.r, m.K, m.r, false, at + (size_t)g * m.rext,
                                                               nullptr, m.K, m.rext, ext_ld)
                                                    : PrepJob{},
                                        static_cast<const uint16_t*>(proj[g].W),
                                        tw ? reinterpret_cast<uint16_t*>(base + w.wt[g]) : nullptr};
            }
            MC_TRY(launch_lora_bwd_operands(calls, count, m.T, m.K, rc, d.scale, keep,
                                            last ? rc + (m.rext - m.r) : rc, ext_ld, st));
        }
    }
    if ((any_dA || any_dB) && cs) {
        // the column reductions over the bf16 planes (one pass over x for
        // every projection's dA, one over each dY_g for dB_g), then the
        // fixed-order split sums
        if (!need_g) {  // no finishing launch carried the Hd^T planes
            PrepJob preps[kMaxProj];
            MC_TRY(prep_all(preps, hd_preps(preps), st));
        }
        ColsplitJob cj[1 + kMaxProj];
        SumJob sj[2 * kMaxProj];
        int nc = 0, ns = 0;
        double bytes = 0, flops = 0;
        const int sa = colsplit_splits(m.T, m.K);
        float* pa = reinterpret_cast<float*>(base + w.part_a);
        if (any_dA) {
            cj[nc++] = ColsplitJob{static_cast<const uint16_t*>(x), m.K, gd_hi, gd_lo, rtot, sa, pa};
            bytes += 2.0 * m.T * m.K + 4.0 * m.T * rtot;
            flops += 2.0 * m.T * m.K * rtot;
            for (int g = 0; g < count; ++g)
                if (dA[g])
                    sj[ns++] = SumJob{pa + (size_t)g * m.r * m.K, sa, m.K, (int64_t)colreduce_rows(rtot) * m.K, m.r,
                                      1.0f, true, dA[g]};
        }
        for (int g = 0; g < count; ++g) {
            if (!(dB && dB[g])) continue;
            const int sb = colsplit_splits(m.T, Ns[g]);
            float* pb = reinterpret_cast<float*>(base + w.part_b[g]);
            cj[nc++] = ColsplitJob{static_cast<const uint16_t*>(dY[g]), Ns[g], hd_hi + (size_t)g * m.r * m.T,
                                   hd_lo + (size_t)g * m.r * m.T, m.r, sb, pb};
            sj[ns++] = SumJob{pb, sb, Ns[g], (int64_t)colreduce_rows(m.r) * Ns[g], m.r, d.scale, false, dB[g]};
            bytes += 2.0 * m.T * Ns[g] + 4.0 * m.T * m.r;
            flops += 2.0 * m.T * Ns[g] * m.r;
        }
        auto sc = prof::Scope(prof::kLowRank, st, flops, bytes);
        MC_TRY(launch_colsplit_bf16(m.T, cj, nc, st));
        MC_TRY(launch_split_sum(sj, ns, st));
    } else if (any_dA || any_dB) {
        // dA_g = x^T.Gd_g for every g from one pass over x (all ranks), and
        // dB_g = s Hd_g^T.dY_g: split-T column reductions, then the fixed-order
        // split sums
        ColJob cj[1 + kMaxProj];
        SumJob sj[2 * kMaxProj];
        int nc = 0, ns = 0;
        double bytes = 0, flops = 0;
        const int sa = colreduce_splits(m.T, m.K);
        float* pa = reinterpret_cast<float*>(base + w.part_a);
        if (any_dA) {
            cj[nc++] = ColJob{static_cast<const uint16_t*>(x), m.K, gdt, rtot, sa, pa};
            bytes += 2.0 * m.T * m.K + 4.0 * m.T * rtot;
            flops += 2.0 * m.T * m.K * rtot;
            for (int g = 0; g < count; ++g)
                if (dA[g])
                    sj[ns++] = SumJob{pa + (size_t)g * m.r * m.K, sa, m.K, (int64_t)colreduce_rows(rtot) * m.K, m.r,
                                      1.0f, true, dA[g]};
        }
        for (int g = 0; g < count; ++g) {
            if (!(dB && dB[g])) continue;
            const int sb = colreduce_splits(m.T, Ns[g]);
            float* pb = reinterpret_cast<float*>(base + w.part_b[g]);
            cj[nc++] = ColJob{static_cast<const uint16_t*>(dY[g]), Ns[g], h_save[g], m.r, sb, pb};
            sj[ns++] = SumJob{pb, sb, Ns[g], (int64_t)colreduce_rows(m.r) * Ns[g], m.r, d.scale, false, dB[g]};
            bytes += 2.0 * m.T * Ns[g] + 4.0 * m.T * m.r;
            flops += 2.0 * m.T * Ns[g] * m.r;
        }
        auto sc = prof::Scope(prof::kLowRank, st, flops, bytes);
        MC_TRY(launch_colreduce_bf16(m.T, cj, nc, st));
        MC_TRY(launch_split_sum(sj, ns, st));
    }
    if (dX) {
        GemmSeg segs[kGemmMaxSeg];
        int nseg = 0;
        int64_t kbase = 0;
        for (int g = 0; g < count; ++g)
            if (proj[g].W) {
                const uint16_t* wt = proj[g].Wt ? static_cast<const uint16_t*>(proj[g].Wt)
                                                : reinterpret_cast<const uint16_t*>(base + w.wt[g]);
                segs[nseg++] = GemmSeg{static_cast<const uint16_t*>(dY[g]), Ns[g], wt, Ns[g], Ns[g]};
                kbase += Ns[g];
            }
        segs[nseg++] = GemmSeg{gd, ext_ld, at, ext_ld, ext_ld};
        auto sc = gemm_scope(st, m.T, m.K, kbase, ext_ld, rtot, 2);
        MC_TRY(launch_gemm_bf16(m.T, m.K, segs, nseg, nullptr, static_cast<uint16_t*>(dX), m.K, st));
    }
    return hipSuccess;
}

}  // namespace mc
