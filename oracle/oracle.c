/*
 * CPU oracle (test infrastructure only; never linked into the product).
 * Every function restates a reference composite; see oracle.h for the
 * reference file:line each one follows and the checks that pin it.
 *
 * Accumulation is fp64 in the order of the composite's ops; results are
 * stored as fp32. OpenMP parallelises over independent rows/columns only,
 * so results do not depend on the thread count.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int nthreads(int threads) {
#ifdef _OPENMP
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

/* ---------------------------------------------------------------- Philox */
/* Philox4x32-10, Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
 * easy as 1, 2, 3", SC'11: round multipliers 0xD2511F53 / 0xCD9E8D57, Weyl
 * key increments 0x9E3779B9 / 0xBB67AE85. */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c1 ^ k0;
        uint32_t n2 = hi0 ^ c3 ^ k1;
        c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

void oracle_dropout_mask(uint64_t seed, float p, int64_t rows, int32_t rank, uint8_t* mask) {
    const int64_t n = rows * (int64_t)rank;
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    for (int64_t blk = 0; blk * 4 < n; ++blk) {
        uint32_t ctr[4] = {(uint32_t)blk, (uint32_t)((uint64_t)blk >> 32), 0u, 0u};
        uint32_t w[4];
        oracle_philox4x32_10(ctr, key, w);
        for (int q = 0; q < 4 && blk * 4 + q < n; ++q) {
            float u = (float)(w[q] >> 8) * (1.0f / 16777216.0f);
            mask[blk * 4 + q] = (uint8_t)(u >= p);
        }
    }
}

/* ------------------------------------------------------------------ LoRA */
/* Dropout scale as candle-nn computes it: kept values times 1/(1-p) in fp32. */
static float keep_scale(float p) { return 1.0f / (1.0f - p); }

/* Row blocks of the LoRA loops: a block of token rows shares each pass over a
 * row of W (or B^T), which keeps W in cache across the block. */
#define ORACLE_ROWS 8

/* acc[j] = sum_k xr[k] * A[k*r + j] for j < r, each sum over ascending k (the
 * j loop is innermost so that the r independent sums vectorise; every sum
 * still sees the same sequence of fp64 operations). */
static void rank_proj(const float* xr, int64_t K, const float* A, int32_t r, double* acc) {
    for (int32_t j = 0; j < r; ++j) acc[j] = 0.0;
    for (int64_t k = 0; k < K; ++k) {
        const double xv = (double)xr[k];
        const float* ar = A + k * r;
        for (int32_t j = 0; j < r; ++j) acc[j] += xv * (double)ar[j];
    }
}

void oracle_lora_fwd(int64_t T, int64_t K, int64_t N, int32_t r, float scale, float p,
                     const float* x, const float* W, const float* bias,
                     const float* A, const float* B, const uint8_t* mask,
                     float* y, float* hd_out, int threads) {
    const float ks = mask ? keep_scale(p) : 1.0f;
    const int64_t nblk = (T + ORACLE_ROWS - 1) / ORACLE_ROWS;
#pragma omp parallel for schedule(dynamic) num_threads(nthreads(threads))
    for (int64_t blk = 0; blk < nblk; ++blk) {
        const int64_t t0 = blk * ORACLE_ROWS;
        const int64_t nt = T - t0 < ORACLE_ROWS ? T - t0 : ORACLE_ROWS;
        double* h = (double*)malloc(sizeof(double) * (size_t)(ORACLE_ROWS * r));
        double* acc = (double*)malloc(sizeof(double) * (size_t)r);
        for (int64_t i = 0; i < nt; ++i) {
            const int64_t t = t0 + i;
            /* lora.rs:323  hidden = input.broadcast_matmul(A) */
            rank_proj(x + t * K, K, A, r, acc);
            for (int32_t j = 0; j < r; ++j) {
                /* fp32 storage of the matmul result, as candle keeps it */
                float hf = (float)acc[j];
                /* lora.rs:326-330  dropout on the rank-r hidden */
                if (mask) hf = mask[t * r + j] ? hf * ks : 0.0f;
                h[i * r + j] = hf;
                if (hd_out) hd_out[t * r + j] = hf;
            }
        }
        for (int64_t n = 0; n < N; ++n) {
            /* candle_nn::Linear: x . W^T (+ b); one sum per row of the block,
             * each over ascending k */
            double base[ORACLE_ROWS] = {0};
            if (W) {
                const float* wr = W + n * K;
                for (int64_t k = 0; k < K; ++k) {
                    const double wv = (double)wr[k];
                    for (int64_t i = 0; i < nt; ++i) base[i] += (double)x[(t0 + i) * K + k] * wv;
                }
            }
            for (int64_t i = 0; i < nt; ++i) {
                /* lora.rs:336-339  (hidden . B) then affine(scale) */
                double d = 0.0;
                for (int32_t j = 0; j < r; ++j) d += h[i * r + j] * (double)B[(int64_t)j * N + n];
                double out = (double)scale * d;
                if (W) {
                    out += base[i];
                    if (bias) out += (double)bias[n];
                }
                y[(t0 + i) * N + n] = (float)out;
            }
        }
        free(acc);
        free(h);
    }
}

void oracle_lora_bwd(int64_t T, int64_t K, int64_t N, int32_t r, float scale, float p,
                     const float* x, const float* W, const float* A, const float* B,
                     const uint8_t* mask, const float* dy,
                     float* dx, float* dA, float* dB, int threads) {
    const float ks = mask ? keep_scale(p) : 1.0f;
    const int nt = nthreads(threads);
    /* Hd (forward hidden after dropout) and Gd (gradient of the hidden). */
    double* hd = (double*)malloc(sizeof(double) * (size_t)(T * r));
    double* gd = (double*)malloc(sizeof(double) * (size_t)(T * r));
    /* B^T [N][r], so that the r sums of G = dY.B^T run side by side */
    float* bt = (float*)malloc(sizeof(float) * (size_t)(N * r));
    for (int32_t j = 0; j < r; ++j)
        for (int64_t n = 0; n < N; ++n) bt[n * r + j] = B[(int64_t)j * N + n];
#pragma omp parallel num_threads(nt)
    {
        double* hacc = (double*)malloc(sizeof(double) * (size_t)r);
        double* gacc = (double*)malloc(sizeof(double) * (size_t)r);
#pragma omp for schedule(static)
        for (int64_t t = 0; t < T; ++t) {
            rank_proj(x + t * K, K, A, r, hacc);
            rank_proj(dy + t * N, N, bt, r, gacc);
            for (int32_t j = 0; j < r; ++j) {
                double g = gacc[j] * (double)scale;
                float hf = (float)hacc[j];
                if (mask) {
                    int keep = mask[t * r + j];
                    hf = keep ? hf * ks : 0.0f;
                    g = keep ? g * (double)ks : 0.0;
                }
                hd[t * r + j] = (double)hf;
                gd[t * r + j] = g;
            }
        }
        free(gacc);
        free(hacc);
    }
    free(bt);
    if (dx) {
        /* dx[t][k] = sum_n dy[t][n] W[n][k] (ascending n), then + sum_j
         * gd[t][j] A[k][j] (ascending j); rows of W are read contiguously */
        const int64_t nblk = (T + ORACLE_ROWS - 1) / ORACLE_ROWS;
#pragma omp parallel for schedule(dynamic) num_threads(nt)
        for (int64_t blk = 0; blk < nblk; ++blk) {
            const int64_t t0 = blk * ORACLE_ROWS;
            const int64_t nr = T - t0 < ORACLE_ROWS ? T - t0 : ORACLE_ROWS;
            double* acc = (double*)calloc((size_t)(ORACLE_ROWS * K), sizeof(double));
            if (W)
                for (int64_t n = 0; n < N; ++n) {
                    const float* wr = W + n * K;
                    for (int64_t i = 0; i < nr; ++i) {
                        const double dv = (double)dy[(t0 + i) * N + n];
                        double* ai = acc + i * K;
                        for (int64_t k = 0; k < K; ++k) ai[k] += dv * (double)wr[k];
                    }
                }
            for (int64_t i = 0; i < nr; ++i) {
                const int64_t t = t0 + i;
                for (int64_t k = 0; k < K; ++k) {
                    double a = acc[i * K + k];
                    for (int32_t j = 0; j < r; ++j) a += gd[t * r + j] * (double)A[k * r + j];
                    dx[t * K + k] = (float)a;
                }
            }
            free(acc);
        }
    }
    /* dA[k][j] = sum_t x[t][k] gd[t][j] and dB[j][n] = s sum_t hd[t][j] dy[t][n]:
     * columns are processed in blocks of 64 so x / dy rows are read
     * contiguously; each sum still runs over t in ascending order. */
    if (dA) {
#pragma omp parallel for schedule(dynamic) num_threads(nt)
        for (int64_t k0 = 0; k0 < K; k0 += 64) {
            const int64_t kn = K - k0 < 64 ? K - k0 : 64;
            double* acc = (double*)calloc((size_t)(kn * r), sizeof(double));
            for (int64_t t = 0; t < T; ++t)
                for (int64_t k = 0; k < kn; ++k) {
                    const double xv = (double)x[t * K + k0 + k];
                    for (int32_t j = 0; j < r; ++j) acc[k * r + j] += xv * gd[t * r + j];
                }
            for (int64_t k = 0; k < kn; ++k)
                for (int32_t j = 0; j < r; ++j) dA[(k0 + k) * r + j] = (float)acc[k * r + j];
            free(acc);
        }
    }
    if (dB) {
#pragma omp parallel for schedule(dynamic) num_threads(nt)
        for (int64_t n0 = 0; n0 < N; n0 += 64) {
            const int64_t nn = N - n0 < 64 ? N - n0 : 64;
            double* acc = (double*)calloc((size_t)(nn * r), sizeof(double));
            for (int64_t t = 0; t < T; ++t)
                for (int64_t n = 0; n < nn; ++n) {
                    const double gv = (double)dy[t * N + n0 + n];
                    for (int32_t j = 0; j < r; ++j) acc[n * r + j] += hd[t * r + j] * gv;
                }
            for (int64_t n = 0; n < nn; ++n)
                for (int32_t j = 0; j < r; ++j)
                    dB[(int64_t)j * N + n0 + n] = (float)((double)scale * acc[n * r + j]);
            free(acc);
        }
    }
    free(hd);
    free(gd);
}

/* --------------------------------------------------------------- RMSNorm */
void oracle_rmsnorm_fwd(int64_t rows, int64_t D, float eps, const float* x, const float* w,
                        float* y, float* rstd_out, int threads) {
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (int64_t i = 0; i < rows; ++i) {
        const float* xr = x + i * D;
        /* tensor.rs:113-115  sqr -> mean_keepdim -> (+eps) -> sqrt */
        double ss = 0.0;
        for (int64_t j = 0; j < D; ++j) ss += (double)xr[j] * (double)xr[j];
        double rms = sqrt(ss / (double)D + (double)eps);
        if (rstd_out) rstd_out[i] = (float)(1.0 / rms);
        for (int64_t j = 0; j < D; ++j) {
            /* tensor.rs:116 broadcast_div, then qwen.rs:321 broadcast_mul(weight) */
            double v = (double)xr[j] / rms;
            if (w) v *= (double)w[j];
            y[i * D + j] = (float)v;
        }
    }
}

void oracle_rmsnorm_bwd(int64_t rows, int64_t D, float eps, const float* x, const float* w,
                        const float* dy, float* dx, float* dw, int threads) {
    const int nt = nthreads(threads);
    double* rs = (double*)malloc(sizeof(double) * (size_t)(rows > 0 ? rows : 1));
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < rows; ++i) {
        const float* xr = x + i * D;
        const float* dyr = dy + i * D;
        double ss = 0.0;
        for (int64_t j = 0; j < D; ++j) ss += (double)xr[j] * (double)xr[j];
        double r = 1.0 / sqrt(ss / (double)D + (double)eps);
        rs[i] = r;
        if (dx) {
            double gx = 0.0;
            for (int64_t j = 0; j < D; ++j) {
                double g = (double)dyr[j] * (w ? (double)w[j] : 1.0);
                gx += g * (double)xr[j];
            }
            double c = r * r * r * gx / (double)D;
            for (int64_t j = 0; j < D; ++j) {
                double g = (double)dyr[j] * (w ? (double)w[j] : 1.0);
                dx[i * D + j] = (float)(r * g - (double)xr[j] * c);
            }
        }
    }
    if (dw) {
#pragma omp parallel for schedule(static) num_threads(nt)
        for (int64_t j = 0; j < D; ++j) {
            double acc = 0.0;
            for (int64_t i = 0; i < rows; ++i) acc += (double)dy[i * D + j] * (double)x[i * D + j] * rs[i];
            dw[j] = (float)acc;
        }
    }
    free(rs);
}

/* --------------------------------------------------------------- softmax */
static int64_t causal_limit(int64_t row, int64_t D, int64_t causal_rows) {
    /* last unmasked column of this row (inclusive) */
    if (causal_rows <= 0) return D - 1;
    return row % causal_rows + (D - causal_rows);
}

static void softmax_fwd_impl(int64_t rows, int64_t D, int64_t causal_rows, const int64_t* row_ids,
                             const float* s, float* p, int threads) {
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (int64_t i = 0; i < rows; ++i) {
        const float* sr = s + i * D;
        float* pr = p + i * D;
        int64_t lim = causal_limit(row_ids ? row_ids[i] : i, D, causal_rows);
        /* tensor.rs:93 max_keepdim (masked entries are -inf and never the max) */
        double m = -INFINITY;
        for (int64_t j = 0; j <= lim; ++j) if ((double)sr[j] > m) m = (double)sr[j];
        /* tensor.rs:94-96  sub, exp, sum_keepdim */
        double sum = 0.0;
        for (int64_t j = 0; j <= lim; ++j) sum += exp((double)sr[j] - m);
        /* tensor.rs:97 broadcast_div; exp(-inf) = 0 exactly at masked entries */
        for (int64_t j = 0; j < D; ++j)
            pr[j] = j <= lim ? (float)(exp((double)sr[j] - m) / sum) : 0.0f;
    }
}

static void softmax_bwd_impl(int64_t rows, int64_t D, int64_t causal_rows, const int64_t* row_ids,
                             const float* p, const float* dp, float* ds, int threads) {
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (int64_t i = 0; i < rows; ++i) {
        const float* pr = p + i * D;
        const float* dpr = dp + i * D;
        int64_t lim = causal_limit(row_ids ? row_ids[i] : i, D, causal_rows);
        double dot = 0.0;
        for (int64_t j = 0; j <= lim; ++j) dot += (double)pr[j] * (double)dpr[j];
        for (int64_t j = 0; j < D; ++j)
            ds[i * D + j] = j <= lim ? (float)((double)pr[j] * ((double)dpr[j] - dot)) : 0.0f;
    }
}

void oracle_softmax_fwd(int64_t rows, int64_t D, int64_t causal_rows, const float* s, float* p,
                        int threads) {
    softmax_fwd_impl(rows, D, causal_rows, NULL, s, p, threads);
}

void oracle_softmax_bwd(int64_t rows, int64_t D, int64_t causal_rows, const float* p,
                        const float* dp, float* ds, int threads) {
    softmax_bwd_impl(rows, D, causal_rows, NULL, p, dp, ds, threads);
}

void oracle_softmax_fwd_rows(int64_t n, int64_t D, int64_t causal_rows, const int64_t* row_ids,
                             const float* s, float* p, int threads) {
    softmax_fwd_impl(n, D, causal_rows, row_ids, s, p, threads);
}

void oracle_softmax_bwd_rows(int64_t n, int64_t D, int64_t causal_rows, const int64_t* row_ids,
                             const float* p, const float* dp, float* ds, int threads) {
    softmax_bwd_impl(n, D, causal_rows, row_ids, p, dp, ds, threads);
}

/* ------------------------------------------------------------- attention */
/* Attention::forward (src/models/transformer.rs:258-283) for one (b, h, i)
 * score row, in the reference's op order: q.k^T (matmul, 264), scaled (266;
 * the reference divides by sqrt(d), callers pass scale = 1/sqrt(d)), the
 * broadcast mask added (268-272), softmax_stable (tensor.rs:91-98: max, sub,
 * exp, sum, divide). The causal mask is -inf where key j > query i. K/V head
 * of query head h: h / (H / Hkv), the order repeat_kv builds (295-319).
 * Returns the row max; *sum receives the exp sum; p[j] the probabilities. */
static double attn_row(int64_t S, int D, double scale, int causal, const float* qi, const float* kh,
                       const float* mrow, int64_t i, double* p, double* sum) {
    double m = -INFINITY;
    for (int64_t j = 0; j < S; ++j) {
        double s = 0.0;
        const float* kj = kh + j * D;
        for (int d = 0; d < D; ++d) s += (double)qi[d] * (double)kj[d];
        s *= scale;
        if (mrow) s += (double)mrow[j];
        if (causal && j > i) s = -INFINITY;
        p[j] = s;
        if (s > m) m = s;
    }
    double z = 0.0;
    for (int64_t j = 0; j < S; ++j) {
        p[j] = exp(p[j] - m); /* all -inf: exp(nan) = nan, as the reference */
        z += p[j];
    }
    for (int64_t j = 0; j < S; ++j) p[j] /= z;
    *sum = z;
    return m;
}

void oracle_attention_fwd(int64_t B, int32_t H, int32_t Hkv, int64_t S, int32_t D, float scale, int causal,
                          const float* q, const float* k, const float* v, const float* mask, float* o,
                          float* lse, int threads) {
    const int rep = H / Hkv;
#pragma omp parallel num_threads(nthreads(threads))
    {
        double* p = (double*)malloc(sizeof(double) * (size_t)S);
        double* acc = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 16)
        for (int64_t row = 0; row < B * H * S; ++row) {
            const int64_t bh = row / S, i = row % S;
            const int64_t b = bh / H, h = bh % H;
            const int64_t bhk = b * Hkv + h / rep;
            const float* kh = k + bhk * S * D;
            const float* vh = v + bhk * S * D;
            double z;
            const double m = attn_row(S, D, scale, causal, q + (bh * S + i) * D, kh, mask ? mask + i * S : NULL,
                                      i, p, &z);
            for (int d = 0; d < D; ++d) acc[d] = 0.0;
            for (int64_t j = 0; j < S; ++j) {
                if (p[j] == 0.0) continue;
                const float* vj = vh + j * D;
                for (int d = 0; d < D; ++d) acc[d] += p[j] * (double)vj[d];
            }
            /* transpose(1, 2) + reshape to [B, S, H * D] (transformer.rs:280-282) */
            float* orow = o + ((b * S + i) * H + h) * D;
            for (int d = 0; d < D; ++d) orow[d] = (float)acc[d];
            if (lse) lse[bh * S + i] = (float)(m + log(z));
        }
        free(p);
        free(acc);
    }
}

/* Gradients of the forward above (candle autograd of transformer.rs:264-278,
 * no reference kernel): with P the probabilities and dO [B, S, H * D],
 *   dV_j = sum_i P_ij dO_i            dP_ij = dO_i . v_j
 *   dS_ij = P_ij (dP_ij - sum_k P_ik dP_ik)
 *   dQ_i = scale sum_j dS_ij k_j      dK_j = scale sum_i dS_ij q_i
 * dK and dV of a K/V head sum over the H / Hkv query heads that read it (the
 * backward of repeat_kv's concatenation). dq [B, H, S, D], dk, dv
 * [B, Hkv, S, D]. */
void oracle_attention_bwd(int64_t B, int32_t H, int32_t Hkv, int64_t S, int32_t D, float scale, int causal,
                          const float* q, const float* k, const float* v, const float* mask, const float* dout,
                          float* dq, float* dk, float* dv, int threads) {
    /* tasks: (b, h, chunk of 128 queries); each writes its dq rows and its own
     * dK / dV partial [S, D], summed afterwards per K/V head in (h, chunk) order */
    const int rep = H / Hkv;
    const int64_t CH = 128, nch = (S + CH - 1) / CH, ntask = B * H * nch;
    double* part = (double*)calloc((size_t)ntask * 2 * (size_t)S * D, sizeof(double));
#pragma omp parallel num_threads(nthreads(threads))
    {
        double* p = (double*)malloc(sizeof(double) * (size_t)S);
        double* dp = (double*)malloc(sizeof(double) * (size_t)S);
        double* gq = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
        for (int64_t task = 0; task < ntask; ++task) {
            const int64_t bh = task / nch, ch = task % nch;
            const int64_t b = bh / H, h = bh % H;
            const int64_t bhk = b * Hkv + h / rep;
            const float* kh = k + bhk * S * D;
            const float* vh = v + bhk * S * D;
            double* gk = part + (size_t)task * 2 * S * D;
            double* gv = gk + (size_t)S * D;
            for (int64_t i = ch * CH; i < S && i < (ch + 1) * CH; ++i) {
                const float* qi = q + (bh * S + i) * D;
                const float* doi = dout + ((b * S + i) * H + h) * D;
                double z;
                attn_row(S, D, scale, causal, qi, kh, mask ? mask + i * S : NULL, i, p, &z);
                double dot = 0.0;
                for (int64_t j = 0; j < S; ++j) {
                    double sv = 0.0;
                    const float* vj = vh + j * D;
                    for (int d = 0; d < D; ++d) sv += (double)doi[d] * (double)vj[d];
                    dp[j] = sv;
                    dot += p[j] * sv;
                }
                for (int d = 0; d < D; ++d) gq[d] = 0.0;
                for (int64_t j = 0; j < S; ++j) {
                    if (p[j] == 0.0) continue;
                    const double ds = p[j] * (dp[j] - dot) * (double)scale;
                    const float* kj = kh + j * D;
                    for (int d = 0; d < D; ++d) {
                        gq[d] += ds * (double)kj[d];
                        gk[j * D + d] += ds * (double)qi[d];
                        gv[j * D + d] += p[j] * (double)doi[d];
                    }
                }
                float* dqi = dq + (bh * S + i) * D;
                for (int d = 0; d < D; ++d) dqi[d] = (float)gq[d];
            }
        }
        free(p);
        free(dp);
        free(gq);
#pragma omp for schedule(static)
        for (int64_t bhk = 0; bhk < B * Hkv; ++bhk) {
            const int64_t b = bhk / Hkv, hk = bhk % Hkv;
            for (int64_t e = 0; e < S * D; ++e) {
                double sk = 0.0, sv = 0.0;
                for (int64_t h = hk * rep; h < (hk + 1) * rep; ++h)
                    for (int64_t ch = 0; ch < nch; ++ch) {
                        const double* gk = part + (size_t)((b * H + h) * nch + ch) * 2 * S * D;
                        sk += gk[e];
                        sv += gk[(size_t)S * D + e];
                    }
                dk[bhk * S * D + e] = (float)sk;
                dv[bhk * S * D + e] = (float)sv;
            }
        }
    }
    free(part);
}

/* ----------------------------------------------------------------- AdamW */
/* AdamW::step (src/training/optimizer.rs:227-281) as the reference evaluates
 * it: candle fp32 tensor ops, one rounding each, in this order. `tensor * f64`
 * and `tensor + f64` are candle's affine(mul, add) = v * mul + add in fp32
 * (candle-core 0.9 CPU backend, not vendored), `tensor / f64` is
 * affine(1 / x, 0) with the reciprocal taken in f64. beta^t is f32::powi
 * (optimizer.rs:257-258), which a run-time exponent lowers to right-to-left
 * binary exponentiation in fp32. The Makefile builds with -ffp-contract=off,
 * so no multiply-add is fused. */
static float powi_f32(float base, int32_t t) {
    float r = 1.0f;
    for (;;) {
        if (t & 1) r *= base;
        t /= 2;
        if (t == 0) break;
        base *= base;
    }
    return r;
}

static float affine0(float x, float mul) {
    const float y = x * mul;
    return y + 0.0f;
}

void oracle_adamw_step(int64_t n, float lr, float beta1, float beta2, float eps, float wd, int64_t step,
                       const float* param, const float* grad, float* m, float* v, float* param_out) {
    const float omb1 = 1.0f - beta1, omb2 = 1.0f - beta2;                   /* 243, 248 */
    const float c1 = (float)(1.0 / (double)(1.0f - powi_f32(beta1, (int32_t)step)));  /* 260 */
    const float c2 = (float)(1.0 / (double)(1.0f - powi_f32(beta2, (int32_t)step)));  /* 261 */
    const float wdlr = wd * lr;                                              /* 272 */
    for (int64_t i = 0; i < n; ++i) {
        const float g = grad[i], p = param[i];
        const float m1 = affine0(m[i], beta1) + affine0(g, omb1);           /* 242-243 */
        const float g2 = g * g;                                              /* 246 */
        const float v1 = affine0(v[i], beta2) + affine0(g2, omb2);          /* 247-248 */
        const float mh = affine0(m1, c1);                                    /* 260 */
        const float vh = affine0(v1, c2);                                    /* 261 */
        const float sq = sqrtf(vh);                                          /* 264 */
        const float den = sq * 1.0f + eps;                                   /* 265 */
        const float u = mh / den;                                            /* 266 */
        const float lru = affine0(u, lr);                                    /* 269 */
        const float wdu = affine0(p, wdlr);                                  /* 272 */
        const float p1 = p - lru;                                            /* 275 */
        param_out[i] = p1 - wdu;
        m[i] = m1;                                                           /* 278-279 */
        v[i] = v1;
    }
}

/* ------------------------------------------------------------- LayerNorm */
/* LayerNormOp::cpu_fwd (src/backend/custom_ops.rs, the two-pass loop: mean,
 * then the centred variance, then (x - mean) * 1/sqrt(var + eps)), with the
 * weight and bias of MetalLayerNorm::forward (src/embeddings/metal_bert.rs:
 * 30-72). fp64 accumulation. mean / rstd [rows] may be NULL. */
void oracle_layernorm_fwd(int64_t rows, int64_t D, float eps, const float* x, const float* w, const float* b,
                          float* y, float* mean, float* rstd, int threads) {
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (int64_t i = 0; i < rows; ++i) {
        const float* xr = x + i * D;
        double m = 0.0;
        for (int64_t j = 0; j < D; ++j) m += xr[j];
        m /= (double)D;
        double v = 0.0;
        for (int64_t j = 0; j < D; ++j) v += ((double)xr[j] - m) * ((double)xr[j] - m);
        v /= (double)D;
        const double r = 1.0 / sqrt(v + (double)eps);
        for (int64_t j = 0; j < D; ++j) {
            double t = ((double)xr[j] - m) * r;
            if (w) t *= (double)w[j];
            if (b) t += (double)b[j];
            y[i * D + j] = (float)t;
        }
        if (mean) mean[i] = (float)m;
        if (rstd) rstd[i] = (float)r;
    }
}

/* Gradients of the forward above (no reference kernel): xh = (x - mean) r,
 * g = dy w: dx = r (g - mean(g) - xh mean(g xh)); dw = sum_rows dy xh,
 * db = sum_rows dy (dw, db may be NULL). */
void oracle_layernorm_bwd(int64_t rows, int64_t D, float eps, const float* x, const float* w, const float* dy,
                          float* dx, float* dw, float* db, int threads) {
    double* gw = (double*)calloc((size_t)D, sizeof(double));
    double* gb = (double*)calloc((size_t)D, sizeof(double));
    for (int64_t i = 0; i < rows; ++i) {
        const float* xr = x + i * D;
        const float* gr = dy + i * D;
        double m = 0.0, v = 0.0;
        for (int64_t j = 0; j < D; ++j) m += xr[j];
        m /= (double)D;
        for (int64_t j = 0; j < D; ++j) v += ((double)xr[j] - m) * ((double)xr[j] - m);
        const double r = 1.0 / sqrt(v / (double)D + (double)eps);
        double mg = 0.0, mgx = 0.0;
        for (int64_t j = 0; j < D; ++j) {
            const double g = (double)gr[j] * (w ? (double)w[j] : 1.0);
            mg += g;
            mgx += g * ((double)xr[j] - m) * r;
        }
        mg /= (double)D;
        mgx /= (double)D;
        for (int64_t j = 0; j < D; ++j) {
            const double xh = ((double)xr[j] - m) * r;
            const double g = (double)gr[j] * (w ? (double)w[j] : 1.0);
            dx[i * D + j] = (float)(r * (g - mg - xh * mgx));
            gw[j] += (double)gr[j] * xh;
            gb[j] += (double)gr[j];
        }
    }
    for (int64_t j = 0; j < D; ++j) {
        if (dw) dw[j] = (float)gw[j];
        if (db) db[j] = (float)gb[j];
    }
    free(gw);
    free(gb);
    (void)threads;
}

/* ----------------------------------------------- log-softmax, cross entropy */
/* candle_nn::ops::log_softmax as cross_entropy_loss uses it
 * (src/training/loss.rs:108; candle-nn 0.9, not vendored): max_keepdim,
 * broadcast_sub, exp, sum_keepdim, log, broadcast_sub. Returns the row's
 * log-sum-exp. */
static double log_softmax_row(int64_t D, const float* x, double* out) {
    double m = -INFINITY;
    for (int64_t j = 0; j < D; ++j)
        if ((double)x[j] > m) m = x[j];
    double sum = 0.0;
    for (int64_t j = 0; j < D; ++j) sum += exp((double)x[j] - m);
    const double ls = log(sum);
    if (out)
        for (int64_t j = 0; j < D; ++j) out[j] = ((double)x[j] - m) - ls;
    return m + ls;
}

void oracle_log_softmax_fwd(int64_t rows, int64_t D, const float* x, float* y, int threads) {
#pragma omp parallel num_threads(nthreads(threads))
    {
        double* t = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(static)
        for (int64_t i = 0; i < rows; ++i) {
            log_softmax_row(D, x + i * D, t);
            for (int64_t j = 0; j < D; ++j) y[i * D + j] = (float)t[j];
        }
        free(t);
    }
}

/* dx = dy - exp(y) sum(dy) */
void oracle_log_softmax_bwd(int64_t rows, int64_t D, const float* y, const float* dy, float* dx, int threads) {
#pragma omp parallel for schedule(static) num_threads(nthreads(threads))
    for (int64_t i = 0; i < rows; ++i) {
        double s = 0.0;
        for (int64_t j = 0; j < D; ++j) s += dy[i * D + j];
        for (int64_t j = 0; j < D; ++j)
            dx[i * D + j] = (float)((double)dy[i * D + j] - exp((double)y[i * D + j]) * s);
    }
}

/* cross_entropy_loss (loss.rs:58-148): log-softmax of each row, gather of
 * the target's log-probability, mask of targets != ignore_index (ignore < 0:
 * none), sum / count, negated; with smoothing s (loss.rs:208-245):
 * (1 - s) * that + s * (-mean of every log-probability of every row).
 * Returns NaN where the reference returns an error (count 0, target out of
 * range). lse [rows] may be NULL; *count receives the count. */
double oracle_cross_entropy_fwd(int64_t rows, int64_t V, const float* logits, const uint32_t* targets,
                                int64_t ignore_index, float smoothing, float* lse, double* count) {
    double nll = 0.0, all = 0.0, cnt = 0.0;
    int bad = 0;
    for (int64_t i = 0; i < rows; ++i) {
        const float* xr = logits + i * V;
        const double l = log_softmax_row(V, xr, NULL);
        if (lse) lse[i] = (float)l;
        double rs = 0.0;
        for (int64_t j = 0; j < V; ++j) rs += (double)xr[j] - l;
        all += rs;
        const int ignored = ignore_index >= 0 && (int64_t)targets[i] == ignore_index;
        if (ignored) continue;
        if ((int64_t)targets[i] >= V) {
            bad = 1;
            continue;
        }
        nll += l - (double)xr[targets[i]];
        cnt += 1.0;
    }
    if (count) *count = cnt;
    if (bad || cnt == 0.0) return NAN;
    double loss = nll / cnt;
    if (smoothing != 0.0f) loss = (1.0 - smoothing) * loss + smoothing * (-all / ((double)rows * (double)V));
    return loss;
}

/* d loss / d logits, times dloss: (1 - s) [counted] (p - onehot) / count + s (p - 1/V) / rows. */
void oracle_cross_entropy_bwd(int64_t rows, int64_t V, const float* logits, const uint32_t* targets,
                              int64_t ignore_index, float smoothing, float dloss, float* dlogits) {
    double cnt = 0.0;
    for (int64_t i = 0; i < rows; ++i)
        if (!(ignore_index >= 0 && (int64_t)targets[i] == ignore_index)) cnt += 1.0;
    for (int64_t i = 0; i < rows; ++i) {
        const float* xr = logits + i * V;
        const double l = log_softmax_row(V, xr, NULL);
        const int valid = !(ignore_index >= 0 && (int64_t)targets[i] == ignore_index);
        for (int64_t j = 0; j < V; ++j) {
            const double p = exp((double)xr[j] - l);
            double g = smoothing * (p - 1.0 / (double)V) / (double)rows;
            if (valid) g += (1.0 - smoothing) * (p - (j == (int64_t)targets[i] ? 1.0 : 0.0)) / cnt;
            dlogits[i * V + j] = (float)(dloss * g);
        }
    }
}

/* ------------------------------------------------------------------ bf16 */
void oracle_round_bf16(const float* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t u;
        memcpy(&u, &in[i], 4);
        if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
            u |= 0x00400000u; /* quiet NaN */
        } else {
            u += 0x7fffu + ((u >> 16) & 1u);
        }
        u &= 0xffff0000u;
        memcpy(&out[i], &u, 4);
    }
}
