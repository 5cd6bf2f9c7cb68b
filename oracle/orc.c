/* ORACLE -- test infrastructure only (see orc.h).  A restatement of the
 * reference CPU path; each function cites the reference code it follows. */
#include "orc.h"

#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ======================= GEMM family ======================= */

/* Block sizes of the reference kernel (reference src/gemm.c:22-39).  Every
 * C element of the main region is one serial FMA chain over k = 0..K-1
 * starting from +0, whatever the blocking; the tails are serial
 * multiply-then-add chains that skip a == 0 (reference src/gemm.c:52-62). */
#define O_MR 6
#define O_NR 16
#define O_KC 384
#define O_NC 1024
#define O_MC 120
#define O_APAD 16

static void tail_block(int M, int N, int K, const float *A, const float *B, float *C, int n0,
                       int n1) {
    for (int i = 0; i < M; i++)
        for (int k = 0; k < K; k++) {
            const float av = A[(long)i * K + k];
            if (av == 0.0f) continue;
            const float *brow = B + (long)k * N;
            float *crow = C + (long)i * N;
            for (int j = n0; j < n1; j++) crow[j] += av * brow[j];
        }
}

/* 6x16 tile: 12 accumulators of 8 lanes, b row pair, broadcast a */
static void tile6x16(const float *Ap, long lda, const float *Bp, float *C, long ldc, int Ki,
                     int first) {
    __m256 acc[O_MR][2];
    for (int r = 0; r < O_MR; r++) {
        if (first) {
            acc[r][0] = _mm256_setzero_ps();
            acc[r][1] = _mm256_setzero_ps();
        } else {
            acc[r][0] = _mm256_loadu_ps(C + r * ldc);
            acc[r][1] = _mm256_loadu_ps(C + r * ldc + 8);
        }
    }
    for (int k = 0; k < Ki; k++) {
        const __m256 b0 = _mm256_load_ps(Bp + (long)k * O_NR);
        const __m256 b1 = _mm256_load_ps(Bp + (long)k * O_NR + 8);
        for (int r = 0; r < O_MR; r++) {
            const __m256 a = _mm256_broadcast_ss(Ap + r * lda + k);
            acc[r][0] = _mm256_fmadd_ps(b0, a, acc[r][0]);
            acc[r][1] = _mm256_fmadd_ps(b1, a, acc[r][1]);
        }
    }
    for (int r = 0; r < O_MR; r++) {
        _mm256_storeu_ps(C + r * ldc, acc[r][0]);
        _mm256_storeu_ps(C + r * ldc + 8, acc[r][1]);
    }
}

int orc_sgemm(int M, int N, int K, const float *A, const float *B, float *C, int nthreads) {
    if (M <= 0 || N <= 0) return 0;
    memset(C, 0, sizeof(float) * (size_t)M * (size_t)N);
    if (K <= 0) return 0;
#ifdef _OPENMP
    if (nthreads < 1) nthreads = 1;
    if (nthreads > omp_get_max_threads()) nthreads = omp_get_max_threads();
#else
    nthreads = 1;
#endif
    const int Nfull = N / O_NR * O_NR;
    const int Mfull = M / O_MR * O_MR;
    if (Nfull == 0 || Mfull == 0) {
        tail_block(M, N, K, A, B, C, 0, N);
        return 0;
    }
    const size_t panel = (size_t)O_KC * O_NR;
    float *Bp = (float *)aligned_alloc(32, sizeof(float) * panel * (O_NC / O_NR));
    const int mc_rows = O_MC < Mfull ? O_MC : Mfull;
    float *Ap = (float *)aligned_alloc(32, sizeof(float) * (size_t)mc_rows * (O_KC + O_APAD));
    if (!Bp || !Ap) { free(Bp); free(Ap); return -1; }
    const long lda = O_KC + O_APAD;
    for (int jc = 0; jc < Nfull; jc += O_NC) {
        const int jend = jc + O_NC < Nfull ? jc + O_NC : Nfull;
        const int npan = (jend - jc) / O_NR;
        for (int kk = 0; kk < K; kk += O_KC) {
            const int Ki = kk + O_KC <= K ? O_KC : K - kk;
            for (int p = 0; p < npan; p++)
                for (int k2 = 0; k2 < Ki; k2++)
                    memcpy(Bp + p * panel + (size_t)k2 * O_NR,
                           B + (long)(kk + k2) * N + jc + (long)p * O_NR, sizeof(float) * O_NR);
            for (int ic = 0; ic < Mfull; ic += O_MC) {
                const int mi = ic + O_MC <= Mfull ? O_MC : Mfull - ic;
                for (int r = 0; r < mi; r++)
                    memcpy(Ap + (size_t)r * lda, A + (long)(ic + r) * K + kk, sizeof(float) * Ki);
#ifdef _OPENMP
#pragma omp parallel for num_threads(nthreads) schedule(static) collapse(2)
#endif
                for (int p = 0; p < npan; p++)
                    for (int ig = 0; ig < mi; ig += O_MR)
                        tile6x16(Ap + (size_t)ig * lda, lda, Bp + p * panel,
                                 C + (long)(ic + ig) * N + jc + (long)p * O_NR, N, Ki, kk == 0);
            }
        }
    }
    free(Bp);
    free(Ap);
    if (Mfull < M) tail_block(M - Mfull, N, K, A + (long)Mfull * K, B, C + (long)Mfull * N, 0, Nfull);
    if (Nfull < N) tail_block(M, N, K, A, B, C, Nfull, N);
    return 0;
}

void orc_matmul_naive(int M, int N, int K, const float *A, const float *B, float *C) {
    memset(C, 0, sizeof(float) * (size_t)M * (size_t)N);
    for (int m = 0; m < M; m++)
        for (int k = 0; k < K; k++) {
            const float av = A[(long)m * K + k];
            if (av == 0.0f) continue;
            const float *brow = B + (long)k * N;
            float *orow = C + (long)m * N;
            for (int n = 0; n < N; n++) orow[n] += av * brow[n];
        }
}

void orc_matmul_nt(int M, int N, int K, const float *X, const float *Y, float *R) {
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(static)
#endif
    for (int m = 0; m < M; m++)
        for (int n = 0; n < N; n++) {
            const float *xr = X + (long)m * K, *yr = Y + (long)n * K;
            float s = 0.0f;
            for (int k = 0; k < K; k++) s += xr[k] * yr[k];
            R[(long)m * N + n] = s;
        }
}

void orc_matmul_tn(int M, int N, int K, const float *X, const float *Y, float *R) {
    memset(R, 0, sizeof(float) * (size_t)M * (size_t)N);
#ifdef _OPENMP
#pragma omp parallel for schedule(static)
#endif
    for (int m = 0; m < M; m++)
        for (int k = 0; k < K; k++) {
            const float xv = X[(long)k * M + m];
            const float *yr = Y + (long)k * N;
            float *rr = R + (long)m * N;
            for (int n = 0; n < N; n++) rr[n] += xv * yr[n];
        }
}

void orc_sgemm_a_bt(int M, int N, long K, const float *A, const float *B, float *C) {
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(static)
#endif
    for (int i = 0; i < M; i++)
        for (int j = 0; j < N; j++) {
            const float *a = A + (long)i * K, *b = B + (long)j * K;
            float s = 0.0f;
            for (long k = 0; k < K; k++) s += a[k] * b[k];
            C[(long)i * N + j] = s;
        }
}

/* ======================= spatial ======================= */

void orc_im2col(const float *x, int N, int C, int H, int W, int HH, int WW, int ph, int pw,
                int sh, int sw, float *col) {
    const int Ho = (H + 2 * ph - HH) / sh + 1, Wo = (W + 2 * pw - WW) / sw + 1;
    const long HoWo = (long)Ho * Wo, Ncol = (long)N * HoWo;
    const int Kc = C * HH * WW;
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(static)
#endif
    for (int c = 0; c < Kc; c++)
        for (int n = 0; n < N; n++) {
            const int kw = c % WW, kh = (c / WW) % HH, ci = c / (HH * WW);
            const float *img = x + ((long)n * C + ci) * H * W;
            float *dst = col + (long)c * Ncol + (long)n * HoWo;
            for (int ho = 0; ho < Ho; ho++) {
                const int hi = ho * sh - ph + kh;
                for (int wo = 0; wo < Wo; wo++) {
                    const int wi = wo * sw - pw + kw;
                    dst[ho * Wo + wo] =
                        (hi >= 0 && hi < H && wi >= 0 && wi < W) ? img[(long)hi * W + wi] : 0.0f;
                }
            }
        }
}

void orc_col2im(const float *col, int N, int C, int H, int W, int HH, int WW, int ph, int pw,
                int sh, int sw, float *x) {
    memset(x, 0, sizeof(float) * (size_t)N * C * H * W);
    const int Ho = (H + 2 * ph - HH) / sh + 1, Wo = (W + 2 * pw - WW) / sw + 1;
    const long HoWo = (long)Ho * Wo, Ncol = (long)N * HoWo;
    const int Kc = C * HH * WW;
    for (int c = 0; c < Kc; c++) {
        const int kw = c % WW, kh = (c / WW) % HH, ci = c / (HH * WW);
        for (int n = 0; n < N; n++) {
            float *img = x + ((long)n * C + ci) * H * W;
            const float *src = col + (long)c * Ncol + (long)n * HoWo;
            for (int ho = 0; ho < Ho; ho++) {
                const int hi = ho * sh - ph + kh;
                for (int wo = 0; wo < Wo; wo++) {
                    const int wi = wo * sw - pw + kw;
                    if (hi >= 0 && hi < H && wi >= 0 && wi < W)
                        img[(long)hi * W + wi] += src[ho * Wo + wo];
                }
            }
        }
    }
}

int orc_conv2d_fwd(const float *x, int N, int C, int H, int W, const float *w, int F, int HH,
                   int WW, const float *b, int sh, int sw, int ph, int pw, float *out,
                   int nthreads) {
    const int Ho = (H + 2 * ph - HH) / sh + 1, Wo = (W + 2 * pw - WW) / sw + 1;
    const int Kc = C * HH * WW;
    const long HoWo = (long)Ho * Wo, Ncol = (long)N * HoWo;
    float *col = (float *)malloc(sizeof(float) * (size_t)Kc * Ncol);
    float *gm = (float *)malloc(sizeof(float) * (size_t)F * Ncol);
    if (!col || !gm) { free(col); free(gm); return -1; }
    orc_im2col(x, N, C, H, W, HH, WW, ph, pw, sh, sw, col);
    int rc = orc_sgemm(F, (int)Ncol, Kc, w, col, gm, nthreads);
    if (rc == 0) {
#ifdef _OPENMP
#pragma omp parallel for collapse(2) schedule(static)
#endif
        for (int n = 0; n < N; n++)
            for (int f = 0; f < F; f++) {
                const float bv = b ? b[f] : 0.0f;
                const float *src = gm + (long)f * Ncol + (long)n * HoWo;
                float *dst = out + ((long)n * F + f) * HoWo;
                for (long i = 0; i < HoWo; i++) dst[i] = src[i] + bv;
            }
    }
    free(col);
    free(gm);
    return rc;
}

void orc_bias_grad(const float *g, int N, int F, int HW, float *db) {
    for (int f = 0; f < F; f++) {
        float s = 0.0f;
        for (int n = 0; n < N; n++)
            for (int i = 0; i < HW; i++) s += g[((long)n * F + f) * HW + i];
        db[f] = s;
    }
}

int orc_conv2d_bwd(const float *x, int N, int C, int H, int W, const float *w, int F, int HH,
                   int WW, const float *g, int sh, int sw, int ph, int pw, float *dx, float *dw,
                   float *db, int nthreads) {
    const int Ho = (H + 2 * ph - HH) / sh + 1, Wo = (W + 2 * pw - WW) / sw + 1;
    const int Kc = C * HH * WW;
    const long HoWo = (long)Ho * Wo, Ncol = (long)N * HoWo;
    if (db) orc_bias_grad(g, N, F, (int)HoWo, db);
    if (!dw && !dx) return 0;
    float *gp = (float *)malloc(sizeof(float) * (size_t)F * Ncol);   /* (F, N*HW) permute */
    if (!gp) return -1;
    for (int f = 0; f < F; f++)
        for (int n = 0; n < N; n++)
            memcpy(gp + (long)f * Ncol + (long)n * HoWo, g + ((long)n * F + f) * HoWo,
                   sizeof(float) * HoWo);
    int rc = 0;
    if (dw) {
        float *col = (float *)malloc(sizeof(float) * (size_t)Kc * Ncol);
        if (!col) { free(gp); return -1; }
        orc_im2col(x, N, C, H, W, HH, WW, ph, pw, sh, sw, col);
        orc_sgemm_a_bt(F, Kc, Ncol, gp, col, dw);
        free(col);
    }
    if (dx) {
        float *wt = (float *)malloc(sizeof(float) * (size_t)F * Kc);
        float *dcol = (float *)malloc(sizeof(float) * (size_t)Kc * Ncol);
        if (!wt || !dcol) { free(wt); free(dcol); free(gp); return -1; }
        for (int f = 0; f < F; f++)
            for (int k = 0; k < Kc; k++) wt[(long)k * F + f] = w[(long)f * Kc + k];
        rc = orc_sgemm(Kc, (int)Ncol, F, wt, gp, dcol, nthreads);
        if (rc == 0) orc_col2im(dcol, N, C, H, W, HH, WW, ph, pw, sh, sw, dx);
        free(wt);
        free(dcol);
    }
    free(gp);
    return rc;
}

void orc_maxpool_fwd(const float *x, int N, int C, int H, int W, int ph, int pw, int sh, int sw,
                     float *y) {
    const int Ho = (H - ph) / sh + 1, Wo = (W - pw) / sw + 1;
    for (long nc = 0; nc < (long)N * C; nc++)
        for (int ho = 0; ho < Ho; ho++)
            for (int wo = 0; wo < Wo; wo++) {
                float m = -INFINITY;
                for (int kh = 0; kh < ph; kh++)
                    for (int kw = 0; kw < pw; kw++) {
                        const float v = x[nc * H * W + (long)(ho * sh + kh) * W + wo * sw + kw];
                        if (v > m) m = v;
                    }
                y[nc * Ho * Wo + (long)ho * Wo + wo] = m;
            }
}

void orc_maxpool_bwd(const float *x, const float *g, int N, int C, int H, int W, int ph, int pw,
                     int sh, int sw, float *dx) {
    const int Ho = (H - ph) / sh + 1, Wo = (W - pw) / sw + 1;
    memset(dx, 0, sizeof(float) * (size_t)N * C * H * W);
    for (long nc = 0; nc < (long)N * C; nc++)
        for (int ho = 0; ho < Ho; ho++)
            for (int wo = 0; wo < Wo; wo++) {
                float m = -INFINITY;
                int bh = ho * sh, bw = wo * sw;
                for (int kh = 0; kh < ph; kh++)
                    for (int kw = 0; kw < pw; kw++) {
                        const float v = x[nc * H * W + (long)(ho * sh + kh) * W + wo * sw + kw];
                        if (v > m) { m = v; bh = ho * sh + kh; bw = wo * sw + kw; }
                    }
                dx[nc * H * W + (long)bh * W + bw] += g[nc * Ho * Wo + (long)ho * Wo + wo];
            }
}

void orc_avgpool_fwd(const float *x, int N, int C, int H, int W, int ph, int pw, int sh, int sw,
                     float *y) {
    const int Ho = (H - ph) / sh + 1, Wo = (W - pw) / sw + 1;
    const float norm = 1.0f / (float)(ph * pw);
    for (long nc = 0; nc < (long)N * C; nc++)
        for (int ho = 0; ho < Ho; ho++)
            for (int wo = 0; wo < Wo; wo++) {
                float s = 0.0f;
                for (int kh = 0; kh < ph; kh++)
                    for (int kw = 0; kw < pw; kw++)
                        s += x[nc * H * W + (long)(ho * sh + kh) * W + wo * sw + kw];
                y[nc * Ho * Wo + (long)ho * Wo + wo] = s * norm;
            }
}

void orc_avgpool_bwd(const float *g, int N, int C, int H, int W, int ph, int pw, int sh, int sw,
                     float *dx) {
    const int Ho = (H - ph) / sh + 1, Wo = (W - pw) / sw + 1;
    const float norm = 1.0f / (float)(ph * pw);
    memset(dx, 0, sizeof(float) * (size_t)N * C * H * W);
    for (long nc = 0; nc < (long)N * C; nc++)
        for (int ho = 0; ho < Ho; ho++)
            for (int wo = 0; wo < Wo; wo++) {
                const float gv = g[nc * Ho * Wo + (long)ho * Wo + wo] * norm;
                for (int kh = 0; kh < ph; kh++)
                    for (int kw = 0; kw < pw; kw++)
                        dx[nc * H * W + (long)(ho * sh + kh) * W + wo * sw + kw] += gv;
            }
}

/* ======================= elementwise / rows ======================= */

void orc_relu_fwd(const float *x, float *y, long n) {
    for (long i = 0; i < n; i++) y[i] = x[i] > 0.0f ? x[i] : 0.0f;
}

void orc_relu_bwd(const float *x, const float *g, float *dx, long n) {
    for (long i = 0; i < n; i++) dx[i] = x[i] > 0.0f ? g[i] : 0.0f;
}

void orc_softmax_fwd(const float *x, float *y, long rows, int cols) {
    for (long r = 0; r < rows; r++) {
        const float *xr = x + r * cols;
        float *yr = y + r * cols;
        float m = -INFINITY;
        for (int j = 0; j < cols; j++) if (xr[j] > m) m = xr[j];
        if (m == -INFINITY) {
            for (int j = 0; j < cols; j++) yr[j] = 1.0f / (float)cols;
            continue;
        }
        float s = 0.0f;
        for (int j = 0; j < cols; j++) { const float e = expf(xr[j] - m); yr[j] = e; s += e; }
        for (int j = 0; j < cols; j++) yr[j] /= s;
    }
}

void orc_softmax_bwd(const float *s, const float *g, float *dx, long rows, int cols) {
    for (long r = 0; r < rows; r++) {
        const float *sr = s + r * cols, *gr = g + r * cols;
        float d = 0.0f;
        for (int j = 0; j < cols; j++) d += gr[j] * sr[j];
        for (int j = 0; j < cols; j++) dx[r * cols + j] = sr[j] * (gr[j] - d);
    }
}

void orc_padones_fwd(const float *x, float *y, long M, long K) {
    for (long m = 0; m < M; m++) {
        memcpy(y + m * (K + 1), x + m * K, sizeof(float) * (size_t)K);
        y[m * (K + 1) + K] = 1.0f;
    }
}

void orc_padones_bwd(const float *g, float *dx, long M, long K) {
    for (long m = 0; m < M; m++) memcpy(dx + m * K, g + m * (K + 1), sizeof(float) * (size_t)K);
}

double orc_ce_seed(const float *p, const int *labels, long rows, int cols, float *seed) {
    double loss = 0.0;
    const float fr = (float)rows;
    for (long r = 0; r < rows; r++) {
        const int y = labels[r];
        for (int j = 0; j < cols; j++) {
            const float d = p[r * cols + j] - (j == y ? 1.0f : 0.0f);
            seed[r * cols + j] = d / fr;
        }
        float py = (y >= 0 && y < cols) ? p[r * cols + y] : 0.0f;
        if (py < 1e-12f) py = 1e-12f;
        loss -= log((double)py);
    }
    return loss / (double)rows;
}

/* ======================= whole steps ======================= */

double orc_mlp_step(int B, int d0, int d1, int d2, int d3, const float *x, const int *labels,
                    const float *W1, const float *W2, const float *W3, float *logits, float *probs,
                    float *dW1, float *dW2, float *dW3, int nthreads) {
    const long k0 = d0 + 1, k1 = d1 + 1, k2 = d2 + 1;
    float *a0 = malloc(sizeof(float) * B * k0), *z1 = malloc(sizeof(float) * B * d1);
    float *h1 = malloc(sizeof(float) * B * d1), *a1 = malloc(sizeof(float) * B * k1);
    float *z2 = malloc(sizeof(float) * B * d2), *h2 = malloc(sizeof(float) * B * d2);
    float *a2 = malloc(sizeof(float) * B * k2), *seed = malloc(sizeof(float) * B * d3);
    float *ga2 = malloc(sizeof(float) * B * k2), *gh2 = malloc(sizeof(float) * B * d2);
    float *gz2 = malloc(sizeof(float) * B * d2), *ga1 = malloc(sizeof(float) * B * k1);
    float *gh1 = malloc(sizeof(float) * B * d1), *gz1 = malloc(sizeof(float) * B * d1);
    float *ga0 = malloc(sizeof(float) * B * k0);
    double loss = NAN;
    if (!a0 || !z1 || !h1 || !a1 || !z2 || !h2 || !a2 || !seed || !ga2 || !gh2 || !gz2 || !ga1 ||
        !gh1 || !gz1 || !ga0)
        goto out;
    /* forward: reference tests/gate_mnist_mlp.py:68-71 */
    orc_padones_fwd(x, a0, B, d0);
    orc_sgemm(B, d1, (int)k0, a0, W1, z1, nthreads);
    orc_relu_fwd(z1, h1, (long)B * d1);
    orc_padones_fwd(h1, a1, B, d1);
    orc_sgemm(B, d2, (int)k1, a1, W2, z2, nthreads);
    orc_relu_fwd(z2, h2, (long)B * d2);
    orc_padones_fwd(h2, a2, B, d2);
    orc_sgemm(B, d3, (int)k2, a2, W3, logits, nthreads);
    orc_softmax_fwd(logits, probs, B, d3);
    loss = orc_ce_seed(probs, labels, B, d3, seed);
    /* backward, reverse topological order (reference src/autograd.c:682-702) */
    orc_matmul_nt(B, (int)k2, d3, seed, W3, ga2);      /* matmul: dA */
    orc_matmul_tn((int)k2, d3, B, a2, seed, dW3);      /* matmul: dB */
    orc_padones_bwd(ga2, gh2, B, d2);
    orc_relu_bwd(z2, gh2, gz2, (long)B * d2);
    orc_matmul_nt(B, (int)k1, d2, gz2, W2, ga1);
    orc_matmul_tn((int)k1, d2, B, a1, gz2, dW2);
    orc_padones_bwd(ga1, gh1, B, d1);
    orc_relu_bwd(z1, gh1, gz1, (long)B * d1);
    orc_matmul_nt(B, (int)k0, d1, gz1, W1, ga0);      /* computed and dropped, as the reference */
    orc_matmul_tn((int)k0, d1, B, a0, gz1, dW1);
out:
    free(a0); free(z1); free(h1); free(a1); free(z2); free(h2); free(a2); free(seed);
    free(ga2); free(gh2); free(gz2); free(ga1); free(gh1); free(gz1); free(ga0);
    return loss;
}

double orc_cnn_step(int B, int C0, int H, int W, int F1, int F2, int classes, const float *x,
                    const int *labels, const float *w1, const float *b1, const float *w2,
                    const float *b2, const float *wfc, float *logits, float *probs, float *dw1,
                    float *db1, float *dw2, float *db2, float *dwfc, int nthreads) {
    const int H2 = H / 2, W2 = W / 2, H4 = H2 / 2, W4 = W2 / 2;
    const long n1 = (long)B * F1 * H * W, p1n = (long)B * F1 * H2 * W2;
    const long n2 = (long)B * F2 * H2 * W2, p2n = (long)B * F2 * H4 * W4;
    const long D = (long)F2 * H4 * W4;
    float *c1 = malloc(sizeof(float) * n1), *r1 = malloc(sizeof(float) * n1);
    float *p1 = malloc(sizeof(float) * p1n), *c2 = malloc(sizeof(float) * n2);
    float *r2 = malloc(sizeof(float) * n2), *p2 = malloc(sizeof(float) * p2n);
    float *a = malloc(sizeof(float) * B * (D + 1)), *seed = malloc(sizeof(float) * B * classes);
    float *ga = malloc(sizeof(float) * B * (D + 1)), *gp2 = malloc(sizeof(float) * p2n);
    float *gr2 = malloc(sizeof(float) * n2), *gc2 = malloc(sizeof(float) * n2);
    float *gp1 = malloc(sizeof(float) * p1n), *gr1 = malloc(sizeof(float) * n1);
    float *gc1 = malloc(sizeof(float) * n1);
    double loss = NAN;
    if (!c1 || !r1 || !p1 || !c2 || !r2 || !p2 || !a || !seed || !ga || !gp2 || !gr2 || !gc2 ||
        !gp1 || !gr1 || !gc1)
        goto out;
    /* forward: conv -> relu -> maxpool, twice; reshape (a copy) -> padones -> matmul */
    if (orc_conv2d_fwd(x, B, C0, H, W, w1, F1, 3, 3, b1, 1, 1, 1, 1, c1, nthreads)) goto out;
    orc_relu_fwd(c1, r1, n1);
    orc_maxpool_fwd(r1, B, F1, H, W, 2, 2, 2, 2, p1);
    if (orc_conv2d_fwd(p1, B, F1, H2, W2, w2, F2, 3, 3, b2, 1, 1, 1, 1, c2, nthreads)) goto out;
    orc_relu_fwd(c2, r2, n2);
    orc_maxpool_fwd(r2, B, F2, H2, W2, 2, 2, 2, 2, p2);
    orc_padones_fwd(p2, a, B, D);
    orc_sgemm(B, classes, (int)(D + 1), a, wfc, logits, nthreads);
    orc_softmax_fwd(logits, probs, B, classes);
    loss = orc_ce_seed(probs, labels, B, classes, seed);
    /* backward */
    orc_matmul_nt(B, (int)(D + 1), classes, seed, wfc, ga);
    orc_matmul_tn((int)(D + 1), classes, B, a, seed, dwfc);
    orc_padones_bwd(ga, gp2, B, D);   /* reshape backward is a plain copy: same buffer */
    orc_maxpool_bwd(r2, gp2, B, F2, H2, W2, 2, 2, 2, 2, gr2);
    orc_relu_bwd(c2, gr2, gc2, n2);
    if (orc_conv2d_bwd(p1, B, F1, H2, W2, w2, F2, 3, 3, gc2, 1, 1, 1, 1, gp1, dw2, db2, nthreads))
        { loss = NAN; goto out; }
    orc_maxpool_bwd(r1, gp1, B, F1, H, W, 2, 2, 2, 2, gr1);
    orc_relu_bwd(c1, gr1, gc1, n1);
    if (orc_conv2d_bwd(x, B, C0, H, W, w1, F1, 3, 3, gc1, 1, 1, 1, 1, NULL, dw1, db1, nthreads))
        loss = NAN;
out:
    free(c1); free(r1); free(p1); free(c2); free(r2); free(p2); free(a); free(seed);
    free(ga); free(gp2); free(gr2); free(gc2); free(gp1); free(gr1); free(gc1);
    return loss;
}

/* ======================= seeded inputs ======================= */

static uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ULL);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

static double u01(uint64_t *s) { return (double)(splitmix64(s) >> 11) * (1.0 / 9007199254740992.0); }

void orc_fill_uniform(float *x, long n, float lo, float hi, unsigned long long seed) {
    uint64_t s = seed;
    for (long i = 0; i < n; i++) x[i] = (float)(lo + (hi - lo) * u01(&s));
}

void orc_fill_normal(float *x, long n, float stddev, unsigned long long seed) {
    uint64_t s = seed;
    for (long i = 0; i < n; i += 2) {
        double u1 = u01(&s), u2 = u01(&s);
        if (u1 < 1e-300) u1 = 1e-300;
        const double r = sqrt(-2.0 * log(u1));
        x[i] = (float)(stddev * r * cos(6.283185307179586 * u2));
        if (i + 1 < n) x[i + 1] = (float)(stddev * r * sin(6.283185307179586 * u2));
    }
}

void orc_fill_labels(int *y, long n, int classes, unsigned long long seed) {
    uint64_t s = seed;
    for (long i = 0; i < n; i++) y[i] = (int)(splitmix64(&s) % (uint64_t)classes);
}
