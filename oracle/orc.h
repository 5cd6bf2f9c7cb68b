/* ORACLE -- test infrastructure only.
 *
 * A CPU restatement, in plain C, of the reference tinytorch hot path.  It is
 * the parity checker of the GPU backend and the "port" CPU baseline timed by
 * bench.py; nothing in the product library links, loads or calls it.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * Every function names the reference file:line it follows.  Arithmetic
 * order is the reference's, and the library is compiled with the
 * reference's flags (-O3 -mavx2 -mfma -fopenmp -std=c11, which keeps
 * ISO C's no-contraction rule), so for the same inputs the outputs are
 * bit-identical to the reference's -- tests/test_oracle.py checks exactly
 * that against the reference compiled from its own sources (oracle/_ref),
 * and checks the oracle against closed forms, brute force and central
 * finite differences where the reference build is absent.
 *
 * All arrays are row-major fp32; images are NCHW. */
#ifndef ORC_H
#define ORC_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- GEMM family ---- */
/* C = A*B with the reference's blocked AVX2+FMA kernel (6x16 register tile,
 * KC=384, NC=1024, MC=120) and scalar tails.  C is overwritten.
 * reference src/gemm.c:52-62, 70-567, 569-641 */
int  orc_sgemm(int M, int N, int K, const float *A, const float *B, float *C, int nthreads);
/* naive tt_matmul: skips a == 0. reference src/ops.c:84-102 */
void orc_matmul_naive(int M, int N, int K, const float *A, const float *B, float *C);
/* R(MxN) = X(MxK) * Y(NxK)^T, dot form. reference src/autograd.c:66-84 */
void orc_matmul_nt(int M, int N, int K, const float *X, const float *Y, float *R);
/* R(MxN) = X(KxM)^T * Y(KxN), axpy form. reference src/autograd.c:87-103 */
void orc_matmul_tn(int M, int N, int K, const float *X, const float *Y, float *R);
/* C(MxN) = A(MxK) * B(NxK)^T, dot form. reference src/autograd.c:439-454 */
void orc_sgemm_a_bt(int M, int N, long K, const float *A, const float *B, float *C);

/* ---- spatial ---- */
/* reference src/ops_spatial.c:37-69 */
void orc_im2col(const float *x, int N, int C, int H, int W, int HH, int WW, int ph, int pw,
                int sh, int sw, float *col);
/* reference src/autograd.c:406-434 (zeroes x first) */
void orc_col2im(const float *col, int N, int C, int H, int W, int HH, int WW, int ph, int pw,
                int sh, int sw, float *x);
/* im2col + GEMM + bias + (F, N*HW) -> NCHW. reference src/ops_spatial.c:71-127 */
int  orc_conv2d_fwd(const float *x, int N, int C, int H, int W, const float *w, int F, int HH,
                    int WW, const float *b, int sh, int sw, int ph, int pw, float *out,
                    int nthreads);
/* db, dW, dX of a conv node (each output nullable = not required).
 * reference src/autograd.c:456-553 */
int  orc_conv2d_bwd(const float *x, int N, int C, int H, int W, const float *w, int F, int HH,
                    int WW, const float *g, int sh, int sw, int ph, int pw, float *dx,
                    float *dw, float *db, int nthreads);
/* db[f] = sum_{n,ho,wo} g (serial). reference src/autograd.c:467-482 */
void orc_bias_grad(const float *g, int N, int F, int HW, float *db);
/* reference src/ops_spatial.c:129-164 */
void orc_maxpool_fwd(const float *x, int N, int C, int H, int W, int ph, int pw, int sh, int sw,
                     float *y);
/* reference src/autograd.c:555-594 (dx zeroed first) */
void orc_maxpool_bwd(const float *x, const float *g, int N, int C, int H, int W, int ph, int pw,
                     int sh, int sw, float *dx);
/* reference src/ops_spatial.c:166-201 */
void orc_avgpool_fwd(const float *x, int N, int C, int H, int W, int ph, int pw, int sh, int sw,
                     float *y);
/* reference src/autograd.c:596-628 */
void orc_avgpool_bwd(const float *g, int N, int C, int H, int W, int ph, int pw, int sh, int sw,
                     float *dx);

/* ---- elementwise / rows ---- */
void orc_relu_fwd(const float *x, float *y, long n);                   /* src/ops.c:104-106 */
void orc_relu_bwd(const float *x, const float *g, float *dx, long n);  /* src/autograd.c:318-327 */
void orc_softmax_fwd(const float *x, float *y, long rows, int cols);   /* src/ops.c:108-145 */
void orc_softmax_bwd(const float *s, const float *g, float *dx, long rows, int cols); /* src/autograd.c:329-346 */
void orc_padones_fwd(const float *x, float *y, long M, long K);        /* src/autograd.c:195-212 */
void orc_padones_bwd(const float *g, float *dx, long M, long K);       /* src/autograd.c:348-359 */
/* seed = (p - onehot(y)) / rows in fp32, as NumPy computes it in the
 * reference harness (tests/gate_cifar_cnn.py:175-181); returns the mean CE
 * loss -log(max(p[y], 1e-12)) in double. */
double orc_ce_seed(const float *p, const int *labels, long rows, int cols, float *seed);

/* ---- whole training steps (forward + softmax + CE seed + full backward) ----
 * MLP of tests/gate_mnist_mlp.py:68-71 with dims d0->d1->d2->d3:
 *   x (B x d0), W1 (d0+1 x d1), W2 (d1+1 x d2), W3 (d2+1 x d3)
 * Outputs logits, probs (B x d3) and dW1..dW3; returns the loss (or NaN on OOM). */
double orc_mlp_step(int B, int d0, int d1, int d2, int d3, const float *x, const int *labels,
                    const float *W1, const float *W2, const float *W3, float *logits, float *probs,
                    float *dW1, float *dW2, float *dW3, int nthreads);
/* CNN of BASELINE config 4 (tests/gate_cifar_cnn.py:101-111 with two conv
 * blocks): x (B x C0 x H x W) -> conv3x3 pad1 F1 -> relu -> maxpool2 ->
 * conv3x3 pad1 F2 -> relu -> maxpool2 -> reshape -> padones -> matmul Wfc
 * ((F2*H/4*W/4 + 1) x classes).  Outputs logits/probs and all grads. */
double orc_cnn_step(int B, int C0, int H, int W, int F1, int F2, int classes, const float *x,
                    const int *labels, const float *w1, const float *b1, const float *w2,
                    const float *b2, const float *wfc, float *logits, float *probs, float *dw1,
                    float *db1, float *dw2, float *db2, float *dwfc, int nthreads);

/* ---- seeded input generation (splitmix64 + Box-Muller), shared with bench ---- */
void orc_fill_uniform(float *x, long n, float lo, float hi, unsigned long long seed);
void orc_fill_normal(float *x, long n, float stddev, unsigned long long seed);
void orc_fill_labels(int *y, long n, int classes, unsigned long long seed);

#ifdef __cplusplus
}
#endif
#endif
