/* Device-level C ABI of the MI355X backend: runtime control and the HIP
 * kernels behind tensor.h / autograd.h, callable on raw device pointers.
 *
 * All pointers named d* / the kernel operands are DEVICE pointers obtained
 * from tth_malloc (or any hipMalloc'd memory of the current device); sizes
 * are element counts unless stated.  Every kernel is enqueued on the
 * library's single HIP stream (tth_stream) and returns 0 on a successful
 * launch, negative on bad arguments or launch failure.  Completion is
 * observed with tth_sync / tth_event_* or any copy back to the host.
 *
 * Each kernel cites the reference function it replaces. */
#ifndef TINYTORCH_TT_HIP_H
#define TINYTORCH_TT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime ---- */
int    tth_available(void);            /* 1 when a GPU is usable */
int    tth_device_name(char *buf, int len);
void  *tth_stream(void);               /* hipStream_t every kernel runs on */
int    tth_sync(void);                 /* wait for the stream; 0 ok */
int    tth_last_error(void);           /* last runtime error code (0 none) */
void  *tth_malloc(size_t bytes);       /* cached device allocation; NULL on OOM */
void   tth_free(void *d);
void   tth_release_cache(void);
/* Test hook: every device allocation after the next n fails (n < 0: none
 * fails), as TT_FAIL_ALLOC_AFTER=n in the environment does from the first
 * allocation; exercises the NULL-on-out-of-memory paths of the C ABI. */
int    tth_fail_alloc_after(long n);
size_t tth_bytes_in_use(void);
int    tth_h2d(void *d, const void *h, size_t bytes);
int    tth_d2h(void *h, const void *d, size_t bytes);
/* device payload of a tensor (uploads a host-modified mirror first) */
struct Tensor;
float *tt_dev(struct Tensor *t);
/* stream-ordered timing: events recorded on tth_stream */
void  *tth_event_create(void);
int    tth_event_record(void *ev);
float  tth_event_elapsed_ms(void *start, void *stop);  /* syncs on stop */
void   tth_event_destroy(void *ev);

/* ---- GEMM (gemm.hip) ----
 * C[M x N] = opA[M x K] * opB[K x N], fp32 in / fp32 MFMA accumulate / fp32 out.
 *   transA = 0: A is M x K row-major, element (m,k) at A[m*lda + k]
 *   transA = 1: A is K x M row-major, element (m,k) at A[k*lda + m]
 *   transB = 0: B is K x N row-major, element (k,n) at B[k*ldb + n]
 *   transB = 1: B is N x K row-major, element (k,n) at B[n*ldb + k]
 * (0,0) replaces tt_sgemm_rowmajor   reference src/gemm.c:569-641
 * (0,1) replaces matmul_nt (dA=dC*B^T) reference src/autograd.c:66-84
 * (1,0) replaces matmul_tn (dB=A^T*dC) reference src/autograd.c:87-103 */
int tt_k_gemm(int M, int N, int K,
              const float *A, int lda, int transA,
              const float *B, int ldb, int transB,
              float *C, int ldc);

/* C = A * B + bias (row-major; bias a row of N) with the softmax-CE of C's
 * rows in the GEMM's split-K reduction: probs, seed = (p - onehot(label)) *
 * scale and rowloss[r] = -log max(p[label], 1e-12), labels on the host
 * (M <= TT_CE_ARG_ROWS, N <= 32) -- the matmul of the classifier and
 * softmax-CE of the reference harness (tests/gate_cifar_cnn.py:175-181)
 * in one pass over the partial products, bit for bit the GEMM followed by
 * tt_k_softmax_ce_mean_hostlab (whose mean the row losses give, summed in
 * its order, by tt_k_ce_mean_rows).  0: all written; 1: only C (the GEMM
 * took no split-K path; run the softmax-CE); < 0: error. */
int tt_k_gemm_bias_ce(int M, int N, int K, const float *A, const float *B, const float *bias,
                      float *C, const int32_t *host_labels, float *probs, float *seed,
                      float *rowloss, float scale);
/* loss[0] = the mean of rowloss (rows floats) summed as
 * tt_k_softmax_ce_mean_hostlab sums its row losses (the loss of a
 * tt_k_gemm_bias_ce pass) */
int tt_k_ce_mean_rows(const float *rowloss, float *loss, int rows);

/* tt_k_gemm without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as tt_k_gemm (bit-identical), but the
 * workspace some shapes need (split-K partials) comes from one static
 * device array of TT_GEMM_SCRATCH_BYTES per GPU, held until the process
 * ends, instead of the caching allocator.  A shape whose workspace exceeds it returns
 * TT_E_SCRATCH with nothing launched (also reported by tth_last_error).
 * Every call on a GPU shares that GPU's array and leaves its contents behind
 * (the kernels write every workspace element before reading it, so nothing
 * needs clearing).  Calls that could overlap on one GPU race on the array:
 * the library enqueues all of them on its one stream, which orders them; do
 * not run them from several threads or processes on one GPU at once. */
#define TT_GEMM_SCRATCH_BYTES (32L << 20)
#define TT_E_SCRATCH (-4)
int tt_k_gemm_noalloc(int M, int N, int K,
                      const float *A, int lda, int transA,
                      const float *B, int ldb, int transB,
                      float *C, int ldc);

/* Tuning hook: force the GEMM tile (0: 128x128, 1: 128x64, 2: 64x64, 3: 32x256,
 * 4: 64x256, 5: 256x256, 6: 256x128, 7: 64x128, 8: 32x128, 9: 64x64 with 64-k
 * stages, 10: 32x128 with 64-k stages) and/or split-K count for every later
 * call; -1 restores the automatic choice. */
int tth_gemm_config(int tile, int splits);
/* Tuning hook: 0 disables, 1 (default) enables the direct-to-LDS kernel used
 * for plain GEMMs (any transposition) on whole 256x256 tiles. */
int tth_gemm_direct(int on);
/* Tuning hook: 0 disables, 1 (default) enables the 64x64 direct-load kernel
 * used for plain GEMMs too small for 128x128 tiles on every CU (and for
 * ragged or unaligned operands); 2 enables it with the k tiles shared by the
 * workgroup's waves (a barrier a tile) instead of a load ring per wave (same
 * results); a forced tile (tth_gemm_config) bypasses it. */
int tth_gemm_mid(int on);
/* Tuning hook for tests: 1 sends every plain GEMM that the 64x64
 * direct-load kernel covers to it whatever its size (below the sizes where
 * it pays off, and ahead of the 32x32 register kernel); 0 (default) off. */
int tth_gemm_mid_force(int on);
/* Tuning hook: 0 disables, 1 (default) enables the 32x32-tile register
 * kernel (K split over the waves of a workgroup, no split-K workspace) used
 * for plain GEMMs below 2^29 flops with at least 128 output tiles whose
 * k-contiguous operands have 16-byte aligned rows. */
int tth_gemm_small(int on);
/* Tuning hook: 0 disables, 1 (default) enables the 16x16-tile kernels (K
 * split over eight waves, each loading its whole slice before its MFMAs):
 * tt_k_gemm_bias_relu_pad's for 256-1024 output tiles of 16x16, K <= 1024,
 * 16-byte aligned A rows; and the split-K partials of GEMMs with N <= 16
 * and K >= 2048 (at most 128 tiles). */
int tth_gemm_t16(int on);
/* Diagnostics: how many classifier backward rules took the input gradients
   that the classifier's softmax-CE launch formed with the seed (instead of a
   classifier backward kernel).  No counterpart in the reference. */
long tth_ce_spec_count(void);

/* Convolution GEMMs over the im2col matrix col[(c,kh,kw)][(n,ho,wo)]
 * (Kc = C*HH*WW rows, Ncol = N*Ho*Wo columns, HW = Ho*Wo):
 *   conv_fwd : out[n][f][hw] = sum_c W[f][c] col[c][p] + bias[f] (bias may be NULL)
 *              reference src/ops_spatial.c:96-121 (GEMM + bias + NCHW permute)
 *   conv_dw  : dW[f][c] = sum_p g[n][f][hw] col[c][p]
 *              reference src/autograd.c:487-507 (g_perm + sgemm_A_Bt_local)
 *   conv_dcol: dcol[c][p] = sum_f W[f][c] g[n][f][hw]
 *              reference src/autograd.c:515-539 (W^T copy + g_perm + sgemm) */
int tt_k_conv_fwd(int F, int Kc, long Ncol, int HW,
                  const float *W, const float *col, const float *bias, float *out);
int tt_k_conv_dw(int F, int Kc, long Ncol, int HW,
                 const float *g, const float *col, float *dW);
int tt_k_conv_dcol(int F, int Kc, long Ncol, int HW,
                   const float *W, const float *g, float *dcol);
/* conv_dw fused with the bias gradient (reference src/autograd.c:467-482):
 * col1 is the im2col matrix with one extra row of ones (Kc + 1 rows, see
 * tt_k_im2col_ones), db[f] = sum_p g[n][f][hw] comes out of the same GEMM. */
int tt_k_conv_dw_bias(int F, int Kc, long Ncol, int HW,
                      const float *g, const float *col1, float *dW, float *db);

/* dW = [X, 1]^T * G ((Kx+1) x N) for X (rows x Kx) and G (rows x N): the
 * weight gradient of a matmul of padones(X) (reference src/autograd.c:168-171
 * on src/autograd.c:195-212's output) computed from X itself, the ones
 * column taken as a row of ones in the MFMA tiles -- bit for bit tt_k_gemm on
 * the padded matrix, where that takes the small-GEMM kernel; -1 elsewhere,
 * nothing launched.  dW == NULL: 0 when the shape is covered, -1 when not. */
int tt_k_gemm_tn_padones(int rows, int Kx, int N, const float *X, const float *G, float *dW);

/* ---- bandwidth kernels (elementwise.hip / spatial.hip) ---- */
int tt_k_fill(float *x, long n, float v);
int tt_k_copy(float *dst, const float *src, long n);
int tt_k_add_inplace(float *dst, const float *src, long n);          /* accum: src/autograd.c:52-63 */
int tt_k_relu_fwd(const float *x, float *y, long n);                  /* src/ops.c:104-106 */
int tt_k_relu_bwd(const float *x, const float *g, float *dx, long n); /* src/autograd.c:318-327 */
int tt_k_binary(const float *a, const float *b, float *y, long n, int op); /* 0 add, 1 mul: src/ops.c:26-52 */
int tt_k_scalar(const float *a, float *y, long n, float s, int op);        /* 0 add, 1 mul: src/ops.c:71-78 */
int tt_k_softmax_fwd(const float *x, float *y, long rows, int cols);       /* src/ops.c:108-145 */
int tt_k_softmax_bwd(const float *s, const float *g, float *dx, long rows, int cols); /* src/autograd.c:329-346 */
/* probs = softmax(logits); loss_rows[r] = -log(max(probs[r][y_r], 1e-12));
 * seed = (probs - onehot(y)) * scale.  Harness math of
 * reference tests/gate_cifar_cnn.py:175-181 on the device. */
int tt_k_softmax_ce(const float *logits, const int32_t *labels, float *probs,
                    float *loss_rows, float *seed, long rows, int cols, float scale);
/* Same, for rows <= TT_CE_MEAN_MAX_ROWS, in one launch that also reduces the
 * mean loss into loss_mean[0] (fixed reduction order). */
#define TT_CE_MEAN_MAX_ROWS 8192
int tt_k_softmax_ce_mean(const float *logits, const int32_t *labels, float *probs,
                         float *loss_mean, float *seed, long rows, int cols, float scale);
/* Same, with the labels read from HOST memory at the call and handed to the
 * kernel inside its launch arguments (no device label buffer, no copy before
 * the launch); rows <= TT_CE_ARG_ROWS. */
#define TT_CE_ARG_ROWS 512
int tt_k_softmax_ce_mean_hostlab(const float *logits, const int32_t *host_labels, float *probs,
                                 float *loss_mean, float *seed, long rows, int cols, float scale);
/* Backward of a classifier layer, one launch: dW (K x N) = A^T * G summed over m
 * ascending (reference matmul_tn, src/autograd.c:87-103) and dA (M x K) =
 * G * W^T summed over j ascending (reference matmul_nt, :66-84), both
 * bit-identical to the reference loops; either may be NULL.  d1 / d2
 * (optional, need dA): dA without its last column (M x (K-1)) -- the
 * padones backward (:348-359); d2 is masked by R > 0 when R is given (the
 * relu backward through the relu output R, :318-327).  N <= 32 and, with
 * dW, M <= 480 (a block of A is staged in LDS), else -1. */
int tt_k_head_bwd(const float *A, int M, int K, const float *W, int N, const float *G,
                  float *dW, float *dA, float *d1, float *d2, const float *R);
/* tt_k_head_bwd (R = NULL) where d2 is the gradient of a 2x2 / stride-2 max
 * pool (F x Ho2 x Wo2 per row, K - 1 = F * Ho2 * Wo2) of a relu output whose
 * windows' codes are given (tt_k_conv2d_relu_pool_fwd_lds): dc (N x F x
 * 2Ho2 x 2Wo2) gets the pool + relu backward of d2 in the same launch (the
 * reference's src/autograd.c:555-594 then :318-327), bit for bit
 * tt_k_maxpool2x2_code_relu_bwd of d2 (d1 and d2 themselves may be NULL;
 * dA is required).  -1: shapes or alignment outside it. */
int tt_k_head_bwd_pool(const float *A, int M, int K, const float *W, int N, const float *G,
                       float *dW, float *dA, float *d1, float *d2, const unsigned char *codes,
                       float *dc, int F, int Ho2, int Wo2);
/* Both gradients of a matmul C = A * B (A M x K, B K x N; reference
 * src/autograd.c:66-103, matmul_nt for dA = G * B^T and matmul_tn for
 * dB = A^T * G) in ONE launch, when tt_k_gemm would compute each with its
 * small-GEMM kernel -- the same values as the two tt_k_gemm calls -- with
 * the d1 / d2 / R epilogue of tt_k_head_bwd on dA.  -1: not covered,
 * nothing launched. */
int tt_k_matmul_bwd_small(const float *A, int M, int K, const float *B, int N, const float *G,
                          float *dB, float *dA, float *d1, float *d2, const float *R);
/* y = x * s[0], s a device scalar (chain rule through a scalar loss) */
int tt_k_scale_by_dev(const float *x, const float *s, float *y, long n);
int tt_k_padones_fwd(const float *x, float *y, long M, long K);      /* src/autograd.c:195-212 */
/* c = x (M*K floats) and y = padones(x) (M x K+1) from one read of x: a
 * reshape (src/ops_spatial.c:22-34, a copy) followed by ag_padones
 * (src/autograd.c:195-212).  M < 65536, K < 2^30, else -1. */
int tt_k_copy_padones_fwd(const float *x, float *c, float *y, long M, long K);
/* r = relu(x) (M*K floats) and y = padones(r) (M x K+1) from one read of x:
 * ag_relu (src/ops.c:104-106) followed by ag_padones (src/autograd.c:195-212).
 * M < 65536, K < 2^30, else -1. */
int tt_k_relu_padones_fwd(const float *x, float *r, float *y, long M, long K);
/* C = A * B (row-major, contiguous; ag_matmul, reference
 * src/autograd.c:168-171) with the relu and padones that follow it in an MLP
 * layer (src/autograd.c:173-193, src/autograd.c:195-212): R = relu(C), P = [R, 1]
 * (M x N+1).  The three outputs of tt_k_gemm then tt_k_relu_padones_fwd,
 * bit for bit, written by the GEMM's split-K reduction when it has one. */
int tt_k_gemm_relu_pad(int M, int N, int K, const float *A, const float *B, float *C, float *R,
                       float *P);
/* C = A * B + bias (A M x K, B K x N row-major, contiguous; bias a row of N
 * added to every row of C), and when R, P are given R = relu(C),
 * P = [R, 1]: ag_matmul of a padones output (src/autograd.c:168-171,
 * 195-212) computed from the padones input X and the weights W, as
 * X * W[:K] + W[K] -- the same sum as the padded product, not the same
 * rounding order.  R and P both or neither. */
int tt_k_gemm_bias_relu_pad(int M, int N, int K, const float *A, const float *B,
                            const float *bias, float *C, float *R, float *P);
/* padones backward (src/autograd.c:348-359) written to two buffers: d1 and
 * d2 both get g without its last column; the backward pass uses it when the
 * padded tensor is a reshape (src/autograd.c:361-369, a copy of the
 * gradient) so the reshape's input gradient needs no second pass.
 * M < 65536, K < 2^30, else -1. */
int tt_k_padones_bwd2(const float *g, float *d1, float *d2, long M, long K);
int tt_k_padones_bwd(const float *g, float *dx, long M, long K);     /* src/autograd.c:348-359 */
/* padones backward and the backward of the relu whose output r (M x K) was
 * padded, in one pass: dr = g without its last column, dx = dr where r > 0
 * else +0.0f (src/autograd.c:348-359 followed by src/autograd.c:318-327 of
 * the reference).  -1: M >= 65536 (the caller runs the two steps). */
int tt_k_padones_relu_bwd(const float *g, const float *r, float *dr, float *dx, long M, long K);
int tt_k_im2col(const float *x, float *col, int N, int C, int H, int W,
                int HH, int WW, int sh, int sw, int ph, int pw, int Ho, int Wo);  /* src/ops_spatial.c:37-69 */
/* im2col followed by a row of Ncol ones (col has Kc + 1 rows) */
int tt_k_im2col_ones(const float *x, float *col, int N, int C, int H, int W,
                     int HH, int WW, int sh, int sw, int ph, int pw, int Ho, int Wo);
int tt_k_col2im(const float *col, float *x, int N, int C, int H, int W,
                int HH, int WW, int sh, int sw, int ph, int pw, int Ho, int Wo);  /* src/autograd.c:406-434 */
int tt_k_bias_grad(const float *g, float *db, int N, int F, int HW);              /* src/autograd.c:467-482 */
int tt_k_maxpool_fwd(const float *x, float *y, int N, int C, int H, int W,
                     int ph, int pw, int sh, int sw, int Ho, int Wo);             /* src/ops_spatial.c:129-164 */
int tt_k_maxpool_bwd(const float *x, const float *g, float *dx, int N, int C, int H, int W,
                     int ph, int pw, int sh, int sw, int Ho, int Wo);             /* src/autograd.c:555-594 */
/* 2x2 / stride-2 max pool backward and the backward of the relu whose output
 * x is the pool's input, in one pass: dx as tt_k_maxpool_bwd, dxr = dx where
 * x > 0 else +0.0f (src/autograd.c:555-594 followed by src/autograd.c:318-327
 * of the reference, which runs them as two steps).  dx may be NULL: then only
 * dxr is written.  -1: shape or alignment outside the 2x2 kernel. */
int tt_k_maxpool2x2_relu_bwd(const float *x, const float *g, float *dx, float *dxr, int N, int C,
                             int H, int W, int Ho, int Wo);
/* The same from the relu's INPUT xpre: the relu (xpre > 0 ? xpre : +0) is
 * taken as each value is read, so the results are bit for bit those of
 * tt_k_maxpool2x2_relu_bwd on the relu's output (for callers that did not
 * store that output). */
int tt_k_maxpool2x2_prerelu_bwd(const float *xpre, const float *g, float *dx, float *dxr, int N,
                                int C, int H, int W, int Ho, int Wo);
/* dxr of tt_k_maxpool2x2_relu_bwd from the pool windows' codes of
 * tt_k_conv2d_relu_pool_fwd_lds instead of the relu output (H = 2 Ho,
 * W = 2 Wo, W % 4 == 0): bit for bit the same, reading a byte per window
 * instead of four floats.  -1: shape or alignment outside the kernel. */
int tt_k_maxpool2x2_code_relu_bwd(const unsigned char *codes, const float *g, float *dxr, int N,
                                  int C, int H, int W, int Ho, int Wo);
int tt_k_avgpool_fwd(const float *x, float *y, int N, int C, int H, int W,
                     int ph, int pw, int sh, int sw, int Ho, int Wo);             /* src/ops_spatial.c:166-201 */
int tt_k_avgpool_bwd(const float *g, float *dx, int N, int C, int H, int W,
                     int ph, int pw, int sh, int sw, int Ho, int Wo);             /* src/autograd.c:596-628 */
/* C (M x N) = A (M x K) * B (K x N), row-major, with the arithmetic of the
 * reference's naive tt_matmul (src/ops.c:84-101): per output, +0.0 plus
 * a*b for k ascending, terms with a == 0 skipped (a NaN or Inf in B meets a
 * zero of A without reaching C); bit-identical to it. */
int tt_k_matmul_naive(const float *A, const float *B, float *C, int M, int N, int K);
int tt_k_sgd(float *w, const float *g, long n, float lr);  /* harness SGD: tests/gate_mnist_mlp.py:121-124 */
/* w[i] -= lr * g[i] for count <= TT_SGD_MAX tensors in one launch */
#define TT_SGD_MAX 16
int tt_k_sgd_multi(float *const *w, const float *const *g, const long *n, int count, float lr);
/* SGD with momentum, per tensor i (count <= TT_SGD_MAX, one launch), fp32 as
 * NumPy evaluates tests/gate_mnist_mlp.py:121-124:
 *   v = (mu * v) - (lr * g);  w = w + v                                  */
int tt_k_momentum_multi(float *const *w, const float *const *g, float *const *v, const long *n,
                        int count, float lr, float mu);
/* Adam, per tensor i (count <= TT_SGD_MAX, one launch), as NumPy evaluates
 * tests/gate_cifar_cnn.py:92-98 (fp32 moments, fp64 step):
 *   m = b1*m + omb1*g;  v = b2*v + omb2*(g*g)          (fp32)
 *   w = fp32( fp64(w) - (lr_t * fp64(m)) / fp64(sqrtf(v) + eps) )         */
int tt_k_adam_multi(float *const *w, const float *const *g, float *const *m, float *const *v,
                    const long *n, int count, float b1, float omb1, float b2, float omb2,
                    float eps, double lr_t);
/* Implicit-GEMM convolution: the im2col matrix is never formed; the GEMM's
 * B operand reads x (or the output gradient) directly.  Same results as the
 * explicit im2col + GEMM forms above, to GEMM rounding.  Return -1 (nothing
 * launched) for shapes they do not cover: tensors of 2^31 elements or more;
 * for dX, stride != 1 or padding > kernel-1.
 *   fwd: out (N,F,Ho,Wo) = conv(x, w) + bias        src/ops_spatial.c:71-127
 *   dw:  dw (F, C*HH*WW), db (F, optional)         src/autograd.c:467-513
 *   dx:  dx (N,C,H,W) = conv_transpose(g, w)       src/autograd.c:515-539,406-434 */
/* Convolutions whose im2col matrix would take at least implicit_min_bytes
 * use these implicit forms inside tt_conv2d / ag_conv2d (default 256 MiB;
 * a negative value restores it, 0 uses them wherever they apply). */
int tth_conv_config(long implicit_min_bytes);
int tt_k_conv2d_fwd_implicit(const float *x, const float *w, const float *bias, float *out,
                             int N, int C, int H, int W, int F, int HH, int WW,
                             int sh, int sw, int ph, int pw, int Ho, int Wo);
int tt_k_conv2d_dw_implicit(const float *g, const float *x, float *dw, float *db,
                            int N, int C, int H, int W, int F, int HH, int WW,
                            int sh, int sw, int ph, int pw, int Ho, int Wo);
int tt_k_conv2d_dx_implicit(const float *g, const float *w, float *dx,
                            int N, int C, int H, int W, int F, int HH, int WW,
                            int sh, int sw, int ph, int pw, int Ho, int Wo);

/* Direct convolution with the image rows staged in LDS (conv.hip): the
 * MFMA operands are read through im2col addressing of the staged slab, so
 * no im2col matrix is formed.  Used by tt_conv2d / ag_conv2d wherever
 * tt_k_conv2d_lds_plan reports coverage (bit 0 forward, bit 1 dW/db, bit 2
 * dX; dX needs stride 1 and padding <= kernel-1).  Each entry returns -1
 * (nothing launched) for shapes it does not cover, -2 out of memory, -3
 * launch failure.  tth_conv_lds(0) switches them off (1 on, <0 query); the
 * previous setting is returned.
 *   fwd: out (N,F,Ho,Wo) = conv(x, w) + bias        src/ops_spatial.c:71-127
 *   dw:  dw (F, C*HH*WW), db (F, optional)         src/autograd.c:456-513
 *   dx:  dx (N,C,H,W)                              src/autograd.c:515-539,406-434 */
int tth_conv_lds(int on);
/* 1 (default): tt_k_conv2d_dw_lds uses the tiled, pipelined weight-gradient
 * kernel (blocks of filters x taps x pixels, the next unit staged while the
 * current one multiplies) where it applies (W % 4 == 0, Wo % 8 == 0, 16-byte
 * aligned operands); 0: the per-image kernel.  <0 queries; returns the
 * previous setting. */
int tth_conv_dwt(int on);
/* 1 (default): ag_conv2d leaves its direct-convolution launch pending until
 * the next library call, and an ag_relu on its output computes both in one
 * launch (tt_k_conv2d_relu_fwd_lds); ag_reshape's copy and any other
 * ag_relu likewise, fused with an ag_padones of their output
 * (tt_k_copy_padones_fwd, tt_k_relu_padones_fwd); 0: every convolution,
 * reshape and relu launches at once.
 * <0 queries; the previous setting is returned. */
int tth_conv_relu_fuse(int on);
/* Tuning hook: 0 disables, 1 (default) enables running a conv -> relu ->
 * 2x2 pool -> conv -> relu -> 2x2 pool chain of ag_* calls (the
 * tt_k_conv2d_chain_fwd shape) as one launch; the convolutions' outputs are
 * then recomputed from a snapshot of their filters on first read.  The
 * backward then runs the second convolution's input gradient and the first
 * one's weight gradient as one launch too (tt_k_conv2d_chain_bwd).  Returns
 * the previous setting; -1 only queries. */
int tth_conv_chain(int on);
int tt_k_conv2d_lds_plan(int N, int C, int H, int W, int F, int HH, int WW,
                         int sh, int sw, int ph, int pw, int Ho, int Wo);
int tt_k_conv2d_fwd_lds(const float *x, const float *w, const float *bias, float *out,
                        int N, int C, int H, int W, int F, int HH, int WW,
                        int sh, int sw, int ph, int pw, int Ho, int Wo);
/* Forward convolution and the relu applied to its output in one launch:
 * out = conv(x, w) + bias as tt_k_conv2d_fwd_lds, rout = out > 0 ? out : 0
 * (NaN -> 0), bit-identical to tt_k_conv2d_fwd_lds + tt_k_relu_fwd.
 * Replaces tt_conv2d followed by tt_relu (src/ops_spatial.c:71-127,
 * src/ops.c:55-69,104-106) when the relu consumes the convolution. */
int tt_k_conv2d_relu_fwd_lds(const float *x, const float *w, const float *bias, float *out,
                             float *rout, int N, int C, int H, int W, int F, int HH, int WW,
                             int sh, int sw, int ph, int pw, int Ho, int Wo);
/* The same convolution, its relu and the 2x2 / stride-2 max pool of the relu
 * (reference src/ops_spatial.c:129-164) in one launch: out, rout as in
 * tt_k_conv2d_relu_fwd_lds and pout (N x F x Ho/2 x Wo/2), bit-identical to
 * the three separate steps; cout / dout (may be NULL): the pool output
 * flattened per image once more, as a copy (a reshape to N x F*Ho*Wo/4,
 * src/ops_spatial.c:22-34) and padded with a last column of ones (padones
 * of that, src/autograd.c:195-212).  3x3 kernels with even Ho, Wo whose
 * output rows pair up inside the kernel's pixel blocks (Wo = 32, or
 * 32 % Wo == 0 with 32 / Wo even); -1 otherwise, nothing launched.  rout
 * may be NULL (the relu is pooled but not stored); codes (optional): one
 * byte per pool window, N x F x Ho/2 x Wo/2 -- bits 0-1 the window's argmax
 * (first maximum in top-left, top-right, bottom-left, bottom-right order, as
 * src/autograd.c:555-594 scans), bits 2-5 which relu values are > 0 -- for
 * tt_k_maxpool2x2_code_relu_bwd. */
int tt_k_conv2d_relu_pool_fwd_lds(const float *x, const float *w, const float *bias, float *out,
                                  float *rout, float *pout, float *cout, float *dout,
                                  unsigned char *codes, int N, int C, int H, int W, int F, int HH,
                                  int WW, int sh, int sw, int ph, int pw, int Ho, int Wo);
/* Two tt_k_conv2d_relu_pool_fwd_lds in one launch, for the CNN feature
 * extractor's shape (reference src/ops_spatial.c:71-164 twice, each followed
 * by the relu of src/ops.c:104-106): x (N x C1 x 32 x 32, C1 <= 4) -> 3x3 pad
 * 1 conv with w1 (32 x C1 x 3 x 3) + b1 -> relu -> 2x2 pool = pool1 (N x 32
 * x 16 x 16, codes1) -> 3x3 pad 1 conv with w2 (64 x 32 x 3 x 3) + b2 -> relu
 * -> 2x2 pool = pool2 (N x 64 x 8 x 8, codes2).  The convolutions' outputs
 * are not written; snap1 / snap2 (optional, both or neither; 32*C1*9 + 32
 * and 18432 + 64 floats) get w1 | b1 and w2 | b2 as read (zeros for a NULL
 * bias), from which tt_k_conv2d_fwd_lds recomputes them.  copy2 (pool2 again) and pad2 (N x
 * 4097, pool2 flattened then 1) are optional; b1 / b2 may be NULL.  Bit for
 * bit the two separate launches.  fcpart (optional, fcn == 10 classes): a
 * classifier's partial logits, fcpart[h][n][j] = sum over the 2048 features
 * of image n's half h (flattened pool2, h * 32 + (0..31) of each channel's
 * 64) of feature * fcw[feature][j] (fcw: 4096 x 10 rows, row-major; bias not
 * included) -- the matmul of the flattened pool2 split over the halves.  -1: shape or alignment not covered (H, W,
 * F1, F2 must be 32, 32, 32, 64; x, w2, pool1, pool2, copy2, codes1, codes2
 * 16-byte aligned), nothing launched. */
int tt_k_conv2d_chain_fwd(const float *x, const float *w1, const float *b1, const float *w2,
                          const float *b2, float *pool1, unsigned char *codes1, float *pool2,
                          float *copy2, float *pad2, unsigned char *codes2, float *snap1,
                          float *snap2, const float *fcw, int fcn, float *fcpart, int N,
                          int C1, int H, int W, int F1, int F2);
/* The backward between the chain's two convolutions in one launch (plus the
 * weight-gradient reduction): dx2 (N x 32 x 16 x 16) = the input gradient of
 * the second convolution (w2 64 x 32 x 3 x 3, pad 1) from its output
 * gradient dc2 (N x 64 x 16 x 16) -- the reference's src/autograd.c:515-539
 * + col2im :406-434, bit for bit tt_k_conv2d_dx_lds -- then, through the 2x2
 * pool + relu backward of the pool codes codes1 (src/autograd.c:555-594,
 * :318-327), dw1 / db1 of the first convolution (x N x C1 x 32 x 32, C1 <=
 * 3, 32 filters, 3x3, pad 1; src/autograd.c:456-513), bit for bit
 * tt_k_conv2d_dw_lds_pooled of dx2; with dw2 (db2 optional), in the same
 * grid, the second convolution's weight gradient from dc2 and its input x2
 * (N x 32 x 16 x 16), bit for bit tt_k_conv2d_dw_lds.  -1: not covered
 * (nothing launched). */
int tt_k_conv2d_chain_bwd(const float *dc2, const float *w2, const unsigned char *codes1,
                          const float *x, float *dx2, float *dw1, float *db1, const float *x2,
                          float *dw2, float *db2, int N, int C1);
int tt_k_conv2d_dw_lds(const float *g, const float *x, float *dw, float *db,
                       int N, int C, int H, int W, int F, int HH, int WW,
                       int sh, int sw, int ph, int pw, int Ho, int Wo);
/* dw / db of tt_k_conv2d_dw_lds when the output gradient is that of a relu
 * followed by a 2x2 / stride-2 max pool: computed from the pool's gradient
 * gp (N x F x Ho/2 x Wo/2) and the windows' codes of
 * tt_k_conv2d_relu_pool_fwd_lds, the output gradient decoded in LDS and
 * never stored -- bit for bit tt_k_maxpool2x2_code_relu_bwd followed by
 * tt_k_conv2d_dw_lds (the reference's src/autograd.c:555-594, 318-327 and
 * src/ops_spatial.c:71-127 backward in one step).  dw == NULL: 0 when the
 * shape is covered, -1 when not (nothing launched). */
int tt_k_conv2d_dw_lds_pooled(const float *gp, const unsigned char *codes, const float *x,
                              float *dw, float *db, int N, int C, int H, int W, int F, int HH,
                              int WW, int sh, int sw, int ph, int pw, int Ho, int Wo);
int tt_k_conv2d_dx_lds(const float *g, const float *w, float *dx,
                       int N, int C, int H, int W, int F, int HH, int WW,
                       int sh, int sw, int ph, int pw, int Ho, int Wo);

/* Dataset batch gather + normalisation (see tt_data.h):
 * out[r, j] = ((float)src[idx[r]*sample + j] / 255 - mean[c]) / stdv[c],
 * c = j / plane, channels = sample / plane <= 4.  idx values must be in
 * [0, nsrc): the caller checks them (the kernel trusts them). */
int tt_k_gather_u8_norm(const uint8_t *src, long nsrc, long sample, long plane, int channels,
                        const int64_t *idx, long n, const float *mean, const float *stdv,
                        float *out);

#ifdef __cplusplus
}
#endif
#endif
