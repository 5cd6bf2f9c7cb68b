/* Internal runtime interface shared by the host C layer (tensor.c, ops.c,
 * autograd.c) and the HIP kernel launchers (*.hip).  Everything here is
 * C-ABI; nothing in this header is part of the public tensor.h/autograd.h
 * surface.
 *
 * Execution model: one process, one GPU, one in-order HIP stream owned by
 * the library.  Every kernel is launched on that stream, so a device buffer
 * released back to the caching allocator may be handed out again at once:
 * any later kernel that writes it is ordered after every earlier kernel that
 * read it.  The host only waits on the stream when it copies results out
 * (tt_data / ag_value readers) or when the caller asks (tth_sync). */
#ifndef TT_RT_H
#define TT_RT_H

#include <stddef.h>
#include <stdint.h>
#include "tt_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- runtime (runtime.c) ---- */
int    ttrt_init(void);                 /* 0 ok, <0 no usable GPU */
void  *ttrt_stream(void);               /* hipStream_t of the library */
void  *ttrt_alloc(size_t bytes);        /* stream-ordered cached device alloc; NULL on OOM */
void   ttrt_free(void *p);              /* return to cache (no sync) */
void   ttrt_release_cache(void);        /* hipFree every cached block (syncs) */
int    ttrt_sync(void);                 /* wait for the stream; 0 ok */
int    ttrt_h2d(void *dst, const void *src, size_t bytes);   /* sync copy */
int    ttrt_d2h(void *dst, const void *src, size_t bytes);   /* sync copy */
int    ttrt_h2d_async(void *dst, const void *src, size_t bytes); /* stream-ordered, src reusable at return */
void  *ttrt_host_alloc(size_t bytes);   /* pinned (cached) host block, 64-B aligned; NULL on OOM */
void   ttrt_host_free(void *p);         /* only for ttrt_host_alloc blocks */
int    ttrt_host_is_pinned(const void *p);
void   ttrt_set_error(int code);
int    ttrt_last_error(void);
size_t ttrt_bytes_in_use(void);
size_t ttrt_bytes_cached(void);
/* elementwise.hip: c[m][n] = cin[m][n] + c[m][n] for every (m, n) of the
 * M x N matrices outside the leading mb x nb block */
int    ttk_add_outside(float *c, const float *cin, int M, int N, int mb, int nb);
/* elementwise.hip: c[m][n] += bias[n] for the M x N matrix c, and when r / p
 * are given r = relu(c), p = [r, 1] (M x N+1) */
int    ttk_bias_relu_pad(float *c, const float *bias, float *r, float *p, int M, int N);
/* elementwise.hip: the split-K reduction of a GEMM (ws: S partial M x N
 * products, summed as gemm.hip's reduce_one does with zl lanes an element)
 * plus bias into C, and the softmax-CE of C's rows in the same launch:
 * probs, seed = (p - onehot(label)) * scale, rowloss[r] = -log p[label];
 * labels on the host (rows <= TT_CE_ARG_ROWS).  1: shape not covered
 * (N * zl > 1024, N > 32), nothing launched. */
typedef struct {
    const float *bias;
    const int32_t *host_labels;
    float *probs, *seed, *rowloss;
    float scale;
} TTCeHook;
int    ttk_reduce_ce(const float *ws, float *C, int M, int N, int S, int zl, const TTCeHook *h);
/* head.hip: tt_k_head_bwd / tt_k_head_bwd_pool (codes non-NULL) whose
 * output gradient is the seed of a softmax-CE of the logits formed by the
 * kernel itself from two partial sums per logit (part: 2 x M x N), the bias
 * and the labels -- the values splitk_reduce_ce would give -- and whose
 * workgroup 0 also writes that reduction's outputs (logits, probs, seed,
 * rowloss; each may be NULL).  -1: not covered (nothing launched). */
typedef struct {
    const float *part, *bias;
    const int32_t *labels;
    float scale;
    float *logits, *probs, *seed, *rowloss;
} TTHeadCeArgs;
int    ttk_head_bwd_ce(const float *A, int M, int K, const float *W, int N, const TTHeadCeArgs *a,
                       float *dW, float *dA, float *d1, float *d2, const float *R,
                       const unsigned char *codes, float *dc, int F, int Ho2, int Wo2);
/* conv.hip: a weight gradient whose tiled kernel ran but whose reduction is
 * still to run: the partial sums (owned), the outputs (dw, db; either may
 * be NULL: not written) and the reduction's shape */
typedef struct {
    float *part;
    float *dw, *db;
    int nu, nfb, jbp, F, K, zl, nblk;
} TTDwtJob;
/* conv.hip: tt_k_conv2d_dw_lds (codes NULL) or tt_k_conv2d_dw_lds_pooled
 * (gr the pool gradient) without the reduction, described in *job.  0:
 * launched; -1: not covered (nothing launched); < -1: error. */
int    ttk_conv2d_dwt_defer(const float *gr, const unsigned char *codes, const float *x,
                            float *dw, float *db, const int geo[13], TTDwtJob *job);
/* conv.hip: the CNN chain's middle backward in one launch: dx2 = the input
 * gradient of the second convolution (tt_k_conv2d_dx_lds bits) and the first
 * convolution's weight gradient through the pool codes1 (the job
 * tt_k_conv2d_dw_lds_pooled would defer); with dw2 (db2 optional), the
 * second convolution's weight gradient from dc2 and its input x2 in the same
 * grid (the job tt_k_conv2d_dw_lds would defer, *job2).  -1: not covered. */
int    ttk_conv2d_chain_bwd(const float *dc2, const float *w2, const unsigned char *codes1,
                            const float *x, float *dx2, float *dw1, float *db1, int N, int C1,
                            TTDwtJob *job, const float *x2, float *dw2, float *db2,
                            TTDwtJob *job2);
/* conv.hip: the reductions of n jobs in one launch (the same values as
 * each job's own reduction), then their partials freed; 0 ok */
int    ttk_dwt_reduce_jobs(const TTDwtJob *jobs, int n);
/* conv.hip: the reductions of nj <= 4 jobs and an SGD step (w -= lr * g) in
 * one launch: job q's dw / db are written and, when wdw[q] / wdb[q] are
 * given, those weights stepped with them; the np plain tensors pw are
 * stepped with pg.  Then the jobs' partials are freed.  0 ok; 1: too many
 * jobs or tensors, nothing launched. */
int    ttk_dwt_reduce_sgd(const TTDwtJob *jobs, float *const *wdw, float *const *wdb, int nj,
                          float *const *pw, const float *const *pg, const long *pn, int np,
                          float lr);
/* gemm.hip: tt_k_gemm_tn_padones (dW) with the SGD step wsgd -= lr * dW and
 * the plain steps pw -= lr * pg (np <= TT_SGD_MAX) in one launch; 1: not
 * covered, nothing launched. */
int    ttk_gemm_tn_padones_sgd(int rows, int Kx, int N, const float *X, const float *G,
                               float *dW, float *wsgd, float lr, float *const *pw,
                               const float *const *pg, const long *pn, int np);
/* gemm.hip: tt_k_gemm_tn_padones on every shape its tiles index (not only
 * where the planner picks them); NULL dW only asks.  0 ok, -1 not covered */
int    ttk_gemm_tn_padones_any(int rows, int Kx, int N, const float *X, const float *G,
                               float *dW);
/* the same for up to two jobs (dW = [X, 1]^T G, wsgd -= lr * dW each) */
typedef struct {
    int rows, Kx, N;
    const float *X, *G;
    float *dW, *wsgd;
} TTTnSgdJob;
int    ttk_gemm_tn_padones_sgd_jobs(const TTTnSgdJob *jobs, int nj, float lr, float *const *pw,
                                    const float *const *pg, const long *pn, int np);
/* conv.hip: free a job's partials without reducing them */
void   ttk_dwt_job_drop(TTDwtJob *job);
/* elementwise.hip: C = A * B + bias (A M x K, B K x N row-major) for N <= 16,
 * one workgroup per 16 rows (K < 16: per row), with R = relu(C) / P = [relu(C), 1] when given, or
 * with the softmax-CE of each row when ce is given (ce->bias unused).  1:
 * not covered (N > 16, K > 1024; with ce, M > TT_CE_ARG_ROWS), nothing
 * launched. */
int    ttk_gemm_rows(const float *A, const float *B, const float *bias, float *C, float *R,
                     float *P, int M, int N, int K, const TTCeHook *ce);
/* ttk_gemm_rows with ce and, for the rows' softmax-CE seed g, the backward
 * of the layer's input [A, 1] (B's rows followed by the bias row, bias == B +
 * K * N): dA = g [B; bias]^T (M x (K + 1)), d1 = dA without its last column
 * and d2 = d1 where A > 0 (d1, d2 may be NULL) -- the classifier backward
 * kernel's dA outputs, bit for bit.  1: not covered (the 16-row kernel only:
 * 16 <= K < 512, N <= 16, (K + 1) * N <= 4096), nothing launched. */
int    ttk_gemm_rows_da(const float *A, const float *B, const float *bias, float *C, float *R,
                        float *P, int M, int N, int K, const TTCeHook *ce, float *dA, float *d1,
                        float *d2);

/* gemm.hip: look up, on the current device, the device address of the
 * static scratch array behind tt_k_gemm_noalloc; 0 ok */
int    ttg_scratch_setup(void);

#ifdef __cplusplus
}
#endif
#endif
