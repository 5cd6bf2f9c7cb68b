/* Internal declarations shared by tensor.c, ops.c and autograd.c. */
#ifndef TT_INTERNAL_H
#define TT_INTERNAL_H

#include "tensor.h"
#include "autograd.h"
#include "tt_hip.h"
#include "tt_rt.h"

#define TT_V_DEV  1
#define TT_V_HOST 2
/* valid == 0: no copy is current (the kernel that was to write it failed) */

/* device tensor without zero fill (the producing kernel writes every element) */
Tensor *tt_empty_dev(const long *shape, int ndim);
Tensor *tt_empty_like(const Tensor *a);
void    tt_mark_dev_written(Tensor *t);

/* conv2d forward that can hand back its im2col matrix (Kc x Ncol floats of
 * device memory owned by the caller, release with ttrt_free); with ones_row
 * the matrix gets a (Kc+1)-th row of ones for the fused bias gradient */
int tt_conv_use_implicit(long col_bytes);
Tensor *tt_conv2d_keepcol(const Tensor *a, const Tensor *w, const Tensor *b,
                          int stride_h, int stride_w, int pad_h, int pad_w, float **col_out,
                          int ones_row);

/* A forward convolution of ag_conv2d (or the copy of ag_reshape) whose
 * launch waits for the next call into the library: when that call is ag_relu
 * on the convolution's output, the relu is computed by the same launch
 * (tt_k_conv2d_relu_fwd_lds); ag_padones on the copy's output likewise
 * (tt_k_copy_padones_fwd); any other call
 * launches it first (tt_flush_pending from tt_dev, tt_data, tth_sync and
 * ag_release), so every later kernel is still enqueued after it. */
#define TT_PEND_CONV 1
#define TT_PEND_COPY 2        /* ag_reshape's copy; ag_padones of it fuses */
#define TT_PEND_RELU 3        /* ag_relu; ag_padones of it fuses */
#define TT_PEND_MATMUL 4      /* ag_matmul (x * w); ag_relu of it waits with it */
#define TT_PEND_MATMUL_RELU 5 /* ag_matmul and ag_relu of it (r); ag_padones of r fuses */
#define TT_PEND_CONV_RELU 6   /* ag_conv2d and ag_relu of it (r); a 2x2 ag_maxpool2d of r waits too */
#define TT_PEND_CONV_RELU_POOL 7  /* ... and the 2x2 max pool of r (p); ag_reshape of p waits too */
#define TT_PEND_CONV_RELU_POOL_COPY 8  /* ... and that reshape's copy (c); ag_padones of c fuses */
/* with tt_pend1 (a two-convolution chain): ... and the padones of c (d) */
#define TT_PEND_CHAIN_PAD 9
/* ... and the matmul of d (fco = c * fcw[:K] + fcw[K], fcn columns): an
 * ag_softmax_ce of fco takes the classifier's partial sums from the chain's
 * own launch */
#define TT_PEND_CHAIN_FC 10
typedef struct {
    int active;               /* 0 or one of TT_PEND_* */
    Tensor *out;              /* the pending output (owned by its node) */
    Tensor *r;                /* *_RELU* kinds: the relu output (owned by its node) */
    Tensor *p, *c;            /* the pool output, the reshape's copy (owned by their nodes) */
    const float *x, *w, *b;   /* device operands, retained by the node's parents (matmul: b is
                                 the weights' last row when x is a padones input) */
    Tensor *xt;               /* conv kinds: the input tensor x belongs to */
    Tensor *d;                /* TT_PEND_CHAIN_*: the padded copy */
    Tensor *fco;              /* TT_PEND_CHAIN_FC: the classifier's output, */
    const float *fcw;         /* its weights (K + 1 rows of fcn, the last the bias) */
    int fcn;
    int geo[13];              /* conv: N C H W F HH WW sh sw ph pw Ho Wo; matmul: M N K */
    Tensor *codes;            /* *_POOL* kinds: the pool windows' codes (bytes in a float */
    Tensor **codes_dst;       /* tensor, or NULL), handed to the pool node's field here
                                 once written */
} TTPendConv;
extern TTPendConv tt_pend;
/* The first convolution of a chain conv -> relu -> pool -> conv (kind
 * TT_PEND_CONV_RELU_POOL, its pool output the input of the convolution
 * pending in tt_pend): when the second one has its relu and pool too, one
 * launch runs both (tt_k_conv2d_chain_fwd); otherwise it is flushed first. */
extern TTPendConv tt_pend1;
int tt_flush_pending(void);   /* 0 ok; <0 the pending output is invalid */
/* whether the pending chain (tt_pend1 + tt_pend) can run as one launch */
int tt_chain_ready(void);
/* the chain tt_pend1 + tt_pend (pooled) in one launch, with the padded copy
 * and the classifier of the TT_PEND_CHAIN_* kinds; fcpart (TT_PEND_CHAIN_FC
 * only): the classifier's partial sums go there (2 x rows x fcn) and its
 * output is left to the caller, else the classifier's GEMM runs after the
 * chain.  0 launched (both cleared), 1 not possible here (nothing done) */
int tt_chain_launch(float *fcpart);
int tt_flush_first(void);
int tt_chain_enabled(void);   /* tth_conv_chain on (and deferral on) */     /* launch tt_pend1 by itself (tt_pend stays pending) */
/* out = conv(x, w) + b by the direct kernel, else the GEMM path; q holds
 * N C H W F HH WW sh sw ph pw Ho Wo.  0 ok */
int tt_conv_fwd_any(const float *x, const float *w, const float *b, float *out, const int *q);
/* t (allocated, unwritten) = conv(x, w) + b with w | b the F*K + F floats of
 * snap (device memory the recipe then owns and frees), q as above; written on
 * first use.  0 ok, -1 no memory (snap is not taken) */
int tt_lazy_conv(Tensor *t, Tensor *x, float *snap, const int *q);
/* t (allocated, unwritten) = relu(src), written on first use (tensor.c) */
int tt_lazy_relu(Tensor *t, Tensor *src);
int tt_lazy_padones(Tensor *t, Tensor *src);  /* t (M x K+1) = padones(src (M x K)) */
int tt_lazy_ce_mean(Tensor *t, Tensor *src);  /* t (1) = mean of the row losses src */
/* dw, db (db may be NULL) = the pending reduction job; 0 ok, -1 (no memory):
 * run the job now */
int tt_lazy_dwt(Tensor *dw, Tensor *db, const TTDwtJob *job);
/* w[i] -= lr * g[i] (count <= TT_SGD_MAX) with every pending reduction in the
 * same launch when some g[i] is one's output; 1: none is (or the step does
 * not fit one launch) -- take the plain way, nothing done; 0 ok; < 0 error */
int tt_lazy_dwt_sgd(float *const *w, Tensor *const *g, const long *n, int count, float lr);
/* dw (Kx+1 x N) = [x, 1]^T g, the weight gradient of a matmul of padones(x)
 * (x rows x Kx, g rows x N), written on first use; 0 ok, -1 no memory */
int tt_lazy_gemm_tn_padones(Tensor *dw, Tensor *x, Tensor *g, int rows, int Kx, int N);
/* t (M x K elements) = src (M x (K + 1)) without its last column -- the
 * padones backward -- written on first use; 0 ok, -1 no memory */
int tt_lazy_padones_bwd(Tensor *t, Tensor *src, long M, long K);
/* *flag = 1 when src is about to be written in place or through its host
 * copy (the accesses that run recipes reading src); tt_lazy_guard_drop
 * removes the guards of flag.  0 ok, -1 no memory */
int tt_lazy_guard(Tensor *src, int *flag);
void tt_lazy_guard_drop(int *flag);
/* as tt_lazy_dwt_sgd, for one or two pending tt_lazy_gemm_tn_padones
 * gradients: the GEMMs (stepping their weights) and the other tensors' steps
 * in one launch */
int tt_lazy_gemm_sgd(float *const *w, Tensor *const *g, const long *n, int count, float lr);
/* out = logits, probs, seed, row losses of a softmax-CE (allocated,
 * unwritten): one ttk_reduce_ce of ws (2 x M x N partial sums, then owned by
 * the recipe), the bias (the last row of the classifier weights w, which the
 * recipe retains) and the labels (copied), run on the first use of any of
 * them.  0 ok, -1 no memory (nothing registered) */
int tt_lazy_ce_job(Tensor *const out[4], Tensor *w, float *ws, const float *bias,
                   const int32_t *labels, int M, int N, float scale);
/* t pending in such a job: its arguments for ttk_head_bwd_ce (*job set); -1
 * otherwise.  tt_lazy_ce_done(job): a kernel wrote the job's outputs */
int tt_lazy_ce_args(const Tensor *t, TTHeadCeArgs *a, void **job);
void tt_lazy_ce_done(void *job);
/* t is about to be changed in place: run the recipes that read it */
void tt_lazy_before_write(Tensor *t);
Tensor *tt_lazy_relu_src(const Tensor *t);  /* src while t is still unwritten */
int tt_defer_enabled(void);
Tensor *tt_reshape_ex(const Tensor *a, const long *new_shape, int new_ndim, int defer);
Tensor *tt_conv2d_keepcol_ex(const Tensor *a, const Tensor *w, const Tensor *b,
                             int stride_h, int stride_w, int pad_h, int pad_w, float **col_out,
                             int ones_row, int defer);

#endif
