/* tt_* tensor ops on the GPU.
 *
 * Each op keeps the reference's argument validation and NULL-on-error
 * behaviour and allocates a fresh output, but the arithmetic is one (or a
 * few) kernel launches on the library stream:
 *   elementwise / scalar / relu / softmax   reference src/ops.c:26-145
 *   matmul (naive, fast, omp)               reference src/ops.c:84-102, src/gemm.c:644-671
 *   reshape / conv2d / maxpool / avgpool     reference src/ops_spatial.c:12-201
 * All three matmul entry points run the same MFMA GEMM; `nthreads` of
 * tt_matmul_omp has no meaning on the GPU and is ignored. */
#include "tt_internal.h"

#include <stdlib.h>
#include <string.h>

static int same_shape(const Tensor *a, const Tensor *b) {
    if (a->ndim != b->ndim) return 0;
    for (int i = 0; i < a->ndim; i++)
        if (a->shape[i] != b->shape[i]) return 0;
    return 1;
}

static Tensor *fail(Tensor *out) {
    tt_release(out);
    return NULL;
}

static Tensor *binary(const Tensor *a, const Tensor *b, int op) {
    if (!a || !b || !same_shape(a, b)) return NULL;
    const float *x = tt_dev((Tensor *)a), *y = tt_dev((Tensor *)b);
    if (!x || !y) return NULL;
    Tensor *out = tt_empty_like(a);
    if (!out) return NULL;
    if (tt_k_binary(x, y, out->dev, a->numel, op)) return fail(out);
    return out;
}

Tensor *tt_add(const Tensor *a, const Tensor *b) { return binary(a, b, 0); }
Tensor *tt_mul(const Tensor *a, const Tensor *b) { return binary(a, b, 1); }

static Tensor *scalar(const Tensor *a, float s, int op) {
    if (!a) return NULL;
    const float *x = tt_dev((Tensor *)a);
    if (!x) return NULL;
    Tensor *out = tt_empty_like(a);
    if (!out) return NULL;
    if (tt_k_scalar(x, out->dev, a->numel, s, op)) return fail(out);
    return out;
}

Tensor *tt_addscalar(const Tensor *a, float s) { return scalar(a, s, 0); }
Tensor *tt_mulscalar(const Tensor *a, float s) { return scalar(a, s, 1); }

static Tensor *matmul2d(const Tensor *a, const Tensor *b) {
    if (!a || !b || a->ndim != 2 || b->ndim != 2) return NULL;
    if (a->shape[1] != b->shape[0]) return NULL;
    if (a->shape[0] > 0x7fffffffL || a->shape[1] > 0x7fffffffL || b->shape[1] > 0x7fffffffL)
        return NULL;
    const int M = (int)a->shape[0], K = (int)a->shape[1], N = (int)b->shape[1];
    const float *x = tt_dev((Tensor *)a), *y = tt_dev((Tensor *)b);
    if (!x || !y) return NULL;
    const long shp[2] = {M, N};
    Tensor *out = tt_empty_dev(shp, 2);
    if (!out) return NULL;
    if (tt_k_gemm(M, N, K, x, K, 0, y, N, 0, out->dev, N)) return fail(out);
    return out;
}

/* The reference's naive matmul (src/ops.c:84-101) keeps its own arithmetic
 * here -- serial k order, zeros of a skipped -- so its results, NaN masking
 * included, are the reference's bit for bit; the fast entries below run the
 * MFMA GEMM. */
Tensor *tt_matmul(const Tensor *a, const Tensor *b) {
    if (!a || !b || a->ndim != 2 || b->ndim != 2) return NULL;
    if (a->shape[1] != b->shape[0]) return NULL;
    if (a->shape[0] > 0x7fffffffL || a->shape[1] > 0x7fffffffL || b->shape[1] > 0x7fffffffL)
        return NULL;
    const int M = (int)a->shape[0], K = (int)a->shape[1], N = (int)b->shape[1];
    const float *x = tt_dev((Tensor *)a), *y = tt_dev((Tensor *)b);
    if (!x || !y) return NULL;
    const long shp[2] = {M, N};
    Tensor *out = tt_empty_dev(shp, 2);
    if (!out) return NULL;
    if (tt_k_matmul_naive(x, y, out->dev, M, N, K)) return fail(out);
    return out;
}
Tensor *tt_matmul_fast(const Tensor *a, const Tensor *b) { return matmul2d(a, b); }
Tensor *tt_matmul_omp(const Tensor *a, const Tensor *b, int nthreads) {
    (void)nthreads;
    return matmul2d(a, b);
}

/* Host pointers in and out, as the reference (src/gemm.c:569-641).  The
 * reference overwrites C only on its main block -- the leading
 * (M/6*6) x (N/16*16) rows and columns, when K > 0 and that block is not
 * empty -- and ADDS the product into C everywhere else (its scalar tails
 * accumulate; with K == 0 or fewer than 16 columns nothing is overwritten).
 * The same contract here: C is uploaded when any element accumulates and
 * added to the product outside the overwritten block. */
int tt_sgemm_rowmajor(int M, int N, int K, const float *A, const float *B, float *C,
                      int nthreads) {
    (void)nthreads;
    if (M <= 0 || N <= 0 || K < 0 || !C || (K > 0 && (!A || !B))) return -1;
    const int Nfull = N / 16 * 16, Msfx = M / 6 * 6;
    const int over = Nfull > 0 && K > 0 && Msfx > 0;
    const int mb = over ? Msfx : 0, nb = over ? Nfull : 0;
    const int accum = !(mb == M && nb == N);
    const size_t sa = sizeof(float) * (size_t)M * (size_t)K;
    const size_t sb = sizeof(float) * (size_t)K * (size_t)N;
    const size_t sc = sizeof(float) * (size_t)M * (size_t)N;
    float *dA = (float *)ttrt_alloc(sa ? sa : 4);
    float *dB = (float *)ttrt_alloc(sb ? sb : 4);
    float *dC = (float *)ttrt_alloc(sc);
    float *dCin = accum ? (float *)ttrt_alloc(sc) : NULL;
    int rc = -1;
    if (dA && dB && dC && (dCin || !accum) && ttrt_h2d(dA, A, sa) == 0 &&
        ttrt_h2d(dB, B, sb) == 0 && (!accum || ttrt_h2d(dCin, C, sc) == 0) &&
        tt_k_gemm(M, N, K, dA, K, 0, dB, N, 0, dC, N) == 0 &&
        (!accum || ttk_add_outside(dC, dCin, M, N, mb, nb) == 0) && ttrt_d2h(C, dC, sc) == 0)
        rc = 0;
    ttrt_free(dA);
    ttrt_free(dB);
    ttrt_free(dC);
    ttrt_free(dCin);
    return rc;
}

Tensor *tt_relu(const Tensor *a) {
    if (!a) return NULL;
    const float *x = tt_dev((Tensor *)a);
    if (!x) return NULL;
    Tensor *out = tt_empty_like(a);
    if (!out) return NULL;
    if (tt_k_relu_fwd(x, out->dev, a->numel)) return fail(out);
    return out;
}

Tensor *tt_softmax(const Tensor *a) {
    if (!a || a->ndim < 1) return NULL;
    const long N = a->shape[a->ndim - 1];
    if (N > 0x7fffffffL) return NULL;
    const float *x = tt_dev((Tensor *)a);
    if (!x) return NULL;
    Tensor *out = tt_empty_like(a);
    if (!out) return NULL;
    if (tt_k_softmax_fwd(x, out->dev, a->numel / N, (int)N)) return fail(out);
    return out;
}

/* ---- spatial ---- */

static int valid_conv_params(int HH, int WW, int sh, int sw, int ph, int pw) {
    return HH > 0 && WW > 0 && sh > 0 && sw > 0 && ph >= 0 && pw >= 0;
}

static int valid_pool_params(int ph, int pw, int sh, int sw) {
    return ph > 0 && pw > 0 && sh > 0 && sw > 0;
}

TTPendConv tt_pend;
TTPendConv tt_pend1;
/* defer ag_conv2d / ag_reshape launches so a relu / padones can fuse */
static int g_conv_relu = 1;
/* a conv -> relu -> pool -> conv -> relu -> pool chain as one launch */
static int g_conv_chain = 1;

int tt_chain_enabled(void) { return g_conv_relu && g_conv_chain; }

int tth_conv_chain(int on) {
    const int prev = g_conv_chain;
    if (on >= 0) {
        tt_flush_pending();
        g_conv_chain = on ? 1 : 0;
    }
    return prev;
}

int tt_defer_enabled(void) { return g_conv_relu; }

Tensor *tt_reshape(const Tensor *a, const long *new_shape, int new_ndim) {
    return tt_reshape_ex(a, new_shape, new_ndim, 0);
}

/* defer: the copy may be left pending in tt_pend (ag_reshape) */
Tensor *tt_reshape_ex(const Tensor *a, const long *new_shape, int new_ndim, int defer) {
    if (!a || !new_shape || new_ndim <= 0 || new_ndim > 8) return NULL;
    long numel = 1;
    for (int i = 0; i < new_ndim; i++) {
        if (new_shape[i] <= 0) return NULL;
        numel *= new_shape[i];
    }
    if (numel != a->numel) return NULL;
    const float *x = tt_dev((Tensor *)a);
    if (!x) return NULL;
    Tensor *out = tt_empty_dev(new_shape, new_ndim);
    if (!out) return NULL;
    if (defer && g_conv_relu) {
        tt_flush_pending();
        tt_pend.out = out;
        tt_pend.x = x;
        tt_pend.active = TT_PEND_COPY;
        return out;
    }
    if (tt_k_copy(out->dev, x, numel)) return fail(out);
    return out;
}

/* Convolutions whose im2col matrix would reach this many bytes run as
 * implicit GEMMs (the matrix is never formed); below it the explicit
 * im2col + GEMM is as fast or faster at the sizes measured, and the forward
 * matrix is kept for the weight gradient. */
static long g_implicit_min_bytes = 256L << 20;

int tth_conv_config(long implicit_min_bytes) {
    g_implicit_min_bytes = implicit_min_bytes < 0 ? (256L << 20) : implicit_min_bytes;
    return 0;
}

int tt_conv_use_implicit(long col_bytes) { return col_bytes >= g_implicit_min_bytes; }


int tth_conv_relu_fuse(int on) {
    const int prev = g_conv_relu;
    if (on >= 0) {
        tt_flush_pending();
        g_conv_relu = on ? 1 : 0;
    }
    return prev;
}

/* The forward convolution without the LDS-staged kernel: the implicit GEMM
 * where it applies (no im2col matrix), else im2col + GEMM.  q holds
 * N C H W F HH WW sh sw ph pw Ho Wo.  0 ok. */
static int conv_fwd_gemm(const float *x, const float *wd, const float *bd, float *out,
                         const int *q) {
    const int N = q[0], C = q[1], H = q[2], W = q[3], F = q[4], HH = q[5], WW = q[6];
    const int sh = q[7], sw = q[8], ph = q[9], pw = q[10], Ho = q[11], Wo = q[12];
    const int Kc = C * HH * WW;
    const long Ncol = (long)N * Ho * Wo;
    if (tt_k_conv2d_fwd_implicit(x, wd, bd, out, N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho,
                                 Wo) == 0)
        return 0;
    float *col = (float *)ttrt_alloc(sizeof(float) * (size_t)Kc * (size_t)Ncol);
    if (!col) return -2;
    const int rc = tt_k_im2col(x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo) ||
                   tt_k_conv_fwd(F, Kc, Ncol, Ho * Wo, wd, col, bd, out);
    ttrt_free(col);
    return rc ? -3 : 0;
}

int tt_conv_fwd_any(const float *x, const float *w, const float *b, float *out, const int *q) {
    if (tt_k_conv2d_fwd_lds(x, w, b, out, q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7], q[8],
                            q[9], q[10], q[11], q[12]) == 0)
        return 0;
    return conv_fwd_gemm(x, w, b, out, q);
}

/* The geometry tt_k_conv2d_chain_fwd takes: q1 the first convolution (C1 <=
 * 4 channels of 32x32 -> 32 filters, 3x3, stride 1, pad 1), q2 the second
 * (its pool output -> 64 filters, the same kernel). */
static int chain_geometry(const int *q1, const int *q2) {
    static const int k[8] = {3, 3, 1, 1, 1, 1};
    for (int i = 0; i < 6; i++)
        if (q1[5 + i] != k[i] || q2[5 + i] != k[i]) return 0;
    return q1[1] >= 1 && q1[1] <= 4 && q1[2] == 32 && q1[3] == 32 && q1[4] == 32 &&
           q1[11] == 32 && q1[12] == 32 && q2[0] == q1[0] && q2[1] == 32 && q2[2] == 16 &&
           q2[3] == 16 && q2[4] == 64 && q2[11] == 16 && q2[12] == 16;
}

/* The convolution outputs of a launched chain were not written: each becomes
 * a recipe recomputing it from the chain's snapshot of its filters and bias
 * (or, without memory for the recipe, is computed now), and its relu a
 * recipe of it. */
static int chain_outputs(const TTPendConv *p, float *snap) {
    int rc = 0;
    if (tt_lazy_conv(p->out, p->xt, snap, p->geo) != 0) {
        rc = tt_conv_fwd_any(p->x, snap, snap + (long)p->geo[4] * p->geo[1] * 9, p->out->dev,
                             p->geo);
        ttrt_free(snap);
    }
    if (rc == 0 && tt_lazy_relu(p->r, p->out) != 0)
        rc = tt_k_relu_fwd(p->out->dev, p->r->dev, p->r->numel);
    if (rc != 0) {
        p->out->valid = 0;
        p->r->valid = 0;
    }
    return rc;
}

int tt_chain_ready(void) {
    const int k = tt_pend.active;
    return tt_pend1.active == TT_PEND_CONV_RELU_POOL &&
           (k == TT_PEND_CONV_RELU_POOL || k == TT_PEND_CONV_RELU_POOL_COPY ||
            k == TT_PEND_CHAIN_PAD || k == TT_PEND_CHAIN_FC) &&
           tt_pend1.codes && tt_pend.codes && tt_pend1.xt && tt_pend.xt == tt_pend1.p &&
           chain_geometry(tt_pend1.geo, tt_pend.geo);
}

/* the classifier of a TT_PEND_CHAIN_FC (the matmul of the padded copy): its
 * GEMM from the flattened copy, the weights' last row added as the bias */
static int chain_fc_gemm(const TTPendConv *b) {
    const int M = (int)b->c->shape[0], K = (int)b->c->shape[1];
    return tt_k_gemm_bias_relu_pad(M, b->fcn, K, b->c->dev, b->fcw, b->fcw + (long)K * b->fcn,
                                   b->fco->dev, NULL, NULL);
}

int tt_chain_launch(float *fcpart) {
    if (!tt_chain_ready() || (fcpart && tt_pend.active != TT_PEND_CHAIN_FC)) return 1;
    const TTPendConv a = tt_pend1, b = tt_pend;
    Tensor *c = b.active != TT_PEND_CONV_RELU_POOL ? b.c : NULL;
    Tensor *pad = b.active >= TT_PEND_CHAIN_PAD ? b.d : NULL;
    const long n1 = 32L * a.geo[1] * 9 + 32, n2 = 64L * 32 * 9 + 64;
    float *s1 = (float *)ttrt_alloc(sizeof(float) * (size_t)n1);
    float *s2 = s1 ? (float *)ttrt_alloc(sizeof(float) * (size_t)n2) : NULL;
    if (!s2 || tt_k_conv2d_chain_fwd(a.x, a.w, a.b, b.w, b.b, a.p->dev,
                                     (unsigned char *)a.codes->dev, b.p->dev,
                                     c ? c->dev : NULL, pad ? pad->dev : NULL,
                                     (unsigned char *)b.codes->dev, s1, s2,
                                     fcpart ? b.fcw : NULL, fcpart ? b.fcn : 0, fcpart,
                                     a.geo[0], a.geo[1], 32, 32, 32, 64) != 0) {
        ttrt_free(s1);
        ttrt_free(s2);
        return 1;
    }
    tt_pend1.active = 0;
    tt_pend.active = 0;
    *a.codes_dst = a.codes;  /* the pool nodes own them now */
    *b.codes_dst = b.codes;
    const int rc1 = chain_outputs(&a, s1), rc2 = chain_outputs(&b, s2);
    int rc3 = 0;
    if (b.active == TT_PEND_CHAIN_FC && !fcpart && (rc3 = chain_fc_gemm(&b)) != 0)
        b.fco->valid = 0;
    if (rc1 || rc2 || rc3) ttrt_set_error(-3);
    return 0;
}

/* Launch the pending kernel.  A convolution whose direct kernel cannot be
 * launched after all runs through conv_fwd_gemm instead.  When nothing can
 * produce the output, the output tensor is marked as holding no valid data,
 * so tt_dev / tt_data on it return NULL (and every op reading it returns
 * NULL), as an op failing at its call would have. */
static int flush_one(void);

int tt_flush_first(void) {
    if (!tt_pend1.active) return 0;
    const TTPendConv second = tt_pend;
    tt_pend = tt_pend1;
    tt_pend1.active = 0;
    const int rc = flush_one();
    tt_pend = second;
    return rc;
}

int tt_flush_pending(void) {
    if (tt_pend1.active) {
        if (tt_chain_launch(NULL) == 0) return 0;
        /* the first convolution by itself, then the second as it stands */
        const TTPendConv second = tt_pend;
        tt_pend = tt_pend1;
        tt_pend1.active = 0;
        const int rc1 = flush_one();
        tt_pend = second;
        const int rc2 = flush_one();
        return rc1 ? rc1 : rc2;
    }
    return flush_one();
}

static int flush_one(void) {
    if (!tt_pend.active) return 0;
    const int kind = tt_pend.active;
    tt_pend.active = 0;
    int rc;
    if (kind == TT_PEND_COPY || kind == TT_PEND_RELU) {
        rc = kind == TT_PEND_COPY ? tt_k_copy(tt_pend.out->dev, tt_pend.x, tt_pend.out->numel)
                                  : tt_k_relu_fwd(tt_pend.x, tt_pend.out->dev, tt_pend.out->numel);
    } else if (kind == TT_PEND_MATMUL || kind == TT_PEND_MATMUL_RELU) {
        const int M = tt_pend.geo[0], N = tt_pend.geo[1], K = tt_pend.geo[2];
        rc = tt_pend.b ? tt_k_gemm_bias_relu_pad(M, N, K, tt_pend.x, tt_pend.w, tt_pend.b,
                                                 tt_pend.out->dev, NULL, NULL)
                       : tt_k_gemm(M, N, K, tt_pend.x, K, 0, tt_pend.w, N, 0, tt_pend.out->dev, N);
        if (kind == TT_PEND_MATMUL_RELU) {
            if (rc == 0) rc = tt_k_relu_fwd(tt_pend.out->dev, tt_pend.r->dev, tt_pend.r->numel);
            if (rc != 0) tt_pend.r->valid = 0;
        }
    } else if (kind == TT_PEND_CONV_RELU || kind == TT_PEND_CONV_RELU_POOL ||
               kind == TT_PEND_CONV_RELU_POOL_COPY || kind == TT_PEND_CHAIN_PAD ||
               kind == TT_PEND_CHAIN_FC) {
        const int *q = tt_pend.geo;
        Tensor *p = kind != TT_PEND_CONV_RELU ? tt_pend.p : NULL;
        Tensor *c = kind >= TT_PEND_CONV_RELU_POOL_COPY ? tt_pend.c : NULL;
        Tensor *d = kind >= TT_PEND_CHAIN_PAD ? tt_pend.d : NULL;
        /* with the pool, the relu output is not stored: it becomes a recipe
         * (relu of the convolution output) run on first use */
        Tensor *codes = p ? tt_pend.codes : NULL;
        rc = p ? tt_k_conv2d_relu_pool_fwd_lds(tt_pend.x, tt_pend.w, tt_pend.b, tt_pend.out->dev,
                                               NULL, p->dev, c ? c->dev : NULL, d ? d->dev : NULL,
                                               codes ? (unsigned char *)codes->dev : NULL,
                                               q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7],
                                               q[8], q[9], q[10], q[11], q[12])
               : -1;
        if (rc == 0 && codes) {
            *tt_pend.codes_dst = codes;  /* the pool node owns them now */
            codes = NULL;
        }
        tt_release(codes);  /* not written: the backward reads the relu values */
        if (rc == 0 && tt_lazy_relu(tt_pend.r, tt_pend.out) != 0)
            rc = tt_k_relu_fwd(tt_pend.out->dev, tt_pend.r->dev, tt_pend.r->numel) ? -2 : 0;
        if (rc != 0) {  /* the convolution + relu, then the pool and the copy by themselves */
            rc = tt_k_conv2d_relu_fwd_lds(tt_pend.x, tt_pend.w, tt_pend.b, tt_pend.out->dev,
                                          tt_pend.r->dev, q[0], q[1], q[2], q[3], q[4], q[5],
                                          q[6], q[7], q[8], q[9], q[10], q[11], q[12]);
            if (rc != 0) {
                rc = conv_fwd_gemm(tt_pend.x, tt_pend.w, tt_pend.b, tt_pend.out->dev, q);
                if (rc == 0)
                    rc = tt_k_relu_fwd(tt_pend.out->dev, tt_pend.r->dev, tt_pend.r->numel);
            }
            if (rc == 0 && p)
                rc = tt_k_maxpool_fwd(tt_pend.r->dev, p->dev, q[0], q[4], q[11], q[12], 2, 2, 2,
                                      2, q[11] / 2, q[12] / 2);
            if (rc == 0 && c) rc = tt_k_copy(c->dev, p->dev, c->numel);
            if (rc == 0 && d) rc = tt_k_padones_fwd(c->dev, d->dev, c->shape[0], c->shape[1]);
        }
        if (rc == 0 && kind == TT_PEND_CHAIN_FC && chain_fc_gemm(&tt_pend) != 0) {
            tt_pend.fco->valid = 0;
            ttrt_set_error(-3);
        }
        if (rc != 0) {
            tt_pend.r->valid = 0;
            if (p) p->valid = 0;
            if (c) c->valid = 0;
            if (d) d->valid = 0;
            if (kind == TT_PEND_CHAIN_FC) tt_pend.fco->valid = 0;
        }
    } else {
        const int *q = tt_pend.geo;
        rc = tt_k_conv2d_fwd_lds(tt_pend.x, tt_pend.w, tt_pend.b, tt_pend.out->dev, q[0], q[1],
                                 q[2], q[3], q[4], q[5], q[6], q[7], q[8], q[9], q[10], q[11],
                                 q[12]);
        if (rc != 0) rc = conv_fwd_gemm(tt_pend.x, tt_pend.w, tt_pend.b, tt_pend.out->dev, q);
    }
    if (rc != 0) {
        tt_pend.out->valid = 0;
        ttrt_set_error(-3);
        return -3;
    }
    return 0;
}

Tensor *tt_conv2d_keepcol(const Tensor *a, const Tensor *w, const Tensor *b, int sh, int sw,
                          int ph, int pw, float **col_out, int ones_row) {
    return tt_conv2d_keepcol_ex(a, w, b, sh, sw, ph, pw, col_out, ones_row, 0);
}

/* defer: the direct-convolution launch may be left pending in tt_pend */
Tensor *tt_conv2d_keepcol_ex(const Tensor *a, const Tensor *w, const Tensor *b, int sh, int sw,
                             int ph, int pw, float **col_out, int ones_row, int defer) {
    if (col_out) *col_out = NULL;
    if (!a || !w || a->ndim != 4 || w->ndim != 4) return NULL;
    const int N = (int)a->shape[0], C = (int)a->shape[1], H = (int)a->shape[2],
              W = (int)a->shape[3];
    const int F = (int)w->shape[0], Cw = (int)w->shape[1], HH = (int)w->shape[2],
              WW = (int)w->shape[3];
    if (C != Cw) return NULL;
    if (b && (b->ndim != 1 || b->shape[0] != F)) return NULL;
    if (!valid_conv_params(HH, WW, sh, sw, ph, pw)) return NULL;
    const int Ho = (H + 2 * ph - HH) / sh + 1;
    const int Wo = (W + 2 * pw - WW) / sw + 1;
    if (Ho <= 0 || Wo <= 0) return NULL;

    /* the input is the pool output of a pending conv -> relu -> pool: that
     * launch stays pending (stashed here) so both convolutions can run as
     * one chain; it is put back (and flushed first) if this one is not
     * deferred after all */
    const int q[13] = {N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo};
    TTPendConv first;
    first.active = 0;
    if (defer && g_conv_relu && g_conv_chain && tt_pend.active == TT_PEND_CONV_RELU_POOL &&
        tt_pend.p == a && !tt_pend1.active && chain_geometry(tt_pend.geo, q)) {
        first = tt_pend;
        tt_pend.active = 0;
    }
    const float *x = first.active ? a->dev : tt_dev((Tensor *)a), *wd = tt_dev((Tensor *)w);
    const float *bd = b ? tt_dev((Tensor *)b) : NULL;
    const long shp[4] = {N, F, Ho, Wo};
    Tensor *out = x && wd && (!b || bd) ? tt_empty_dev(shp, 4) : NULL;
    if (!out) {
        if (first.active) tt_pend = first;
        return NULL;
    }
    const int Kc = C * HH * WW;
    const long Ncol = (long)N * Ho * Wo;
    /* LDS-staged direct convolution: taken when it also covers the weight
     * gradient the caller will ask for (that reads x, so no col is kept) */
    const int lds = tt_k_conv2d_lds_plan(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo);
    const int direct = (lds & 1) && (!col_out || (lds & 2));
    if (direct && defer && g_conv_relu) {
        tt_flush_pending();
        tt_pend.out = out;
        tt_pend.x = x; tt_pend.w = wd; tt_pend.b = bd;
        tt_pend.xt = (Tensor *)a;
        for (int i = 0; i < 13; i++) tt_pend.geo[i] = q[i];
        tt_pend.active = TT_PEND_CONV;
        if (first.active) tt_pend1 = first;
        return out;
    }
    if (first.active) {  /* not deferred: the first convolution runs now */
        tt_pend = first;
        if (!(x = tt_dev((Tensor *)a))) return fail(out);
    }
    if (direct) {
        if (tt_k_conv2d_fwd_lds(x, wd, bd, out->dev, N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho,
                                Wo) == 0)
            return out;
    }
    if (tt_conv_use_implicit(sizeof(float) * (long)Kc * Ncol) &&
        tt_k_conv2d_fwd_implicit(x, wd, bd, out->dev, N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho,
                                 Wo) == 0)
        return out;  /* no col: the backward pass reads x directly too */
    const int rows = (col_out && ones_row) ? Kc + 1 : Kc;
    float *col = (float *)ttrt_alloc(sizeof(float) * (size_t)rows * (size_t)Ncol);
    if (!col) return fail(out);
    if ((rows > Kc ? tt_k_im2col_ones(x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo)
                   : tt_k_im2col(x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo)) ||
        tt_k_conv_fwd(F, Kc, Ncol, Ho * Wo, wd, col, bd, out->dev)) {
        ttrt_free(col);
        return fail(out);
    }
    if (col_out) *col_out = col;
    else ttrt_free(col);
    return out;
}

Tensor *tt_conv2d(const Tensor *a, const Tensor *w, const Tensor *b, int sh, int sw, int ph,
                  int pw) {
    return tt_conv2d_keepcol(a, w, b, sh, sw, ph, pw, NULL, 0);
}

static Tensor *pool(const Tensor *a, int ph, int pw, int sh, int sw, int is_max) {
    if (!a || a->ndim != 4) return NULL;
    if (!valid_pool_params(ph, pw, sh, sw)) return NULL;
    const int N = (int)a->shape[0], C = (int)a->shape[1], H = (int)a->shape[2],
              W = (int)a->shape[3];
    const int Ho = (H - ph) / sh + 1;
    const int Wo = (W - pw) / sw + 1;
    if (Ho <= 0 || Wo <= 0 || ph > H || pw > W) return NULL;
    const float *x = tt_dev((Tensor *)a);
    if (!x) return NULL;
    const long shp[4] = {N, C, Ho, Wo};
    Tensor *out = tt_empty_dev(shp, 4);
    if (!out) return NULL;
    int rc = is_max ? tt_k_maxpool_fwd(x, out->dev, N, C, H, W, ph, pw, sh, sw, Ho, Wo)
                    : tt_k_avgpool_fwd(x, out->dev, N, C, H, W, ph, pw, sh, sw, Ho, Wo);
    if (rc) return fail(out);
    return out;
}

Tensor *tt_maxpool2d(const Tensor *a, int ph, int pw, int sh, int sw) {
    return pool(a, ph, pw, sh, sw, 1);
}

Tensor *tt_avgpool2d(const Tensor *a, int ph, int pw, int sh, int sw) {
    return pool(a, ph, pw, sh, sw, 0);
}
