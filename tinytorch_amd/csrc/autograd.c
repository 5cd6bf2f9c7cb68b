/* Reverse-mode autograd: host-side graph, device-side arithmetic.
 *
 * Follows the reference src/autograd.c:
 *   node construction / ownership           :105-275
 *   accum (first grad = copy, then +=)      :44-63
 *   backward rules                          :283-628
 *   iterative post-order topo sort          :649-680
 *   reverse propagation                     :682-702
 *   seeding and mismatch rule               :704-727
 *
 * Differences that do not change any observable value:
 *   * A gradient a parent does not require is never computed (the reference
 *     computes dA of every matmul and throws it away when A is a constant).
 *   * A freshly computed gradient temporary is moved into an empty parent
 *     grad instead of being copied (same bits, one copy fewer).
 *   * conv2d keeps its forward im2col matrix for the backward pass instead
 *     of recomputing it (reference :495 recomputes identical values).
 *   * The NCHW <-> F x (N*Ho*Wo) permutes and W^T are folded into the GEMM
 *     operand addressing instead of materialised (reference :498-533).
 * Backward rules that fail to allocate skip silently, as in the reference. */
#include "tt_internal.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef enum {
    OP_LEAF, OP_ADD, OP_MUL, OP_ADDSCALAR, OP_MULSCALAR, OP_MATMUL, OP_RELU,
    OP_SOFTMAX, OP_PADONES, OP_RESHAPE, OP_CONV2D, OP_MAXPOOL2D, OP_AVGPOOL2D,
    OP_SOFTMAX_CE
} OpKind;

struct AGNode {
    Tensor *val;
    Tensor *grad;
    AGNode *parents[3];
    int     nparents;
    OpKind  kind;
    float   scalar;
    int     params[4];
    int     requires_grad;
    int     mark;        /* DFS state: 0 new, 1 on stack, 2 done */
    int     uses;        /* backward: edges from nodes of this pass to this node */
    int     grad_done;   /* backward: this relu's / reshape's backward already ran fused */
    int     refcount;
    float  *col;         /* conv2d: forward im2col matrix (device) */
    int     col_ones;    /* conv2d: col carries the extra row of ones */
    Tensor *aux;         /* softmax_ce: probabilities */
    Tensor *aux2;        /* softmax_ce: per-row seed (p - onehot)/rows; NULL once
                            moved into the logits' gradient */
    int32_t *labels;     /* softmax_ce: host copy of the labels (seed recompute) */
};

/* ---------- gradient accumulation ---------- */

/* p->grad += g, or p->grad = copy(g) if it has none (g is borrowed) */
static void accum_copy(AGNode *p, Tensor *g) {
    if (!p || !p->requires_grad || !g) return;
    const float *gd = tt_dev(g);
    if (!gd) return;
    if (!p->grad) {
        Tensor *c = tt_empty_like(g);
        if (!c) return;
        if (tt_k_copy(c->dev, gd, g->numel)) { tt_release(c); return; }
        p->grad = c;
        return;
    }
    float *pd = tt_dev(p->grad);
    if (!pd) return;
    tt_k_add_inplace(pd, gd, g->numel);
    tt_mark_dev_written(p->grad);
}

/* same, but g is an owned temporary: moved in when p has no grad yet */
static void accum_move(AGNode *p, Tensor *g) {
    if (!g) return;
    if (p && p->requires_grad && !p->grad) {
        p->grad = g;
        return;
    }
    accum_copy(p, g);
    tt_release(g);
}

static int needs(const AGNode *p) { return p && p->requires_grad; }

/* ---------- node construction ---------- */

static AGNode *node_new(Tensor *val, int requires_grad) {
    if (!val) return NULL;
    AGNode *n = (AGNode *)calloc(1, sizeof(AGNode));
    if (!n) { tt_release(val); return NULL; }
    n->val = val;
    n->requires_grad = requires_grad;
    n->refcount = 1;
    return n;
}

static AGNode *node_unary(AGNode *a, Tensor *val, OpKind k) {
    AGNode *n = node_new(val, a->requires_grad);
    if (!n) return NULL;
    n->parents[0] = ag_retain(a);
    n->nparents = 1;
    n->kind = k;
    return n;
}

static AGNode *node_binary(AGNode *a, AGNode *b, Tensor *val, OpKind k) {
    AGNode *n = node_new(val, a->requires_grad || b->requires_grad);
    if (!n) return NULL;
    n->parents[0] = ag_retain(a);
    n->parents[1] = ag_retain(b);
    n->nparents = 2;
    n->kind = k;
    return n;
}

AGNode *ag_leaf(Tensor *t, int requires_grad) {
    if (!t) return NULL;
    AGNode *n = node_new(tt_retain(t), requires_grad);
    if (n) n->kind = OP_LEAF;
    return n;
}

AGNode *ag_add(AGNode *a, AGNode *b) {
    if (!a || !b) return NULL;
    return node_binary(a, b, tt_add(a->val, b->val), OP_ADD);
}

AGNode *ag_mul(AGNode *a, AGNode *b) {
    if (!a || !b) return NULL;
    return node_binary(a, b, tt_mul(a->val, b->val), OP_MUL);
}

AGNode *ag_addscalar(AGNode *a, float s) {
    if (!a) return NULL;
    AGNode *n = node_unary(a, tt_addscalar(a->val, s), OP_ADDSCALAR);
    if (n) n->scalar = s;
    return n;
}

AGNode *ag_mulscalar(AGNode *a, float s) {
    if (!a) return NULL;
    AGNode *n = node_unary(a, tt_mulscalar(a->val, s), OP_MULSCALAR);
    if (n) n->scalar = s;
    return n;
}

AGNode *ag_matmul(AGNode *a, AGNode *b) {
    if (!a || !b) return NULL;
    return node_binary(a, b, tt_matmul_omp(a->val, b->val, 0), OP_MATMUL);
}

AGNode *ag_relu(AGNode *a) {
    if (!a) return NULL;
    if (tt_pend.active == TT_PEND_CONV && tt_pend.out == a->val) {
        /* the convolution producing a is still pending: one launch writes
         * it and its relu (same values as tt_relu of the stored output) */
        Tensor *r = tt_empty_like(a->val);
        if (r) {
            const TTPendConv p = tt_pend;
            const int *q = p.geo;
            tt_pend.active = 0;
            if (tt_k_conv2d_relu_fwd_lds(p.x, p.w, p.b, p.out->dev, r->dev, q[0], q[1], q[2],
                                         q[3], q[4], q[5], q[6], q[7], q[8], q[9], q[10], q[11],
                                         q[12]) == 0)
                return node_unary(a, r, OP_RELU);
            tt_pend = p;  /* not launched: the plain convolution runs below */
            tt_release(r);
        }
    }
    if (tt_defer_enabled() && a->val->ndim == 2) {
        /* a relu that a padones may consume (the MLP's hidden layers): left
         * pending like the convolution above */
        const float *x = tt_dev(a->val);
        Tensor *r = x ? tt_empty_like(a->val) : NULL;
        if (!r) return NULL;
        AGNode *n = node_unary(a, r, OP_RELU);
        if (!n) return NULL;
        tt_pend.out = r;
        tt_pend.x = x;
        tt_pend.active = TT_PEND_RELU;
        return n;
    }
    return node_unary(a, tt_relu(a->val), OP_RELU);
}

AGNode *ag_softmax(AGNode *a) {
    if (!a) return NULL;
    return node_unary(a, tt_softmax(a->val), OP_SOFTMAX);
}

AGNode *ag_padones(AGNode *a) {
    if (!a || a->val->ndim != 2) return NULL;
    const long M = a->val->shape[0], K = a->val->shape[1];
    const long shp[2] = {M, K + 1};
    if (tt_pend.active == TT_PEND_COPY && tt_pend.out == a->val) {
        /* a is a reshape whose copy is still pending: one pass writes the
         * copy and the padded tensor */
        Tensor *v = tt_empty_dev(shp, 2);
        if (v) {
            const TTPendConv p = tt_pend;
            tt_pend.active = 0;
            if (tt_k_copy_padones_fwd(p.x, p.out->dev, v->dev, M, K) == 0)
                return node_unary(a, v, OP_PADONES);
            tt_pend = p;  /* not launched: the plain copy runs below */
            tt_release(v);
        }
    }
    if (tt_pend.active == TT_PEND_RELU && tt_pend.out == a->val) {
        Tensor *v = tt_empty_dev(shp, 2);
        if (v) {
            const TTPendConv p = tt_pend;
            tt_pend.active = 0;
            if (tt_k_relu_padones_fwd(p.x, p.out->dev, v->dev, M, K) == 0)
                return node_unary(a, v, OP_PADONES);
            tt_pend = p;  /* not launched: the plain relu runs below */
            tt_release(v);
        }
    }
    const float *x = tt_dev(a->val);
    if (!x) return NULL;
    Tensor *v = tt_empty_dev(shp, 2);
    if (!v) return NULL;
    if (tt_k_padones_fwd(x, v->dev, M, K)) { tt_release(v); return NULL; }
    return node_unary(a, v, OP_PADONES);
}

AGNode *ag_reshape(AGNode *a, const long *new_shape, int new_ndim) {
    if (!a) return NULL;
    Tensor *v = tt_reshape_ex(a->val, new_shape, new_ndim, 1);
    if (!v) return NULL;
    AGNode *n = node_unary(a, v, OP_RESHAPE);
    if (!n && tt_pend.active && tt_pend.out == v) tt_pend.active = 0;  /* v was released */
    return n;
}

AGNode *ag_conv2d(AGNode *a, AGNode *w, AGNode *b, int sh, int sw, int ph, int pw) {
    if (!a || !w) return NULL;
    const int keep = w->requires_grad;
    const int ones = keep && b && b->requires_grad;  /* fuse db into the dW GEMM */
    float *col = NULL;
    Tensor *v = tt_conv2d_keepcol_ex(a->val, w->val, b ? b->val : NULL, sh, sw, ph, pw,
                                     keep ? &col : NULL, ones, 1);
    if (!v) return NULL;
    int req = a->requires_grad || w->requires_grad || (b && b->requires_grad);
    AGNode *n = node_new(v, req);
    if (!n) {
        if (tt_pend.active && tt_pend.out == v) tt_pend.active = 0;  /* v was released */
        ttrt_free(col);
        return NULL;
    }
    n->parents[0] = ag_retain(a);
    n->parents[1] = ag_retain(w);
    n->nparents = 2;
    if (b) {
        n->parents[2] = ag_retain(b);
        n->nparents = 3;
    }
    n->kind = OP_CONV2D;
    n->params[0] = sh; n->params[1] = sw;
    n->params[2] = ph; n->params[3] = pw;
    n->col = col;
    n->col_ones = col && ones;
    return n;
}

static AGNode *pool_node(AGNode *a, Tensor *v, OpKind k, int ph, int pw, int sh, int sw) {
    AGNode *n = node_unary(a, v, k);
    if (!n) return NULL;
    n->params[0] = ph; n->params[1] = pw;
    n->params[2] = sh; n->params[3] = sw;
    return n;
}

AGNode *ag_maxpool2d(AGNode *a, int ph, int pw, int sh, int sw) {
    if (!a) return NULL;
    Tensor *v = tt_maxpool2d(a->val, ph, pw, sh, sw);
    if (!v) return NULL;
    return pool_node(a, v, OP_MAXPOOL2D, ph, pw, sh, sw);
}

AGNode *ag_avgpool2d(AGNode *a, int ph, int pw, int sh, int sw) {
    if (!a) return NULL;
    Tensor *v = tt_avgpool2d(a->val, ph, pw, sh, sw);
    if (!v) return NULL;
    return pool_node(a, v, OP_AVGPOOL2D, ph, pw, sh, sw);
}

/* Fused softmax + mean cross-entropy (no reference counterpart: the
 * reference harness does this in NumPy, tests/gate_cifar_cnn.py:175-181). */
AGNode *ag_softmax_ce(AGNode *logits, const int *labels, long rows) {
    if (!logits || !labels || logits->val->ndim != 2 || logits->val->shape[0] != rows ||
        rows <= 0 || logits->val->shape[1] > 0x7fffffffL)
        return NULL;
    const int cols = (int)logits->val->shape[1];
    const float *x = tt_dev(logits->val);
    if (!x) return NULL;
    const long one = 1;
    Tensor *probs = tt_empty_like(logits->val);
    Tensor *seed = tt_empty_like(logits->val);
    Tensor *loss = tt_empty_dev(&one, 1);
    int32_t *hlab = (int32_t *)malloc(sizeof(int32_t) * (size_t)rows);
    if (hlab)
        for (long r = 0; r < rows; r++) hlab[r] = (int32_t)labels[r];
    /* small batches: the labels travel inside the kernel's arguments */
    if (probs && seed && loss && hlab && rows <= TT_CE_ARG_ROWS &&
        tt_k_softmax_ce_mean_hostlab(x, hlab, probs->dev, loss->dev, seed->dev, rows, cols,
                                     1.0f / (float)rows) == 0) {
        AGNode *n = node_unary(logits, loss, OP_SOFTMAX_CE);
        if (!n) { tt_release(probs); tt_release(seed); free(hlab); return NULL; }
        n->aux = probs;
        n->aux2 = seed;
        n->labels = hlab;
        return n;
    }
    free(hlab);
    int32_t *dlab = (int32_t *)ttrt_alloc(sizeof(int32_t) * (size_t)rows);
    float *rowloss = rows > TT_CE_MEAN_MAX_ROWS ? (float *)ttrt_alloc(sizeof(float) * (size_t)rows)
                                                : NULL;
    int ok = probs && seed && loss && dlab && (rowloss || rows <= TT_CE_MEAN_MAX_ROWS);
    if (ok) {
        int32_t *h = (int32_t *)malloc(sizeof(int32_t) * (size_t)rows);
        ok = h != NULL;
        if (ok) {
            for (long r = 0; r < rows; r++) h[r] = (int32_t)labels[r];
            ok = ttrt_h2d_async(dlab, h, sizeof(int32_t) * (size_t)rows) == 0;
            free(h);
        }
    }
    /* small batches: one workgroup computes probabilities, seed and the mean
     * loss; large ones reduce the per-row losses with a 1 x rows x 1 GEMM
     * against a vector of 1/rows */
    float *inv = NULL;
    if (ok && rows <= TT_CE_MEAN_MAX_ROWS) {
        ok = tt_k_softmax_ce_mean(x, dlab, probs->dev, loss->dev, seed->dev, rows, cols,
                                  1.0f / (float)rows) == 0;
    } else if (ok) {
        inv = (float *)ttrt_alloc(sizeof(float) * (size_t)rows);
        ok = inv && tt_k_fill(inv, rows, 1.0f / (float)rows) == 0 &&
             tt_k_softmax_ce(x, dlab, probs->dev, rowloss, seed->dev, rows, cols,
                             1.0f / (float)rows) == 0 &&
             tt_k_gemm(1, 1, (int)rows, rowloss, (int)rows, 0, inv, 1, 0, loss->dev, 1) == 0;
    }
    ttrt_free(dlab);
    ttrt_free(rowloss);
    ttrt_free(inv);
    if (!ok) {
        tt_release(probs); tt_release(seed); tt_release(loss);
        return NULL;
    }
    AGNode *n = node_unary(logits, loss, OP_SOFTMAX_CE);
    if (!n) { tt_release(probs); tt_release(seed); return NULL; }
    n->aux = probs;
    n->aux2 = seed;
    return n;
}

Tensor *ag_softmax_ce_probs(const AGNode *n) {
    return (n && n->kind == OP_SOFTMAX_CE) ? n->aux : NULL;
}

/* ---------- accessors ---------- */

Tensor *ag_value(const AGNode *n) { return n ? n->val : NULL; }
Tensor *ag_grad(const AGNode *n) { return n ? n->grad : NULL; }
int ag_requires_grad(const AGNode *n) { return n ? n->requires_grad : 0; }

/* ---------- backward rules ---------- */

static void backward_add(AGNode *n) {
    accum_copy(n->parents[0], n->grad);
    accum_copy(n->parents[1], n->grad);
}

static void backward_mul(AGNode *n) {
    AGNode *a = n->parents[0], *b = n->parents[1];
    if (needs(a)) accum_move(a, tt_mul(n->grad, b->val));   /* g * b */
    if (needs(b)) accum_move(b, tt_mul(n->grad, a->val));   /* g * a */
}

static void backward_addscalar(AGNode *n) { accum_copy(n->parents[0], n->grad); }

static void backward_mulscalar(AGNode *n) {
    if (needs(n->parents[0])) accum_move(n->parents[0], tt_mulscalar(n->grad, n->scalar));
}

static void backward_matmul(AGNode *n) {
    AGNode *a = n->parents[0], *b = n->parents[1];
    const int M = (int)a->val->shape[0], K = (int)a->val->shape[1], N = (int)b->val->shape[1];
    const float *g = tt_dev(n->grad);
    if (!g) return;
    if (needs(a)) {  /* dA = g (MxN) * b^T (b is KxN) */
        const float *bd = tt_dev(b->val);
        Tensor *ga = bd ? tt_empty_like(a->val) : NULL;
        if (ga && tt_k_gemm(M, K, N, g, N, 0, bd, N, 1, ga->dev, K) == 0) accum_move(a, ga);
        else tt_release(ga);
    }
    if (needs(b)) {  /* dB = a^T (a is MxK) * g (MxN) */
        const float *ad = tt_dev(a->val);
        Tensor *gb = ad ? tt_empty_like(b->val) : NULL;
        if (gb && tt_k_gemm(K, N, M, ad, K, 1, g, N, 0, gb->dev, N) == 0) accum_move(b, gb);
        else tt_release(gb);
    }
}

static void backward_relu(AGNode *n) {
    AGNode *a = n->parents[0];
    if (!needs(a)) return;
    const float *x = tt_dev(a->val), *g = tt_dev(n->grad);
    if (!x || !g) return;
    Tensor *t = tt_empty_like(a->val);
    if (!t) return;
    if (tt_k_relu_bwd(x, g, t->dev, t->numel)) { tt_release(t); return; }
    accum_move(a, t);
}

static void backward_softmax(AGNode *n) {
    AGNode *a = n->parents[0];
    if (!needs(a)) return;
    const Tensor *s = n->val;
    const long N = s->shape[s->ndim - 1];
    const float *sd = tt_dev(n->val), *g = tt_dev(n->grad);
    if (!sd || !g) return;
    Tensor *t = tt_empty_like(s);
    if (!t) return;
    if (tt_k_softmax_bwd(sd, g, t->dev, s->numel / N, (int)N)) { tt_release(t); return; }
    accum_move(a, t);
}

/* A node whose backward can also run the backward of the relu r feeding it
 * in the same pass: r is used by nothing else in this pass (its gradient is
 * complete once this node's backward has run), starts with no gradient, and
 * its input needs one and has no other consumer -- so every gradient gets
 * the same sums in the same order as with two separate steps. */
static int relu_fusable(const AGNode *r) {
    return r->kind == OP_RELU && r->uses == 1 && !r->grad && needs(r->parents[0]) &&
           r->parents[0]->uses == 1;
}

/* hand the fused pass's two gradients to the relu and its input */
static void fused_relu_done(AGNode *r, Tensor *dr, Tensor *dx) {
    accum_move(r, dr);
    accum_move(r->parents[0], dx);
    r->grad_done = 1;
}

static void backward_padones(AGNode *n) {
    AGNode *a = n->parents[0];
    if (!needs(a)) return;
    const float *g = tt_dev(n->grad);
    if (!g) return;
    if (relu_fusable(a)) {
        const float *r = tt_dev(a->val);
        Tensor *t = r ? tt_empty_like(a->val) : NULL, *u = t ? tt_empty_like(a->val) : NULL;
        if (u && tt_k_padones_relu_bwd(g, r, t->dev, u->dev, a->val->shape[0],
                                       a->val->shape[1]) == 0) {
            fused_relu_done(a, t, u);
            return;
        }
        tt_release(t);
        tt_release(u);
    }
    if (a->kind == OP_RESHAPE && a->uses == 1 && !a->grad && needs(a->parents[0]) &&
        a->parents[0]->uses == 1) {
        /* a reshape (a copy) feeds only this padones: its gradient and its
         * input's gradient are the same values, written by one pass */
        AGNode *x = a->parents[0];
        Tensor *t = tt_empty_like(a->val), *u = t ? tt_empty_like(x->val) : NULL;
        if (u && tt_k_padones_bwd2(g, t->dev, u->dev, a->val->shape[0], a->val->shape[1]) == 0) {
            accum_move(a, t);
            accum_move(x, u);
            a->grad_done = 1;
            return;
        }
        tt_release(t);
        tt_release(u);
    }
    Tensor *t = tt_empty_like(a->val);
    if (!t) return;
    if (tt_k_padones_bwd(g, t->dev, a->val->shape[0], a->val->shape[1])) {
        tt_release(t);
        return;
    }
    accum_move(a, t);
}

static void backward_reshape(AGNode *n) {
    AGNode *a = n->parents[0];
    if (!needs(a)) return;
    accum_move(a, tt_reshape(n->grad, a->val->shape, a->val->ndim));
}

static void backward_conv2d(AGNode *n) {
    AGNode *a = n->parents[0], *w = n->parents[1];
    AGNode *b = n->nparents > 2 ? n->parents[2] : NULL;
    const int sh = n->params[0], sw = n->params[1], ph = n->params[2], pw = n->params[3];
    const Tensor *g = n->grad;
    const int N = (int)a->val->shape[0], C = (int)a->val->shape[1], H = (int)a->val->shape[2],
              W = (int)a->val->shape[3];
    const int F = (int)w->val->shape[0], HH = (int)w->val->shape[2], WW = (int)w->val->shape[3];
    const int Ho = (int)g->shape[2], Wo = (int)g->shape[3];
    const int HW = Ho * Wo;
    const int Kc = C * HH * WW;
    const long Ncol = (long)N * HW;
    const float *gd = tt_dev(n->grad);
    if (!gd) return;

    const long bshp[1] = {F};
    const int lds = tt_k_conv2d_lds_plan(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo);
    int w_done = 0;
    if (needs(w) && !n->col && (lds & 2)) {
        /* LDS-staged forward kept no col: dW (and db) read x */
        const float *x = tt_dev(a->val);
        Tensor *gw = x ? tt_empty_like(w->val) : NULL;
        Tensor *gb = gw && needs(b) ? tt_empty_dev(bshp, 1) : NULL;
        if (gw && (gb || !needs(b)) &&
            tt_k_conv2d_dw_lds(gd, x, gw->dev, gb ? gb->dev : NULL, N, C, H, W, F, HH, WW, sh,
                               sw, ph, pw, Ho, Wo) == 0) {
            if (gb) accum_move(b, gb);
            accum_move(w, gw);
            w_done = 1;
        } else {
            tt_release(gw);
            tt_release(gb);
        }
    }
    if (w_done) {
    } else if (needs(b) && needs(w) && n->col && n->col_ones) {
        /* dW and db from one GEMM against [col; ones] */
        Tensor *gw = tt_empty_like(w->val);
        Tensor *gb = gw ? tt_empty_dev(bshp, 1) : NULL;
        if (gb && tt_k_conv_dw_bias(F, Kc, Ncol, HW, gd, n->col, gw->dev, gb->dev) == 0) {
            accum_move(b, gb);
            accum_move(w, gw);
        } else {
            tt_release(gw);
            tt_release(gb);
        }
    } else if (needs(w) && !n->col && tt_conv_use_implicit(sizeof(float) * (long)Kc * Ncol)) {
        /* implicit forward kept no col: dW (and db, from the ones row) read x */
        const float *x = tt_dev(a->val);
        Tensor *gw = x ? tt_empty_like(w->val) : NULL;
        Tensor *gb = gw && needs(b) ? tt_empty_dev(bshp, 1) : NULL;
        if (gw && (gb || !needs(b)) &&
            tt_k_conv2d_dw_implicit(gd, x, gw->dev, gb ? gb->dev : NULL, N, C, H, W, F, HH, WW,
                                    sh, sw, ph, pw, Ho, Wo) == 0) {
            if (gb) accum_move(b, gb);
            accum_move(w, gw);
        } else {
            tt_release(gw);
            tt_release(gb);
        }
    } else {
        if (needs(b)) {
            Tensor *gb = tt_empty_dev(bshp, 1);
            if (gb && tt_k_bias_grad(gd, gb->dev, N, F, HW) == 0) accum_move(b, gb);
            else tt_release(gb);
        }
        if (needs(w)) {
            float *col = n->col;
            int own = 0;
            if (!col) {
                const float *x = tt_dev(a->val);
                col = x ? (float *)ttrt_alloc(sizeof(float) * (size_t)Kc * (size_t)Ncol) : NULL;
                if (col && tt_k_im2col(x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo)) {
                    ttrt_free(col);
                    col = NULL;
                }
                own = 1;
            }
            Tensor *gw = col ? tt_empty_like(w->val) : NULL;
            if (gw && tt_k_conv_dw(F, Kc, Ncol, HW, gd, col, gw->dev) == 0) accum_move(w, gw);
            else tt_release(gw);
            if (own) ttrt_free(col);
        }
    }
    if (needs(a) && (lds & 4)) {
        const float *wd = tt_dev(w->val);
        Tensor *ga = wd ? tt_empty_like(a->val) : NULL;
        if (ga && tt_k_conv2d_dx_lds(gd, wd, ga->dev, N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho,
                                     Wo) == 0) {
            accum_move(a, ga);
            return;
        }
        tt_release(ga);
    }
    if (needs(a) && tt_conv_use_implicit(sizeof(float) * (long)Kc * Ncol)) {
        /* stride-1 dX as one implicit GEMM; other strides keep dcol + col2im */
        const float *wd = tt_dev(w->val);
        Tensor *ga = wd ? tt_empty_like(a->val) : NULL;
        if (ga && tt_k_conv2d_dx_implicit(gd, wd, ga->dev, N, C, H, W, F, HH, WW, sh, sw, ph, pw,
                                          Ho, Wo) == 0) {
            accum_move(a, ga);
            return;
        }
        tt_release(ga);
    }
    if (needs(a)) {
        const float *wd = tt_dev(w->val);
        float *dcol = wd ? (float *)ttrt_alloc(sizeof(float) * (size_t)Kc * (size_t)Ncol) : NULL;
        Tensor *ga = dcol ? tt_empty_like(a->val) : NULL;
        if (ga && tt_k_conv_dcol(F, Kc, Ncol, HW, wd, gd, dcol) == 0 &&
            tt_k_col2im(dcol, ga->dev, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo) == 0)
            accum_move(a, ga);
        else
            tt_release(ga);
        ttrt_free(dcol);
    }
}

/* A 2x2 / stride-2 max pool whose input is a fusable relu (relu_fusable)
 * runs both backwards in one pass; the relu node's own step is skipped. */
static int backward_maxpool_relu(AGNode *n, AGNode *r, const float *g, const float *x, int N,
                                 int C, int H, int W, int Ho, int Wo) {
    if (!relu_fusable(r) || n->params[0] != 2 || n->params[1] != 2 || n->params[2] != 2 ||
        n->params[3] != 2)
        return 0;
    Tensor *t = tt_empty_like(r->val), *u = t ? tt_empty_like(r->parents[0]->val) : NULL;
    if (!u || tt_k_maxpool2x2_relu_bwd(x, g, t->dev, u->dev, N, C, H, W, Ho, Wo)) {
        tt_release(t);
        tt_release(u);
        return 0;
    }
    fused_relu_done(r, t, u);
    return 1;
}

static void backward_pool(AGNode *n, int is_max) {
    AGNode *a = n->parents[0];
    if (!needs(a)) return;
    const int ph = n->params[0], pw = n->params[1], sh = n->params[2], sw = n->params[3];
    const int N = (int)a->val->shape[0], C = (int)a->val->shape[1], H = (int)a->val->shape[2],
              W = (int)a->val->shape[3];
    const int Ho = (int)n->grad->shape[2], Wo = (int)n->grad->shape[3];
    const float *g = tt_dev(n->grad);
    const float *x = is_max ? tt_dev(a->val) : NULL;
    if (!g || (is_max && !x)) return;
    if (is_max && backward_maxpool_relu(n, a, g, x, N, C, H, W, Ho, Wo)) return;
    Tensor *t = tt_empty_like(a->val);
    if (!t) return;
    int rc = is_max ? tt_k_maxpool_bwd(x, g, t->dev, N, C, H, W, ph, pw, sh, sw, Ho, Wo)
                    : tt_k_avgpool_bwd(g, t->dev, N, C, H, W, ph, pw, sh, sw, Ho, Wo);
    if (rc) { tt_release(t); return; }
    accum_move(a, t);
}

/* the tensor's current copy is the host one and holds exactly 1.0f (the
 * default seed of ag_backward, see backward_impl) */
static int is_host_one(const Tensor *t) {
    return t && t->numel == 1 && t->valid == TT_V_HOST && t->data && t->data[0] == 1.0f;
}

/* d logits = seed * dL (dL is the 1-element incoming gradient).  With dL
 * exactly 1 the product is the seed itself: the first backward moves the
 * seed tensor into the logits' gradient (no kernel); a later one recomputes
 * it (same kernel, same inputs, same bits) from the kept host labels. */
static void backward_softmax_ce(AGNode *n) {
    AGNode *a = n->parents[0];
    if (!needs(a)) return;
    if (!n->aux2 && n->labels) {
        const float *x = tt_dev(a->val);
        const long rows = a->val->shape[0];
        const int cols = (int)a->val->shape[1];
        Tensor *p = tt_empty_like(a->val), *s = tt_empty_like(a->val);
        float *l = (float *)ttrt_alloc(sizeof(float));
        const int ok = x && p && s && l &&
                       tt_k_softmax_ce_mean_hostlab(x, n->labels, p->dev, l, s->dev, rows, cols,
                                                    1.0f / (float)rows) == 0;
        tt_release(p);
        ttrt_free(l);
        if (!ok) { tt_release(s); return; }
        n->aux2 = s;
    }
    if (!n->aux2) return;
    if (is_host_one(n->grad)) {
        if (n->labels && !a->grad) {
            a->grad = n->aux2;
            n->aux2 = NULL;
        } else {
            accum_copy(a, n->aux2);
        }
        return;
    }
    const float *seed = tt_dev(n->aux2), *gl = tt_dev(n->grad);
    if (!seed || !gl) return;
    Tensor *t = tt_empty_like(a->val);
    if (!t) return;
    if (tt_k_scale_by_dev(seed, gl, t->dev, t->numel)) {
        tt_release(t);
        return;
    }
    accum_move(a, t);
}

/* ---------- topological sort + propagation ---------- */

typedef struct {
    AGNode **items;
    size_t len, cap;
} NodeList;

static int list_push(NodeList *l, AGNode *n) {
    if (l->len == l->cap) {
        size_t nc = l->cap ? l->cap * 2 : 64;
        AGNode **ni = (AGNode **)realloc(l->items, nc * sizeof(AGNode *));
        if (!ni) return 0;
        l->items = ni;
        l->cap = nc;
    }
    l->items[l->len++] = n;
    return 1;
}

/* Iterative post-order DFS from root over parents (explicit stack, so a
 * 1000-deep chain does not recurse); order ends with root. */
static int topo_order(AGNode *root, NodeList *order) {
    typedef struct { AGNode *n; int next; } Frame;
    size_t cap = 64, top = 0;
    Frame *st = (Frame *)malloc(cap * sizeof(Frame));
    if (!st) return 0;
    st[top].n = root; st[top].next = 0; top++;
    root->mark = 1;
    int ok = 1;
    while (top > 0) {
        Frame *f = &st[top - 1];
        if (f->next < f->n->nparents) {
            AGNode *c = f->n->parents[f->next++];
            if (c->mark) continue;
            if (top == cap) {
                Frame *ns = (Frame *)realloc(st, 2 * cap * sizeof(Frame));
                if (!ns) { ok = 0; break; }
                st = ns;
                cap *= 2;
            }
            c->mark = 1;
            st[top].n = c; st[top].next = 0; top++;
        } else {
            f->n->mark = 2;
            if (!list_push(order, f->n)) { ok = 0; break; }
            top--;
        }
    }
    free(st);
    return ok;
}

static void propagate(NodeList *order) {
    for (size_t i = order->len; i-- > 0;) {
        AGNode *n = order->items[i];
        if (!n->grad || n->nparents == 0) continue;
        switch (n->kind) {
            case OP_ADD:        backward_add(n); break;
            case OP_MUL:        backward_mul(n); break;
            case OP_ADDSCALAR:  backward_addscalar(n); break;
            case OP_MULSCALAR:  backward_mulscalar(n); break;
            case OP_MATMUL:     backward_matmul(n); break;
            case OP_RELU:
                if (n->grad_done) n->grad_done = 0;
                else backward_relu(n);
                break;
            case OP_SOFTMAX:    backward_softmax(n); break;
            case OP_PADONES:    backward_padones(n); break;
            case OP_RESHAPE:
                if (n->grad_done) n->grad_done = 0;
                else backward_reshape(n);
                break;
            case OP_CONV2D:     backward_conv2d(n); break;
            case OP_MAXPOOL2D:  backward_pool(n, 1); break;
            case OP_AVGPOOL2D:  backward_pool(n, 0); break;
            case OP_SOFTMAX_CE: backward_softmax_ce(n); break;
            default: break;
        }
    }
}

/* seed_kind: 0 = ones, 1 = host floats, 2 = device tensor */
static void backward_impl(AGNode *out, int seed_kind, const float *hseed, const Tensor *dseed) {
    NodeList order = {0};
    if (!topo_order(out, &order)) {
        for (size_t i = 0; i < order.len; i++) order.items[i]->mark = 0;
        free(order.items);
        return;  /* marks of nodes still on the stack stay set only on OOM */
    }
    for (size_t i = 0; i < order.len; i++) order.items[i]->uses = 0;
    for (size_t i = 0; i < order.len; i++)
        for (int j = 0; j < order.items[i]->nparents; j++) order.items[i]->parents[j]->uses++;
    if (!out->grad) out->grad = tt_empty_like(out->val);
    if (out->grad && seed_kind == 0 && out->grad->numel == 1) {
        /* a scalar ones seed is written to the host copy: no kernel, and a
         * rule that only needs to know it is 1 (softmax-CE) reads no device
         * memory; tt_dev uploads it for any rule that does */
        Tensor *t = out->grad;
        if (!t->data) t->data = (float *)ttrt_host_alloc(sizeof(float));
        if (t->data) {
            t->data[0] = 1.0f;
            t->valid = TT_V_HOST;
            propagate(&order);
            for (size_t i = 0; i < order.len; i++) order.items[i]->mark = order.items[i]->grad_done = 0;
            free(order.items);
            return;
        }
    }
    if (out->grad) {
        int rc;
        float *gd = out->grad->dev;
        if (seed_kind == 1) rc = ttrt_h2d_async(gd, hseed, sizeof(float) * (size_t)out->val->numel);
        else if (seed_kind == 2) {
            const float *sd = tt_dev((Tensor *)dseed);
            rc = sd ? tt_k_copy(gd, sd, out->val->numel) : -1;
        } else rc = tt_k_fill(gd, out->grad->numel, 1.0f);
        tt_mark_dev_written(out->grad);
        if (rc == 0) propagate(&order);
    }
    for (size_t i = 0; i < order.len; i++) order.items[i]->mark = order.items[i]->grad_done = 0;
    free(order.items);
}

void ag_backward_from(AGNode *out, const float *seed, size_t seed_numel) {
    if (!out || !out->requires_grad) return;
    if (seed && (!out->val || seed_numel != (size_t)out->val->numel)) return;
    backward_impl(out, seed ? 1 : 0, seed, NULL);
}

void ag_backward(AGNode *out) { ag_backward_from(out, NULL, 0); }

void ag_backward_from_tensor(AGNode *out, const Tensor *seed) {
    if (!out || !out->requires_grad || !seed) return;
    if (!out->val || seed->numel != out->val->numel) return;
    backward_impl(out, 2, NULL, seed);
}

int ag_sgd_step_many(AGNode *const *leaves, int count, float lr) {
    if (count < 0 || (count > 0 && !leaves)) return -1;
    for (int base = 0; base < count; base += TT_SGD_MAX) {
        float *w[TT_SGD_MAX];
        const float *g[TT_SGD_MAX];
        long n[TT_SGD_MAX];
        int k = 0;
        for (int i = base; i < count && i < base + TT_SGD_MAX; i++) {
            AGNode *l = leaves[i];
            if (!l || !l->grad) continue;
            w[k] = tt_dev(l->val);
            g[k] = tt_dev(l->grad);
            if (!w[k] || !g[k]) return -1;
            n[k] = l->val->numel;
            tt_mark_dev_written(l->val);
            k++;
        }
        if (tt_k_sgd_multi(w, g, n, k, lr)) return -1;
    }
    return 0;
}

int ag_sgd_step(AGNode *leaf, float lr) {
    if (!leaf || !leaf->grad) return 0;
    float *w = tt_dev(leaf->val);
    const float *g = tt_dev(leaf->grad);
    if (!w || !g) return -1;
    int rc = tt_k_sgd(w, g, leaf->val->numel, lr);
    tt_mark_dev_written(leaf->val);
    return rc;
}

/* ---------- optimizers with device-resident state ---------- */

/* One state slot per position in the parameter list handed to
 * ag_optim_step: leaves are rebuilt every step around the same tensors, so
 * the slot, not the node, owns the moments.  Hyperparameters are doubles
 * because the reference harness keeps them as Python floats: the fp32
 * factors are the doubles rounded once, as NumPy rounds a Python scalar
 * against a float32 array, and Adam's bias-corrected rate stays a double. */
enum { OPT_MOMENTUM = 1, OPT_ADAM = 2 };

struct AGOptim {
    int kind;
    double lr, mu, b1, b2, eps;
    long t;            /* Adam steps taken */
    int nslots;        /* fixed by the first step */
    long *numel;       /* per slot */
    float **m, **v;    /* per-slot device state (v: Adam only) */
};

static AGOptim *optim_new(int kind) {
    if (ttrt_init() != 0) return NULL;
    AGOptim *o = (AGOptim *)calloc(1, sizeof(AGOptim));
    if (o) o->kind = kind;
    return o;
}

AGOptim *ag_optim_sgd_momentum(double lr, double momentum) {
    AGOptim *o = optim_new(OPT_MOMENTUM);
    if (!o) return NULL;
    o->lr = lr;
    o->mu = momentum;
    return o;
}

AGOptim *ag_optim_adam(double lr, double beta1, double beta2, double eps) {
    if (!(beta1 >= 0.0 && beta1 < 1.0) || !(beta2 >= 0.0 && beta2 < 1.0)) return NULL;
    AGOptim *o = optim_new(OPT_ADAM);
    if (!o) return NULL;
    o->lr = lr;
    o->b1 = beta1;
    o->b2 = beta2;
    o->eps = eps;
    return o;
}

void ag_optim_release(AGOptim *o) {
    if (!o) return;
    for (int i = 0; i < o->nslots; i++) {
        ttrt_free(o->m ? o->m[i] : NULL);
        ttrt_free(o->v ? o->v[i] : NULL);
    }
    free(o->numel);
    free(o->m);
    free(o->v);
    free(o);
}

long ag_optim_steps(const AGOptim *o) { return o ? o->t : -1; }

int ag_optim_set_lr(AGOptim *o, double lr) {
    if (!o) return -1;
    o->lr = lr;
    return 0;
}

double ag_optim_lr(const AGOptim *o) { return o ? o->lr : 0.0; }

/* zero-filled per-slot state on the first step */
static int optim_bind(AGOptim *o, AGNode *const *params, int count) {
    o->numel = (long *)calloc((size_t)count, sizeof(long));
    o->m = (float **)calloc((size_t)count, sizeof(float *));
    o->v = (float **)calloc((size_t)count, sizeof(float *));
    if (!o->numel || !o->m || !o->v) return -1;
    o->nslots = count;
    for (int i = 0; i < count; i++) {
        if (!params[i]) return -1;
        const long n = params[i]->val->numel;
        o->numel[i] = n;
        const size_t bytes = sizeof(float) * (size_t)n;
        o->m[i] = (float *)ttrt_alloc(bytes);
        if (!o->m[i] || tt_k_fill(o->m[i], n, 0.0f)) return -1;
        if (o->kind == OPT_ADAM) {
            o->v[i] = (float *)ttrt_alloc(bytes);
            if (!o->v[i] || tt_k_fill(o->v[i], n, 0.0f)) return -1;
        }
    }
    return 0;
}

int ag_optim_step(AGOptim *o, AGNode *const *params, int count) {
    if (!o || count < 0 || (count > 0 && !params)) return -1;
    if (o->nslots == 0 && count > 0) {
        if (optim_bind(o, params, count)) {
            for (int i = 0; i < o->nslots; i++) {
                ttrt_free(o->m[i]);
                ttrt_free(o->v[i]);
            }
            free(o->numel); free(o->m); free(o->v);
            o->numel = NULL; o->m = o->v = NULL; o->nslots = 0;
            return -1;
        }
    }
    if (count != o->nslots) return -1;
    for (int i = 0; i < count; i++)
        if (!params[i] || params[i]->val->numel != o->numel[i]) return -1;

    double lr_t = 0.0;
    if (o->kind == OPT_ADAM) {
        /* tests/gate_cifar_cnn.py:93-94 */
        o->t++;
        lr_t = o->lr * (sqrt(1.0 - pow(o->b2, (double)o->t)) / (1.0 - pow(o->b1, (double)o->t)));
    }
    for (int base = 0; base < count; base += TT_SGD_MAX) {
        float *w[TT_SGD_MAX], *m[TT_SGD_MAX], *v[TT_SGD_MAX];
        const float *g[TT_SGD_MAX];
        long n[TT_SGD_MAX];
        int k = 0;
        for (int i = base; i < count && i < base + TT_SGD_MAX; i++) {
            AGNode *l = params[i];
            if (!l->grad) continue;   /* no gradient reached it: state untouched */
            w[k] = tt_dev(l->val);
            g[k] = tt_dev(l->grad);
            if (!w[k] || !g[k]) return -1;
            m[k] = o->m[i];
            v[k] = o->v[i];
            n[k] = o->numel[i];
            tt_mark_dev_written(l->val);
            k++;
        }
        int rc;
        if (o->kind == OPT_MOMENTUM)
            rc = tt_k_momentum_multi(w, g, m, n, k, (float)o->lr, (float)o->mu);
        else
            rc = tt_k_adam_multi(w, g, m, v, n, k, (float)o->b1, (float)(1.0 - o->b1),
                                 (float)o->b2, (float)(1.0 - o->b2), (float)o->eps, lr_t);
        if (rc) return -1;
    }
    return 0;
}

/* ---------- lifecycle ---------- */

AGNode *ag_retain(AGNode *n) {
    if (!n) return NULL;
    n->refcount++;
    return n;
}

void ag_release(AGNode *n) {
    if (!n) return;
    if (--n->refcount > 0) return;
    if (tt_pend.active && tt_pend.out == n->val) tt_flush_pending();
    tt_release(n->val);
    tt_release(n->grad);
    tt_release(n->aux);
    tt_release(n->aux2);
    free(n->labels);
    ttrt_free(n->col);
    for (int i = 0; i < n->nparents; i++) ag_release(n->parents[i]);
    free(n);
}
