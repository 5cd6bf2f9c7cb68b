/* Reverse-mode autograd: host-side graph, device-side arithmetic.
 *
 * Behaviour follows the reference src/autograd.c:
 *   node construction / ownership           :105-275
 *   accum (first grad = copy, then +=)      :44-63
 *   backward rules                          :283-628
 *   order the rules run in                  :649-702
 *   seeding and mismatch rule               :704-727
 * The structure is this file's own: each node points at an operation
 * descriptor (its backward rule and the release of its own state), the
 * backward schedule is threaded through the nodes themselves (no node list,
 * no stack allocation, nothing to reset afterwards), and release walks a
 * worklist instead of recursing.
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

/* An operation kind: its name and the rule that turns a node's gradient
 * into gradients of its inputs.  Leaves have no operation. */
typedef struct AGOp {
    const char *name;
    void (*backward)(AGNode *n);
    void (*drop)(AGNode *n);     /* frees the kind's own state; may be NULL */
} AGOp;

/* A graph node.  `in` holds the inputs (retained), packed from index 0.
 * `at` holds what one kind of node needs beyond its inputs.  The trailing
 * fields are scratch of the backward pass that last visited the node. */
struct AGNode {
    const AGOp *op;
    Tensor *val;
    Tensor *grad;                /* NULL until a backward pass reaches the node */
    AGNode *in[3];
    int     n_in;
    int     needs_grad;
    int     refs;
    union {
        float s;                                          /* add/mul scalar */
        struct { int kh, kw, sh, sw; Tensor *codes; } win;  /* pools (codes: one byte a
                                                      2x2 window, or NULL) */
        struct { int sh, sw, ph, pw; float *col; int col_ones; } conv;
        /* softmax-CE; sda: the input gradients of its classifier (see
         * ce_spec), computed with the seed and not yet handed over */
        struct { Tensor *probs, *seed; int32_t *labels; Tensor *sda[3]; int *stale; } ce;
        /* matmul: sda handed over by its softmax-CE; *stale set when the
         * weights they were formed with are about to change */
        struct { Tensor *sda[3]; int *stale; } mm;
    } at;
    unsigned long long pass;     /* backward pass that scheduled the node */
    int     walk;                /* depth-first walk: next input to enter */
    AGNode *up;                  /* depth-first walk: the node it was entered from */
    AGNode *next;                /* schedule: the node whose rule runs after this one */
    int     fanin;               /* edges into the node from nodes of the pass */
    int     fused;               /* its rule already ran inside a consumer's fused rule */
    /* A gradient the fused 2x2 max pool + relu backward did not write,
     * computed by materialise on first need from lazy_g (retained), the
     * pool's output gradient: the relu's own gradient (lazy_codes NULL), or
     * the gradient of the convolution feeding the relu (lazy_codes, retained:
     * the pool windows' codes), whose weight gradient is then computed from
     * lazy_g and the codes directly.  lazy_next links the nodes that hold
     * one. */
    Tensor *lazy_g, *lazy_codes;
    AGNode *lazy_next;
};

static AGNode *g_lazy;           /* nodes whose gradient is still a recipe */

static void backward_add(AGNode *n);
static void backward_mul(AGNode *n);
static void backward_addscalar(AGNode *n);
static void backward_mulscalar(AGNode *n);
static void backward_matmul(AGNode *n);
static void backward_relu(AGNode *n);
static void backward_softmax(AGNode *n);
static void backward_padones(AGNode *n);
static void backward_reshape(AGNode *n);
static void backward_conv2d(AGNode *n);
static int conv_pooled_dw(AGNode *n);
static int conv_dw_deferred(const float *gd, const unsigned char *codes, const float *x,
                            Tensor *gw, Tensor *gb, const int q[13]);
static void backward_maxpool(AGNode *n);
static void backward_avgpool(AGNode *n);
static void backward_softmax_ce(AGNode *n);

static void drop_conv(AGNode *n) { ttrt_free(n->at.conv.col); }
static void drop_pool(AGNode *n) { tt_release(n->at.win.codes); }
static void spec_drop(Tensor *sda[3], int **stale) {
    for (int i = 0; i < 3; i++) { tt_release(sda[i]); sda[i] = NULL; }
    if (*stale) {
        tt_lazy_guard_drop(*stale);
        free(*stale);
        *stale = NULL;
    }
}
static void drop_ce(AGNode *n) {
    tt_release(n->at.ce.probs);
    tt_release(n->at.ce.seed);
    free(n->at.ce.labels);
    spec_drop(n->at.ce.sda, &n->at.ce.stale);
}
static void drop_mm(AGNode *n) { spec_drop(n->at.mm.sda, &n->at.mm.stale); }

static const AGOp OP_ADD = {"add", backward_add, NULL};
static const AGOp OP_MUL = {"mul", backward_mul, NULL};
static const AGOp OP_ADDSCALAR = {"addscalar", backward_addscalar, NULL};
static const AGOp OP_MULSCALAR = {"mulscalar", backward_mulscalar, NULL};
static const AGOp OP_MATMUL = {"matmul", backward_matmul, drop_mm};
static const AGOp OP_RELU = {"relu", backward_relu, NULL};
static const AGOp OP_SOFTMAX = {"softmax", backward_softmax, NULL};
static const AGOp OP_PADONES = {"padones", backward_padones, NULL};
static const AGOp OP_RESHAPE = {"reshape", backward_reshape, NULL};
static const AGOp OP_CONV2D = {"conv2d", backward_conv2d, drop_conv};
static const AGOp OP_MAXPOOL2D = {"maxpool2d", backward_maxpool, drop_pool};
static const AGOp OP_AVGPOOL2D = {"avgpool2d", backward_avgpool, NULL};
static const AGOp OP_SOFTMAX_CE = {"softmax_ce", backward_softmax_ce, drop_ce};

/* ---------- gradient accumulation ---------- */

/* p->grad += g, or p->grad = copy(g) if it has none (g is borrowed) */
static void accum_copy(AGNode *p, Tensor *g) {
    if (!p || !p->needs_grad || !g) return;
    const float *gd = tt_dev(g);
    if (!gd) return;
    if (!p->grad) {
        Tensor *c = tt_empty_like(g);
        if (!c) return;
        if (tt_k_copy(c->dev, gd, g->numel)) { tt_release(c); return; }
        p->grad = c;
        return;
    }
    tt_lazy_before_write(p->grad);  /* a recipe may read this gradient */
    float *pd = tt_dev(p->grad);
    if (!pd) return;
    tt_k_add_inplace(pd, gd, g->numel);
    tt_mark_dev_written(p->grad);
}

/* same, but g is an owned temporary: moved in when p has no grad yet */
static void accum_move(AGNode *p, Tensor *g) {
    if (!g) return;
    if (p && p->needs_grad && !p->grad) {
        p->grad = g;
        return;
    }
    accum_copy(p, g);
    tt_release(g);
}

static int needs(const AGNode *p) { return p && p->needs_grad; }

/* Write the gradient of a node that holds a recipe: the max pool backward
 * of the relu's output with the pool's output gradient (the reference's
 * src/autograd.c:555-594), or for the convolution before the relu that
 * followed by the relu backward (src/autograd.c:318-327) from the windows'
 * codes.  Run on first need -- before ag_grad hands out the node's gradient
 * or the pool's, before a rule other than the convolution's reads it, and
 * before a backward pass that may add into the pool's gradient -- so the
 * recipe's operands are unchanged. */
static void materialise(AGNode *n) {
    for (AGNode **pp = &g_lazy; *pp; pp = &(*pp)->lazy_next)
        if (*pp == n) { *pp = n->lazy_next; break; }
    n->lazy_next = NULL;
    Tensor *g = n->lazy_g, *codes = n->lazy_codes;
    n->lazy_g = n->lazy_codes = NULL;
    const Tensor *v = n->val;
    const int N = (int)v->shape[0], C = (int)v->shape[1], H = (int)v->shape[2],
              W = (int)v->shape[3], Ho = (int)g->shape[2], Wo = (int)g->shape[3];
    const float *x = codes ? NULL : tt_dev((Tensor *)v), *gd = tt_dev(g);
    const unsigned char *cd = codes ? (const unsigned char *)tt_dev(codes) : NULL;
    Tensor *t = ((x || cd) && gd) ? tt_empty_like(v) : NULL;
    if (t && (cd ? tt_k_maxpool2x2_code_relu_bwd(cd, gd, t->dev, N, C, H, W, Ho, Wo)
                 : tt_k_maxpool_bwd(x, gd, t->dev, N, C, H, W, 2, 2, 2, 2, Ho, Wo)) == 0)
        accum_move(n, t);
    else
        tt_release(t);
    tt_release(g);
    tt_release(codes);
}

/* materialise every recipe that is n's gradient or reads it */
static void materialise_for(const AGNode *n) {
    AGNode *l = g_lazy;
    while (l) {
        AGNode *next = l->lazy_next;
        if (l == n || (n->grad && l->lazy_g == n->grad)) materialise(l);
        l = next;
    }
}

static void lazy_drop(AGNode *n) {
    if (!n->lazy_g) return;
    for (AGNode **pp = &g_lazy; *pp; pp = &(*pp)->lazy_next)
        if (*pp == n) { *pp = n->lazy_next; break; }
    tt_release(n->lazy_g);
    tt_release(n->lazy_codes);
    n->lazy_g = n->lazy_codes = NULL;
    n->lazy_next = NULL;
}

static void lazy_set(AGNode *n, Tensor *g, Tensor *codes) {
    n->lazy_g = tt_retain(g);
    n->lazy_codes = codes ? tt_retain(codes) : NULL;
    n->lazy_next = g_lazy;
    g_lazy = n;
}

/* ---------- node construction ---------- */

/* A node computing `val` (owned; released when the node cannot be made)
 * from up to three inputs; NULL entries of `in` are skipped.  The node needs
 * a gradient when any input does. */
static AGNode *make_node(Tensor *val, const AGOp *op, AGNode *x, AGNode *y, AGNode *z) {
    if (!val) return NULL;
    AGNode *n = (AGNode *)calloc(1, sizeof(AGNode));
    if (!n) { tt_release(val); return NULL; }
    n->op = op;
    n->val = val;
    n->refs = 1;
    AGNode *const in[3] = {x, y, z};
    for (int i = 0; i < 3; i++) {
        if (!in[i]) continue;
        n->needs_grad |= in[i]->needs_grad;
        n->in[n->n_in++] = ag_retain(in[i]);
    }
    return n;
}

AGNode *ag_leaf(Tensor *t, int requires_grad) {
    if (!t) return NULL;
    AGNode *n = make_node(tt_retain(t), NULL, NULL, NULL, NULL);
    if (n) n->needs_grad = requires_grad ? 1 : 0;
    return n;
}

AGNode *ag_add(AGNode *a, AGNode *b) {
    if (!a || !b) return NULL;
    return make_node(tt_add(a->val, b->val), &OP_ADD, a, b, NULL);
}

AGNode *ag_mul(AGNode *a, AGNode *b) {
    if (!a || !b) return NULL;
    return make_node(tt_mul(a->val, b->val), &OP_MUL, a, b, NULL);
}

AGNode *ag_addscalar(AGNode *a, float s) {
    if (!a) return NULL;
    AGNode *n = make_node(tt_addscalar(a->val, s), &OP_ADDSCALAR, a, NULL, NULL);
    if (n) n->at.s = s;
    return n;
}

AGNode *ag_mulscalar(AGNode *a, float s) {
    if (!a) return NULL;
    AGNode *n = make_node(tt_mulscalar(a->val, s), &OP_MULSCALAR, a, NULL, NULL);
    if (n) n->at.s = s;
    return n;
}

/* The backward of a matmul with at most this many output columns (a
 * classifier layer) runs as one launch of tt_k_head_bwd. */
#define HEAD_MAX_N 32

/* The input of a padones node, when a is one: a matmul of a padones output
 * [X, 1] * W is X * W[:K-1] + W[K-1] (the weights' last row added to every
 * row), computed from X's aligned rows without reading the ones column. */
static const Tensor *padones_input(const AGNode *a) {
    if (a->op != &OP_PADONES || !a->in[0]) return NULL;
    const Tensor *x = a->in[0]->val;
    return x && x->ndim == 2 && x->shape[1] >= 1 && a->val->shape[1] == x->shape[1] + 1 ? x
                                                                                       : NULL;
}

AGNode *ag_matmul(AGNode *a, AGNode *b) {
    if (!a || !b) return NULL;
    const Tensor *av = a->val, *bv = b->val;
    if (tt_pend.active == TT_PEND_CHAIN_PAD && tt_pend.d == av && bv->ndim == 2 &&
        bv->shape[0] == av->shape[1] && bv->shape[1] == 10 && padones_input(a) == tt_pend.c) {
        /* the classifier of a pending conv chain (10 classes): it waits too;
         * a softmax-CE of it takes its partial sums from the chain's launch,
         * anything else runs the chain and then this GEMM */
        const TTPendConv s1 = tt_pend1, s2 = tt_pend;
        tt_pend1.active = tt_pend.active = 0;  /* the weights' device copy, nothing flushed */
        const float *wd = tt_dev(b->val);
        tt_pend1 = s1;
        tt_pend = s2;
        const long shp[2] = {av->shape[0], 10};
        Tensor *out = wd ? tt_empty_dev(shp, 2) : NULL;
        AGNode *n = out ? make_node(out, &OP_MATMUL, a, b, NULL) : NULL;
        if (!n) return NULL;
        tt_pend.fco = out;
        tt_pend.fcw = wd;
        tt_pend.fcn = 10;
        tt_pend.active = TT_PEND_CHAIN_FC;
        return n;
    }
    if (av->ndim == 2 && bv->ndim == 2 && av->shape[1] == bv->shape[0] && av->shape[0] > 0 &&
        av->shape[1] > 0 && bv->shape[1] > 0 && av->shape[0] <= 0x7fffffffL &&
        av->shape[1] <= 0x7fffffffL && bv->shape[1] <= 0x7fffffffL) {
        const Tensor *xv = padones_input(a);
        const int M = (int)av->shape[0], N = (int)bv->shape[1], K = (int)av->shape[1];
        const float *x = tt_dev((Tensor *)(xv ? xv : av)), *y = tt_dev(b->val);
        if (!x || !y) return NULL;
        const float *bias = xv ? y + (long)(K - 1) * N : NULL;
        const int Kx = xv ? K - 1 : K;
        const long shp[2] = {M, N};
        Tensor *out = tt_empty_dev(shp, 2);
        if (!out) return NULL;
        AGNode *n = make_node(out, &OP_MATMUL, a, b, NULL);
        if (!n) return NULL;
        if (tt_defer_enabled()) {
            /* left pending: a relu + padones of the product is then computed
             * by the GEMM's own epilogue */
            tt_pend.out = out;
            tt_pend.r = NULL;
            tt_pend.x = x;
            tt_pend.w = y;
            tt_pend.b = bias;
            tt_pend.geo[0] = M;
            tt_pend.geo[1] = N;
            tt_pend.geo[2] = Kx;
            tt_pend.active = TT_PEND_MATMUL;
            return n;
        }
        const int rc = bias ? tt_k_gemm_bias_relu_pad(M, N, Kx, x, y, bias, out->dev, NULL, NULL)
                            : tt_k_gemm(M, N, K, x, K, 0, y, N, 0, out->dev, N);
        if (rc != 0) {
            ag_release(n);
            return NULL;
        }
        return n;
    }
    return make_node(tt_matmul_omp(a->val, b->val, 0), &OP_MATMUL, a, b, NULL);
}

AGNode *ag_relu(AGNode *a) {
    if (!a) return NULL;
    if (tt_pend.active == TT_PEND_MATMUL && tt_pend.out == a->val) {
        /* the matmul producing a is still pending: its relu waits with it
         * (a padones of the relu then fuses all three) */
        Tensor *r = tt_empty_like(a->val);
        if (!r) return NULL;
        AGNode *n = make_node(r, &OP_RELU, a, NULL, NULL);
        if (!n) return NULL;
        tt_pend.r = r;
        tt_pend.active = TT_PEND_MATMUL_RELU;
        return n;
    }
    if (tt_pend.active == TT_PEND_CONV && tt_pend.out == a->val) {
        /* the convolution producing a is still pending: its relu waits with
         * it, and one launch writes both (same values as tt_relu of the
         * stored output) -- with a 2x2 max pool of the relu too when that is
         * the next call */
        Tensor *r = tt_empty_like(a->val);
        if (!r) return NULL;
        AGNode *n = make_node(r, &OP_RELU, a, NULL, NULL);
        if (!n) return NULL;
        tt_pend.r = r;
        tt_pend.active = TT_PEND_CONV_RELU;
        return n;
    }
    if (tt_defer_enabled() && a->val->ndim == 2) {
        /* a relu that a padones may consume (the MLP's hidden layers): left
         * pending like the convolution above */
        const float *x = tt_dev(a->val);
        Tensor *r = x ? tt_empty_like(a->val) : NULL;
        if (!r) return NULL;
        AGNode *n = make_node(r, &OP_RELU, a, NULL, NULL);
        if (!n) return NULL;
        tt_pend.out = r;
        tt_pend.x = x;
        tt_pend.active = TT_PEND_RELU;
        return n;
    }
    return make_node(tt_relu(a->val), &OP_RELU, a, NULL, NULL);
}

AGNode *ag_softmax(AGNode *a) {
    if (!a) return NULL;
    return make_node(tt_softmax(a->val), &OP_SOFTMAX, a, NULL, NULL);
}

AGNode *ag_padones(AGNode *a) {
    if (!a || a->val->ndim != 2) return NULL;
    const long M = a->val->shape[0], K = a->val->shape[1];
    const long shp[2] = {M, K + 1};
    if (tt_pend1.active && tt_pend.active == TT_PEND_CONV_RELU_POOL_COPY && tt_pend.c == a->val) {
        /* both convolutions of a conv -> relu -> pool chain, the second's
         * flattening copy and this padones in one launch -- left pending
         * too, so that a classifier matmul of this padones and its
         * softmax-CE can join it */
        Tensor *v = tt_chain_ready() ? tt_empty_dev(shp, 2) : NULL;
        if (v) {
            AGNode *n = make_node(v, &OP_PADONES, a, NULL, NULL);
            if (n) {
                tt_pend.d = v;
                tt_pend.active = TT_PEND_CHAIN_PAD;
            }
            return n;
        }
        tt_flush_first();  /* the first by itself; the second and this padones below */
    }
    if (tt_pend.active == TT_PEND_CONV_RELU_POOL_COPY && tt_pend.c == a->val) {
        /* convolution, relu, pool, flattening copy and this padones in one
         * launch */
        Tensor *v = tt_empty_dev(shp, 2);
        if (v) {
            const TTPendConv p = tt_pend;
            const int *q = p.geo;
            tt_pend.active = 0;
            /* the relu output is not stored: a recipe run on first use */
            if (tt_k_conv2d_relu_pool_fwd_lds(p.x, p.w, p.b, p.out->dev, NULL, p.p->dev,
                                              p.c->dev, v->dev,
                                              p.codes ? (unsigned char *)p.codes->dev : NULL,
                                              q[0], q[1], q[2], q[3],
                                              q[4], q[5], q[6], q[7], q[8], q[9], q[10], q[11],
                                              q[12]) == 0) {
                if (p.codes) *p.codes_dst = p.codes;
                if (tt_lazy_relu(p.r, p.out) != 0 &&
                    tt_k_relu_fwd(p.out->dev, p.r->dev, p.r->numel) != 0)
                    p.r->valid = 0;
                return make_node(v, &OP_PADONES, a, NULL, NULL);
            }
            tt_pend = p;  /* not launched: the chain runs below, then the padones */
            tt_release(v);
        }
    }
    if (tt_pend.active == TT_PEND_COPY && tt_pend.out == a->val) {
        /* a is a reshape whose copy is still pending: one pass writes the
         * copy and the padded tensor */
        Tensor *v = tt_empty_dev(shp, 2);
        if (v) {
            const TTPendConv p = tt_pend;
            tt_pend.active = 0;
            if (tt_k_copy_padones_fwd(p.x, p.out->dev, v->dev, M, K) == 0)
                return make_node(v, &OP_PADONES, a, NULL, NULL);
            tt_pend = p;  /* not launched: the plain copy runs below */
            tt_release(v);
        }
    }
    if (tt_pend.active == TT_PEND_MATMUL_RELU && tt_pend.r == a->val) {
        /* matmul, relu and padones in one GEMM + reduction */
        Tensor *v = tt_empty_dev(shp, 2);
        if (v) {
            const TTPendConv p = tt_pend;
            tt_pend.active = 0;
            if ((p.b ? tt_k_gemm_bias_relu_pad(p.geo[0], p.geo[1], p.geo[2], p.x, p.w, p.b,
                                               p.out->dev, p.r->dev, v->dev)
                     : tt_k_gemm_relu_pad(p.geo[0], p.geo[1], p.geo[2], p.x, p.w, p.out->dev,
                                          p.r->dev, v->dev)) == 0)
                return make_node(v, &OP_PADONES, a, NULL, NULL);
            tt_pend = p;  /* not launched: the plain matmul and relu run below */
            tt_release(v);
        }
    }
    if (tt_pend.active == TT_PEND_RELU && tt_pend.out == a->val) {
        Tensor *v = tt_empty_dev(shp, 2);
        if (v) {
            const TTPendConv p = tt_pend;
            tt_pend.active = 0;
            if (tt_k_relu_padones_fwd(p.x, p.out->dev, v->dev, M, K) == 0)
                return make_node(v, &OP_PADONES, a, NULL, NULL);
            tt_pend = p;  /* not launched: the plain relu runs below */
            tt_release(v);
        }
    }
    const float *x = tt_dev(a->val);
    if (!x) return NULL;
    Tensor *v = tt_empty_dev(shp, 2);
    if (!v) return NULL;
    /* an input that needs no gradient (never changed in place by the
     * library): the padded copy is a recipe, written when first read -- a
     * matmul of it reads the input itself, forward (ag_matmul) and for its
     * weight gradient (tt_k_gemm_tn_padones) */
    if (!(tt_defer_enabled() && !needs(a) && tt_lazy_padones(v, a->val) == 0) &&
        tt_k_padones_fwd(x, v->dev, M, K)) {
        tt_release(v);
        return NULL;
    }
    return make_node(v, &OP_PADONES, a, NULL, NULL);
}

AGNode *ag_reshape(AGNode *a, const long *new_shape, int new_ndim) {
    if (!a) return NULL;
    if (tt_pend.active == TT_PEND_CONV_RELU_POOL && tt_pend.p == a->val && new_shape &&
        new_ndim == 2 && new_shape[0] == a->val->shape[0] &&
        new_shape[0] > 0 && new_shape[1] == a->val->numel / new_shape[0] &&
        new_shape[0] * new_shape[1] == a->val->numel) {
        /* a flattening reshape of a pending pool output: its copy waits too */
        Tensor *v = tt_empty_dev(new_shape, 2);
        if (!v) return NULL;
        AGNode *n = make_node(v, &OP_RESHAPE, a, NULL, NULL);
        if (!n) return NULL;
        tt_pend.c = v;
        tt_pend.active = TT_PEND_CONV_RELU_POOL_COPY;
        return n;
    }
    Tensor *v = tt_reshape_ex(a->val, new_shape, new_ndim, 1);
    if (!v) return NULL;
    AGNode *n = make_node(v, &OP_RESHAPE, a, NULL, NULL);
    if (!n && tt_pend.active && tt_pend.out == v) tt_pend.active = 0;  /* v was released */
    return n;
}

AGNode *ag_conv2d(AGNode *a, AGNode *w, AGNode *b, int sh, int sw, int ph, int pw) {
    if (!a || !w) return NULL;
    const int keep = w->needs_grad;
    const int ones = keep && b && b->needs_grad;  /* fuse db into the dW GEMM */
    float *col = NULL;
    Tensor *v = tt_conv2d_keepcol_ex(a->val, w->val, b ? b->val : NULL, sh, sw, ph, pw,
                                     keep ? &col : NULL, ones, 1);
    if (!v) return NULL;
    AGNode *n = make_node(v, &OP_CONV2D, a, w, b);
    if (!n) {
        if (tt_pend.active && tt_pend.out == v) tt_pend.active = 0;  /* v was released */
        ttrt_free(col);
        return NULL;
    }
    n->at.conv.sh = sh; n->at.conv.sw = sw;
    n->at.conv.ph = ph; n->at.conv.pw = pw;
    n->at.conv.col = col;
    n->at.conv.col_ones = col && ones;
    return n;
}

static AGNode *pool_node(AGNode *a, Tensor *v, const AGOp *op, int ph, int pw, int sh, int sw) {
    AGNode *n = make_node(v, op, a, NULL, NULL);
    if (!n) return NULL;
    n->at.win.kh = ph; n->at.win.kw = pw;
    n->at.win.sh = sh; n->at.win.sw = sw;
    return n;
}

AGNode *ag_maxpool2d(AGNode *a, int ph, int pw, int sh, int sw) {
    if (!a) return NULL;
    if (tt_pend.active == TT_PEND_CONV_RELU && tt_pend.r == a->val && ph == 2 && pw == 2 &&
        sh == 2 && sw == 2 && a->val->ndim == 4 && a->val->shape[2] % 2 == 0 &&
        a->val->shape[3] % 2 == 0) {
        /* the convolution and relu producing a are still pending: this pool
         * waits with them (one launch writes all three, and a flattening
         * reshape + padones of the pool's output can join it) */
        const long shp[4] = {a->val->shape[0], a->val->shape[1], a->val->shape[2] / 2,
                             a->val->shape[3] / 2};
        Tensor *v = tt_empty_dev(shp, 4);
        if (!v) return NULL;
        AGNode *n = pool_node(a, v, &OP_MAXPOOL2D, ph, pw, sh, sw);
        if (!n) return NULL;
        tt_pend.p = v;
        /* the launch also writes each window's argmax + relu mask (a byte),
         * from which the backward runs without reading the relu values */
        const long cshp[1] = {(v->numel + 3) / 4};
        tt_pend.codes = tt_empty_dev(cshp, 1);
        tt_pend.codes_dst = &n->at.win.codes;
        tt_pend.active = TT_PEND_CONV_RELU_POOL;
        return n;
    }
    Tensor *v = tt_maxpool2d(a->val, ph, pw, sh, sw);
    if (!v) return NULL;
    return pool_node(a, v, &OP_MAXPOOL2D, ph, pw, sh, sw);
}

AGNode *ag_avgpool2d(AGNode *a, int ph, int pw, int sh, int sw) {
    if (!a) return NULL;
    Tensor *v = tt_avgpool2d(a->val, ph, pw, sh, sw);
    if (!v) return NULL;
    return pool_node(a, v, &OP_AVGPOOL2D, ph, pw, sh, sw);
}

/* Fused softmax + mean cross-entropy (no reference counterpart: the
 * reference harness does this in NumPy, tests/gate_cifar_cnn.py:175-181). */
/* The classifier logits = padones(relu(h)) x W pending, its softmax-CE
 * about to run in the GEMM's launch: the same launch also forms, from each
 * row's seed, the gradients the classifier's backward would give the
 * padones node, the relu node and h (dA = seed [W]^T, d1, d2; the
 * classifier backward kernel's values bit for bit), in sda.  They are the
 * backward's when it starts from this loss with the default seed and the
 * three nodes have no other consumer (backward_matmul checks); otherwise
 * they are dropped.  0: launched (logits, probs, seed, row losses and sda
 * written); else nothing launched, sda empty. */
static int ce_spec(AGNode *logits, const TTPendConv *p, const int32_t *hlab, Tensor *probs,
                   Tensor *seed, Tensor *rl, Tensor *sda[3], int **stale) {
    if (!tt_defer_enabled() || logits->op != &OP_MATMUL) return -1;
    AGNode *a = logits->in[0];
    if (!a || a->op != &OP_PADONES || !needs(a)) return -1;
    AGNode *x = a->in[0];
    if (!x || x->op != &OP_RELU || !needs(x->in[0]) || !x->val || p->x != x->val->dev ||
        !p->b || p->b != p->w + (long)p->geo[2] * p->geo[1])
        return -1;
    sda[0] = tt_empty_like(a->val);
    sda[1] = sda[0] ? tt_empty_like(x->val) : NULL;
    sda[2] = sda[1] ? tt_empty_like(x->in[0]->val) : NULL;
    const TTCeHook hk = {p->b, hlab, probs->dev, seed->dev, rl->dev,
                         1.0f / (float)p->geo[0]};
    /* sda[1] (dA without its ones column) is left to a recipe of sda[0] */
    const int rc = sda[2] ? ttk_gemm_rows_da(p->x, p->w, p->b, p->out->dev, NULL, NULL,
                                             p->geo[0], p->geo[1], p->geo[2], &hk, sda[0]->dev,
                                             NULL, sda[2]->dev)
                          : -1;
    if (rc != 0) {
        for (int i = 0; i < 3; i++) { tt_release(sda[i]); sda[i] = NULL; }
        return -1;
    }
    tt_mark_dev_written(sda[0]);
    tt_mark_dev_written(sda[2]);
    /* formed with W as it is now: a write to W before the backward makes
     * them stale (the backward then computes its own) */
    *stale = (int *)calloc(1, sizeof(int));
    if (!*stale || tt_lazy_guard(logits->in[1]->val, *stale) != 0) **stale = 1;
    return 0;
}

AGNode *ag_softmax_ce(AGNode *logits, const int *labels, long rows) {
    if (!logits || !labels || logits->val->ndim != 2 || logits->val->shape[0] != rows ||
        rows <= 0 || logits->val->shape[1] > 0x7fffffffL)
        return NULL;
    const int cols = (int)logits->val->shape[1];
    const long one = 1;
    Tensor *probs = tt_empty_like(logits->val);
    Tensor *seed = tt_empty_like(logits->val);
    Tensor *loss = tt_empty_dev(&one, 1);
    int32_t *hlab = (int32_t *)malloc(sizeof(int32_t) * (size_t)rows);
    if (hlab)
        for (long r = 0; r < rows; r++) hlab[r] = (int32_t)labels[r];
    if (tt_pend.active == TT_PEND_CHAIN_FC && tt_pend.fco == logits->val && probs && seed &&
        loss && hlab && rows <= TT_CE_ARG_ROWS) {
        /* the conv chain, its classifier and this softmax-CE pending: the
         * chain's launch leaves the classifier's two partial sums per row
         * (the halves of each image), and one reduction adds them, the bias
         * and runs the softmax-CE (the mean loss a recipe, as below) */
        const TTPendConv p = tt_pend;
        const int K = (int)p.c->shape[1];
        const float *bias = p.fcw + (long)K * cols;
        Tensor *rl = tt_empty_dev(&rows, 1);
        float *ws = rl ? (float *)ttrt_alloc(sizeof(float) * 2 * (size_t)rows * cols) : NULL;
        if (ws && tt_chain_launch(ws) == 0) {
            /* the reduction is a recipe of all four outputs: the classifier's
             * backward forms the seed itself and writes them, any earlier
             * read runs it (ttk_reduce_ce) */
            Tensor *const out4[4] = {logits->val, probs, seed, rl};
            int rc = tt_lazy_ce_job(out4, logits->in[1]->val, ws, bias, hlab, (int)rows, cols,
                                    1.0f / (float)rows);
            if (rc != 0) {
                const TTCeHook hk = {bias, hlab, probs->dev, seed->dev, rl->dev,
                                     1.0f / (float)rows};
                rc = ttk_reduce_ce(ws, logits->val->dev, (int)rows, cols, 2, 1, &hk);
                ttrt_free(ws);
            }
            if (rc == 0 && (tt_lazy_ce_mean(loss, rl) == 0 ||
                            tt_k_ce_mean_rows(tt_dev(rl), loss->dev, (int)rows) == 0)) {
                tt_release(rl);
                AGNode *n = make_node(loss, &OP_SOFTMAX_CE, logits, NULL, NULL);
                if (!n) { tt_release(probs); tt_release(seed); free(hlab); return NULL; }
                n->at.ce.probs = probs;
                n->at.ce.seed = seed;
                n->at.ce.labels = hlab;
                return n;
            }
            /* the reduction did not run: the logits from the GEMM (the
             * softmax-CE runs below) */
            if (rc != 0 && tt_k_gemm_bias_relu_pad((int)rows, cols, K, p.c->dev, p.fcw, bias,
                                                   logits->val->dev, NULL, NULL) != 0)
                logits->val->valid = 0;
        } else {
            ttrt_free(ws);
        }
        tt_release(rl);
    }
    if (tt_pend.active == TT_PEND_MATMUL && tt_pend.out == logits->val && tt_pend.b && probs &&
        seed && loss && hlab && rows <= TT_CE_ARG_ROWS && cols <= 32) {
        /* the classifier's GEMM is still pending: the softmax-CE runs in its
         * split-K reduction, and the mean loss becomes a recipe of the row
         * losses (nothing in the backward reads it) */
        Tensor *rl = tt_empty_dev(&rows, 1);
        const TTPendConv p = tt_pend;
        tt_pend.active = 0;
        Tensor *sda[3] = {NULL, NULL, NULL};
        int *stale = NULL;
        int rc = rl ? ce_spec(logits, &p, hlab, probs, seed, rl, sda, &stale) : -1;
        if (rc != 0)
            rc = rl ? tt_k_gemm_bias_ce(p.geo[0], p.geo[1], p.geo[2], p.x, p.w, p.b, p.out->dev,
                                        hlab, probs->dev, seed->dev, rl->dev, 1.0f / (float)rows)
                    : -1;
        if (rc == 0 && (tt_lazy_ce_mean(loss, rl) == 0 ||
                        tt_k_ce_mean_rows(rl->dev, loss->dev, (int)rows) == 0)) {
            tt_release(rl);
            AGNode *n = make_node(loss, &OP_SOFTMAX_CE, logits, NULL, NULL);
            if (!n) {
                tt_release(probs); tt_release(seed); free(hlab);
                spec_drop(sda, &stale);
                return NULL;
            }
            n->at.ce.probs = probs;
            n->at.ce.seed = seed;
            n->at.ce.labels = hlab;
            for (int i = 0; i < 3; i++) n->at.ce.sda[i] = sda[i];
            n->at.ce.stale = stale;
            return n;
        }
        spec_drop(sda, &stale);
        tt_release(rl);
        if (rc < 0) tt_pend = p;  /* not run: the pending GEMM is launched below */
        /* else the GEMM wrote the logits: the softmax-CE runs below */
    }
    const float *x = tt_dev(logits->val);
    if (!x) {
        tt_release(probs); tt_release(seed); tt_release(loss); free(hlab);
        return NULL;
    }
    /* small batches: the labels travel inside the kernel's arguments */
    if (probs && seed && loss && hlab && rows <= TT_CE_ARG_ROWS &&
        tt_k_softmax_ce_mean_hostlab(x, hlab, probs->dev, loss->dev, seed->dev, rows, cols,
                                     1.0f / (float)rows) == 0) {
        AGNode *n = make_node(loss, &OP_SOFTMAX_CE, logits, NULL, NULL);
        if (!n) { tt_release(probs); tt_release(seed); free(hlab); return NULL; }
        n->at.ce.probs = probs;
        n->at.ce.seed = seed;
        n->at.ce.labels = hlab;
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
    AGNode *n = make_node(loss, &OP_SOFTMAX_CE, logits, NULL, NULL);
    if (!n) { tt_release(probs); tt_release(seed); return NULL; }
    n->at.ce.probs = probs;
    n->at.ce.seed = seed;
    return n;
}

Tensor *ag_softmax_ce_probs(const AGNode *n) {
    return (n && n->op == &OP_SOFTMAX_CE) ? n->at.ce.probs : NULL;
}

/* ---------- accessors ---------- */

Tensor *ag_value(const AGNode *n) { return n ? n->val : NULL; }
Tensor *ag_grad(const AGNode *n) {
    if (!n) return NULL;
    if (g_lazy) materialise_for(n);
    return n->grad;
}
int ag_requires_grad(const AGNode *n) { return n ? n->needs_grad : 0; }

/* ---------- backward rules ---------- */

static void backward_add(AGNode *n) {
    accum_copy(n->in[0], n->grad);
    accum_copy(n->in[1], n->grad);
}

static void backward_mul(AGNode *n) {
    AGNode *a = n->in[0], *b = n->in[1];
    if (needs(a)) accum_move(a, tt_mul(n->grad, b->val));   /* g * b */
    if (needs(b)) accum_move(b, tt_mul(n->grad, a->val));   /* g * a */
}

static void backward_addscalar(AGNode *n) { accum_copy(n->in[0], n->grad); }

static void backward_mulscalar(AGNode *n) {
    if (needs(n->in[0])) accum_move(n->in[0], tt_mulscalar(n->grad, n->at.s));
}

static int relu_fusable(const AGNode *r);

/* Both gradients of matmul n in one launch and, when A is a padones used
 * only here whose input is used only by it, that input's gradient too --
 * and, when the input is a reshape or a fusable relu, the gradient of the
 * node before it: the classifier-layer kernel (tt_k_head_bwd) for at most
 * HEAD_MAX_N output columns, else the paired small-GEMM kernel
 * (tt_k_matmul_bwd_small, which needs both gradients).  The nodes whose
 * rules this covers are marked `fused`.  0 when done; -1: not taken,
 * nothing launched. */
static int backward_matmul_fused(AGNode *n, const float *g, const TTHeadCeArgs *ce) {
    AGNode *a = n->in[0], *b = n->in[1];
    const int M = (int)a->val->shape[0], K = (int)a->val->shape[1], N = (int)b->val->shape[1];
    const int head = N <= HEAD_MAX_N;
    if (!head && !(needs(a) && needs(b))) return -1;
    if (ce && !head) return -1;
    const float *ad = needs(b) ? tt_dev(a->val) : NULL;
    const float *bd = needs(a) ? tt_dev(b->val) : NULL;
    if ((needs(b) && !ad) || (needs(a) && !bd)) return -1;
    AGNode *x = NULL, *y = NULL;
    const float *R = NULL;
    if (needs(a) && a->op == &OP_PADONES && a->fanin == 1 && !a->grad && needs(a->in[0]) &&
        a->in[0]->fanin == 1 && !a->in[0]->grad) {
        x = a->in[0];
        AGNode *z = x->in[0];
        if (x->op == &OP_RESHAPE && needs(z) && z->fanin == 1 && !z->grad) {
            y = z;
        } else if (relu_fusable(x)) {
            y = z;
            R = tt_dev(x->val);
            if (!R) return -1;
        }
    }
    /* y a 2x2 max pool (with its windows' codes) of a fusable relu: the head
     * kernel writes the relu input's gradient too (the pool and relu rules
     * are covered; the relu's own gradient stays a recipe) */
    AGNode *pr = NULL;
    const unsigned char *codes = NULL;
    if (head && y && !R && x->op == &OP_RESHAPE && y->op == &OP_MAXPOOL2D && y->at.win.codes &&
        y->at.win.kh == 2 && y->at.win.kw == 2 && y->at.win.sh == 2 && y->at.win.sw == 2 &&
        y->val->ndim == 4 && relu_fusable(y->in[0]) &&
        y->in[0]->val->shape[2] == 2 * y->val->shape[2] &&
        y->in[0]->val->shape[3] == 2 * y->val->shape[3]) {
        codes = (const unsigned char *)tt_dev(y->at.win.codes);
        if (codes) pr = y->in[0];
    }
    Tensor *gb = needs(b) ? tt_empty_like(b->val) : NULL;
    Tensor *ga = needs(a) ? tt_empty_like(a->val) : NULL;
    Tensor *tx = x ? tt_empty_like(x->val) : NULL;
    Tensor *ty = y ? tt_empty_like(y->val) : NULL;
    Tensor *tc = pr ? tt_empty_like(pr->in[0]->val) : NULL;
    int rc = -1;
    if ((!needs(b) || gb) && (!needs(a) || ga) && (!x || tx) && (!y || ty) && (!pr || tc)) {
        float *dB = gb ? gb->dev : NULL, *dA = ga ? ga->dev : NULL;
        float *d1 = tx ? tx->dev : NULL, *d2 = ty ? ty->dev : NULL;
        /* with the pool's backward in the launch (the convolution's output
         * gradient written), the reshape's and the pool's own gradients --
         * dA without its ones column -- are recipes of dA (written if read) */
        const int lazy12 = pr && dA && tt_defer_enabled();
        if (pr)
            rc = ce ? ttk_head_bwd_ce(ad, M, K, bd, N, ce, dB, dA, lazy12 ? NULL : d1,
                                      lazy12 ? NULL : d2, NULL, codes, tc->dev,
                                      (int)y->val->shape[1], (int)y->val->shape[2],
                                      (int)y->val->shape[3])
                    : tt_k_head_bwd_pool(ad, M, K, bd, N, g, dB, dA, lazy12 ? NULL : d1,
                                         lazy12 ? NULL : d2, codes, tc->dev,
                                         (int)y->val->shape[1], (int)y->val->shape[2],
                                         (int)y->val->shape[3]);
        if (rc == 0 && pr && lazy12) {
            if (tx && tt_lazy_padones_bwd(tx, ga, M, K - 1) != 0)
                rc = tt_k_padones_bwd(dA, d1, M, K - 1);
            if (rc == 0 && ty && tt_lazy_padones_bwd(ty, ga, M, K - 1) != 0)
                rc = tt_k_padones_bwd(dA, d2, M, K - 1);
        }
        if (rc != 0) {
            tt_release(tc);
            tc = NULL;
            pr = NULL;
            rc = ce ? ttk_head_bwd_ce(ad, M, K, bd, N, ce, dB, dA, d1, d2, R, NULL, NULL, 0, 0, 0)
                 : head ? tt_k_head_bwd(ad, M, K, bd, N, g, dB, dA, d1, d2, R)
                        : tt_k_matmul_bwd_small(ad, M, K, bd, N, g, dB, dA, d1, d2, R);
        }
    }
    if (rc != 0) {
        tt_release(gb); tt_release(ga); tt_release(tx); tt_release(ty); tt_release(tc);
        return -1;
    }
    if (gb) accum_move(b, gb);
    if (ga) accum_move(a, ga);
    if (tx) { accum_move(x, tx); a->fused = 1; }
    if (ty) { accum_move(y, ty); x->fused = 1; }
    if (pr) {
        lazy_set(pr, y->grad, NULL);
        accum_move(pr->in[0], tc);
        y->fused = 1;
        pr->fused = 1;
    }
    return 0;
}

/* The input gradients its softmax-CE formed with the seed (ce_spec), when
 * they are this pass's: the node's gradient is still exactly that seed (the
 * loss its only consumer), the weights have not been written since (no
 * optimizer step, no host access), and the padones and relu feed only this
 * node, as backward_matmul_fused requires for the same outputs.  Then only dB is left:
 * a recipe the optimizer's step runs in its own launch.  0 when taken. */
static long g_spec_taken;  /* backward rules that took them (tth_ce_spec_count) */
long tth_ce_spec_count(void) { return g_spec_taken; }

static int backward_matmul_spec(AGNode *n) {
    Tensor *sda[3] = {n->at.mm.sda[0], n->at.mm.sda[1], n->at.mm.sda[2]};
    for (int i = 0; i < 3; i++) n->at.mm.sda[i] = NULL;
    const int stale = !n->at.mm.stale || *n->at.mm.stale;
    if (n->at.mm.stale) {
        tt_lazy_guard_drop(n->at.mm.stale);
        free(n->at.mm.stale);
        n->at.mm.stale = NULL;
    }
    AGNode *a = n->in[0], *b = n->in[1];
    AGNode *x = a->in[0];
    const int M = (int)a->val->shape[0], K = (int)a->val->shape[1], N = (int)b->val->shape[1];
    const int ok = !stale && n->fanin == 1 && a->op == &OP_PADONES && a->fanin == 1 && !a->grad &&
                   relu_fusable(x) && !x->grad && needs(b) && tt_defer_enabled() &&
                   ttk_gemm_tn_padones_any(M, K - 1, N, NULL, NULL, NULL) == 0;
    Tensor *gb = ok ? tt_empty_like(b->val) : NULL;
    if (!gb || tt_lazy_gemm_tn_padones(gb, x->val, n->grad, M, K - 1, N) != 0) {
        tt_release(gb);
        for (int i = 0; i < 3; i++) tt_release(sda[i]);
        return -1;
    }
    if (tt_lazy_padones_bwd(sda[1], sda[0], M, K - 1) != 0 &&
        tt_k_padones_bwd(sda[0]->dev, sda[1]->dev, M, K - 1) != 0) {
        tt_release(gb);
        for (int i = 0; i < 3; i++) tt_release(sda[i]);
        return -1;
    }
    accum_move(b, gb);
    accum_move(a, sda[0]);
    accum_move(x, sda[1]);
    a->fused = 1;
    accum_move(x->in[0], sda[2]);
    x->fused = 1;
    g_spec_taken++;
    return 0;
}

static void backward_matmul(AGNode *n) {
    AGNode *a = n->in[0], *b = n->in[1];
    const int M = (int)a->val->shape[0], K = (int)a->val->shape[1], N = (int)b->val->shape[1];
    if (n->at.mm.sda[0] && backward_matmul_spec(n) == 0) return;
    /* the output gradient is a softmax-CE seed still to be reduced from the
     * logits' partial sums: the classifier kernel forms it itself (and
     * writes the softmax-CE's outputs) */
    TTHeadCeArgs ce;
    void *job = NULL;
    if (tt_defer_enabled() && tt_lazy_ce_args(n->grad, &ce, &job) == 0 &&
        backward_matmul_fused(n, NULL, &ce) == 0) {
        tt_lazy_ce_done(job);
        return;
    }
    const float *g = tt_dev(n->grad);
    if (!g) return;
    if (tt_defer_enabled() && backward_matmul_fused(n, g, NULL) == 0) return;
    if (needs(b) && !needs(a) && a->op == &OP_PADONES && K > 1) {
        /* dB from the padones input: the padded copy is not read; with the
         * deferral, dB is a recipe that the optimizer's step runs in its own
         * launch (or the first read runs by itself) */
        if (tt_defer_enabled() &&
            tt_k_gemm_tn_padones(M, K - 1, N, NULL, NULL, NULL) == 0) {
            Tensor *gb = tt_empty_like(b->val);
            if (gb && tt_lazy_gemm_tn_padones(gb, a->in[0]->val, n->grad, M, K - 1, N) == 0) {
                accum_move(b, gb);
                return;
            }
            tt_release(gb);
        }
        const float *xd = tt_dev(a->in[0]->val);
        Tensor *gb = xd ? tt_empty_like(b->val) : NULL;
        if (gb && tt_k_gemm_tn_padones(M, K - 1, N, xd, g, gb->dev) == 0) {
            accum_move(b, gb);
            return;
        }
        tt_release(gb);
    }
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
    AGNode *a = n->in[0];
    if (!needs(a)) return;
    const float *x = tt_dev(a->val), *g = tt_dev(n->grad);
    if (!x || !g) return;
    Tensor *t = tt_empty_like(a->val);
    if (!t) return;
    if (tt_k_relu_bwd(x, g, t->dev, t->numel)) { tt_release(t); return; }
    accum_move(a, t);
}

static void backward_softmax(AGNode *n) {
    AGNode *a = n->in[0];
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
    return r->op == &OP_RELU && r->fanin == 1 && !r->grad && !r->lazy_g && needs(r->in[0]) &&
           r->in[0]->fanin == 1;
}

/* hand the fused pass's two gradients to the relu and its input */
static void fused_relu_done(AGNode *r, Tensor *dr, Tensor *dx) {
    accum_move(r, dr);
    accum_move(r->in[0], dx);
    r->fused = 1;
}

static void backward_padones(AGNode *n) {
    AGNode *a = n->in[0];
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
    if (a->op == &OP_RESHAPE && a->fanin == 1 && !a->grad && needs(a->in[0]) &&
        a->in[0]->fanin == 1) {
        /* a reshape (a copy) feeds only this padones: its gradient and its
         * input's gradient are the same values, written by one pass */
        AGNode *x = a->in[0];
        Tensor *t = tt_empty_like(a->val), *u = t ? tt_empty_like(x->val) : NULL;
        if (u && tt_k_padones_bwd2(g, t->dev, u->dev, a->val->shape[0], a->val->shape[1]) == 0) {
            accum_move(a, t);
            accum_move(x, u);
            a->fused = 1;
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
    AGNode *a = n->in[0];
    if (!needs(a)) return;
    accum_move(a, tt_reshape(n->grad, a->val->shape, a->val->ndim));
}

static int conv_takes_pooled(const AGNode *c);
static void conv_geo(const AGNode *c, int q[13]);

/* The second convolution of a conv -> relu -> 2x2 pool -> conv chain (the
 * tt_k_conv2d_chain_fwd shape): its input gradient (the pool's gradient,
 * complete here: the pool feeds only this convolution) and, through the pool
 * codes, the first convolution's weight gradient in one launch
 * (ttk_conv2d_chain_bwd, its reduction deferred like conv_dw_deferred's),
 * and in the same grid this convolution's own weight gradient.  The first
 * convolution's rule then has nothing left to do (its input needs no
 * gradient; its own gradient stays the recipe the pool's rule leaves).
 * 0: not taken, nothing launched; 1: done without this convolution's weight
 * gradient; 2: with it. */
static int conv_chain_bwd(AGNode *n, const float *gd) {
    AGNode *p = n->in[0];
    if (!tt_chain_enabled() || !needs(p) || p->op != &OP_MAXPOOL2D || !p->at.win.codes ||
        p->fanin != 1 || p->grad || p->lazy_g || p->at.win.kh != 2 || p->at.win.kw != 2 ||
        p->at.win.sh != 2 || p->at.win.sw != 2)
        return 0;
    AGNode *r = p->in[0];
    if (!relu_fusable(r)) return 0;
    AGNode *c = r->in[0];
    if (!conv_takes_pooled(c)) return 0;
    int q1[13], q2[13];
    conv_geo(c, q1);
    conv_geo(n, q2);
    static const int k[6] = {3, 3, 1, 1, 1, 1};
    for (int i = 0; i < 6; i++)
        if (q1[5 + i] != k[i] || q2[5 + i] != k[i]) return 0;
    if (q1[2] != 32 || q1[3] != 32 || q1[4] != 32 || q2[0] != q1[0] || q2[1] != 32 ||
        q2[2] != 16 || q2[3] != 16 || q2[4] != 64)
        return 0;
    AGNode *w1 = c->in[1], *b1 = c->n_in > 2 ? c->in[2] : NULL;
    const long bshp[1] = {32};
    const float *w2 = tt_dev(n->in[1]->val), *x = tt_dev(c->in[0]->val);
    const unsigned char *codes = (const unsigned char *)tt_dev(p->at.win.codes);
    Tensor *ga = w2 && x && codes ? tt_empty_like(p->val) : NULL;
    Tensor *gw = ga ? tt_empty_like(w1->val) : NULL;
    Tensor *gb = gw && needs(b1) ? tt_empty_dev(bshp, 1) : NULL;
    if (!gw || (needs(b1) && !gb)) {
        tt_release(ga);
        tt_release(gw);
        tt_release(gb);
        return 0;
    }
    /* this convolution's own weight gradient (and bias) in the same grid,
     * when its LDS path would compute it (the forward kept no col) */
    AGNode *w2n = n->in[1], *b2n = n->n_in > 2 ? n->in[2] : NULL;
    const long b2shp[1] = {64};
    const float *x2 = needs(w2n) && !n->at.conv.col ? tt_dev(p->val) : NULL;
    Tensor *gw2 = x2 ? tt_empty_like(w2n->val) : NULL;
    Tensor *gb2 = gw2 && needs(b2n) ? tt_empty_dev(b2shp, 1) : NULL;
    if (gw2 && needs(b2n) && !gb2) {
        tt_release(gw2);
        gw2 = NULL;
    }
    TTDwtJob job, job2;
    int rc = gw2 ? ttk_conv2d_chain_bwd(gd, w2, codes, x, ga->dev, gw->dev, gb ? gb->dev : NULL,
                                        q1[0], q1[1], &job, x2, gw2->dev, gb2 ? gb2->dev : NULL,
                                        &job2)
                 : -1;
    if (rc != 0) {
        tt_release(gw2);
        tt_release(gb2);
        gw2 = gb2 = NULL;
        rc = ttk_conv2d_chain_bwd(gd, w2, codes, x, ga->dev, gw->dev, gb ? gb->dev : NULL, q1[0],
                                  q1[1], &job, NULL, NULL, NULL, NULL);
    }
    if (rc != 0) {
        tt_release(ga);
        tt_release(gw);
        tt_release(gb);
        return 0;
    }
    if (gw2) {
        if (tt_lazy_dwt(gw2, gb2, &job2) != 0) ttk_dwt_reduce_jobs(&job2, 1);
        if (gb2) accum_move(b2n, gb2);
        accum_move(w2n, gw2);
    }
    if (tt_lazy_dwt(gw, gb, &job) != 0) ttk_dwt_reduce_jobs(&job, 1);
    accum_move(p, ga);
    if (gb) accum_move(b1, gb);
    accum_move(w1, gw);
    c->fused = 1;
    return gw2 ? 2 : 1;
}

static void backward_conv2d(AGNode *n) {
    if (n->lazy_codes) {
        if (conv_pooled_dw(n)) return;
        materialise(n);
        if (!n->grad) return;  /* could not be written (out of memory) */
    }
    AGNode *a = n->in[0], *w = n->in[1];
    AGNode *b = n->n_in > 2 ? n->in[2] : NULL;
    const int sh = n->at.conv.sh, sw = n->at.conv.sw, ph = n->at.conv.ph, pw = n->at.conv.pw;
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

    /* the second convolution of a chain: its input gradient, the first
     * convolution's weight gradient and, in the same launch, its own */
    const int chained = conv_chain_bwd(n, gd);
    if (chained == 2) return;
    const long bshp[1] = {F};
    const int lds = tt_k_conv2d_lds_plan(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo);
    int w_done = 0;
    if (needs(w) && !n->at.conv.col && (lds & 2)) {
        /* LDS-staged forward kept no col: dW (and db) read x */
        const float *x = tt_dev(a->val);
        Tensor *gw = x ? tt_empty_like(w->val) : NULL;
        Tensor *gb = gw && needs(b) ? tt_empty_dev(bshp, 1) : NULL;
        const int q[13] = {N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo};
        if (gw && (gb || !needs(b)) &&
            (conv_dw_deferred(gd, NULL, x, gw, gb, q) == 0 ||
             tt_k_conv2d_dw_lds(gd, x, gw->dev, gb ? gb->dev : NULL, N, C, H, W, F, HH, WW, sh,
                                sw, ph, pw, Ho, Wo) == 0)) {
            if (gb) accum_move(b, gb);
            accum_move(w, gw);
            w_done = 1;
        } else {
            tt_release(gw);
            tt_release(gb);
        }
    }
    if (w_done) {
    } else if (needs(b) && needs(w) && n->at.conv.col && n->at.conv.col_ones) {
        /* dW and db from one GEMM against [col; ones] */
        Tensor *gw = tt_empty_like(w->val);
        Tensor *gb = gw ? tt_empty_dev(bshp, 1) : NULL;
        if (gb && tt_k_conv_dw_bias(F, Kc, Ncol, HW, gd, n->at.conv.col, gw->dev, gb->dev) == 0) {
            accum_move(b, gb);
            accum_move(w, gw);
        } else {
            tt_release(gw);
            tt_release(gb);
        }
    } else if (needs(w) && !n->at.conv.col && tt_conv_use_implicit(sizeof(float) * (long)Kc * Ncol)) {
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
            float *col = n->at.conv.col;
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
    if (chained) return;
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
/* dW (and db) on the tiled LDS path with the reduction deferred: gw and gb
 * become recipes, and every pending reduction runs in one launch when the
 * first of them is read (the optimizer's step, ag_grad, ...).  codes: gd is
 * the pool gradient of tt_k_conv2d_dw_lds_pooled.  0 done; -1 not covered. */
static int conv_dw_deferred(const float *gd, const unsigned char *codes, const float *x,
                            Tensor *gw, Tensor *gb, const int q[13]) {
    TTDwtJob job;
    const int rc = ttk_conv2d_dwt_defer(gd, codes, x, gw->dev, gb ? gb->dev : NULL, q, &job);
    if (rc != 0) return rc < -1 ? rc : -1;
    if (tt_lazy_dwt(gw, gb, &job) != 0) return ttk_dwt_reduce_jobs(&job, 1);
    return 0;
}

/* geometry of a convolution node: N C H W F HH WW sh sw ph pw Ho Wo */
static void conv_geo(const AGNode *c, int q[13]) {
    const Tensor *x = c->in[0]->val, *w = c->in[1]->val;
    const int v[13] = {(int)x->shape[0], (int)x->shape[1], (int)x->shape[2], (int)x->shape[3],
                       (int)w->shape[0], (int)w->shape[2], (int)w->shape[3], c->at.conv.sh,
                       c->at.conv.sw, c->at.conv.ph, c->at.conv.pw, (int)c->val->shape[2],
                       (int)c->val->shape[3]};
    for (int i = 0; i < 13; i++) q[i] = v[i];
}

/* A convolution whose rule can take its output gradient as (pool gradient,
 * pool codes): only its weight (and bias) gradient is wanted -- its input
 * needs none -- on the LDS path the pooled form covers. */
static int conv_takes_pooled(const AGNode *c) {
    if (c->op != &OP_CONV2D || c->fanin != 1 || c->grad || c->lazy_g || needs(c->in[0]) ||
        !needs(c->in[1]) || c->at.conv.col)
        return 0;
    int q[13];
    conv_geo(c, q);
    return (tt_k_conv2d_lds_plan(q[0], q[1], q[2], q[3], q[4], q[5], q[6], q[7], q[8], q[9],
                                 q[10], q[11], q[12]) & 2) &&
           tt_k_conv2d_dw_lds_pooled(NULL, NULL, NULL, NULL, NULL, q[0], q[1], q[2], q[3], q[4],
                                     q[5], q[6], q[7], q[8], q[9], q[10], q[11], q[12]) == 0;
}

/* The rule of such a convolution: dW (and db) from the pool gradient and
 * codes; its own gradient stays a recipe.  0: not done (the caller
 * materialises the gradient and takes the ordinary rule). */
static int conv_pooled_dw(AGNode *n) {
    AGNode *a = n->in[0], *w = n->in[1];
    AGNode *b = n->n_in > 2 ? n->in[2] : NULL;
    if (needs(a) || !needs(w)) return 0;
    int q[13];
    conv_geo(n, q);
    const long bshp[1] = {q[4]};
    const float *x = tt_dev(a->val), *gp = tt_dev(n->lazy_g);
    const unsigned char *cd = (const unsigned char *)tt_dev(n->lazy_codes);
    Tensor *gw = x && gp && cd ? tt_empty_like(w->val) : NULL;
    Tensor *gb = gw && needs(b) ? tt_empty_dev(bshp, 1) : NULL;
    if (gw && (gb || !needs(b)) &&
        (conv_dw_deferred(gp, cd, x, gw, gb, q) == 0 ||
         tt_k_conv2d_dw_lds_pooled(gp, cd, x, gw->dev, gb ? gb->dev : NULL, q[0], q[1], q[2],
                                   q[3], q[4], q[5], q[6], q[7], q[8], q[9], q[10], q[11],
                                   q[12]) == 0)) {
        if (gb) accum_move(b, gb);
        accum_move(w, gw);
        return 1;
    }
    tt_release(gw);
    tt_release(gb);
    return 0;
}

static int backward_maxpool_relu(AGNode *n, AGNode *r, const float *g, int N, int C, int H,
                                 int W, int Ho, int Wo) {
    if (!relu_fusable(r) || n->at.win.kh != 2 || n->at.win.kw != 2 || n->at.win.sh != 2 ||
        n->at.win.sw != 2)
        return 0;
    /* from the windows' codes written by the fused forward; else, a relu
     * output still unwritten (a recipe of its input): the kernel reads the
     * relu's input and takes the relu on load */
    const unsigned char *codes =
        n->at.win.codes ? (const unsigned char *)tt_dev(n->at.win.codes) : NULL;
    if (codes && conv_takes_pooled(r->in[0])) {
        /* the convolution's weight gradient reads the pool's gradient and
         * the codes itself: neither gradient is written here */
        lazy_set(r, n->grad, NULL);
        lazy_set(r->in[0], n->grad, n->at.win.codes);
        r->fused = 1;
        return 1;
    }
    Tensor *pre = codes ? NULL : tt_lazy_relu_src(r->val);
    const float *x = codes ? NULL : pre ? tt_dev(pre) : tt_dev(r->val);
    if (!codes && !x) return 0;
    /* the relu's own gradient is left as a recipe (nothing in the pass reads
     * it: the relu feeds only this pool and its rule is skipped); the pool's
     * gradient is complete here, as every consumer's rule has run */
    Tensor *u = tt_empty_like(r->in[0]->val);
    if (!u || (codes ? tt_k_maxpool2x2_code_relu_bwd(codes, g, u->dev, N, C, H, W, Ho, Wo)
               : pre ? tt_k_maxpool2x2_prerelu_bwd(x, g, NULL, u->dev, N, C, H, W, Ho, Wo)
                     : tt_k_maxpool2x2_relu_bwd(x, g, NULL, u->dev, N, C, H, W, Ho, Wo))) {
        tt_release(u);
        return 0;
    }
    lazy_set(r, n->grad, NULL);
    accum_move(r->in[0], u);
    r->fused = 1;
    return 1;
}

static void backward_pool(AGNode *n, int is_max) {
    AGNode *a = n->in[0];
    if (!needs(a)) return;
    const int ph = n->at.win.kh, pw = n->at.win.kw, sh = n->at.win.sh, sw = n->at.win.sw;
    const int N = (int)a->val->shape[0], C = (int)a->val->shape[1], H = (int)a->val->shape[2],
              W = (int)a->val->shape[3];
    const int Ho = (int)n->grad->shape[2], Wo = (int)n->grad->shape[3];
    const float *g = tt_dev(n->grad);
    if (!g) return;
    if (is_max && backward_maxpool_relu(n, a, g, N, C, H, W, Ho, Wo)) return;
    const float *x = is_max ? tt_dev(a->val) : NULL;
    if (is_max && !x) return;
    Tensor *t = tt_empty_like(a->val);
    if (!t) return;
    int rc = is_max ? tt_k_maxpool_bwd(x, g, t->dev, N, C, H, W, ph, pw, sh, sw, Ho, Wo)
                    : tt_k_avgpool_bwd(g, t->dev, N, C, H, W, ph, pw, sh, sw, Ho, Wo);
    if (rc) { tt_release(t); return; }
    accum_move(a, t);
}

static void backward_maxpool(AGNode *n) { backward_pool(n, 1); }
static void backward_avgpool(AGNode *n) { backward_pool(n, 0); }

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
    AGNode *a = n->in[0];
    if (!needs(a)) return;
    if (!n->at.ce.seed && n->at.ce.labels) {
        const float *x = tt_dev(a->val);
        const long rows = a->val->shape[0];
        const int cols = (int)a->val->shape[1];
        Tensor *p = tt_empty_like(a->val), *s = tt_empty_like(a->val);
        float *l = (float *)ttrt_alloc(sizeof(float));
        const int ok = x && p && s && l &&
                       tt_k_softmax_ce_mean_hostlab(x, n->at.ce.labels, p->dev, l, s->dev, rows, cols,
                                                    1.0f / (float)rows) == 0;
        tt_release(p);
        ttrt_free(l);
        if (!ok) { tt_release(s); return; }
        n->at.ce.seed = s;
    }
    if (!n->at.ce.seed) return;
    if (is_host_one(n->grad)) {
        if (n->at.ce.labels && !a->grad) {
            a->grad = n->at.ce.seed;
            n->at.ce.seed = NULL;
            if (n->at.ce.sda[0] && a->op == &OP_MATMUL && !a->at.mm.sda[0]) {
                /* the seed is the logits' gradient as it stands: the
                 * classifier's input gradients formed with it go along */
                for (int i = 0; i < 3; i++) {
                    a->at.mm.sda[i] = n->at.ce.sda[i];
                    n->at.ce.sda[i] = NULL;
                }
                a->at.mm.stale = n->at.ce.stale;
                n->at.ce.stale = NULL;
            }
        } else {
            accum_copy(a, n->at.ce.seed);
        }
        return;
    }
    const float *seed = tt_dev(n->at.ce.seed), *gl = tt_dev(n->grad);
    if (!seed || !gl) return;
    Tensor *t = tt_empty_like(a->val);
    if (!t) return;
    if (tt_k_scale_by_dev(seed, gl, t->dev, t->numel)) {
        tt_release(t);
        return;
    }
    accum_move(a, t);
}

/* ---------- scheduling and running the backward pass ---------- */

static unsigned long long g_pass = 0;

/* The order in which the rules run: the reverse of the post-order of a
 * depth-first walk from `root` that enters each node's inputs in index order
 * and every node once (a node is placed only after every input reachable
 * through it; the reference's order, src/autograd.c:650-686, which fixes the
 * order gradients are summed in).  The walk keeps its state in the nodes --
 * `up` links back to the node a node was entered from, `walk` is its next
 * input -- so it needs no stack of its own and cannot fail; finished nodes
 * are pushed onto the front of the list through `next`, which leaves the
 * list in running order, root first.  `fanin` counts the pass's edges into
 * each node (the fused rules need to know a node has one consumer). */
static AGNode *schedule(AGNode *root) {
    const unsigned long long pass = ++g_pass;
    AGNode *head = NULL;
    root->pass = pass;
    root->walk = 0;
    root->fanin = 0;
    root->up = NULL;
    AGNode *cur = root;
    while (cur) {
        if (cur->walk < cur->n_in) {
            AGNode *c = cur->in[cur->walk++];
            if (c->pass != pass) {       /* first visit: enter it */
                c->pass = pass;
                c->walk = 0;
                c->fanin = 0;
                c->up = cur;
                cur = c;
            }
            c->fanin++;
        } else {                         /* every input placed: place it */
            cur->next = head;
            head = cur;
            cur = cur->up;
        }
    }
    return head;
}

static void run_rules(AGNode *head) {
    for (AGNode *n = head; n; n = n->next) {
        if ((!n->grad && !n->lazy_g) || !n->op) continue;
        if (n->fused) continue;          /* its consumer's rule did its work */
        /* a gradient still a recipe: only the convolution's rule reads one */
        if (n->lazy_g && n->op != &OP_CONV2D) {
            materialise(n);
            if (!n->grad) continue;  /* could not be written (out of memory) */
        }
        n->op->backward(n);
    }
    for (AGNode *n = head; n; n = n->next) n->fused = 0;
}

/* seed_kind: 0 = ones, 1 = host floats, 2 = device tensor */
static void backward_impl(AGNode *out, int seed_kind, const float *hseed, const Tensor *dseed) {
    AGNode *head = schedule(out);
    if (g_lazy)
        for (AGNode *n = head; n && g_lazy; n = n->next) materialise_for(n);
    tt_lazy_before_write(out->grad);  /* the seed overwrites it below */
    if (!out->grad) out->grad = tt_empty_like(out->val);
    if (!out->grad) return;
    if (seed_kind == 0 && out->grad->numel == 1) {
        /* a scalar ones seed is written to the host copy: no kernel, and a
         * rule that only needs to know it is 1 (softmax-CE) reads no device
         * memory; tt_dev uploads it for any rule that does */
        Tensor *t = out->grad;
        if (!t->data) t->data = (float *)ttrt_host_alloc(sizeof(float));
        if (t->data) {
            t->data[0] = 1.0f;
            t->valid = TT_V_HOST;
            run_rules(head);
            return;
        }
    }
    int rc;
    float *gd = out->grad->dev;
    if (seed_kind == 1) rc = ttrt_h2d_async(gd, hseed, sizeof(float) * (size_t)out->val->numel);
    else if (seed_kind == 2) {
        const float *sd = tt_dev((Tensor *)dseed);
        rc = sd ? tt_k_copy(gd, sd, out->val->numel) : -1;
    } else rc = tt_k_fill(gd, out->grad->numel, 1.0f);
    tt_mark_dev_written(out->grad);
    if (rc == 0) run_rules(head);
}

void ag_backward_from(AGNode *out, const float *seed, size_t seed_numel) {
    if (!out || !out->needs_grad) return;
    if (seed && (!out->val || seed_numel != (size_t)out->val->numel)) return;
    backward_impl(out, seed ? 1 : 0, seed, NULL);
}

void ag_backward(AGNode *out) { ag_backward_from(out, NULL, 0); }

void ag_backward_from_tensor(AGNode *out, const Tensor *seed) {
    if (!out || !out->needs_grad || !seed) return;
    if (!out->val || seed->numel != out->val->numel) return;
    backward_impl(out, 2, NULL, seed);
}

int ag_sgd_step_many(AGNode *const *leaves, int count, float lr) {
    if (count < 0 || (count > 0 && !leaves)) return -1;
    for (int base = 0; base < count; base += TT_SGD_MAX) {
        float *w[TT_SGD_MAX];
        const float *g[TT_SGD_MAX];
        Tensor *gt[TT_SGD_MAX];
        long n[TT_SGD_MAX];
        int k = 0;
        /* pending recipes that read a value about to change (a padded copy
         * or a weight gradient of this very tensor) run first */
        for (int i = base; i < count && i < base + TT_SGD_MAX; i++)
            if (leaves[i] && leaves[i]->grad) tt_lazy_before_write(leaves[i]->val);
        for (int i = base; i < count && i < base + TT_SGD_MAX; i++) {
            AGNode *l = leaves[i];
            if (!l || !l->grad) continue;
            w[k] = tt_dev(l->val);
            if (!w[k]) return -1;
            gt[k] = l->grad;
            n[k] = l->val->numel;
            k++;
        }
        /* gradients whose reduction is still pending: the reductions and
         * the step in one launch */
        int rc = tt_lazy_dwt_sgd(w, gt, n, k, lr);
        if (rc == 1) rc = tt_lazy_gemm_sgd(w, gt, n, k, lr);
        if (rc < 0) return -1;
        if (rc == 1) {
            for (int i = 0; i < k; i++)
                if (!(g[i] = tt_dev(gt[i]))) return -1;
            if (tt_k_sgd_multi(w, g, n, k, lr)) return -1;
        }
        for (int i = base; i < count && i < base + TT_SGD_MAX; i++)
            if (leaves[i] && leaves[i]->grad) tt_mark_dev_written(leaves[i]->val);
    }
    return 0;
}

int ag_sgd_step(AGNode *leaf, float lr) {
    if (!leaf || !leaf->grad) return 0;
    tt_lazy_before_write(leaf->val);
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
        for (int i = base; i < count && i < base + TT_SGD_MAX; i++)
            if (params[i]->grad) tt_lazy_before_write(params[i]->val);
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
    n->refs++;
    return n;
}

/* Dropping the last reference frees the node and releases its inputs; the
 * nodes whose count reaches zero that way wait on a list linked through
 * `next` (no recursion, so a long chain frees in constant stack). */
void ag_release(AGNode *n) {
    if (!n || --n->refs > 0) return;
    n->next = NULL;
    AGNode *dead = n;
    while (dead) {
        AGNode *d = dead;
        dead = d->next;
        if ((tt_pend.active && (tt_pend.out == d->val || tt_pend.r == d->val ||
                                tt_pend.p == d->val || tt_pend.c == d->val ||
                                (tt_pend.active >= TT_PEND_CHAIN_PAD && tt_pend.d == d->val) ||
                                (tt_pend.active == TT_PEND_CHAIN_FC && tt_pend.fco == d->val))) ||
            (tt_pend1.active && (tt_pend1.out == d->val || tt_pend1.r == d->val ||
                                 tt_pend1.p == d->val)))
            tt_flush_pending();  /* the launch writes into d's tensors */
        tt_release(d->val);
        tt_release(d->grad);
        lazy_drop(d);
        if (d->op && d->op->drop) d->op->drop(d);
        for (int i = 0; i < d->n_in; i++) {
            AGNode *p = d->in[i];
            if (--p->refs == 0) {
                p->next = dead;
                dead = p;
            }
        }
        free(d);
    }
}
