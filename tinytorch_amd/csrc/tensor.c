/* Tensor lifecycle and accessors with device residency.
 *
 * Reference: src/tensor.c:1-75 (tt_alloc validation, calloc zero-fill,
 * refcounting, accessors).  Validation is the same -- ndim in 1..8, every
 * dim > 0, no long overflow, at most 2^40 elements -- so the hostile-shape
 * cases return NULL before anything is allocated.
 *
 * Residency: the payload lives in `dev`.  `valid` records which copy is
 * current (TT_V_DEV / TT_V_HOST).  tt_data() downloads into the host mirror
 * and, because the caller may write through the returned pointer, leaves the
 * HOST copy authoritative; tt_dev() (used by every op) uploads it again when
 * needed.  valid == 0 marks a tensor whose producing kernel failed to
 * launch: both accessors return NULL for it.  The host mirror is a pinned block from the runtime's host cache
 * (direct DMA on download).  Internal outputs are created with tt_empty_dev (no zero fill); the
 * public tt_new keeps the reference's zero-filled contract. */
#include "tt_internal.h"

#include <hip/hip_runtime_api.h>
#include <limits.h>
#include <stdlib.h>
#include <string.h>

#define TT_MAX_NUMEL (1L << 40)

static Tensor *alloc_meta(const long *shape, int ndim) {
    if (!shape || ndim <= 0 || ndim > 8) return NULL;
    long numel = 1;
    for (int i = 0; i < ndim; i++) {
        if (shape[i] <= 0) return NULL;
        if (numel > LONG_MAX / shape[i]) return NULL;
        numel *= shape[i];
    }
    if (numel > TT_MAX_NUMEL) return NULL;
    Tensor *t = (Tensor *)calloc(1, sizeof(Tensor));
    if (!t) return NULL;
    t->shape = (long *)malloc(sizeof(long) * (size_t)ndim);
    t->strides = (long *)malloc(sizeof(long) * (size_t)ndim);
    if (!t->shape || !t->strides) {
        free(t->shape); free(t->strides); free(t);
        return NULL;
    }
    long st = 1;
    for (int i = ndim - 1; i >= 0; i--) {
        t->shape[i] = shape[i];
        t->strides[i] = st;
        st *= shape[i];
    }
    t->ndim = ndim;
    t->numel = numel;
    t->refcount = 1;
    return t;
}

static void free_meta(Tensor *t) {
    ttrt_host_free(t->data);
    free(t->shape);
    free(t->strides);
    free(t);
}

Tensor *tt_empty_dev(const long *shape, int ndim) {
    Tensor *t = alloc_meta(shape, ndim);
    if (!t) return NULL;
    t->dev = (float *)ttrt_alloc(sizeof(float) * (size_t)t->numel);
    if (!t->dev) { free_meta(t); return NULL; }
    t->valid = TT_V_DEV;
    return t;
}

Tensor *tt_empty_like(const Tensor *a) { return tt_empty_dev(a->shape, a->ndim); }

Tensor *tt_new(const long *shape, int ndim) {
    Tensor *t = tt_empty_dev(shape, ndim);
    if (!t) return NULL;
    if (tt_k_fill(t->dev, t->numel, 0.0f) != 0) { tt_release(t); return NULL; }
    return t;
}

Tensor *tt_fromdata(const float *data, const long *shape, int ndim) {
    Tensor *t = alloc_meta(shape, ndim);
    if (!t) return NULL;
    if (!data) { free_meta(t); return NULL; }
    t->dev = (float *)ttrt_alloc(sizeof(float) * (size_t)t->numel);
    if (!t->dev) { free_meta(t); return NULL; }
    if (ttrt_h2d_async(t->dev, data, sizeof(float) * (size_t)t->numel) != 0) {
        tt_release(t);
        return NULL;
    }
    t->valid = TT_V_DEV;
    return t;
}

Tensor *tt_retain(Tensor *t) {
    if (!t) return NULL;
    t->refcount++;
    return t;
}

/* Tensors whose payload is a recipe not yet run: t = relu(src),
 * t = padones(src) or t = the mean loss of the row losses src, written by the first accessor that needs it (tt_dev /
 * tt_data of t), or before the host may write src (tt_data of src).  src is
 * retained meanwhile; a tensor released unread is never written.  The fused
 * convolution + relu + pool forward registers its relu output this way (the
 * pool is computed from the relu values in registers and the pool backward
 * reads the convolution output or the windows' codes), ag_padones the
 * padded copy of an input that needs no gradient (the matmul reads the
 * input itself, forward and backward), and ag_softmax_ce the loss of a
 * softmax-CE computed in its classifier's GEMM (the backward reads only
 * the seed). */
/* a deferred weight-gradient reduction, shared by its dw and db tensors */
typedef struct {
    TTDwtJob job;
    int refs;
} TTDwtShared;

/* a softmax-CE whose reduction (two partial sums per logit -> logits,
 * probabilities, seed, row losses: ttk_reduce_ce) has not run, shared by the
 * entries of its four outputs */
typedef struct {
    float *ws;                 /* 2 x M x N partial sums (owned) */
    const float *bias;         /* the classifier weights' last row */
    int32_t *labels;           /* M labels (owned) */
    int M, N;
    float scale;
    Tensor *out[4];            /* logits, probs, seed, row losses; NULL once released */
    int refs;
} TTCeJob;

typedef struct TTLazyVal {
    Tensor *t, *src;
    int kind;                  /* 0: relu(src); 1: padones(src); 2: mean of src;
                                  3: the reduction `dwt` (every pending one runs
                                  in the same launch); 4: [src, 1]^T src2, the
                                  weight gradient of a matmul of padones(src)
                                  (tt_k_gemm_tn_padones, dims rows Kx N); 5:
                                  conv(src, buf) -- a convolution output the
                                  two-convolution chain did not store; 6: see
                                  ce (every output is written at once); 7:
                                  src without its last column (padones
                                  backward, dims M K); 8: a guard (flag) */
    TTDwtShared *dwt;
    Tensor *src2;
    int dims[3];
    float *buf;                /* kind 5: the filters | bias snapshot (owned) */
    TTCeJob *ce;               /* kind 6: one output of the softmax-CE job `ce` (src:
                                  the classifier weights the bias belongs to) */
    int q[13];                 /* kind 5: N C H W F HH WW sh sw ph pw Ho Wo */
    int *flag;                 /* kind 8 (a guard, t NULL): set to 1 when src is about
                                  to be written */
    struct TTLazyVal *next;
} TTLazyVal;
static TTLazyVal *g_lazy_vals;

static int lazy_add(Tensor *t, Tensor *src, int kind) {
    TTLazyVal *l = (TTLazyVal *)malloc(sizeof(TTLazyVal));
    if (!l) return -1;
    l->t = t;
    l->src = tt_retain(src);
    l->kind = kind;
    l->dwt = NULL;
    l->src2 = NULL;
    l->buf = NULL;
    l->ce = NULL;
    l->flag = NULL;
    l->next = g_lazy_vals;
    g_lazy_vals = l;
    return 0;
}

int tt_lazy_relu(Tensor *t, Tensor *src) { return lazy_add(t, src, 0); }
int tt_lazy_padones(Tensor *t, Tensor *src) { return lazy_add(t, src, 1); }
int tt_lazy_ce_mean(Tensor *t, Tensor *src) { return lazy_add(t, src, 2); }
int tt_lazy_guard(Tensor *src, int *flag) {
    if (lazy_add(NULL, src, 8) != 0) return -1;
    g_lazy_vals->flag = flag;
    return 0;
}

void tt_lazy_guard_drop(int *flag) {
    for (TTLazyVal **pp = &g_lazy_vals; *pp;) {
        TTLazyVal *l = *pp;
        if (l->kind == 8 && l->flag == flag) {
            *pp = l->next;
            tt_release(l->src);
            free(l);
        } else {
            pp = &l->next;
        }
    }
}

int tt_lazy_padones_bwd(Tensor *t, Tensor *src, long M, long K) {
    if (M > 0x7fffffffL || K > 0x7fffffffL || lazy_add(t, src, 7) != 0) return -1;
    g_lazy_vals->dims[0] = (int)M;
    g_lazy_vals->dims[1] = (int)K;
    return 0;
}

int tt_lazy_gemm_tn_padones(Tensor *dw, Tensor *x, Tensor *g, int rows, int Kx, int N) {
    if (lazy_add(dw, x, 4) != 0) return -1;
    g_lazy_vals->src2 = tt_retain(g);
    g_lazy_vals->dims[0] = rows;
    g_lazy_vals->dims[1] = Kx;
    g_lazy_vals->dims[2] = N;
    return 0;
}

int tt_lazy_conv(Tensor *t, Tensor *x, float *snap, const int *q) {
    if (lazy_add(t, x, 5) != 0) return -1;
    g_lazy_vals->buf = snap;
    memcpy(g_lazy_vals->q, q, sizeof(g_lazy_vals->q));
    return 0;
}

Tensor *tt_lazy_relu_src(const Tensor *t) {
    for (TTLazyVal *l = g_lazy_vals; l; l = l->next)
        if (l->t == t && l->kind == 0) return l->src;
    return NULL;
}

int tt_lazy_dwt(Tensor *dw, Tensor *db, const TTDwtJob *job) {
    TTDwtShared *sh = (TTDwtShared *)malloc(sizeof(TTDwtShared));
    TTLazyVal *a = (TTLazyVal *)malloc(sizeof(TTLazyVal));
    TTLazyVal *b = db ? (TTLazyVal *)malloc(sizeof(TTLazyVal)) : NULL;
    if (!sh || !a || (db && !b)) {
        free(sh); free(a); free(b);
        return -1;
    }
    sh->job = *job;
    sh->refs = db ? 2 : 1;
    a->t = dw; a->src = NULL; a->kind = 3; a->dwt = sh; a->src2 = NULL;
    a->buf = NULL; a->ce = NULL;
    a->next = g_lazy_vals;
    g_lazy_vals = a;
    if (b) {
        b->t = db; b->src = NULL; b->kind = 3; b->dwt = sh; b->src2 = NULL;
        b->buf = NULL; b->ce = NULL;
        b->next = g_lazy_vals;
        g_lazy_vals = b;
    }
    return 0;
}

/* every pending reduction (up to 32 at a time) in one launch; their tensors
 * become current */
static void dwt_flush_all(void) {
    for (;;) {
        TTDwtShared *sh[32];
        TTDwtJob jobs[32];
        int n = 0;
        for (TTLazyVal *l = g_lazy_vals; l && n < 32; l = l->next) {
            if (l->kind != 3) continue;
            int seen = 0;
            for (int i = 0; i < n; i++) seen |= sh[i] == l->dwt;
            if (!seen) { sh[n] = l->dwt; jobs[n] = l->dwt->job; n++; }
        }
        if (!n) return;
        const int rc = ttk_dwt_reduce_jobs(jobs, n);  /* frees the partials */
        TTLazyVal **pp = &g_lazy_vals;
        while (*pp) {
            TTLazyVal *l = *pp;
            int mine = 0;
            for (int i = 0; l->kind == 3 && i < n; i++) mine |= sh[i] == l->dwt;
            if (!mine) { pp = &l->next; continue; }
            *pp = l->next;
            if (rc != 0) l->t->valid = 0;
            else tt_mark_dev_written(l->t);
            free(l);
        }
        for (int i = 0; i < n; i++) free(sh[i]);
    }
}

static TTLazyVal *dwt_entry(const Tensor *t) {
    for (TTLazyVal *l = g_lazy_vals; l; l = l->next)
        if (l->kind == 3 && l->t == t) return l;
    return NULL;
}

int tt_lazy_dwt_sgd(float *const *w, Tensor *const *g, const long *n, int count, float lr) {
    if (count <= 0 || count > TT_SGD_MAX || !g_lazy_vals) return 1;
    int any = 0;
    for (int i = 0; i < count; i++) {
        if (dwt_entry(g[i])) any = 1;
        for (int k = 0; k < i; k++)
            if (g[k] == g[i] || w[k] == w[i]) return 1;  /* a tensor twice: the plain way */
    }
    if (!any) return 1;
    /* every pending job (the step reads the gradients they write) */
    TTDwtShared *sh[4];
    TTDwtJob jobs[4];
    float *wdw[4], *wdb[4];
    int nj = 0;
    for (TTLazyVal *l = g_lazy_vals; l; l = l->next) {
        if (l->kind != 3) continue;
        int seen = 0;
        for (int q = 0; q < nj; q++) seen |= sh[q] == l->dwt;
        if (seen) continue;
        if (nj == 4) return 1;
        sh[nj] = l->dwt;
        jobs[nj] = l->dwt->job;
        wdw[nj] = wdb[nj] = NULL;
        nj++;
    }
    float *pw[TT_SGD_MAX];
    const float *pg[TT_SGD_MAX];
    long pn[TT_SGD_MAX];
    int np = 0;
    for (int i = 0; i < count; i++) {
        TTLazyVal *l = dwt_entry(g[i]);
        if (!l) {
            pw[np] = w[i];
            pn[np] = n[i];
            pg[np] = tt_dev(g[i]);  /* no pending reduction: nothing flushed */
            if (!pg[np]) return -1;
            np++;
            continue;
        }
        for (int q = 0; q < nj; q++) {
            if (sh[q] != l->dwt) continue;
            if (g[i]->dev == jobs[q].dw) wdw[q] = w[i];
            else if (g[i]->dev == jobs[q].db) wdb[q] = w[i];
        }
    }
    const int rc = ttk_dwt_reduce_sgd(jobs, wdw, wdb, nj, pw, pg, pn, np, lr);
    if (rc == 1) return 1;
    /* the jobs ran (or failed): their tensors leave the registry */
    TTLazyVal **pp = &g_lazy_vals;
    while (*pp) {
        TTLazyVal *l = *pp;
        int mine = 0;
        for (int q = 0; l->kind == 3 && q < nj; q++) mine |= sh[q] == l->dwt;
        if (!mine) { pp = &l->next; continue; }
        *pp = l->next;
        if (rc != 0) l->t->valid = 0;
        else tt_mark_dev_written(l->t);
        free(l);
    }
    for (int q = 0; q < nj; q++) free(sh[q]);
    return rc;
}

int tt_lazy_gemm_sgd(float *const *w, Tensor *const *g, const long *n, int count, float lr) {
    if (count <= 0 || count > TT_SGD_MAX || !g_lazy_vals) return 1;
    TTLazyVal *pend[2] = {NULL, NULL};
    int at[2] = {-1, -1}, nj = 0;
    for (int i = 0; i < count; i++) {
        for (TTLazyVal *l = g_lazy_vals; l; l = l->next)
            if (l->kind == 4 && l->t == g[i]) {
                if (nj == 2) return 1;  /* two such gradients a launch */
                pend[nj] = l;
                at[nj++] = i;
            }
        for (int k = 0; k < i; k++)
            if (g[k] == g[i] || w[k] == w[i]) return 1;
    }
    if (!nj) return 1;
    TTTnSgdJob jobs[2];
    for (int q = 0; q < nj; q++) {
        const float *x = tt_dev(pend[q]->src), *gg = tt_dev(pend[q]->src2);
        if (!x || !gg) return -1;
        jobs[q].rows = pend[q]->dims[0];
        jobs[q].Kx = pend[q]->dims[1];
        jobs[q].N = pend[q]->dims[2];
        jobs[q].X = x;
        jobs[q].G = gg;
        jobs[q].dW = pend[q]->t->dev;
        jobs[q].wsgd = w[at[q]];
    }
    float *pw[TT_SGD_MAX];
    const float *pg[TT_SGD_MAX];
    long pn[TT_SGD_MAX];
    int np = 0;
    for (int i = 0; i < count; i++) {
        if (i == at[0] || i == at[1]) continue;
        pw[np] = w[i];
        pn[np] = n[i];
        if (!(pg[np] = tt_dev(g[i]))) return -1;
        np++;
    }
    const int rc = ttk_gemm_tn_padones_sgd_jobs(jobs, nj, lr, pw, pg, pn, np);
    if (rc == 1) return 1;
    for (int q = 0; q < nj; q++) {
        for (TTLazyVal **pp = &g_lazy_vals; *pp; pp = &(*pp)->next)
            if (*pp == pend[q]) { *pp = pend[q]->next; break; }
        if (rc != 0) pend[q]->t->valid = 0;
        else tt_mark_dev_written(pend[q]->t);
        tt_release(pend[q]->src);
        tt_release(pend[q]->src2);
        free(pend[q]);
    }
    return rc;
}

/* a pending reduction's output released unread: the reduction skips it (and
 * is dropped when nothing of it is left) */
static void dwt_drop_entry(TTLazyVal **pp) {
    TTLazyVal *l = *pp;
    TTDwtShared *sh = l->dwt;
    *pp = l->next;
    if (sh->job.dw == l->t->dev) sh->job.dw = NULL;
    if (sh->job.db == l->t->dev) sh->job.db = NULL;
    if (--sh->refs == 0) {
        ttk_dwt_job_drop(&sh->job);
        free(sh);
    }
    free(l);
}

int tt_lazy_ce_job(Tensor *const out[4], Tensor *w, float *ws, const float *bias,
                   const int32_t *labels, int M, int N, float scale) {
    TTCeJob *j = (TTCeJob *)calloc(1, sizeof(TTCeJob));
    int32_t *lab = (int32_t *)malloc(sizeof(int32_t) * (size_t)M);
    TTLazyVal *e[4] = {NULL, NULL, NULL, NULL};
    int ok = j && lab;
    for (int i = 0; i < 4 && ok; i++) ok = (e[i] = (TTLazyVal *)malloc(sizeof(TTLazyVal))) != NULL;
    if (!ok) {
        for (int i = 0; i < 4; i++) free(e[i]);
        free(j);
        free(lab);
        return -1;
    }
    memcpy(lab, labels, sizeof(int32_t) * (size_t)M);
    j->ws = ws;
    j->bias = bias;
    j->labels = lab;
    j->M = M;
    j->N = N;
    j->scale = scale;
    j->refs = 4;
    for (int i = 0; i < 4; i++) {
        j->out[i] = out[i];
        e[i]->t = out[i];
        e[i]->src = tt_retain(w);
        e[i]->src2 = NULL;
        e[i]->kind = 6;
        e[i]->dwt = NULL;
        e[i]->buf = NULL;
        e[i]->ce = j;
        e[i]->next = g_lazy_vals;
        g_lazy_vals = e[i];
    }
    return 0;
}

/* the job's entries leave the registry (outputs written, or not: invalid) */
static void ce_job_finish(TTCeJob *j, int written) {
    TTLazyVal **pp = &g_lazy_vals;
    while (*pp) {
        TTLazyVal *l = *pp;
        if (l->kind != 6 || l->ce != j) { pp = &l->next; continue; }
        *pp = l->next;
        if (written) tt_mark_dev_written(l->t);
        else l->t->valid = 0;
        tt_release(l->src);
        free(l);
    }
    ttrt_free(j->ws);  /* stream-ordered: after the kernel that read it */
    free(j->labels);
    free(j);
}

static void ce_job_run(TTCeJob *j) {
    float *tmp[4] = {NULL, NULL, NULL, NULL}, *dst[4];
    int ok = 1;
    for (int i = 0; i < 4; i++) {
        if (j->out[i]) { dst[i] = j->out[i]->dev; continue; }
        const size_t n = i == 3 ? (size_t)j->M : (size_t)j->M * j->N;
        ok &= (dst[i] = tmp[i] = (float *)ttrt_alloc(sizeof(float) * n)) != NULL;
    }
    if (ok) {
        const TTCeHook hk = {j->bias, j->labels, dst[1], dst[2], dst[3], j->scale};
        ok = ttk_reduce_ce(j->ws, dst[0], j->M, j->N, 2, 1, &hk) == 0;
    }
    for (int i = 0; i < 4; i++) ttrt_free(tmp[i]);
    ce_job_finish(j, ok);
}

static void ce_drop_entry(TTLazyVal **pp) {
    TTLazyVal *l = *pp;
    TTCeJob *j = l->ce;
    *pp = l->next;
    for (int i = 0; i < 4; i++)
        if (j->out[i] == l->t) j->out[i] = NULL;
    tt_release(l->src);
    free(l);
    if (--j->refs == 0) {
        ttrt_free(j->ws);
        free(j->labels);
        free(j);
    }
}

int tt_lazy_ce_args(const Tensor *t, TTHeadCeArgs *a, void **job) {
    for (TTLazyVal *l = g_lazy_vals; l; l = l->next) {
        if (l->kind != 6 || l->t != t) continue;
        TTCeJob *j = l->ce;
        a->part = j->ws;
        a->bias = j->bias;
        a->labels = j->labels;
        a->scale = j->scale;
        a->logits = j->out[0] ? j->out[0]->dev : NULL;
        a->probs = j->out[1] ? j->out[1]->dev : NULL;
        a->seed = j->out[2] ? j->out[2]->dev : NULL;
        a->rowloss = j->out[3] ? j->out[3]->dev : NULL;
        *job = j;
        return 0;
    }
    return -1;
}

void tt_lazy_ce_done(void *job) { ce_job_finish((TTCeJob *)job, 1); }

/* unlink the entries of t (as the recipe's output, or every entry computed
 * from t when `from`), running their recipes unless `drop`; a recipe's run
 * may change the list, so the walk restarts after each */
static void lazy_take(const Tensor *t, int from, int drop) {
restart:
    for (TTLazyVal **pp = &g_lazy_vals; *pp; pp = &(*pp)->next) {
        TTLazyVal *l = *pp;
        if (from ? (l->src != t && l->src2 != t) : l->t != t) continue;
        if (l->kind == 3) {
            if (drop) dwt_drop_entry(pp);
            else dwt_flush_all();
            goto restart;
        }
        if (l->kind == 6) {
            if (drop && !from) ce_drop_entry(pp);
            else ce_job_run(l->ce);
            goto restart;
        }
        if (l->kind == 8) {  /* a guard: its source is about to change */
            *pp = l->next;
            *l->flag = 1;
            tt_release(l->src);
            free(l);
            goto restart;
        }
        *pp = l->next;
        if (!drop) {
            const float *x = tt_dev(l->src);
            const float *x2 = l->src2 ? tt_dev(l->src2) : NULL;
            const int rc = !x || (l->src2 && !x2) ? -1
                           : l->kind == 1 ? tt_k_padones_fwd(x, l->t->dev, l->t->shape[0],
                                                             l->t->shape[1] - 1)
                           : l->kind == 2 ? tt_k_ce_mean_rows(x, l->t->dev, (int)l->src->numel)
                           : l->kind == 4 ? ttk_gemm_tn_padones_any(l->dims[0], l->dims[1],
                                                                    l->dims[2], x, x2, l->t->dev)
                           : l->kind == 7 ? tt_k_padones_bwd(x, l->t->dev, l->dims[0], l->dims[1])
                           : l->kind == 5 ? tt_conv_fwd_any(x, l->buf,
                                                            l->buf + (long)l->q[4] * l->q[1] *
                                                                         l->q[5] * l->q[6],
                                                            l->t->dev, l->q)
                                          : tt_k_relu_fwd(x, l->t->dev, l->t->numel);
            if (rc != 0) l->t->valid = 0;
            else tt_mark_dev_written(l->t);
        }
        tt_release(l->src);
        tt_release(l->src2);
        ttrt_free(l->buf);  /* stream-ordered: after the recomputation read it */
        free(l);
        goto restart;
    }
}

void tt_lazy_before_write(Tensor *t) {
    if (g_lazy_vals && t) lazy_take(t, 1, 0);
}

void tt_release(Tensor *t) {
    if (!t) return;
    if (--t->refcount > 0) return;
    if (g_lazy_vals) lazy_take(t, 0, 1);
    ttrt_free(t->dev);
    free_meta(t);
}

float *tt_dev(Tensor *t) {
    if (tt_pend.active || tt_pend1.active) tt_flush_pending();
    if (g_lazy_vals && t) lazy_take(t, 0, 0);
    if (!t || !t->dev || !t->valid) return NULL;
    if (!(t->valid & TT_V_DEV)) {
        if (!t->data || ttrt_h2d_async(t->dev, t->data, sizeof(float) * (size_t)t->numel) != 0)
            return NULL;
        t->valid |= TT_V_DEV;
    }
    return t->dev;
}

/* After the caller has been handed the host pointer, assume it may write:
 * the device copy is re-uploaded before its next use. */
float *tt_data(const Tensor *ct) {
    Tensor *t = (Tensor *)ct;
    if (tt_pend.active || tt_pend1.active) tt_flush_pending();
    if (g_lazy_vals && t) {
        lazy_take(t, 0, 0);
        lazy_take(t, 1, 0);  /* the host may write t: recipes reading it run now */
    }
    if (!t || !t->valid) return NULL;
    if (!(t->valid & TT_V_HOST)) {
        if (!t->data) {
            t->data = (float *)ttrt_host_alloc(sizeof(float) * (size_t)t->numel);
            if (!t->data) return NULL;
        }
        if (ttrt_d2h(t->data, t->dev, sizeof(float) * (size_t)t->numel) != 0) return NULL;
    }
    t->valid = TT_V_HOST;
    return t->data;
}

/* device payload became the only current copy (a kernel wrote it) */
void tt_mark_dev_written(Tensor *t) { t->valid = TT_V_DEV; }

long tt_numel(const Tensor *t) { return t ? t->numel : 0; }
int  tt_ndim(const Tensor *t) { return t ? t->ndim : 0; }

void tt_shape(const Tensor *t, long *out) {
    if (!t || !out) return;
    for (int i = 0; i < t->ndim; i++) out[i] = t->shape[i];
}

void tt_strides(const Tensor *t, long *out) {
    if (!t || !out) return;
    for (int i = 0; i < t->ndim; i++) out[i] = t->strides[i];
}

/* ---- device-level runtime API (tt_hip.h) ---- */

int tth_available(void) { return ttrt_init() == 0; }

int tth_device_name(char *buf, int len) {
    if (!buf || len <= 0 || ttrt_init() != 0) return -1;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return -1;
    strncpy(buf, prop.gcnArchName, (size_t)len - 1);
    buf[len - 1] = 0;
    return 0;
}

void  *tth_stream(void) { return ttrt_init() == 0 ? ttrt_stream() : NULL; }
int    tth_sync(void) {
    const int rc = tt_flush_pending();
    const int rs = ttrt_sync();
    return rc ? rc : rs;
}
int    tth_last_error(void) { return ttrt_last_error(); }
void  *tth_malloc(size_t bytes) { return ttrt_alloc(bytes); }
void   tth_free(void *d) { ttrt_free(d); }
void   tth_release_cache(void) { ttrt_release_cache(); }
size_t tth_bytes_in_use(void) { return ttrt_bytes_in_use(); }
int    tth_h2d(void *d, const void *h, size_t bytes) {
    tt_flush_pending();
    return ttrt_h2d(d, h, bytes);
}
int    tth_d2h(void *h, const void *d, size_t bytes) {
    tt_flush_pending();
    return ttrt_d2h(h, d, bytes);
}

void *tth_event_create(void) {
    if (ttrt_init() != 0) return NULL;
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return NULL;
    return (void *)e;
}

int tth_event_record(void *ev) {
    if (!ev) return -1;
    tt_flush_pending();
    return hipEventRecord((hipEvent_t)ev, (hipStream_t)ttrt_stream()) == hipSuccess ? 0 : -1;
}

float tth_event_elapsed_ms(void *start, void *stop) {
    if (!start || !stop) return -1.0f;
    if (hipEventSynchronize((hipEvent_t)stop) != hipSuccess) return -1.0f;
    float ms = -1.0f;
    if (hipEventElapsedTime(&ms, (hipEvent_t)start, (hipEvent_t)stop) != hipSuccess) return -1.0f;
    return ms;
}

void tth_event_destroy(void *ev) {
    if (ev) hipEventDestroy((hipEvent_t)ev);
}
