/* tinytorch reverse-mode autograd C ABI -- MI355X (gfx950) backend.
 *
 * Drop-in for the reference header include/autograd.h:1-53: same names,
 * signatures, ownership rules and error behaviour.  Node values and
 * gradients are device-resident Tensors; the graph bookkeeping (topological
 * sort, dispatch of backward rules) runs on the host, the arithmetic on the
 * GPU.
 *
 * Ownership (reference src/autograd.c:107-132, 727-745): constructors return
 * a node with refcount 1 owned by the caller; a node retains its parents and
 * releases them when it is released; ag_leaf retains its tensor; ag_value and
 * ag_grad return borrowed pointers.  Gradients of every node that requires
 * grad persist across backward calls and accumulate. */
#ifndef TINYTORCH_AUTOGRAD_H
#define TINYTORCH_AUTOGRAD_H

#include "tensor.h"
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct AGNode AGNode;

/* graph construction -- reference include/autograd.h:14-22 */
AGNode *ag_leaf(Tensor *t, int requires_grad);   /* retains t */
AGNode *ag_add(AGNode *a, AGNode *b);
AGNode *ag_mul(AGNode *a, AGNode *b);
AGNode *ag_addscalar(AGNode *a, float s);
AGNode *ag_mulscalar(AGNode *a, float s);
AGNode *ag_matmul(AGNode *a, AGNode *b);         /* 2D @ 2D */
AGNode *ag_relu(AGNode *a);
AGNode *ag_softmax(AGNode *a);                   /* last axis */
AGNode *ag_padones(AGNode *a);                   /* append ones column */

/* spatial & shape nodes -- reference include/autograd.h:25-31 */
AGNode *ag_reshape(AGNode *a, const long *new_shape, int new_ndim);
AGNode *ag_conv2d(AGNode *a, AGNode *w, AGNode *b,
                  int stride_h, int stride_w, int pad_h, int pad_w);
AGNode *ag_maxpool2d(AGNode *a, int pool_h, int pool_w,
                     int stride_h, int stride_w);
AGNode *ag_avgpool2d(AGNode *a, int pool_h, int pool_w,
                     int stride_h, int stride_w);

/* accessors -- reference include/autograd.h:34-36 */
Tensor *ag_value(const AGNode *n);
Tensor *ag_grad(const AGNode *n);                /* NULL until backward */
int     ag_requires_grad(const AGNode *n);

/* reverse-mode AD -- reference include/autograd.h:38-45.
 * ag_backward(out): seed out->grad with 1.0.
 * ag_backward_from(out, seed, seed_numel): copy seed (seed_numel host floats)
 * into out->grad; seed_numel must equal the value's numel, otherwise the call
 * returns without touching any gradient.  Callers must surface that as an
 * error. */
void    ag_backward(AGNode *out);
void    ag_backward_from(AGNode *out, const float *seed, size_t seed_numel);

void    ag_release(AGNode *n);                   /* refcounted node */
AGNode *ag_retain(AGNode *n);

/* ---- additions of this backend (no reference counterpart) ---- */

/* Softmax + mean cross-entropy over the last axis of a 2-D logits node, with
 * integer labels (host array of `rows` ints).  Value: a 1-element tensor
 * holding -mean(log(max(p[r, y_r], 1e-12))).  Backward seeds the logits with
 * (p - onehot(y)) / rows times the incoming gradient -- exactly what the
 * reference harnesses compute in NumPy and pass to ag_backward_from
 * (reference tests/gate_cifar_cnn.py:175-181, tests/gate_mnist_mlp.py:112-119).
 * ag_softmax_ce_probs returns the softmax probabilities (borrowed). */
AGNode *ag_softmax_ce(AGNode *logits, const int *labels, long rows);
Tensor *ag_softmax_ce_probs(const AGNode *loss);

/* Backward seeded from a device-resident tensor of the value's shape
 * (no host round trip); same mismatch rule as ag_backward_from. */
void    ag_backward_from_tensor(AGNode *out, const Tensor *seed);

/* In-place SGD on a leaf value: value -= lr * grad (no-op without grad);
 * the _many form updates `count` leaves in one kernel launch.  The update
 * the reference harness does in NumPy (tests/gate_mnist_mlp.py:121-124). */
int     ag_sgd_step(AGNode *leaf, float lr);
int     ag_sgd_step_many(AGNode *const *leaves, int count, float lr);

/* Optimizers whose state (velocity / Adam moments) stays on the device.
 * State slot i belongs to position i of the `params` list given to
 * ag_optim_step; the first step fixes the list length and each slot's
 * element count (a later mismatch returns -1 without updating anything).
 * Parameters without a gradient are skipped.  Each call updates the leaf
 * values in place in one launch per TT_SGD_MAX parameters.
 *   sgd_momentum: v = momentum*v - lr*g; w += v
 *                 (reference tests/gate_mnist_mlp.py:121-124)
 *   adam:         t += 1; lr_t = lr*sqrt(1-b2^t)/(1-b1^t);
 *                 m = b1*m + (1-b1)*g; v = b2*v + (1-b2)*g*g;
 *                 w -= lr_t*m/(sqrt(v)+eps)
 *                 (reference tests/gate_cifar_cnn.py:81-98)
 * Arithmetic matches NumPy's on float32 arrays with Python-float
 * hyperparameters.  Returns NULL / -1 on bad arguments or OOM. */
typedef struct AGOptim AGOptim;
AGOptim *ag_optim_sgd_momentum(double lr, double momentum);
AGOptim *ag_optim_adam(double lr, double beta1, double beta2, double eps);
int      ag_optim_step(AGOptim *opt, AGNode *const *params, int count);
long     ag_optim_steps(const AGOptim *opt);     /* Adam's t; -1 for NULL */
/* learning-rate schedule: the CIFAR harness decays Adam's lr between epochs
 * (reference tests/gate_cifar_cnn.py:159-160); takes effect at the next step */
int      ag_optim_set_lr(AGOptim *opt, double lr);
double   ag_optim_lr(const AGOptim *opt);
void     ag_optim_release(AGOptim *opt);

#ifdef __cplusplus
}
#endif
#endif
