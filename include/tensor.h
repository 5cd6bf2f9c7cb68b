/* tinytorch tensor C ABI -- MI355X (gfx950) backend.
 *
 * Drop-in for the reference header include/tensor.h:1-55.  Every declaration
 * below keeps the reference's name, signature and meaning; the Tensor struct
 * keeps the reference's six leading fields in the same order (reference
 * include/tensor.h:10-17; callers mirror them with ctypes) and appends the
 * device-residency fields after them.
 *
 * Storage: the payload lives in GPU memory.  `data` is a host mirror that is
 * (re)filled on demand: call tt_data() -- as every reference caller does --
 * to get a valid host pointer.  After tt_data() the host copy is treated as
 * authoritative (the caller may write through it) and is uploaded again the
 * next time an op reads the tensor.
 *
 * Errors: constructors and ops return NULL on bad arguments, shape mismatch,
 * out-of-memory, or when no GPU is usable (reference include/tensor.h:32).
 * tth_last_error() (tt_hip.h) tells which. */
#ifndef TINYTORCH_H
#define TINYTORCH_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct Tensor {
    float *data;     /* host mirror; valid after tt_data() (may be NULL before) */
    long  *shape;    /* ndim entries */
    long  *strides;  /* in elements; informational: always contiguous row-major */
    int    ndim;
    long   numel;
    int    refcount;
    /* ---- appended: not part of the reference layout ---- */
    float *dev;      /* device payload, numel floats */
    int    valid;    /* bit 0: device copy current, bit 1: host copy current */
} Tensor;

/* lifecycle -- reference include/tensor.h:20-23, src/tensor.c:10-61 */
Tensor *tt_new(const long *shape, int ndim);                          /* zero-filled */
Tensor *tt_fromdata(const float *data, const long *shape, int ndim);  /* copies (H2D) */
Tensor *tt_retain(Tensor *t);
void    tt_release(Tensor *t);

/* accessors -- reference include/tensor.h:26-30 */
float  *tt_data(const Tensor *t);   /* syncs the device result into the host mirror */
long    tt_numel(const Tensor *t);
int     tt_ndim(const Tensor *t);
void    tt_shape(const Tensor *t, long *out);
void    tt_strides(const Tensor *t, long *out);

/* ops (allocate fresh output; NULL on shape/arg error) -- reference include/tensor.h:33-41 */
Tensor *tt_add(const Tensor *a, const Tensor *b);
Tensor *tt_mul(const Tensor *a, const Tensor *b);
Tensor *tt_addscalar(const Tensor *a, float s);
Tensor *tt_mulscalar(const Tensor *a, float s);
Tensor *tt_matmul(const Tensor *a, const Tensor *b);                   /* 2D @ 2D */
Tensor *tt_matmul_fast(const Tensor *a, const Tensor *b);              /* 2D @ 2D, MFMA */
Tensor *tt_matmul_omp(const Tensor *a, const Tensor *b, int nthreads); /* nthreads ignored */
Tensor *tt_relu(const Tensor *a);
Tensor *tt_softmax(const Tensor *a);                                   /* along last axis */

/* spatial & shape ops -- reference include/tensor.h:44-50 */
Tensor *tt_reshape(const Tensor *a, const long *new_shape, int new_ndim); /* copy, not a view */
Tensor *tt_conv2d(const Tensor *a, const Tensor *w, const Tensor *b,
                  int stride_h, int stride_w, int pad_h, int pad_w);
Tensor *tt_maxpool2d(const Tensor *a, int pool_h, int pool_w,
                     int stride_h, int stride_w);
Tensor *tt_avgpool2d(const Tensor *a, int pool_h, int pool_w,
                     int stride_h, int stride_w);

/* Row-major C = A*B on host pointers (A MxK, B KxN, C MxN), computed on the
 * GPU.  As in the reference, C is overwritten on the leading
 * (M/6*6) x (N/16*16) block when K > 0 and that block is not empty, and the
 * product is added into C everywhere else.  Exported without a header by the
 * reference (src/gemm.c:569-641); returns 0, or -1 on allocation/launch failure.
 * nthreads is accepted for ABI compatibility and ignored. */
int tt_sgemm_rowmajor(int M, int N, int K, const float *A, const float *B,
                      float *C, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
