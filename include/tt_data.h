/* Device-resident datasets for the reference harnesses -- MI355X backend.
 *
 * The reference harnesses read MNIST (idx files, gzip'd) and CIFAR-10 into
 * NumPy, normalise on the host and copy every minibatch to the library
 * (reference tests/gate_mnist_mlp.py:37-53,83-87 and
 * tests/gate_cifar_cnn.py:47-68,165-167).  Here the raw uint8 samples are
 * uploaded once (a quarter of the float32 bytes) and stay in HBM; a batch
 * is one gather kernel that picks the rows, converts and normalises them:
 *     out[r, c, ...] = ((float)u8[idx[r], c, ...] / 255 - mean[c]) / std[c]
 * in float32 with correctly rounded division -- the NumPy expressions of
 * the harnesses, bit for bit.
 *
 * Loaders read local files only (no download).  Formats:
 *   idx   (LeCun's MNIST format): big-endian magic 0x00000800 | ndim (type
 *         byte 0x08 = unsigned byte), ndim big-endian uint32 dims, then the
 *         data; gzip'd or plain (zlib detects which).
 *   CIFAR-10 binary version (data_batch_N.bin / test_batch.bin): records of
 *         1 label byte + 3072 pixel bytes (3 x 32 x 32, channel-major).
 * Every call returns NULL / -1 on a missing or malformed file, bad
 * arguments or OOM. */
#ifndef TINYTORCH_TT_DATA_H
#define TINYTORCH_TT_DATA_H

#include <stddef.h>
#include <stdint.h>
#include "tensor.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct TTDataset TTDataset;

/* Header of an idx file (host only, no GPU needed): fills ndim (<= 8) and
 * dims; returns 0, or -1 when the file is not a uint8 idx file. */
int tt_idx_probe(const char *path, int *ndim, long *dims);

/* MNIST-style pair: images idx (n x rows x cols, or any n x ...) and labels
 * idx (n).  Samples have 1 channel of rows*cols bytes. */
TTDataset *tt_dataset_idx(const char *images_path, const char *labels_path);

/* CIFAR-10 binary batches, concatenated in the order given. */
TTDataset *tt_dataset_cifar10_bin(const char *const *paths, int npaths);

/* Raw samples from host memory: n samples of c x h x w bytes, labels. */
TTDataset *tt_dataset_from_u8(const uint8_t *samples, const int32_t *labels, long n, int c,
                              int h, int w);

long tt_dataset_len(const TTDataset *d);
/* sample shape (c, h, w) */
int  tt_dataset_shape(const TTDataset *d, int *c, int *h, int *w);
/* labels of all samples (host array of tt_dataset_len ints) */
int  tt_dataset_labels(const TTDataset *d, int32_t *out);

/* Batch of the samples idx[0..n): a new float tensor of shape (n, c, h, w),
 * or (n, c*h*w) when flat != 0.  mean/std hold one value per channel
 * (c <= 4).  labels_out (host, n ints, may be NULL) receives their labels.
 * Indices are checked on the host before anything is launched. */
Tensor *tt_dataset_batch(const TTDataset *d, const long *idx, long n, const float *mean,
                         const float *std, int flat, int32_t *labels_out);

void tt_dataset_release(TTDataset *d);

#ifdef __cplusplus
}
#endif
#endif
