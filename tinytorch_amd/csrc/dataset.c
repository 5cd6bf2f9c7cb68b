/* Device-resident uint8 datasets: file parsing on the host (zlib reads
 * gzip'd and plain files alike), one upload of the raw bytes, and batches
 * built on the device by tt_k_gather_u8_norm.
 *
 * Reference behaviour followed: the MNIST harness parses the idx header and
 * takes the bytes after it (reference tests/gate_mnist_mlp.py:44-53), then
 * normalises ((x / 255.0) - mean) / std in float32 (:83-87); the CIFAR
 * harness reshapes each record to (3, 32, 32) and normalises per channel
 * (reference tests/gate_cifar_cnn.py:56-68,165).  The CIFAR reader takes
 * the binary distribution of the same data instead of the Python pickles,
 * which cannot be read without executing code from the file. */
#include "tt_internal.h"
#include "tt_data.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <zlib.h>

_Static_assert(sizeof(long) == sizeof(int64_t), "batch indices are passed as int64");

struct TTDataset {
    uint8_t *dev;      /* n * sample bytes, device */
    int32_t *labels;   /* n, host */
    long n;
    int c, h, w;
};

static long sample_bytes(const TTDataset *d) { return (long)d->c * d->h * d->w; }

static int read_all(gzFile f, void *buf, size_t bytes) {
    uint8_t *p = (uint8_t *)buf;
    while (bytes > 0) {
        const unsigned chunk = bytes > (1u << 30) ? (1u << 30) : (unsigned)bytes;
        const int got = gzread(f, p, chunk);
        if (got <= 0) return -1;
        p += got;
        bytes -= (size_t)got;
    }
    return 0;
}

static uint32_t be32(const uint8_t *b) {
    return ((uint32_t)b[0] << 24) | ((uint32_t)b[1] << 16) | ((uint32_t)b[2] << 8) | b[3];
}

/* opens `path`, parses the idx header; returns the open file positioned at
 * the data, or NULL */
static gzFile idx_open(const char *path, int *ndim, long *dims, long *count) {
    if (!path || !ndim || !dims) return NULL;
    gzFile f = gzopen(path, "rb");
    if (!f) return NULL;
    uint8_t hdr[4];
    if (read_all(f, hdr, 4) || hdr[0] != 0 || hdr[1] != 0 || hdr[2] != 0x08 || hdr[3] == 0 ||
        hdr[3] > 8) {
        gzclose(f);
        return NULL;
    }
    *ndim = hdr[3];
    long total = 1;
    for (int i = 0; i < *ndim; i++) {
        uint8_t b[4];
        if (read_all(f, b, 4)) { gzclose(f); return NULL; }
        dims[i] = (long)be32(b);
        if (dims[i] <= 0 || total > (1L << 40) / dims[i]) { gzclose(f); return NULL; }
        total *= dims[i];
    }
    if (count) *count = total;
    return f;
}

int tt_idx_probe(const char *path, int *ndim, long *dims) {
    gzFile f = idx_open(path, ndim, dims, NULL);
    if (!f) return -1;
    gzclose(f);
    return 0;
}

static TTDataset *upload(uint8_t *host, int32_t *labels, long n, int c, int h, int w) {
    TTDataset *d = (TTDataset *)calloc(1, sizeof(TTDataset));
    if (!d) return NULL;
    d->n = n; d->c = c; d->h = h; d->w = w;
    d->labels = labels;
    const size_t bytes = (size_t)n * (size_t)sample_bytes(d);
    d->dev = (uint8_t *)ttrt_alloc(bytes);
    if (!d->dev || ttrt_h2d(d->dev, host, bytes) != 0) {
        ttrt_free(d->dev);
        free(d);
        return NULL;
    }
    return d;
}

TTDataset *tt_dataset_idx(const char *images_path, const char *labels_path) {
    if (ttrt_init() != 0) return NULL;
    int nd = 0, ndl = 0;
    long dims[8], ldims[8], count = 0, lcount = 0;
    gzFile fi = idx_open(images_path, &nd, dims, &count);
    if (!fi) return NULL;
    gzFile fl = idx_open(labels_path, &ndl, ldims, &lcount);
    if (!fl || nd < 2 || ndl != 1 || ldims[0] != dims[0] || count / dims[0] > 0x7fffffffL) {
        gzclose(fi);
        if (fl) gzclose(fl);
        return NULL;
    }
    const long n = dims[0];
    uint8_t *img = (uint8_t *)malloc((size_t)count);
    uint8_t *lab8 = (uint8_t *)malloc((size_t)n);
    int32_t *lab = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    TTDataset *d = NULL;
    if (img && lab8 && lab && !read_all(fi, img, (size_t)count) && !read_all(fl, lab8, (size_t)n)) {
        for (long i = 0; i < n; i++) lab[i] = lab8[i];
        /* rows x cols for 3-D files; a flat sample otherwise */
        const int hh = nd == 3 ? (int)dims[1] : 1;
        const int ww = (int)(count / n / hh);
        d = upload(img, lab, n, 1, hh, ww);
    }
    gzclose(fi);
    gzclose(fl);
    free(img);
    free(lab8);
    if (!d) free(lab);
    return d;
}

#define CIFAR_REC (1 + 3 * 32 * 32)

TTDataset *tt_dataset_cifar10_bin(const char *const *paths, int npaths) {
    if (ttrt_init() != 0 || !paths || npaths <= 0) return NULL;
    long total = 0;
    long *recs = (long *)calloc((size_t)npaths, sizeof(long));
    if (!recs) return NULL;
    for (int i = 0; i < npaths; i++) {
        FILE *f = paths[i] ? fopen(paths[i], "rb") : NULL;
        if (!f) { free(recs); return NULL; }
        fseek(f, 0, SEEK_END);
        const long sz = ftell(f);
        fclose(f);
        if (sz <= 0 || sz % CIFAR_REC) { free(recs); return NULL; }
        recs[i] = sz / CIFAR_REC;
        total += recs[i];
    }
    uint8_t *img = (uint8_t *)malloc((size_t)total * (CIFAR_REC - 1));
    int32_t *lab = (int32_t *)malloc(sizeof(int32_t) * (size_t)total);
    uint8_t *rec = (uint8_t *)malloc(CIFAR_REC);
    int ok = img && lab && rec;
    long k = 0;
    for (int i = 0; ok && i < npaths; i++) {
        FILE *f = fopen(paths[i], "rb");
        if (!f) { ok = 0; break; }
        for (long r = 0; r < recs[i]; r++, k++) {
            if (fread(rec, 1, CIFAR_REC, f) != CIFAR_REC || rec[0] > 9) { ok = 0; break; }
            lab[k] = rec[0];
            memcpy(img + (size_t)k * (CIFAR_REC - 1), rec + 1, CIFAR_REC - 1);
        }
        fclose(f);
    }
    TTDataset *d = ok ? upload(img, lab, total, 3, 32, 32) : NULL;
    free(recs);
    free(img);
    free(rec);
    if (!d) free(lab);
    return d;
}

TTDataset *tt_dataset_from_u8(const uint8_t *samples, const int32_t *labels, long n, int c,
                              int h, int w) {
    if (ttrt_init() != 0 || !samples || n <= 0 || c <= 0 || h <= 0 || w <= 0) return NULL;
    if ((long)c * h * w > 0x7fffffffL) return NULL;
    int32_t *lab = (int32_t *)malloc(sizeof(int32_t) * (size_t)n);
    if (!lab) return NULL;
    if (labels) memcpy(lab, labels, sizeof(int32_t) * (size_t)n);
    else memset(lab, 0, sizeof(int32_t) * (size_t)n);
    TTDataset *d = upload((uint8_t *)samples, lab, n, c, h, w);
    if (!d) free(lab);
    return d;
}

long tt_dataset_len(const TTDataset *d) { return d ? d->n : -1; }

int tt_dataset_shape(const TTDataset *d, int *c, int *h, int *w) {
    if (!d || !c || !h || !w) return -1;
    *c = d->c; *h = d->h; *w = d->w;
    return 0;
}

int tt_dataset_labels(const TTDataset *d, int32_t *out) {
    if (!d || !out) return -1;
    memcpy(out, d->labels, sizeof(int32_t) * (size_t)d->n);
    return 0;
}

Tensor *tt_dataset_batch(const TTDataset *d, const long *idx, long n, const float *mean,
                         const float *std, int flat, int32_t *labels_out) {
    if (!d || !idx || n <= 0 || !mean || !std || d->c > 4) return NULL;
    for (long r = 0; r < n; r++)
        if (idx[r] < 0 || idx[r] >= d->n) return NULL;
    const long S = sample_bytes(d);
    const long shp4[4] = {n, d->c, d->h, d->w};
    const long shp2[2] = {n, S};
    Tensor *out = flat ? tt_empty_dev(shp2, 2) : tt_empty_dev(shp4, 4);
    if (!out) return NULL;
    int64_t *didx = (int64_t *)ttrt_alloc(sizeof(int64_t) * (size_t)n);
    int rc = -1;
    if (didx && ttrt_h2d_async(didx, idx, sizeof(int64_t) * (size_t)n) == 0)
        rc = tt_k_gather_u8_norm(d->dev, d->n, S, (long)d->h * d->w, d->c, didx, n, mean, std,
                                 out->dev);
    ttrt_free(didx);
    if (rc) { tt_release(out); return NULL; }
    if (labels_out)
        for (long r = 0; r < n; r++) labels_out[r] = d->labels[idx[r]];
    return out;
}

void tt_dataset_release(TTDataset *d) {
    if (!d) return;
    ttrt_free(d->dev);
    free(d->labels);
    free(d);
}
