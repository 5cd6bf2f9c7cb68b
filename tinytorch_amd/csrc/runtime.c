/* Device runtime: the library's HIP stream, a caching device allocator and
 * the host<->device copy helpers.
 *
 * The reference allocates every tensor with calloc (reference
 * src/tensor.c:19-21); on the GPU the equivalent, hipMalloc/hipFree per
 * tensor, costs tens of microseconds and hipFree waits for the whole device.
 * So freed blocks go to per-size free lists and are handed out again
 * directly.  That is safe without events because the library issues every
 * kernel and copy on ONE in-order stream: whatever writes a recycled block
 * is queued after whatever read it before it was freed.
 *
 * Rounding: requests are rounded up to 256 B below 1 MiB, to 64 KiB below
 * 64 MiB and to 2 MiB above, so a training step that rebuilds the same graph
 * every iteration reuses the same blocks.  On hipMalloc failure the cache is
 * returned to the device and the allocation retried once.
 *
 * TT_FAIL_ALLOC_AFTER=n (environment) makes every device allocation after
 * the first n fail, so the NULL-on-OOM paths of the C ABI can be exercised.
 *
 * Single-threaded by contract, like the reference's non-atomic refcounts
 * (reference src/tensor.c:48-61). */
#include "tt_rt.h"

#include <hip/hip_runtime_api.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int g_state = 0; /* 0 = not tried, 1 = ready, -1 = no device */
static hipStream_t g_stream = NULL;
static int g_err = 0;
static long g_fail_after = -1;
static long g_alloc_count = 0;
static size_t g_in_use = 0, g_cached = 0;

/* ---- live-block table: device pointer -> rounded size (open addressing) ---- */
typedef struct { void *p; size_t sz; } Live;
static Live *g_live = NULL;
static size_t g_live_cap = 0, g_live_n = 0;

static size_t hash_ptr(void *p, size_t cap) {
    uint64_t x = (uint64_t)(uintptr_t)p;
    x ^= x >> 33; x *= 0xff51afd7ed558ccdULL; x ^= x >> 33;
    return (size_t)x & (cap - 1);
}

static int live_grow(void) {
    size_t ncap = g_live_cap ? g_live_cap * 2 : 1024;
    Live *nt = (Live *)calloc(ncap, sizeof(Live));
    if (!nt) return 0;
    for (size_t i = 0; i < g_live_cap; i++) {
        if (!g_live[i].p) continue;
        size_t h = hash_ptr(g_live[i].p, ncap);
        while (nt[h].p) h = (h + 1) & (ncap - 1);
        nt[h] = g_live[i];
    }
    free(g_live);
    g_live = nt;
    g_live_cap = ncap;
    return 1;
}

static int live_put(void *p, size_t sz) {
    if ((g_live_n + 1) * 2 > g_live_cap && !live_grow()) return 0;
    size_t h = hash_ptr(p, g_live_cap);
    while (g_live[h].p) h = (h + 1) & (g_live_cap - 1);
    g_live[h].p = p;
    g_live[h].sz = sz;
    g_live_n++;
    return 1;
}

/* remove p; returns its size or 0 when unknown */
static size_t live_take(void *p) {
    if (!g_live_cap) return 0;
    size_t h = hash_ptr(p, g_live_cap);
    while (g_live[h].p) {
        if (g_live[h].p == p) {
            size_t sz = g_live[h].sz;
            /* backward-shift deletion keeps probe chains intact */
            size_t i = h, j = h;
            for (;;) {
                j = (j + 1) & (g_live_cap - 1);
                if (!g_live[j].p) break;
                size_t k = hash_ptr(g_live[j].p, g_live_cap);
                /* entry j may fill hole i unless its home k lies in (i, j] */
                int stays = (i <= j) ? (i < k && k <= j) : (i < k || k <= j);
                if (!stays) { g_live[i] = g_live[j]; i = j; }
            }
            g_live[i].p = NULL;
            g_live[i].sz = 0;
            g_live_n--;
            return sz;
        }
        h = (h + 1) & (g_live_cap - 1);
    }
    return 0;
}

/* ---- free lists keyed by rounded size ---- */
typedef struct { size_t sz; void **ptrs; int n, cap; } Bin;
static Bin *g_bins = NULL;
static int g_nbins = 0, g_bins_cap = 0;

static Bin *bin_for(size_t sz, int create) {
    for (int i = 0; i < g_nbins; i++)
        if (g_bins[i].sz == sz) return &g_bins[i];
    if (!create) return NULL;
    if (g_nbins == g_bins_cap) {
        int nc = g_bins_cap ? g_bins_cap * 2 : 64;
        Bin *nb = (Bin *)realloc(g_bins, sizeof(Bin) * (size_t)nc);
        if (!nb) return NULL;
        g_bins = nb;
        g_bins_cap = nc;
    }
    Bin *b = &g_bins[g_nbins++];
    memset(b, 0, sizeof(*b));
    b->sz = sz;
    return b;
}

static size_t round_size(size_t bytes) {
    if (bytes == 0) bytes = 1;
    size_t q;
    if (bytes < ((size_t)1 << 20)) q = 256;
    else if (bytes < ((size_t)64 << 20)) q = (size_t)64 << 10;
    else q = (size_t)2 << 20;
    return (bytes + q - 1) / q * q;
}

int ttrt_init(void) {
    if (g_state) return g_state > 0 ? 0 : -1;
    g_state = -1;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) { (void)hipGetLastError(); return -1; }
    if (hipSetDevice(0) != hipSuccess) return -1;
    if (hipStreamCreate(&g_stream) != hipSuccess) return -1;
    /* device address of the no-allocation GEMM's scratch array (gemm.hip) */
    if (ttg_scratch_setup() != 0) return -1;
    const char *fa = getenv("TT_FAIL_ALLOC_AFTER");
    if (fa && *fa) g_fail_after = atol(fa);
    g_state = 1;
    return 0;
}

void *ttrt_stream(void) { return (void *)g_stream; }

void ttrt_set_error(int code) { g_err = code; }

int tth_fail_alloc_after(long n) {
    if (ttrt_init() != 0) return -1;
    g_fail_after = n < 0 ? -1 : g_alloc_count + n;
    return 0;
}
int ttrt_last_error(void) { return g_err; }
size_t ttrt_bytes_in_use(void) { return g_in_use; }
size_t ttrt_bytes_cached(void) { return g_cached; }

void ttrt_release_cache(void) {
    if (g_state <= 0) return;
    hipStreamSynchronize(g_stream);
    for (int i = 0; i < g_nbins; i++) {
        for (int j = 0; j < g_bins[i].n; j++) hipFree(g_bins[i].ptrs[j]);
        g_cached -= g_bins[i].sz * (size_t)g_bins[i].n;
        g_bins[i].n = 0;
    }
}

void *ttrt_alloc(size_t bytes) {
    if (ttrt_init() != 0) { g_err = -10; return NULL; }
    if (g_fail_after >= 0 && g_alloc_count >= g_fail_after) { g_err = -11; return NULL; }
    g_alloc_count++;
    const size_t sz = round_size(bytes);
    Bin *b = bin_for(sz, 0);
    void *p = NULL;
    if (b && b->n > 0) {
        p = b->ptrs[--b->n];
        g_cached -= sz;
    } else {
        if (hipMalloc(&p, sz) != hipSuccess) {
            (void)hipGetLastError();
            ttrt_release_cache();
            if (hipMalloc(&p, sz) != hipSuccess) { (void)hipGetLastError(); g_err = -12; return NULL; }
        }
    }
    if (!live_put(p, sz)) {
        hipFree(p);
        g_err = -13;
        return NULL;
    }
    g_in_use += sz;
    return p;
}

void ttrt_free(void *p) {
    if (!p) return;
    size_t sz = live_take(p);
    if (!sz) return; /* not ours */
    g_in_use -= sz;
    Bin *b = bin_for(sz, 1);
    if (!b) { hipFree(p); return; }
    if (b->n == b->cap) {
        int nc = b->cap ? b->cap * 2 : 8;
        void **np = (void **)realloc(b->ptrs, sizeof(void *) * (size_t)nc);
        if (!np) { hipFree(p); return; }
        b->ptrs = np;
        b->cap = nc;
    }
    b->ptrs[b->n++] = p;
    g_cached += sz;
}

int ttrt_sync(void) {
    if (g_state <= 0) return -1;
    return hipStreamSynchronize(g_stream) == hipSuccess ? 0 : -1;
}

int ttrt_h2d(void *dst, const void *src, size_t bytes) {
    if (ttrt_init() != 0) return -1;
    if (!bytes) return 0;
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_stream) != hipSuccess) return -1;
    /* the caller may reuse or free src as soon as we return */
    return hipStreamSynchronize(g_stream) == hipSuccess ? 0 : -1;
}

/* Host-to-device copies of small buffers (tensor construction, backward
 * seeds, labels) go through a ring of pinned staging slots: the bytes are
 * copied into a slot on the host and the DMA is enqueued on the stream, so
 * the caller neither waits for the GPU nor has to keep its buffer alive.  A
 * slot is reused once the event recorded after its copy has completed. */
#define TT_STAGE_SLOTS 8
#define TT_STAGE_BYTES ((size_t)4 << 20)
typedef struct { void *buf; hipEvent_t ev; int pending; } StageSlot;
static StageSlot g_stage[TT_STAGE_SLOTS];
static int g_stage_next = 0;

int ttrt_h2d_async(void *dst, const void *src, size_t bytes) {
    if (ttrt_init() != 0) return -1;
    if (!bytes) return 0;
    if (bytes > TT_STAGE_BYTES) return ttrt_h2d(dst, src, bytes);
    StageSlot *s = &g_stage[g_stage_next];
    if (!s->buf) {
        if (hipHostMalloc(&s->buf, TT_STAGE_BYTES, hipHostMallocDefault) != hipSuccess) {
            (void)hipGetLastError();
            s->buf = NULL;
            return ttrt_h2d(dst, src, bytes);
        }
        if (hipEventCreateWithFlags(&s->ev, hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            hipHostFree(s->buf);
            s->buf = NULL;
            return ttrt_h2d(dst, src, bytes);
        }
    }
    g_stage_next = (g_stage_next + 1) % TT_STAGE_SLOTS;
    if (s->pending && hipEventSynchronize(s->ev) != hipSuccess) return -1;
    memcpy(s->buf, src, bytes);
    if (hipMemcpyAsync(dst, s->buf, bytes, hipMemcpyHostToDevice, g_stream) != hipSuccess) return -1;
    if (hipEventRecord(s->ev, g_stream) != hipSuccess) return -1;
    s->pending = 1;
    return 0;
}

/* Pinned host mirrors.  tt_data() hands the caller a host copy of a device
 * tensor; when that copy lives in page-locked memory the device-to-host DMA
 * writes it directly instead of bouncing through the driver's staging
 * buffers, and NumPy views of it (pybind value(copy=False)) cost nothing.
 * Page-locking is slow (a syscall and page pinning per hipHostMalloc), so
 * freed mirrors go to per-size free lists like device blocks, up to
 * TT_HOST_CACHE_MAX bytes.  A 64-byte header in front of the payload keeps
 * the rounded size and whether the block is pinned (a failed hipHostMalloc
 * falls back to malloc). */
#define TT_HOST_HDR 64
#define TT_HOST_CACHE_MAX ((size_t)1 << 30)
typedef struct { size_t sz; int pinned; } HostHdr;
static Bin *g_hbins = NULL;
static int g_nhbins = 0, g_hbins_cap = 0;
static size_t g_hcached = 0;

static Bin *hbin_for(size_t sz, int create) {
    for (int i = 0; i < g_nhbins; i++)
        if (g_hbins[i].sz == sz) return &g_hbins[i];
    if (!create) return NULL;
    if (g_nhbins == g_hbins_cap) {
        int nc = g_hbins_cap ? g_hbins_cap * 2 : 32;
        Bin *nb = (Bin *)realloc(g_hbins, sizeof(Bin) * (size_t)nc);
        if (!nb) return NULL;
        g_hbins = nb;
        g_hbins_cap = nc;
    }
    Bin *b = &g_hbins[g_nhbins++];
    memset(b, 0, sizeof(*b));
    b->sz = sz;
    return b;
}

static void host_block_free(void *base) {
    HostHdr *h = (HostHdr *)base;
    if (h->pinned) hipHostFree(base);
    else free(base);
}

void *ttrt_host_alloc(size_t bytes) {
    size_t sz = round_size(bytes + TT_HOST_HDR);
    if (sz < 4096) sz = 4096;
    Bin *b = hbin_for(sz, 0);
    void *base = NULL;
    if (b && b->n > 0) {
        base = b->ptrs[--b->n];
        g_hcached -= sz;
    } else {
        int pinned = 0;
        if (ttrt_init() == 0 && hipHostMalloc(&base, sz, hipHostMallocDefault) == hipSuccess) {
            pinned = 1;
        } else {
            (void)hipGetLastError();
            base = malloc(sz);
            if (!base) return NULL;
        }
        ((HostHdr *)base)->sz = sz;
        ((HostHdr *)base)->pinned = pinned;
    }
    return (char *)base + TT_HOST_HDR;
}

void ttrt_host_free(void *p) {
    if (!p) return;
    void *base = (char *)p - TT_HOST_HDR;
    const size_t sz = ((HostHdr *)base)->sz;
    Bin *b = g_hcached + sz <= TT_HOST_CACHE_MAX ? hbin_for(sz, 1) : NULL;
    if (b && b->n == b->cap) {
        int nc = b->cap ? b->cap * 2 : 8;
        void **np = (void **)realloc(b->ptrs, sizeof(void *) * (size_t)nc);
        if (np) { b->ptrs = np; b->cap = nc; } else b = NULL;
    }
    if (!b) { host_block_free(base); return; }
    b->ptrs[b->n++] = base;
    g_hcached += sz;
}

int ttrt_host_is_pinned(const void *p) {
    return p ? ((const HostHdr *)((const char *)p - TT_HOST_HDR))->pinned : 0;
}

int ttrt_d2h(void *dst, const void *src, size_t bytes) {
    if (ttrt_init() != 0) return -1;
    if (!bytes) return 0;
    if (hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_stream) != hipSuccess) return -1;
    return hipStreamSynchronize(g_stream) == hipSuccess ? 0 : -1;
}
