// Bandwidth-bound elementwise and row kernels (HBM roofline).
//
//   relu forward / backward    reference src/ops.c:104-106, src/autograd.c:318-327
//   softmax forward / backward reference src/ops.c:108-145, src/autograd.c:329-346
//   grad accumulation (accum)  reference src/autograd.c:52-63
//   padones forward / backward reference src/autograd.c:195-212, 348-359
//   add / mul / scalar ops     reference src/ops.c:26-78 (API completeness)
//   softmax-cross-entropy seed reference harness tests/gate_cifar_cnn.py:175-181
//
// Flat kernels move 16 bytes per lane per access (float4) when the pointers
// and the length allow it, with a scalar tail; a grid-stride loop sized to a
// few waves per CU keeps every launch at one dispatch.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include "tt_rt.h"
#include "ce_rows.h"

namespace {

inline hipStream_t stream() { return (hipStream_t)ttrt_stream(); }

inline bool a16(const void *p) { return ((uintptr_t)p & 15) == 0; }

inline int grid_for(long n, int per_thread) {
  long blocks = (n / per_thread + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 8192) blocks = 8192;
  return (int)blocks;
}

inline int launched() { return hipGetLastError() == hipSuccess ? 0 : -3; }

// Generic flat map over float4 groups with a scalar tail.
template <typename F>
__global__ void map4_kernel(long n4, long n, F f) {
  const long stride = (long)gridDim.x * blockDim.x;
  const long t0 = (long)blockIdx.x * blockDim.x + threadIdx.x;
  for (long i = t0; i < n4; i += stride) f.vec(i);
  for (long i = n4 * 4 + t0; i < n; i += stride) f.one(i);
}

template <typename F>
__global__ void map1_kernel(long n, F f) {
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) f.one(i);
}

template <typename F>
int run_map(long n, bool vec, F f) {
  if (n <= 0) return 0;
  if (vec) {
    long n4 = n / 4;
    hipLaunchKernelGGL(map4_kernel<F>, dim3(grid_for(n, 4)), dim3(256), 0, stream(), n4, n, f);
  } else {
    hipLaunchKernelGGL(map1_kernel<F>, dim3(grid_for(n, 1)), dim3(256), 0, stream(), n, f);
  }
  return launched();
}

struct FillOp {
  float *x; float v;
  __device__ void vec(long i) const { reinterpret_cast<float4 *>(x)[i] = make_float4(v, v, v, v); }
  __device__ void one(long i) const { x[i] = v; }
};
struct CopyOp {
  float *d; const float *s;
  __device__ void vec(long i) const { reinterpret_cast<float4 *>(d)[i] = reinterpret_cast<const float4 *>(s)[i]; }
  __device__ void one(long i) const { d[i] = s[i]; }
};
struct AddInplaceOp {
  float *d; const float *s;
  __device__ void vec(long i) const {
    float4 a = reinterpret_cast<float4 *>(d)[i];
    const float4 b = reinterpret_cast<const float4 *>(s)[i];
    a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    reinterpret_cast<float4 *>(d)[i] = a;
  }
  __device__ void one(long i) const { d[i] += s[i]; }
};
__device__ __forceinline__ float relu1(float x) { return x > 0.0f ? x : 0.0f; }
struct ReluFwdOp {
  const float *x; float *y;
  __device__ void vec(long i) const {
    const float4 a = reinterpret_cast<const float4 *>(x)[i];
    reinterpret_cast<float4 *>(y)[i] = make_float4(relu1(a.x), relu1(a.y), relu1(a.z), relu1(a.w));
  }
  __device__ void one(long i) const { y[i] = relu1(x[i]); }
};
struct ReluBwdOp {
  const float *x; const float *g; float *dx;
  __device__ void vec(long i) const {
    const float4 a = reinterpret_cast<const float4 *>(x)[i];
    const float4 b = reinterpret_cast<const float4 *>(g)[i];
    reinterpret_cast<float4 *>(dx)[i] = make_float4(a.x > 0.0f ? b.x : 0.0f, a.y > 0.0f ? b.y : 0.0f,
                                                    a.z > 0.0f ? b.z : 0.0f, a.w > 0.0f ? b.w : 0.0f);
  }
  __device__ void one(long i) const { dx[i] = x[i] > 0.0f ? g[i] : 0.0f; }
};
struct BinaryOp {
  const float *a; const float *b; float *y; int op;
  __device__ float f(float u, float v) const { return op == 0 ? u + v : u * v; }
  __device__ void vec(long i) const {
    const float4 u = reinterpret_cast<const float4 *>(a)[i];
    const float4 v = reinterpret_cast<const float4 *>(b)[i];
    reinterpret_cast<float4 *>(y)[i] = make_float4(f(u.x, v.x), f(u.y, v.y), f(u.z, v.z), f(u.w, v.w));
  }
  __device__ void one(long i) const { y[i] = f(a[i], b[i]); }
};
struct ScalarOp {
  const float *a; float *y; float s; int op;
  __device__ float f(float u) const { return op == 0 ? u + s : u * s; }
  __device__ void vec(long i) const {
    const float4 u = reinterpret_cast<const float4 *>(a)[i];
    reinterpret_cast<float4 *>(y)[i] = make_float4(f(u.x), f(u.y), f(u.z), f(u.w));
  }
  __device__ void one(long i) const { y[i] = f(a[i]); }
};
struct SgdOp {
  float *w; const float *g; float lr;
  __device__ void vec(long i) const {
    float4 a = reinterpret_cast<float4 *>(w)[i];
    const float4 b = reinterpret_cast<const float4 *>(g)[i];
    a.x -= lr * b.x; a.y -= lr * b.y; a.z -= lr * b.z; a.w -= lr * b.w;
    reinterpret_cast<float4 *>(w)[i] = a;
  }
  __device__ void one(long i) const { w[i] -= lr * g[i]; }
};

// ---- row kernels ----
// Rows of at most 64 columns run one row per lane with the reference's
// sequential summation order; wider rows run one row per wavefront with a
// butterfly reduction.

// softmax, one row per thread (cols <= 64)
__global__ void softmax_rowthread_kernel(const float *__restrict__ x, float *__restrict__ y,
                                         long rows, int cols) {
  const long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float *xr = x + r * cols;
  float *yr = y + r * cols;
  float mx = -INFINITY;
  for (int j = 0; j < cols; j++) { const float v = xr[j]; if (v > mx) mx = v; }
  if (mx == -INFINITY) {
    const float u = 1.0f / (float)cols;
    for (int j = 0; j < cols; j++) yr[j] = u;
    return;
  }
  float sum = 0.0f;
  for (int j = 0; j < cols; j++) { const float e = expf(xr[j] - mx); yr[j] = e; sum += e; }
  for (int j = 0; j < cols; j++) yr[j] = yr[j] / sum;
}

__device__ __forceinline__ float wave_max(float v) {
  for (int o = 32; o > 0; o >>= 1) { const float t = __shfl_xor(v, o, 64); v = t > v ? t : v; }
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// softmax, one row per wavefront (cols > 64)
__global__ void softmax_rowwave_kernel(const float *__restrict__ x, float *__restrict__ y,
                                       long rows, int cols) {
  const long r = (long)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float *xr = x + r * cols;
  float *yr = y + r * cols;
  float mx = -INFINITY;
  for (int j = lane; j < cols; j += 64) { const float v = xr[j]; if (v > mx) mx = v; }
  mx = wave_max(mx);
  if (mx == -INFINITY) {
    const float u = 1.0f / (float)cols;
    for (int j = lane; j < cols; j += 64) yr[j] = u;
    return;
  }
  float sum = 0.0f;
  for (int j = lane; j < cols; j += 64) { const float e = expf(xr[j] - mx); yr[j] = e; sum += e; }
  sum = wave_sum(sum);
  for (int j = lane; j < cols; j += 64) yr[j] = yr[j] / sum;
}

__global__ void softmax_bwd_rowthread_kernel(const float *__restrict__ s, const float *__restrict__ g,
                                             float *__restrict__ dx, long rows, int cols) {
  const long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float *sr = s + r * cols, *gr = g + r * cols;
  float dot = 0.0f;
  for (int j = 0; j < cols; j++) dot += gr[j] * sr[j];
  for (int j = 0; j < cols; j++) dx[r * cols + j] = sr[j] * (gr[j] - dot);
}

__global__ void softmax_bwd_rowwave_kernel(const float *__restrict__ s, const float *__restrict__ g,
                                           float *__restrict__ dx, long rows, int cols) {
  const long r = (long)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
  const int lane = threadIdx.x & 63;
  if (r >= rows) return;
  const float *sr = s + r * cols, *gr = g + r * cols;
  float dot = 0.0f;
  for (int j = lane; j < cols; j += 64) dot += gr[j] * sr[j];
  dot = wave_sum(dot);
  for (int j = lane; j < cols; j += 64) dx[r * cols + j] = sr[j] * (gr[j] - dot);
}

// Fused softmax + cross-entropy: probs, per-row loss -log(max(p[y],1e-12))
// and the logits gradient seed (p - onehot(y)) * scale, one row per thread.
__global__ void softmax_ce_kernel(const float *__restrict__ x, const int32_t *__restrict__ lab,
                                  float *__restrict__ probs, float *__restrict__ loss,
                                  float *__restrict__ seed, long rows, int cols, float scale) {
  const long r = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float *xr = x + r * cols;
  float *pr = probs + r * cols;
  float mx = -INFINITY;
  for (int j = 0; j < cols; j++) { const float v = xr[j]; if (v > mx) mx = v; }
  if (mx == -INFINITY) {
    for (int j = 0; j < cols; j++) pr[j] = 1.0f / (float)cols;
  } else {
    float sum = 0.0f;
    for (int j = 0; j < cols; j++) { const float e = expf(xr[j] - mx); pr[j] = e; sum += e; }
    for (int j = 0; j < cols; j++) pr[j] = pr[j] / sum;
  }
  const int y = lab[r];
  const bool ok = y >= 0 && y < cols;
  const float py = ok ? pr[y] : 0.0f;
  loss[r] = -logf(fmaxf(py, 1e-12f));
  for (int j = 0; j < cols; j++) seed[r * cols + j] = (pr[j] - (j == y ? 1.0f : 0.0f)) * scale;
}

template <typename I>
__global__ void padones_fwd_kernel(const float *__restrict__ x, float *__restrict__ y, long M, long K) {
  const I total = (I)(M * (K + 1));
  const I K1 = (I)(K + 1);
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I m = i / K1, k = i - m * K1;
    y[i] = k < (I)K ? x[(long)m * K + k] : 1.0f;
  }
}

template <typename I>
__global__ void padones_bwd_kernel(const float *__restrict__ g, float *__restrict__ dx, long M, long K) {
  const I total = (I)(M * K);
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I m = i / (I)K, k = i - m * (I)K;
    dx[i] = g[(long)m * (K + 1) + k];
  }
}

// padones by rows: workgroup (m, chunk) copies 1024 elements of row m with
// no per-element division (grid.y indexes rows, so M < 65536 here)
__global__ void padones_fwd_rows_kernel(const float *__restrict__ x, float *__restrict__ y, int K) {
  const long m = blockIdx.y;
  const float *xr = x + m * K;
  float *yr = y + m * (K + 1);
  for (int k = blockIdx.x * 1024 + threadIdx.x; k <= K && k < (int)(blockIdx.x + 1) * 1024; k += 256)
    yr[k] = k < K ? xr[k] : 1.0f;
}

// padones of a tensor that is itself a fresh copy of x (reshape then
// padones): writes the copy c = x and y = padones(x) from one read of x
__global__ void copy_padones_rows_kernel(const float *__restrict__ x, float *__restrict__ c,
                                         float *__restrict__ y, int K) {
  const long m = blockIdx.y;
  const float *xr = x + m * K;
  float *cr = c + m * K;
  float *yr = y + m * (K + 1);
  for (int k = blockIdx.x * 1024 + threadIdx.x; k <= K && k < (int)(blockIdx.x + 1) * 1024; k += 256) {
    if (k < K) {
      const float v = xr[k];
      cr[k] = v;
      yr[k] = v;
    } else {
      yr[k] = 1.0f;
    }
  }
}

// padones of a relu output that is computed in the same pass: r = relu(x)
// (x > 0 ? x : +0, NaN -> +0) and y = padones(r) from one read of x
__global__ void relu_padones_rows_kernel(const float *__restrict__ x, float *__restrict__ r,
                                         float *__restrict__ y, int K) {
  const long m = blockIdx.y;
  const float *xr = x + m * K;
  float *rr = r + m * K;
  float *yr = y + m * (K + 1);
  for (int k = blockIdx.x * 1024 + threadIdx.x; k <= K && k < (int)(blockIdx.x + 1) * 1024; k += 256) {
    if (k < K) {
      const float v = xr[k];
      const float o = v > 0.0f ? v : 0.0f;
      rr[k] = o;
      yr[k] = o;
    } else {
      yr[k] = 1.0f;
    }
  }
}

// padones backward whose result is also the gradient of a reshape's input
// (same data, another shape): both copies from one read of g
__global__ void padones_bwd2_rows_kernel(const float *__restrict__ g, float *__restrict__ d1,
                                         float *__restrict__ d2, int K) {
  const long m = blockIdx.y;
  const float *gr = g + m * (K + 1);
  const long o = m * K;
  for (int k = blockIdx.x * 1024 + threadIdx.x; k < K && k < (int)(blockIdx.x + 1) * 1024; k += 256) {
    const float v = gr[k];
    d1[o + k] = v;
    d2[o + k] = v;
  }
}

__global__ void padones_bwd_rows_kernel(const float *__restrict__ g, float *__restrict__ dx, int K) {
  const long m = blockIdx.y;
  const float *gr = g + m * (K + 1);
  float *dr = dx + m * K;
  for (int k = blockIdx.x * 1024 + threadIdx.x; k < K && k < (int)(blockIdx.x + 1) * 1024; k += 256)
    dr[k] = gr[k];
}

// padones backward fused with the backward of the relu whose output r is
// the padded tensor: dr = g without its last column, dx = dr where r > 0
// (r > 0 exactly when the relu's input is > 0), else +0.0f.
__global__ void padones_relu_bwd_rows_kernel(const float *__restrict__ g, const float *__restrict__ r,
                                             float *__restrict__ dr, float *__restrict__ dx, int K) {
  const long m = blockIdx.y;
  const float *gr = g + m * (K + 1);
  const long o = m * K;
  for (int k = blockIdx.x * 1024 + threadIdx.x; k < K && k < (int)(blockIdx.x + 1) * 1024; k += 256) {
    const float v = gr[k];
    dr[o + k] = v;
    dx[o + k] = r[o + k] > 0.0f ? v : 0.0f;
  }
}

// Fused softmax + cross-entropy for up to a few thousand rows in ONE
// workgroup (ce_rows_block): probabilities, the seed (p - onehot(y)) * scale
// and the mean loss.  Labels from device memory or, up to TT_CE_ARG_ROWS of
// them, inside the kernel arguments (LabArg: 4 bytes a label; LabU8: one byte,
// for cols <= 255).
struct LabArg {
  int32_t v[TT_CE_ARG_ROWS];
  __device__ int32_t operator[](int r) const { return v[r]; }
};

// LAB: a device pointer to the labels, a LabArg or a LabU8
template <int MAXC, class LAB>
__global__ void __launch_bounds__(256)
softmax_ce_mean_kernel(const float *__restrict__ x, const LAB lab, float *__restrict__ probs,
                       float *__restrict__ loss_mean, float *__restrict__ seed, int rows,
                       int cols, float scale) {
  __shared__ float part[256];
  ce_rows_block<MAXC>(x, lab, probs, loss_mean, seed, rows, cols, scale, part);
}

// general width: the same passes over global memory
template <class LAB>
__global__ void softmax_ce_mean_wide_kernel(const float *__restrict__ x, const LAB lab,
                                            float *__restrict__ probs,
                                            float *__restrict__ loss_mean,
                                            float *__restrict__ seed, int rows, int cols,
                                            float scale) {
  __shared__ float part[256];
  float acc = 0.0f;
  for (int r = threadIdx.x; r < rows; r += blockDim.x) {
    const float *xr = x + (long)r * cols;
    float *pr = probs + (long)r * cols;
    float mx = -INFINITY;
    for (int j = 0; j < cols; j++) { const float v = xr[j]; if (v > mx) mx = v; }
    if (mx == -INFINITY) {
      for (int j = 0; j < cols; j++) pr[j] = 1.0f / (float)cols;
    } else {
      float sum = 0.0f;
      for (int j = 0; j < cols; j++) { const float e = expf(xr[j] - mx); pr[j] = e; sum += e; }
      for (int j = 0; j < cols; j++) pr[j] = pr[j] / sum;
    }
    const int y = lab[r];
    const float py = (y >= 0 && y < cols) ? pr[y] : 0.0f;
    acc += -logf(fmaxf(py, 1e-12f));
    for (int j = 0; j < cols; j++) seed[(long)r * cols + j] = (pr[j] - (j == y ? 1.0f : 0.0f)) * scale;
  }
  part[threadIdx.x] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] += part[threadIdx.x + o];
    __syncthreads();
  }
  if (threadIdx.x == 0) loss_mean[0] = part[0] / (float)rows;
}

// y = x * s[0] with s a device scalar (the incoming gradient of a scalar loss)
__global__ void scale_by_dev_kernel(const float *__restrict__ x, const float *__restrict__ s,
                                    float *__restrict__ y, long n) {
  const float k = s[0];
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) y[i] = x[i] * k;
}

// w_i -= lr * g_i for up to TT_SGD_MAX tensors in one launch: blockIdx.y
// selects the tensor.
struct SgdList {
  float *w[TT_SGD_MAX];
  const float *g[TT_SGD_MAX];
  long n[TT_SGD_MAX];
};

__global__ void sgd_multi_kernel(SgdList L, float lr) {
  const int t = blockIdx.y;
  float *w = L.w[t];
  const float *g = L.g[t];
  const long n = L.n[t];
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) w[i] -= lr * g[i];
}

// SGD with momentum on up to TT_SGD_MAX tensors (blockIdx.y selects one).
// The file is compiled with -ffp-contract=off, so each product is rounded
// before the subtraction exactly as NumPy's separate array operations are.
struct MomList {
  float *w[TT_SGD_MAX];
  const float *g[TT_SGD_MAX];
  float *v[TT_SGD_MAX];
  long n[TT_SGD_MAX];
};

__global__ void momentum_multi_kernel(MomList L, float lr, float mu) {
  const int t = blockIdx.y;
  float *w = L.w[t], *v = L.v[t];
  const float *g = L.g[t];
  const long n = L.n[t];
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float vn = mu * v[i] - lr * g[i];
    v[i] = vn;
    w[i] = w[i] + vn;
  }
}

// Adam on up to TT_SGD_MAX tensors.  Moments are fp32; the parameter step
// is formed in fp64 (lr_t is a double) and rounded once when stored.
struct AdamList {
  float *w[TT_SGD_MAX];
  const float *g[TT_SGD_MAX];
  float *m[TT_SGD_MAX];
  float *v[TT_SGD_MAX];
  long n[TT_SGD_MAX];
};

__global__ void adam_multi_kernel(AdamList L, float b1, float omb1, float b2, float omb2, float eps,
                                  double lr_t) {
  const int t = blockIdx.y;
  float *w = L.w[t], *m = L.m[t], *v = L.v[t];
  const float *g = L.g[t];
  const long n = L.n[t];
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const float gi = g[i];
    const float mn = b1 * m[i] + omb1 * gi;
    const float vn = b2 * v[i] + omb2 * (gi * gi);
    m[i] = mn;
    v[i] = vn;
    const float den = sqrtf(vn) + eps;
    w[i] = (float)((double)w[i] - (lr_t * (double)mn) / (double)den);
  }
}

// Dataset batch: out[r, j] = ((float)src[idx[r], j] / 255 - mean[c]) / std[c]
// with c = j / plane.  Division is IEEE (correctly rounded) and nothing is
// contracted, so the result equals NumPy's float32 evaluation.  blockIdx.y
// strides over rows; the vector path moves 4 bytes in and 16 bytes out per
// lane (needs sample and plane sizes that are multiples of 4).
struct NormParams {
  float mean[4], stdv[4];
};

__device__ __forceinline__ float norm_u8(unsigned v, float m, float s) {
  return ((float)v / 255.0f - m) / s;
}

template <bool VEC>
__global__ void gather_u8_norm_kernel(const uint8_t *__restrict__ src, long S, long plane,
                                      const int64_t *__restrict__ idx, long n, NormParams P,
                                      float *__restrict__ out) {
  const long per = VEC ? S / 4 : S;
  for (long r = blockIdx.y; r < n; r += gridDim.y) {
    const uint8_t *row = src + idx[r] * S;
    float *orow = out + r * S;
    for (long j = (long)blockIdx.x * blockDim.x + threadIdx.x; j < per;
         j += (long)gridDim.x * blockDim.x) {
      if constexpr (VEC) {
        const uchar4 v = *reinterpret_cast<const uchar4 *>(row + 4 * j);
        const int c = (int)((4 * j) / plane);
        const float m = P.mean[c], sd = P.stdv[c];
        *reinterpret_cast<float4 *>(orow + 4 * j) =
            make_float4(norm_u8(v.x, m, sd), norm_u8(v.y, m, sd), norm_u8(v.z, m, sd),
                        norm_u8(v.w, m, sd));
      } else {
        const int c = (int)(j / plane);
        orow[j] = norm_u8(row[j], P.mean[c], P.stdv[c]);
      }
    }
  }
}

// Naive matmul with the reference's arithmetic: C[m][n] starts at +0.0 and
// adds a*B[k][n] for k ascending, skipping every k where a = A[m][k] is zero
// (so 0 * NaN / 0 * Inf in B never reach C), one multiply and one add each
// (this file is compiled without contraction).  One lane per output; the
// lanes of a wave take consecutive n of one row, so B's rows are read
// coalesced and A[m][k] is one broadcast load.
__global__ void __launch_bounds__(256)
matmul_naive_kernel(const float *__restrict__ A, const float *__restrict__ B,
                    float *__restrict__ C, int M, int N, int K) {
  const int n = blockIdx.x * 256 + threadIdx.x;
  if (n >= N) return;
  for (int m = blockIdx.y; m < M; m += gridDim.y) {
    const float *a = A + (long)m * K;
    float acc = 0.0f;
    for (int k = 0; k < K; k++) {
      const float av = a[k];
      if (av == 0.0f) continue;
      acc += av * B[(long)k * N + n];
    }
    C[(long)m * N + n] = acc;
  }
}

// c[m][n] += cin[m][n] for every (m, n) outside the leading mb x nb block
// (tt_sgemm_rowmajor's accumulating tails).
__global__ void __launch_bounds__(256)
add_outside_kernel(float *__restrict__ c, const float *__restrict__ cin, int M, int N, int mb,
                   int nb) {
  const long total = (long)M * N;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int m = (int)(i / N), n = (int)(i % N);
    if (m >= mb || n >= nb) c[i] = cin[i] + c[i];
  }
}

}  // namespace

// The split-K reduction of a GEMM whose rows go straight into softmax-CE
// (the classifier): each element summed exactly as gemm.hip's reduce_one
// (lanes ty = 0..ZL-1 add partials z = ty, ty + ZL, ... in order, then lane
// 0 adds the lanes' sums in lane order) plus bias, stored to C; a workgroup
// holds rpb whole rows (ZL x rpb*N threads), so after a barrier groups of
// MAXC lanes run each row's softmax-CE from LDS (ce_row_group).  The same
// bits as the reduction followed by softmax_ce_mean_kernel (whose per-row
// losses ttk_ce_mean_rows adds).
template <int ZL, int MAXC>
__global__ void __launch_bounds__(1024)
splitk_reduce_ce_kernel(const float *__restrict__ ws, float *__restrict__ C, int M, int N, int S,
                        int rpb, const float *__restrict__ bias, LabU8 lab,
                        float *__restrict__ probs, float *__restrict__ seed,
                        float *__restrict__ rowloss, float scale) {
  extern __shared__ float sm[];
  const int XL = rpb * N;
  float *part = sm, *lv = sm + ZL * XL;
  const int tx = threadIdx.x % XL, ty = threadIdx.x / XL;
  const long total = (long)M * N;
  const long idx = (long)blockIdx.x * XL + tx;
  float s = 0.f;
  if (idx < total) {
#pragma unroll 4
    for (int z = ty; z < S; z += ZL) s += ws[z * total + idx];
  }
  part[ty * XL + tx] = s;
  __syncthreads();
  if (ty == 0) {
    for (int j = 1; j < ZL; j++) s += part[j * XL + tx];
    if (idx < total) {
      const float v = bias ? s + bias[tx % N] : s;
      C[idx] = v;
      lv[tx] = v;
    }
  }
  __syncthreads();
  const int ng = blockDim.x / MAXC;  // groups of MAXC lanes, a row each (ce_row_group)
  if (ng == 0) {
    const int r = threadIdx.x;
    const long row = (long)blockIdx.x * rpb + r;
    if (r < rpb && row < M)
      rowloss[row] = ce_row<MAXC>(lv + r * N, lab[(int)row], probs + row * N, seed + row * N, N,
                                  scale);
    return;
  }
  const int gi = threadIdx.x / MAXC, j = threadIdx.x % MAXC;
  if (gi >= ng) return;
  for (int r = gi; r < rpb; r += ng) {
    const long row = (long)blockIdx.x * rpb + r;
    if (row >= M) break;
    float xj[1] = {j < N ? lv[r * N + j] : 0.0f}, pj[1], sj[1];
    const float loss = ce_row_group<MAXC, 1>(xj, lab[(int)row], N, scale, pj, sj);
    if (j < N) {
      probs[row * N + j] = pj[0];
      seed[row * N + j] = sj[0];
    }
    if (j == 0) rowloss[row] = loss;
  }
}

// loss[0] = the mean of rowloss as softmax_ce_mean_kernel forms it (thread t
// adds rows t, t + 256, ... in order, then ce_mean_tree)
__global__ void __launch_bounds__(256)
ce_mean_rows_kernel(const float *__restrict__ rowloss, float *__restrict__ loss, int rows) {
  __shared__ float part[256];
  float acc = 0.0f;
  for (int r = threadIdx.x; r < rows; r += 256) acc += rowloss[r];
  ce_mean_tree(acc, part, loss, rows);
}

// C = A * B + bias for a skinny B (N <= MAXN columns): one workgroup per
// row of A.  Thread t forms the N dot-product pieces over k = t, t + 256, ...
// (fused multiply-adds, in k order), the 256 pieces of each column are added
// in a fixed tree through LDS, and the row's epilogue follows in the same
// launch: relu / padded relu (R, P), or the softmax-CE of the row (CE:
// probabilities, seed, the row's loss).  For the classifier layer (N = 10),
// where a 64-wide MFMA tile would be 84 % padding and a split-K reduction a
// second launch; with K >= 16 the 16-row form below runs instead.
template <int MAXN, bool CE>
__global__ void __launch_bounds__(256)
gemm_rows_kernel(const float *__restrict__ A, const float *__restrict__ B,
                 const float *__restrict__ bias, float *__restrict__ C, float *__restrict__ R,
                 float *__restrict__ P, int N, int K, LabU8 lab, float *__restrict__ probs,
                 float *__restrict__ seed, float *__restrict__ rowloss, float scale) {
  __shared__ float part[MAXN][256];
  __shared__ float lv[MAXN];
  const int t = threadIdx.x;
  const long m = blockIdx.x;
  const float *__restrict__ a = A + m * K;
  float acc[MAXN];
#pragma unroll
  for (int n = 0; n < MAXN; n++) acc[n] = 0.0f;
#pragma unroll 4
  for (int k = t; k < K; k += 256) {
    const float av = a[k];
    const float *__restrict__ b = B + (long)k * N;
#pragma unroll
    for (int n = 0; n < MAXN; n++)
      if (n < N) acc[n] = fmaf(av, b[n], acc[n]);
  }
#pragma unroll
  for (int n = 0; n < MAXN; n++) part[n][t] = acc[n];
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) {
#pragma unroll
      for (int n = 0; n < MAXN; n++) part[n][t] += part[n][t + o];
    }
    __syncthreads();
  }
  if (t < N) {
    const float v = part[t][0] + bias[t];
    C[m * N + t] = v;
    const float o = v > 0.0f ? v : 0.0f;
    if (R) R[m * N + t] = o;
    if (P) {
      P[m * (N + 1) + t] = o;
      if (t == 0) P[m * (N + 1) + N] = 1.0f;
    }
    lv[t] = v;
  }
  if constexpr (CE) {
    __syncthreads();
    if (t == 0)
      rowloss[m] = ce_row<MAXN>(lv, lab[(int)m], probs + m * N, seed + m * N, N, scale);
  }
}

// The same on 16-row tiles, for K >= 16 (the kernel above takes the rest):
// one workgroup of eight waves per 16 rows, K split over the waves, each
// loading its whole slice (NCH 16-k chunks, 8 registers a chunk) before its
// 16x16x4 MFMAs, so a wave waits for one round trip; the wave sums are added
// in LDS in wave order, then the epilogue of gemm_rows_kernel for the tile's
// rows (the softmax-CE by 16 lanes a row).  Lane l (r = l % 16, q = l / 16)
// feeds A[m0 + r][k] and B[k][r] for k = kb + 4q + i in MFMA i of a chunk;
// loads past the matrix are clamped to it and their values zeroed.  VA:
// 16-byte loads of A's rows (aligned, K % 4 == 0).  MLP step 0.0472 ->
// 0.0463 ms against a workgroup per row.
typedef float f32x4r __attribute__((ext_vector_type(4)));
constexpr int R16W = 8;  // waves per workgroup (sixteen: no faster)
struct R16Da {
  float *dA, *d1, *d2;
};
constexpr int R16_DA_COLS = 64;  // columns of dA a workgroup
template <int NCH, bool VA, bool CE, bool DA = false>
__global__ void __launch_bounds__(64 * R16W)
gemm_rows16_kernel(const float *__restrict__ A, const float *__restrict__ B,
                   const float *__restrict__ bias, float *__restrict__ C, float *__restrict__ R,
                   float *__restrict__ P, int M, int N, int K, int kc, LabU8 lab,
                   float *__restrict__ probs, float *__restrict__ seed,
                   float *__restrict__ rowloss, float scale, R16Da da) {
  __shared__ float red[(R16W - 1) * 4 * 64];
  __shared__ float lv[16][17];
  __shared__ __attribute__((aligned(16))) float gsd[DA ? 16 * 16 : 4];
  __shared__ float bsd[16];
  __shared__ float wsd[DA ? R16_DA_COLS * 16 : 1];
  // dA epilogue: workgroup (tile, blockIdx.y) takes columns [ks0, ks0 +
  // R16_DA_COLS) of [B; bias] and of the tile's rows of A (every workgroup of
  // a tile repeats the tile's GEMM and softmax-CE, which cost little; only the
  // first writes them); lane t takes column ks0 + t % R16_DA_COLS for rows
  // 2 (t / R16_DA_COLS) and the next.  Loaded here, in flight with the GEMM's
  // operands (a load issued where its row is used costs a memory round trip
  // per row): the two A values (for the relu mask) and the slice's rows of B,
  // coalesced, for LDS (each lane then reads its column's N weights there).
  constexpr int DC = R16_DA_COLS;
  const int ks0 = blockIdx.y * DC;
  float ak[2], wv[DA ? (DC * 16 + 64 * R16W - 1) / (64 * R16W) : 1];
  if constexpr (DA) {
    const int rows = min(16, M - (int)blockIdx.x * 16);
    const int kk = min(ks0 + (int)(threadIdx.x % DC), K - 1), r2 = 2 * (threadIdx.x / DC);
#pragma unroll
    for (int u = 0; u < 2; u++)
      ak[u] = A[(long)(blockIdx.x * 16 + min(r2 + u, rows - 1)) * K + kk];
    const int nw = min(DC, K - ks0) * N;  // the slice's floats of B
#pragma unroll
    for (int u = 0; u < (DC * 16 + 64 * R16W - 1) / (64 * R16W); u++)
      wv[u] = B[(long)ks0 * N + min((int)threadIdx.x + 64 * R16W * u, nw - 1)];
  }
  // the epilogue's bias and label, loaded with the operands (a load issued
  // after the reduction is one more memory round trip before the stores)
  const float bnr = bias[min((int)(threadIdx.x & 15), N - 1)];
  const int ylab = CE ? lab[min((int)blockIdx.x * 16 + (int)(threadIdx.x >> 4), M - 1)] : 0;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int m0 = blockIdx.x * 16;
  const int mr = min(m0 + r, M - 1), nr = min(r, N - 1);
  const int k0 = w * kc, k1 = min(K, k0 + kc);
  const float *__restrict__ ap = A + (long)mr * K;
  const float *__restrict__ bp = B + nr;
  float av[NCH][4], bv[NCH][4];
#pragma unroll
  for (int c = 0; c < NCH; c++) {
    const int kq = k0 + 16 * c + 4 * q;
    if constexpr (VA) {
      const float4 v = *reinterpret_cast<const float4 *>(ap + min(kq, K - 4));
      av[c][0] = v.x; av[c][1] = v.y; av[c][2] = v.z; av[c][3] = v.w;
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++) av[c][i] = ap[min(kq + i, K - 1)];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) bv[c][i] = bp[(long)min(kq + i, K - 1) * N];
  }
  f32x4r acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < NCH; c++) {
    const int kq = k0 + 16 * c + 4 * q;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const bool in = kq + i < k1;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(in ? av[c][i] : 0.0f, in ? bv[c][i] : 0.0f, acc,
                                                 0, 0, 0);
    }
  }
  if (w > 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) red[((w - 1) * 4 + i) * 64 + lane] = acc[i];
  }
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int o = 0; o < R16W - 1; o++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc[i] += red[(o * 4 + i) * 64 + lane];
    const int n = r;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int m = m0 + 4 * q + i;
      if (m < M && n < N) {
        const float v = acc[i] + bnr;
        if (blockIdx.y == 0) {
          C[(long)m * N + n] = v;
          const float o = v > 0.0f ? v : 0.0f;
          if (R) R[(long)m * N + n] = o;
          if (P) {
            P[(long)m * (N + 1) + n] = o;
            if (n == N - 1) P[(long)m * (N + 1) + N] = 1.0f;
          }
        }
        lv[4 * q + i][n] = v;
      }
    }
    if (DA && q == 0 && n < N) bsd[n] = bnr;
  }
  if constexpr (CE) {
    // the tile's 16 rows, 16 lanes a row (ce_row_group: the bits of ce_row)
    __syncthreads();
    const int t = threadIdx.x, row = t >> 4, j = t & 15, m = m0 + row;
    if (t < 256 && m < M) {
      float xj[1] = {lv[row][j]}, pj[1], sj[1];
      const float loss = ce_row_group<16, 1>(xj, ylab, N, scale, pj, sj);
      if (blockIdx.y == 0) {
        if (j < N) {
          probs[(long)m * N + j] = pj[0];
          seed[(long)m * N + j] = sj[0];
        }
        if (j == 0) rowloss[m] = loss;
      }
      if constexpr (DA) gsd[row * 16 + j] = sj[0];
    }
    if constexpr (DA) {
      // the backward of the layer's input for the tile's rows from the seed
      // (the logits' gradient when the loss is the only consumer): dA =
      // seed * [B; bias]^T (M x (K + 1), the padones node's gradient), d1 =
      // dA without its last column, d2 = d1 where R > 0 (R = A, the relu
      // output), each sum over j ascending from +0 -- the classifier
      // backward kernel's (head.hip) dA, bit for bit
#pragma unroll
      for (int u = 0; u < (DC * 16 + 64 * R16W - 1) / (64 * R16W); u++) {
        const int i = threadIdx.x + 64 * R16W * u;
        if (i < DC * 16) wsd[i] = wv[u];
      }
      __syncthreads();
      const int K1 = K + 1, rows = min(16, M - m0);
      const int k = ks0 + (int)(threadIdx.x % DC), r2 = 2 * (threadIdx.x / DC);
      if (k < K && r2 < rows) {
        float wk[16];
#pragma unroll
        for (int jj = 0; jj < 16; jj++) wk[jj] = wsd[(k - ks0) * N + min(jj, N - 1)];
        // both rows' seeds read from LDS as 16-byte vectors (one wait, not
        // one a multiply-add)
        float4 gv[2][4];
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
          for (int v = 0; v < 4; v++)
            gv[u][v] = *reinterpret_cast<const float4 *>(gsd + (r2 + u) * 16 + 4 * v);
#pragma unroll
        for (int u = 0; u < 2; u++) {
          const float g[16] = {gv[u][0].x, gv[u][0].y, gv[u][0].z, gv[u][0].w,
                               gv[u][1].x, gv[u][1].y, gv[u][1].z, gv[u][1].w,
                               gv[u][2].x, gv[u][2].y, gv[u][2].z, gv[u][2].w,
                               gv[u][3].x, gv[u][3].y, gv[u][3].z, gv[u][3].w};
          float acc = 0.0f;
#pragma unroll
          for (int jj = 0; jj < 16; jj++)
            if (jj < N) acc = acc + g[jj] * wk[jj];
          if (r2 + u < rows) {
            const long mm = m0 + r2 + u;
            da.dA[mm * K1 + k] = acc;
            if (da.d1) da.d1[mm * K + k] = acc;
            if (da.d2) da.d2[mm * K + k] = ak[u] > 0.0f ? acc : 0.0f;
          }
        }
      }
      // the ones column of dA (the bias row of B): a lane a row, first slice
      if (blockIdx.y == 0 && (int)threadIdx.x < rows) {
        const float *g = gsd + threadIdx.x * 16;
        float acc = 0.0f;
        for (int jj = 0; jj < N; jj++) acc = acc + g[jj] * bsd[jj];
        da.dA[(long)(m0 + threadIdx.x) * K1 + K] = acc;
      }
    }
  }
}

extern "C" {

int tt_k_fill(float *x, long n, float v) { return run_map(n, a16(x), FillOp{x, v}); }
int tt_k_copy(float *d, const float *s, long n) { return run_map(n, a16(d) && a16(s), CopyOp{d, s}); }
int tt_k_add_inplace(float *d, const float *s, long n) {
  return run_map(n, a16(d) && a16(s), AddInplaceOp{d, s});
}
int tt_k_relu_fwd(const float *x, float *y, long n) { return run_map(n, a16(x) && a16(y), ReluFwdOp{x, y}); }
int tt_k_relu_bwd(const float *x, const float *g, float *dx, long n) {
  return run_map(n, a16(x) && a16(g) && a16(dx), ReluBwdOp{x, g, dx});
}
int tt_k_binary(const float *a, const float *b, float *y, long n, int op) {
  return run_map(n, a16(a) && a16(b) && a16(y), BinaryOp{a, b, y, op});
}
int tt_k_scalar(const float *a, float *y, long n, float s, int op) {
  return run_map(n, a16(a) && a16(y), ScalarOp{a, y, s, op});
}
int tt_k_matmul_naive(const float *A, const float *B, float *C, int M, int N, int K) {
  if (M < 0 || N < 0 || K < 0 || (M && N && (!A || !B || !C))) return -1;
  if (M == 0 || N == 0) return 0;
  const dim3 grid((unsigned)((N + 255) / 256), (unsigned)(M < 65535 ? M : 65535));
  hipLaunchKernelGGL(matmul_naive_kernel, grid, dim3(256), 0, stream(), A, B, C, M, N, K);
  return launched();
}
int ttk_add_outside(float *c, const float *cin, int M, int N, int mb, int nb) {
  if (M <= 0 || N <= 0) return 0;
  hipLaunchKernelGGL(add_outside_kernel, dim3(grid_for((long)M * N, 1)), dim3(256), 0, stream(),
                     c, cin, M, N, mb, nb);
  return launched();
}
int tt_k_sgd(float *w, const float *g, long n, float lr) {
  return run_map(n, a16(w) && a16(g), SgdOp{w, g, lr});
}

int tt_k_softmax_fwd(const float *x, float *y, long rows, int cols) {
  if (rows <= 0 || cols <= 0) return 0;
  if (cols <= 64) {
    hipLaunchKernelGGL(softmax_rowthread_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0,
                       stream(), x, y, rows, cols);
  } else {
    hipLaunchKernelGGL(softmax_rowwave_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                       stream(), x, y, rows, cols);
  }
  return launched();
}

int tt_k_softmax_bwd(const float *s, const float *g, float *dx, long rows, int cols) {
  if (rows <= 0 || cols <= 0) return 0;
  if (cols <= 64) {
    hipLaunchKernelGGL(softmax_bwd_rowthread_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256),
                       0, stream(), s, g, dx, rows, cols);
  } else {
    hipLaunchKernelGGL(softmax_bwd_rowwave_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                       stream(), s, g, dx, rows, cols);
  }
  return launched();
}

int tt_k_softmax_ce(const float *logits, const int32_t *labels, float *probs, float *loss_rows,
                    float *seed, long rows, int cols, float scale) {
  if (rows <= 0 || cols <= 0) return 0;
  hipLaunchKernelGGL(softmax_ce_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, stream(),
                     logits, labels, probs, loss_rows, seed, rows, cols, scale);
  return launched();
}

int tt_k_copy_padones_fwd(const float *x, float *c, float *y, long M, long K) {
  if (M <= 0 || K < 0) return 0;
  if (M >= 65536 || K >= (1L << 30) || !x || !c || !y) return -1;
  hipLaunchKernelGGL(copy_padones_rows_kernel, dim3((unsigned)((K + 1 + 1023) / 1024), (unsigned)M),
                     dim3(256), 0, stream(), x, c, y, (int)K);
  return launched();
}

int tt_k_relu_padones_fwd(const float *x, float *r, float *y, long M, long K) {
  if (M <= 0 || K < 0) return 0;
  if (M >= 65536 || K >= (1L << 30) || !x || !r || !y) return -1;
  hipLaunchKernelGGL(relu_padones_rows_kernel, dim3((unsigned)((K + 1 + 1023) / 1024), (unsigned)M),
                     dim3(256), 0, stream(), x, r, y, (int)K);
  return launched();
}

int tt_k_padones_bwd2(const float *g, float *d1, float *d2, long M, long K) {
  if (M <= 0 || K <= 0) return 0;
  if (M >= 65536 || K >= (1L << 30) || !g || !d1 || !d2) return -1;
  hipLaunchKernelGGL(padones_bwd2_rows_kernel, dim3((unsigned)((K + 1023) / 1024), (unsigned)M),
                     dim3(256), 0, stream(), g, d1, d2, (int)K);
  return launched();
}

int tt_k_padones_fwd(const float *x, float *y, long M, long K) {
  if (M <= 0 || K < 0) return 0;
  if (M < 65536 && K < (1L << 30)) {
    hipLaunchKernelGGL(padones_fwd_rows_kernel, dim3((unsigned)((K + 1 + 1023) / 1024), (unsigned)M), dim3(256), 0,
                       stream(), x, y, (int)K);
    return launched();
  }
  const long total = M * (K + 1);
  if (total < (1L << 31))
    hipLaunchKernelGGL(padones_fwd_kernel<unsigned>, dim3(grid_for(total, 1)), dim3(256), 0, stream(), x, y, M, K);
  else
    hipLaunchKernelGGL(padones_fwd_kernel<unsigned long>, dim3(grid_for(total, 1)), dim3(256), 0, stream(), x, y, M, K);
  return launched();
}

int tt_k_padones_relu_bwd(const float *g, const float *r, float *dr, float *dx, long M, long K) {
  if (M <= 0 || K <= 0) return 0;
  if (M >= 65536 || K >= (1L << 30)) return -1;
  hipLaunchKernelGGL(padones_relu_bwd_rows_kernel, dim3((unsigned)((K + 1023) / 1024), (unsigned)M),
                     dim3(256), 0, stream(), g, r, dr, dx, (int)K);
  return launched();
}

int tt_k_padones_bwd(const float *g, float *dx, long M, long K) {
  if (M <= 0 || K <= 0) return 0;
  if (M < 65536 && K < (1L << 30)) {
    hipLaunchKernelGGL(padones_bwd_rows_kernel, dim3((unsigned)((K + 1023) / 1024), (unsigned)M), dim3(256), 0,
                       stream(), g, dx, (int)K);
    return launched();
  }
  const long total = M * K;
  if (total < (1L << 31))
    hipLaunchKernelGGL(padones_bwd_kernel<unsigned>, dim3(grid_for(total, 1)), dim3(256), 0, stream(), g, dx, M, K);
  else
    hipLaunchKernelGGL(padones_bwd_kernel<unsigned long>, dim3(grid_for(total, 1)), dim3(256), 0, stream(), g, dx, M, K);
  return launched();
}

extern "C++" template <class LAB>
static void launch_ce_mean(const float *logits, const LAB &labels, float *probs, float *loss_mean,
                           float *seed, long rows, int cols, float scale) {
  if (cols <= 16)
    hipLaunchKernelGGL((softmax_ce_mean_kernel<16, LAB>), dim3(1), dim3(256), 0, stream(), logits,
                       labels, probs, loss_mean, seed, (int)rows, cols, scale);
  else if (cols <= 32)
    hipLaunchKernelGGL((softmax_ce_mean_kernel<32, LAB>), dim3(1), dim3(256), 0, stream(), logits,
                       labels, probs, loss_mean, seed, (int)rows, cols, scale);
  else
    hipLaunchKernelGGL((softmax_ce_mean_wide_kernel<LAB>), dim3(1), dim3(256), 0, stream(), logits,
                       labels, probs, loss_mean, seed, (int)rows, cols, scale);
}

// c[m][n] += bias[n]; r = relu(c), p = [r, 1] when given (a row per
// blockIdx.y, 1024 columns per blockIdx.x)
__global__ void bias_relu_pad_rows_kernel(float *__restrict__ c, const float *__restrict__ bias,
                                          float *__restrict__ r, float *__restrict__ p, int N) {
  const long m = blockIdx.y;
  float *cr = c + m * N;
  for (int k = blockIdx.x * 1024 + threadIdx.x; k <= N && k < (int)(blockIdx.x + 1) * 1024;
       k += 256) {
    if (k < N) {
      const float v = cr[k] + bias[k];
      cr[k] = v;
      const float o = v > 0.0f ? v : 0.0f;
      if (r) r[m * N + k] = o;
      if (p) p[m * (N + 1) + k] = o;
    } else if (p) {
      p[m * (N + 1) + N] = 1.0f;
    }
  }
}

extern "C" int ttk_bias_relu_pad(float *c, const float *bias, float *r, float *p, int M, int N) {
  if (M <= 0 || N <= 0) return 0;
  if (M >= 65536) return -1;
  hipLaunchKernelGGL(bias_relu_pad_rows_kernel, dim3((unsigned)((N + 1 + 1023) / 1024), (unsigned)M),
                     dim3(256), 0, stream(), c, bias, r, p, N);
  return launched();
}

extern "C" int ttk_gemm_rows(const float *A, const float *B, const float *bias, float *C,
                             float *R, float *P, int M, int N, int K, const TTCeHook *ce) {
  return ttk_gemm_rows_da(A, B, bias, C, R, P, M, N, K, ce, nullptr, nullptr, nullptr);
}

extern "C" int ttk_gemm_rows_da(const float *A, const float *B, const float *bias, float *C,
                                float *R, float *P, int M, int N, int K, const TTCeHook *ce,
                                float *dA, float *d1, float *d2) {
  if (dA && (!ce || K < 16 || K >= 64 * R16W || bias != B + (long)K * N || N > 16 ||
             (long)(K + 1) * N > 4096 || M <= 0 || M > TT_CE_ARG_ROWS || !ce->host_labels))
    return 1;
  // K <= 1024: four k a thread at most (at the CNN classifier's K = 4096
  // with 128 rows, one workgroup a row measured slower than split-K)
  if (M <= 0 || N <= 0 || N > 16 || K < 0 || K > 1024 || !bias || (ce && (M > TT_CE_ARG_ROWS ||
                                                             !ce->host_labels)))
    return 1;
  LabU8 lu;
  if (ce) lab_u8_fill(lu, ce->host_labels, M, N);
  if (K >= 16) {
    const int nch = (K + 16 * R16W - 1) / (16 * R16W);  // 16-k chunks a wave
    const int kc = 16 * nch;
    const bool va = ((uintptr_t)A & 15) == 0 && K % 4 == 0;
    const dim3 grid((unsigned)((M + 15) / 16));
    const dim3 grid_da((unsigned)((M + 15) / 16), (unsigned)((K + R16_DA_COLS - 1) / R16_DA_COLS));
#define TT_R16(NCH_, VA_)                                                                     \
  if (dA)                                                                                     \
    hipLaunchKernelGGL((gemm_rows16_kernel<NCH_, VA_, true, true>), grid_da, dim3(64 * R16W), 0, \
                       stream(), A, B, bias, C, R, P, M, N, K, kc, lu, ce->probs, ce->seed,   \
                       ce->rowloss, ce->scale, R16Da{dA, d1, d2});                            \
  else if (ce)                                                                                \
    hipLaunchKernelGGL((gemm_rows16_kernel<NCH_, VA_, true>), grid, dim3(64 * R16W), 0, stream(), A, \
                       B, bias, C, R, P, M, N, K, kc, lu, ce->probs, ce->seed, ce->rowloss,   \
                       ce->scale, R16Da{});                                                   \
  else                                                                                        \
    hipLaunchKernelGGL((gemm_rows16_kernel<NCH_, VA_, false>), grid, dim3(64 * R16W), 0, stream(),   \
                       A, B, bias, C, R, P, M, N, K, kc, lu, nullptr, nullptr, nullptr, 0.0f, \
                       R16Da{})
#define TT_R16V(NCH_) \
  if (va) { TT_R16(NCH_, true); } else { TT_R16(NCH_, false); }
    switch (nch) {
      case 1: TT_R16V(1); break;
      case 2: TT_R16V(2); break;
      case 3: case 4: TT_R16V(4); break;
      default: TT_R16V(8); break;
    }
#undef TT_R16V
#undef TT_R16
    return launched();
  }
  if (ce)
    hipLaunchKernelGGL((gemm_rows_kernel<16, true>), dim3((unsigned)M), dim3(256), 0, stream(), A,
                       B, bias, C, R, P, N, K, lu, ce->probs, ce->seed, ce->rowloss, ce->scale);
  else
    hipLaunchKernelGGL((gemm_rows_kernel<16, false>), dim3((unsigned)M), dim3(256), 0, stream(),
                       A, B, bias, C, R, P, N, K, lu, nullptr, nullptr, nullptr, 0.0f);
  return launched();
}

extern "C" int ttk_reduce_ce(const float *ws, float *C, int M, int N, int S, int zl,
                             const TTCeHook *h) {
  if (M <= 0 || N <= 0 || N > 32 || M > TT_CE_ARG_ROWS || N * zl > 1024 || !h->host_labels)
    return 1;
  LabU8 lu;
  lab_u8_fill(lu, h->host_labels, M, N);
  const int rpb = 1024 / (zl * N);
  const int XL = rpb * N;
  const size_t lds = sizeof(float) * (size_t)(zl * XL + XL);
  const dim3 grid((unsigned)((M + rpb - 1) / rpb));
#define TT_RCE(ZL_, MC_)                                                                    \
  hipLaunchKernelGGL((splitk_reduce_ce_kernel<ZL_, MC_>), grid, dim3(ZL_ * XL), lds, stream(), \
                     ws, C, M, N, S, rpb, h->bias, lu, h->probs, h->seed, h->rowloss, h->scale)
#define TT_RCE2(ZL_)                  \
  case ZL_:                           \
    if (N <= 16) TT_RCE(ZL_, 16);     \
    else TT_RCE(ZL_, 32);             \
    break;
  switch (zl) {
    TT_RCE2(1) TT_RCE2(2) TT_RCE2(4) TT_RCE2(8) TT_RCE2(16) TT_RCE2(32)
    default: return 1;
  }
#undef TT_RCE2
#undef TT_RCE
  return launched();
}

extern "C" int tt_k_ce_mean_rows(const float *rowloss, float *loss, int rows) {
  if (rows <= 0) return -1;
  hipLaunchKernelGGL(ce_mean_rows_kernel, dim3(1), dim3(256), 0, stream(), rowloss, loss, rows);
  return launched();
}

int tt_k_softmax_ce_mean(const float *logits, const int32_t *labels, float *probs, float *loss_mean,
                         float *seed, long rows, int cols, float scale) {
  if (rows <= 0 || cols <= 0 || rows > TT_CE_MEAN_MAX_ROWS) return -1;
  launch_ce_mean(logits, labels, probs, loss_mean, seed, rows, cols, scale);
  return launched();
}

int tt_k_softmax_ce_mean_hostlab(const float *logits, const int32_t *host_labels, float *probs,
                                 float *loss_mean, float *seed, long rows, int cols, float scale) {
  if (rows <= 0 || cols <= 0 || rows > TT_CE_ARG_ROWS || !host_labels) return -1;
  if (cols <= 255) {
    LabU8 lu;
    lab_u8_fill(lu, host_labels, rows, cols);
    launch_ce_mean(logits, lu, probs, loss_mean, seed, rows, cols, scale);
    return launched();
  }
  LabArg la;
  for (long r = 0; r < rows; r++) la.v[r] = host_labels[r];
  for (long r = rows; r < TT_CE_ARG_ROWS; r++) la.v[r] = 0;
  launch_ce_mean(logits, la, probs, loss_mean, seed, rows, cols, scale);
  return launched();
}

int tt_k_scale_by_dev(const float *x, const float *s, float *y, long n) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(scale_by_dev_kernel, dim3(grid_for(n, 1)), dim3(256), 0, stream(), x, s, y, n);
  return launched();
}

int tt_k_sgd_multi(float *const *w, const float *const *g, const long *n, int count, float lr) {
  if (count < 0 || count > TT_SGD_MAX) return -1;
  if (count == 0) return 0;
  SgdList L;
  long nmax = 0;
  for (int i = 0; i < count; i++) {
    L.w[i] = w[i];
    L.g[i] = g[i];
    L.n[i] = n[i];
    if (n[i] > nmax) nmax = n[i];
  }
  for (int i = count; i < TT_SGD_MAX; i++) { L.w[i] = nullptr; L.g[i] = nullptr; L.n[i] = 0; }
  if (nmax <= 0) return 0;
  hipLaunchKernelGGL(sgd_multi_kernel, dim3(grid_for(nmax, 1), count), dim3(256), 0, stream(), L, lr);
  return launched();
}

int tt_k_momentum_multi(float *const *w, const float *const *g, float *const *v, const long *n,
                        int count, float lr, float mu) {
  if (count < 0 || count > TT_SGD_MAX) return -1;
  if (count == 0) return 0;
  MomList L{};
  long nmax = 0;
  for (int i = 0; i < count; i++) {
    L.w[i] = w[i];
    L.g[i] = g[i];
    L.v[i] = v[i];
    L.n[i] = n[i];
    if (n[i] > nmax) nmax = n[i];
  }
  if (nmax <= 0) return 0;
  hipLaunchKernelGGL(momentum_multi_kernel, dim3(grid_for(nmax, 1), count), dim3(256), 0, stream(),
                     L, lr, mu);
  return launched();
}

int tt_k_adam_multi(float *const *w, const float *const *g, float *const *m, float *const *v,
                    const long *n, int count, float b1, float omb1, float b2, float omb2,
                    float eps, double lr_t) {
  if (count < 0 || count > TT_SGD_MAX) return -1;
  if (count == 0) return 0;
  AdamList L{};
  long nmax = 0;
  for (int i = 0; i < count; i++) {
    L.w[i] = w[i];
    L.g[i] = g[i];
    L.m[i] = m[i];
    L.v[i] = v[i];
    L.n[i] = n[i];
    if (n[i] > nmax) nmax = n[i];
  }
  if (nmax <= 0) return 0;
  hipLaunchKernelGGL(adam_multi_kernel, dim3(grid_for(nmax, 1), count), dim3(256), 0, stream(), L,
                     b1, omb1, b2, omb2, eps, lr_t);
  return launched();
}

int tt_k_gather_u8_norm(const uint8_t *src, long nsrc, long sample, long plane, int channels,
                        const int64_t *idx, long n, const float *mean, const float *stdv,
                        float *out) {
  if (n <= 0) return 0;
  if (!src || !idx || !out || !mean || !stdv || nsrc <= 0 || sample <= 0 || plane <= 0 ||
      channels < 1 || channels > 4 || plane * channels != sample)
    return -1;
  NormParams P{};
  for (int c = 0; c < channels; c++) {
    P.mean[c] = mean[c];
    P.stdv[c] = stdv[c];
  }
  const bool vec = sample % 4 == 0 && plane % 4 == 0 && a16(out);
  const long per = vec ? sample / 4 : sample;
  long gx = (per + 255) / 256;
  if (gx > 64) gx = 64;
  const long gy = n < 65535 ? n : 65535;
  if (vec)
    hipLaunchKernelGGL(gather_u8_norm_kernel<true>, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0,
                       stream(), src, sample, plane, idx, n, P, out);
  else
    hipLaunchKernelGGL(gather_u8_norm_kernel<false>, dim3((unsigned)gx, (unsigned)gy), dim3(256), 0,
                       stream(), src, sample, plane, idx, n, P, out);
  return launched();
}

}  // extern "C"
