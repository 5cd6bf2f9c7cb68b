// Spatial kernels for the im2col convolution and the 2-D pools (HBM roofline).
//
//   im2col          reference src/ops_spatial.c:37-69 (and src/autograd.c:371-404)
//   col2im          reference src/autograd.c:406-434
//   conv bias grad  reference src/autograd.c:467-482
//   maxpool fwd/bwd reference src/ops_spatial.c:129-164, src/autograd.c:555-594
//   avgpool fwd/bwd reference src/ops_spatial.c:166-201, src/autograd.c:596-628
//
// Layouts: images NCHW; the column matrix is (C*HH*WW) x (N*Ho*Wo) with row
// c = (c_im*HH + kh)*WW + kw and column p = (n*Ho + ho)*Wo + wo.
//
// Bit-exactness: col2im and the pool backward passes are written as gathers
// (one thread per input pixel) that visit contributions in exactly the order
// the reference scatters them -- ascending (kh, kw) for col2im, ascending
// (ho, wo) for the pools -- starting from +0.0f, so every sum rounds the same
// way with no atomics.  This file is compiled with -ffp-contract=off so that
// no multiply-add is fused.
#include <hip/hip_runtime.h>
#include <math.h>
#include "tt_rt.h"

namespace {

inline hipStream_t stream() { return (hipStream_t)ttrt_stream(); }
inline int launched() { return hipGetLastError() == hipSuccess ? 0 : -3; }

inline unsigned blocks_for(long n) {
  long b = (n + 255) / 256;
  if (b > 65535L * 16) b = 65535L * 16;
  return (unsigned)(b < 1 ? 1 : b);
}

// One thread per column element; consecutive threads walk consecutive p, so
// the col writes are fully coalesced and the image reads are unit-stride
// along wo for stride-1 convolutions.
__global__ void im2col_kernel(const float *__restrict__ x, float *__restrict__ col, int N, int C,
                              int H, int W, int HH, int WW, int sh, int sw, int ph, int pw, int Ho,
                              int Wo) {
  const long HoWo = (long)Ho * Wo;
  const long Ncol = (long)N * HoWo;
  const long total = (long)C * HH * WW * Ncol;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const long c = i / Ncol, p = i - c * Ncol;
    const int kw = (int)(c % WW), kh = (int)((c / WW) % HH), cim = (int)(c / ((long)HH * WW));
    const long n = p / HoWo;
    const int rem = (int)(p - n * HoWo);
    const int ho = rem / Wo, wo = rem - ho * Wo;
    const int hi = ho * sh - ph + kh, wi = wo * sw - pw + kw;
    float v = 0.0f;
    if (hi >= 0 && hi < H && wi >= 0 && wi < W) v = x[((n * C + cim) * H + hi) * (long)W + wi];
    col[i] = v;
  }
}

// One thread per image pixel (n, c, h, w); sums col[(c,kh,kw)][(n,ho,wo)]
// over the kernel taps that cover it, kh then kw ascending.
__global__ void col2im_kernel(const float *__restrict__ col, float *__restrict__ x, int N, int C,
                              int H, int W, int HH, int WW, int sh, int sw, int ph, int pw, int Ho,
                              int Wo) {
  const long HoWo = (long)Ho * Wo;
  const long Ncol = (long)N * HoWo;
  const long total = (long)N * C * H * W;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int w = (int)(i % W);
    const int h = (int)((i / W) % H);
    const int cim = (int)((i / ((long)W * H)) % C);
    const long n = i / ((long)W * H * C);
    float acc = 0.0f;
    for (int kh = 0; kh < HH; kh++) {
      const int t = h + ph - kh;
      if (t < 0 || t % sh) continue;
      const int ho = t / sh;
      if (ho >= Ho) continue;
      for (int kw = 0; kw < WW; kw++) {
        const int u = w + pw - kw;
        if (u < 0 || u % sw) continue;
        const int wo = u / sw;
        if (wo >= Wo) continue;
        const long c = ((long)cim * HH + kh) * WW + kw;
        acc += col[c * Ncol + n * HoWo + (long)ho * Wo + wo];
      }
    }
    x[i] = acc;
  }
}

__device__ __forceinline__ float wave_sum(float v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// db[f] = sum over (n, hw) of g[n][f][hw]: one workgroup per f, fixed
// per-thread strided partial sums, wavefront butterflies, then the 4 wave
// partials in order -- deterministic for a given shape.
__global__ void bias_grad_kernel(const float *__restrict__ g, float *__restrict__ db, int N, int F,
                                 int HW) {
  const int f = blockIdx.x;
  const long total = (long)N * HW;
  float s = 0.0f;
  for (long i = threadIdx.x; i < total; i += blockDim.x) {
    const long n = i / HW, hw = i - n * HW;
    s += g[(n * F + f) * HW + hw];
  }
  s = wave_sum(s);
  __shared__ float part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) db[f] = ((part[0] + part[1]) + part[2]) + part[3];
}

__global__ void maxpool_fwd_kernel(const float *__restrict__ x, float *__restrict__ y, int N, int C,
                                   int H, int W, int ph, int pw, int sh, int sw, int Ho, int Wo) {
  const long total = (long)N * C * Ho * Wo;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int wo = (int)(i % Wo);
    const int ho = (int)((i / Wo) % Ho);
    const long nc = i / ((long)Wo * Ho);
    const float *xp = x + nc * H * (long)W + (long)(ho * sh) * W + wo * sw;
    float m = -INFINITY;
    for (int kh = 0; kh < ph; kh++)
      for (int kw = 0; kw < pw; kw++) {
        const float v = xp[(long)kh * W + kw];
        if (v > m) m = v;  // strict: NaN never wins, ties keep the first
      }
    y[i] = m;
  }
}

// Position (kh*pw + kw) of the first strict maximum of a window; 0 (the
// top-left) when nothing beats -inf (all -inf or NaN).
__device__ __forceinline__ int window_argmax(const float *xp, int W, int ph, int pw) {
  float m = -INFINITY;
  int am = 0;
  for (int kh = 0; kh < ph; kh++)
    for (int kw = 0; kw < pw; kw++) {
      const float v = xp[(long)kh * W + kw];
      if (v > m) { m = v; am = kh * pw + kw; }
    }
  return am;
}

// General maxpool backward: gather per input pixel over the windows that
// contain it, ho then wo ascending.
__global__ void maxpool_bwd_gather_kernel(const float *__restrict__ x, const float *__restrict__ g,
                                          float *__restrict__ dx, int N, int C, int H, int W,
                                          int ph, int pw, int sh, int sw, int Ho, int Wo) {
  const long total = (long)N * C * H * W;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int w = (int)(i % W);
    const int h = (int)((i / W) % H);
    const long nc = i / ((long)W * H);
    const float *xc = x + nc * H * (long)W;
    const float *gc = g + nc * Ho * (long)Wo;
    // windows ho with ho*sh <= h < ho*sh + ph
    int ho_lo = h - ph + 1 <= 0 ? 0 : (h - ph + 1 + sh - 1) / sh;
    int ho_hi = h / sh; if (ho_hi > Ho - 1) ho_hi = Ho - 1;
    int wo_lo = w - pw + 1 <= 0 ? 0 : (w - pw + 1 + sw - 1) / sw;
    int wo_hi = w / sw; if (wo_hi > Wo - 1) wo_hi = Wo - 1;
    float acc = 0.0f;
    for (int ho = ho_lo; ho <= ho_hi; ho++)
      for (int wo = wo_lo; wo <= wo_hi; wo++) {
        const int am = window_argmax(xc + (long)(ho * sh) * W + wo * sw, W, ph, pw);
        if (ho * sh + am / pw == h && wo * sw + am % pw == w) acc += gc[(long)ho * Wo + wo];
      }
    dx[i] = acc;
  }
}

// Non-overlapping maxpool backward (pool == stride): each thread owns one
// window and writes all of its pixels (the argmax gets 0.0f + g, the rest
// +0.0f); a second pass zeroes rows/cols no window covers.
__global__ void maxpool_bwd_tiled_kernel(const float *__restrict__ x, const float *__restrict__ g,
                                         float *__restrict__ dx, int N, int C, int H, int W, int ph,
                                         int pw, int Ho, int Wo) {
  const long total = (long)N * C * Ho * Wo;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int wo = (int)(i % Wo);
    const int ho = (int)((i / Wo) % Ho);
    const long nc = i / ((long)Wo * Ho);
    const long off = nc * H * (long)W + (long)(ho * ph) * W + wo * pw;
    const int am = window_argmax(x + off, W, ph, pw);
    const float gv = 0.0f + g[i];
    for (int kh = 0; kh < ph; kh++)
      for (int kw = 0; kw < pw; kw++) dx[off + (long)kh * W + kw] = (kh * pw + kw == am) ? gv : 0.0f;
  }
}

__global__ void pool_uncovered_zero_kernel(float *__restrict__ dx, int N, int C, int H, int W,
                                           int hcov, int wcov) {
  const long total = (long)N * C * H * W;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int w = (int)(i % W);
    const int h = (int)((i / W) % H);
    if (h >= hcov || w >= wcov) dx[i] = 0.0f;
  }
}

__global__ void avgpool_fwd_kernel(const float *__restrict__ x, float *__restrict__ y, int N, int C,
                                   int H, int W, int ph, int pw, int sh, int sw, int Ho, int Wo,
                                   float norm) {
  const long total = (long)N * C * Ho * Wo;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int wo = (int)(i % Wo);
    const int ho = (int)((i / Wo) % Ho);
    const long nc = i / ((long)Wo * Ho);
    const float *xp = x + nc * H * (long)W + (long)(ho * sh) * W + wo * sw;
    float s = 0.0f;
    for (int kh = 0; kh < ph; kh++)
      for (int kw = 0; kw < pw; kw++) s += xp[(long)kh * W + kw];
    y[i] = s * norm;
  }
}

__global__ void avgpool_bwd_kernel(const float *__restrict__ g, float *__restrict__ dx, int N, int C,
                                   int H, int W, int ph, int pw, int sh, int sw, int Ho, int Wo,
                                   float norm) {
  const long total = (long)N * C * H * W;
  const long stride = (long)gridDim.x * blockDim.x;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int w = (int)(i % W);
    const int h = (int)((i / W) % H);
    const long nc = i / ((long)W * H);
    const float *gc = g + nc * Ho * (long)Wo;
    int ho_lo = h - ph + 1 <= 0 ? 0 : (h - ph + 1 + sh - 1) / sh;
    int ho_hi = h / sh; if (ho_hi > Ho - 1) ho_hi = Ho - 1;
    int wo_lo = w - pw + 1 <= 0 ? 0 : (w - pw + 1 + sw - 1) / sw;
    int wo_hi = w / sw; if (wo_hi > Wo - 1) wo_hi = Wo - 1;
    float acc = 0.0f;
    for (int ho = ho_lo; ho <= ho_hi; ho++)
      for (int wo = wo_lo; wo <= wo_hi; wo++) {
        const float gv = gc[(long)ho * Wo + wo] * norm;
        acc += gv;
      }
    dx[i] = acc;
  }
}

}  // namespace

extern "C" {

int tt_k_im2col(const float *x, float *col, int N, int C, int H, int W, int HH, int WW, int sh,
                int sw, int ph, int pw, int Ho, int Wo) {
  const long total = (long)C * HH * WW * N * Ho * Wo;
  if (total <= 0) return 0;
  hipLaunchKernelGGL(im2col_kernel, dim3(blocks_for(total)), dim3(256), 0, stream(), x, col, N, C, H,
                     W, HH, WW, sh, sw, ph, pw, Ho, Wo);
  return launched();
}

int tt_k_col2im(const float *col, float *x, int N, int C, int H, int W, int HH, int WW, int sh,
                int sw, int ph, int pw, int Ho, int Wo) {
  const long total = (long)N * C * H * W;
  if (total <= 0) return 0;
  hipLaunchKernelGGL(col2im_kernel, dim3(blocks_for(total)), dim3(256), 0, stream(), col, x, N, C, H,
                     W, HH, WW, sh, sw, ph, pw, Ho, Wo);
  return launched();
}

int tt_k_bias_grad(const float *g, float *db, int N, int F, int HW) {
  if (F <= 0) return 0;
  hipLaunchKernelGGL(bias_grad_kernel, dim3(F), dim3(256), 0, stream(), g, db, N, F, HW);
  return launched();
}

int tt_k_maxpool_fwd(const float *x, float *y, int N, int C, int H, int W, int ph, int pw, int sh,
                     int sw, int Ho, int Wo) {
  const long total = (long)N * C * Ho * Wo;
  if (total <= 0) return 0;
  hipLaunchKernelGGL(maxpool_fwd_kernel, dim3(blocks_for(total)), dim3(256), 0, stream(), x, y, N, C,
                     H, W, ph, pw, sh, sw, Ho, Wo);
  return launched();
}

int tt_k_maxpool_bwd(const float *x, const float *g, float *dx, int N, int C, int H, int W, int ph,
                     int pw, int sh, int sw, int Ho, int Wo) {
  const long total = (long)N * C * H * W;
  if (total <= 0) return 0;
  if (ph == sh && pw == sw) {
    const long nwin = (long)N * C * Ho * Wo;
    hipLaunchKernelGGL(maxpool_bwd_tiled_kernel, dim3(blocks_for(nwin)), dim3(256), 0, stream(), x, g,
                       dx, N, C, H, W, ph, pw, Ho, Wo);
    const int hcov = Ho * ph, wcov = Wo * pw;
    if (hcov < H || wcov < W)
      hipLaunchKernelGGL(pool_uncovered_zero_kernel, dim3(blocks_for(total)), dim3(256), 0, stream(),
                         dx, N, C, H, W, hcov, wcov);
  } else {
    hipLaunchKernelGGL(maxpool_bwd_gather_kernel, dim3(blocks_for(total)), dim3(256), 0, stream(), x,
                       g, dx, N, C, H, W, ph, pw, sh, sw, Ho, Wo);
  }
  return launched();
}

int tt_k_avgpool_fwd(const float *x, float *y, int N, int C, int H, int W, int ph, int pw, int sh,
                     int sw, int Ho, int Wo) {
  const long total = (long)N * C * Ho * Wo;
  if (total <= 0) return 0;
  const float norm = 1.0f / (float)(ph * pw);
  hipLaunchKernelGGL(avgpool_fwd_kernel, dim3(blocks_for(total)), dim3(256), 0, stream(), x, y, N, C,
                     H, W, ph, pw, sh, sw, Ho, Wo, norm);
  return launched();
}

int tt_k_avgpool_bwd(const float *g, float *dx, int N, int C, int H, int W, int ph, int pw, int sh,
                     int sw, int Ho, int Wo) {
  const long total = (long)N * C * H * W;
  if (total <= 0) return 0;
  const float norm = 1.0f / (float)(ph * pw);
  hipLaunchKernelGGL(avgpool_bwd_kernel, dim3(blocks_for(total)), dim3(256), 0, stream(), g, dx, N, C,
                     H, W, ph, pw, sh, sw, Ho, Wo, norm);
  return launched();
}

}  // extern "C"
