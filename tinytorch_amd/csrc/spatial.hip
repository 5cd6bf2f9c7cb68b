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
#include <stdint.h>
#include "tt_rt.h"

namespace {

inline hipStream_t stream() { return (hipStream_t)ttrt_stream(); }
inline int launched() { return hipGetLastError() == hipSuccess ? 0 : -3; }

inline unsigned blocks_for(long n) {
  long b = (n + 255) / 256;
  if (b > 65535L * 16) b = 65535L * 16;
  return (unsigned)(b < 1 ? 1 : b);
}

// One thread per 4 consecutive column elements of one row c; consecutive
// threads walk consecutive p, so the col stores are 16-byte coalesced and the
// image reads are unit-stride along wo for stride-1 convolutions.  Index
// arithmetic runs in I (32-bit whenever the column matrix has < 2^31 entries).
template <typename I, bool VEC>
__global__ void im2col_kernel(const float *__restrict__ x, float *__restrict__ col, int N, int C,
                              int H, int W, int HH, int WW, int sh, int sw, int ph, int pw, int Ho,
                              int Wo) {
  const I HoWo = (I)Ho * Wo;
  const I Ncol = (I)N * HoWo;
  const I P4 = (Ncol + 3) / 4;
  const I total = (I)C * HH * WW * P4;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I c = i / P4;
    const I p0 = (i - c * P4) * 4;
    const int kw = (int)(c % WW), kh = (int)((c / WW) % HH), cim = (int)(c / ((I)HH * WW));
    I n = p0 / HoWo;
    I rem = p0 - n * HoWo;
    int ho = (int)(rem / Wo), wo = (int)(rem - (I)ho * Wo);
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      float t = 0.0f;
      if (p0 + j < Ncol) {
        const int hi = ho * sh - ph + kh, wi = wo * sw - pw + kw;
        if (hi >= 0 && hi < H && wi >= 0 && wi < W)
          t = x[(((long)n * C + cim) * H + hi) * (long)W + wi];
      }
      v[j] = t;
      if (++wo == Wo) { wo = 0; if (++ho == Ho) { ho = 0; ++n; } }
    }
    float *dst = col + (long)c * Ncol + p0;
    if (VEC) {
      *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (p0 + j < Ncol) dst[j] = v[j];
    }
  }
}

// One thread per image pixel (n, c, h, w); sums col[(c,kh,kw)][(n,ho,wo)]
// over the kernel taps that cover it, kh then kw ascending.
template <typename I>
__global__ void col2im_kernel(const float *__restrict__ col, float *__restrict__ x, int N, int C,
                              int H, int W, int HH, int WW, int sh, int sw, int ph, int pw, int Ho,
                              int Wo) {
  const long HoWo = (long)Ho * Wo;
  const long Ncol = (long)N * HoWo;
  const I total = (I)N * C * H * W;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I iw = i / W;
    const int w = (int)(i - iw * W);
    const I ih = iw / H;
    const int h = (int)(iw - ih * H);
    const I ic = ih / C;
    const int cim = (int)(ih - ic * C);
    const long n = (long)ic;
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

// db[f] = sum over (n, hw) of g[n][f][hw], in two deterministic stages:
// workgroup (f, s) sums images [s*per, (s+1)*per) of filter f with float4
// loads into part[f][s] (fixed per-thread order, wavefront butterflies, the
// four wave sums in order); then one thread per f adds its partials in order.
template <bool VEC>
__global__ void bias_grad_partial_kernel(const float *__restrict__ g, float *__restrict__ part,
                                         int N, int F, int HW, int per) {
  const int f = blockIdx.x, sidx = blockIdx.y;
  const int n0 = sidx * per, n1 = min(N, n0 + per);
  float s = 0.0f;
  if (VEC) {
    const int hw4 = HW / 4;
    const int cnt = (n1 - n0) * hw4;
    for (int i = threadIdx.x; i < cnt; i += blockDim.x) {
      const int n = n0 + i / hw4, q = i - (i / hw4) * hw4;
      const float4 v = reinterpret_cast<const float4 *>(g + ((long)n * F + f) * HW)[q];
      s += (v.x + v.y) + (v.z + v.w);
    }
  } else {
    const int cnt = (n1 - n0) * HW;
    for (int i = threadIdx.x; i < cnt; i += blockDim.x) {
      const int n = n0 + i / HW, q = i - (i / HW) * HW;
      s += g[((long)n * F + f) * HW + q];
    }
  }
  s = wave_sum(s);
  __shared__ float ws[4];
  if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) part[(long)f * gridDim.y + sidx] = ((ws[0] + ws[1]) + ws[2]) + ws[3];
}

__global__ void bias_grad_final_kernel(const float *__restrict__ part, float *__restrict__ db,
                                       int F, int S) {
  const int f = blockIdx.x * blockDim.x + threadIdx.x;
  if (f >= F) return;
  float s = 0.0f;
  for (int i = 0; i < S; i++) s += part[(long)f * S + i];
  db[f] = s;
}

// (n*C + c, ho, wo) of output index i, in index type I
#define TT_SPLIT_OUT(I_, i_, Ho_, Wo_, nc_, ho_, wo_)   \
  const I_ q1_ = (i_) / (I_)(Wo_);                     \
  const int wo_ = (int)((i_) - q1_ * (I_)(Wo_));       \
  const I_ nc_##i_ = q1_ / (I_)(Ho_);                  \
  const int ho_ = (int)(q1_ - nc_##i_ * (I_)(Ho_));    \
  const long nc_ = (long)nc_##i_;

template <typename I>
__global__ void maxpool_fwd_kernel(const float *__restrict__ x, float *__restrict__ y, int N, int C,
                                   int H, int W, int ph, int pw, int sh, int sw, int Ho, int Wo) {
  const I total = (I)N * C * Ho * Wo;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    TT_SPLIT_OUT(I, i, Ho, Wo, nc, ho, wo)
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
template <typename I>
__global__ void maxpool_bwd_gather_kernel(const float *__restrict__ x, const float *__restrict__ g,
                                          float *__restrict__ dx, int N, int C, int H, int W,
                                          int ph, int pw, int sh, int sw, int Ho, int Wo) {
  const I total = (I)N * C * H * W;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    TT_SPLIT_OUT(I, i, H, W, nc, h, w)
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
template <typename I>
__global__ void maxpool_bwd_tiled_kernel(const float *__restrict__ x, const float *__restrict__ g,
                                         float *__restrict__ dx, int N, int C, int H, int W, int ph,
                                         int pw, int Ho, int Wo) {
  const I total = (I)N * C * Ho * Wo;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    TT_SPLIT_OUT(I, i, Ho, Wo, nc, ho, wo)
    const long off = nc * H * (long)W + (long)(ho * ph) * W + wo * pw;
    const int am = window_argmax(x + off, W, ph, pw);
    const float gv = 0.0f + g[i];
    for (int kh = 0; kh < ph; kh++)
      for (int kw = 0; kw < pw; kw++) dx[off + (long)kh * W + kw] = (kh * pw + kw == am) ? gv : 0.0f;
  }
}

template <typename I>
__global__ void pool_uncovered_zero_kernel(float *__restrict__ dx, int N, int C, int H, int W,
                                           int hcov, int wcov) {
  const I total = (I)N * C * H * W;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    TT_SPLIT_OUT(I, i, H, W, nc, h, w)
    (void)nc;
    if (h >= hcov || w >= wcov) dx[i] = 0.0f;
  }
}

template <typename I>
__global__ void avgpool_fwd_kernel(const float *__restrict__ x, float *__restrict__ y, int N, int C,
                                   int H, int W, int ph, int pw, int sh, int sw, int Ho, int Wo,
                                   float norm) {
  const I total = (I)N * C * Ho * Wo;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    TT_SPLIT_OUT(I, i, Ho, Wo, nc, ho, wo)
    const float *xp = x + nc * H * (long)W + (long)(ho * sh) * W + wo * sw;
    float s = 0.0f;
    for (int kh = 0; kh < ph; kh++)
      for (int kw = 0; kw < pw; kw++) s += xp[(long)kh * W + kw];
    y[i] = s * norm;
  }
}

template <typename I>
__global__ void avgpool_bwd_kernel(const float *__restrict__ g, float *__restrict__ dx, int N, int C,
                                   int H, int W, int ph, int pw, int sh, int sw, int Ho, int Wo,
                                   float norm) {
  const I total = (I)N * C * H * W;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    TT_SPLIT_OUT(I, i, H, W, nc, h, w)
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

// Launch kernel template K<I> with I = unsigned when every index fits 32 bits.
#define TT_LAUNCH_I(K_, total_, ...)                                                          \
  do {                                                                                        \
    if ((total_) < (1L << 31))                                                                \
      hipLaunchKernelGGL(K_<unsigned>, dim3(blocks_for(total_)), dim3(256), 0, stream(),      \
                         __VA_ARGS__);                                                        \
    else                                                                                      \
      hipLaunchKernelGGL(K_<unsigned long>, dim3(blocks_for(total_)), dim3(256), 0, stream(), \
                         __VA_ARGS__);                                                        \
  } while (0)

extern "C" {

int tt_k_im2col(const float *x, float *col, int N, int C, int H, int W, int HH, int WW, int sh,
                int sw, int ph, int pw, int Ho, int Wo) {
  const long Ncol = (long)N * Ho * Wo;
  const long total = (long)C * HH * WW * ((Ncol + 3) / 4);
  if (total <= 0 || Ncol <= 0) return 0;
  const bool vec = (Ncol % 4 == 0) && (((uintptr_t)col & 15) == 0);
  const bool small = (long)C * HH * WW * Ncol < (1L << 31);
  const dim3 g(blocks_for(total)), b(256);
  if (small && vec)
    hipLaunchKernelGGL((im2col_kernel<unsigned, true>), g, b, 0, stream(), x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
  else if (small)
    hipLaunchKernelGGL((im2col_kernel<unsigned, false>), g, b, 0, stream(), x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
  else if (vec)
    hipLaunchKernelGGL((im2col_kernel<unsigned long, true>), g, b, 0, stream(), x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
  else
    hipLaunchKernelGGL((im2col_kernel<unsigned long, false>), g, b, 0, stream(), x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
  return launched();
}

int tt_k_col2im(const float *col, float *x, int N, int C, int H, int W, int HH, int WW, int sh,
                int sw, int ph, int pw, int Ho, int Wo) {
  const long total = (long)N * C * H * W;
  if (total <= 0) return 0;
  TT_LAUNCH_I(col2im_kernel, total, col, x, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
  return launched();
}

int tt_k_bias_grad(const float *g, float *db, int N, int F, int HW) {
  if (F <= 0) return 0;
  if (N <= 0 || HW <= 0) return tt_k_fill(db, F, 0.0f);
  // ~1024 workgroups in total, each summing at least 4096 floats
  int S = 1024 / F;
  if (S < 1) S = 1;
  const long per_img = HW;
  int per = (N + S - 1) / S;
  if ((long)per * per_img < 4096) per = (int)((4096 + per_img - 1) / per_img);
  if (per > N) per = N;
  S = (N + per - 1) / per;
  float *part = (float *)ttrt_alloc(sizeof(float) * (size_t)F * S);
  if (!part) return -2;
  const bool vec = (HW % 4 == 0) && (((uintptr_t)g & 15) == 0);
  if (vec)
    hipLaunchKernelGGL(bias_grad_partial_kernel<true>, dim3(F, S), dim3(256), 0, stream(), g, part, N, F, HW, per);
  else
    hipLaunchKernelGGL(bias_grad_partial_kernel<false>, dim3(F, S), dim3(256), 0, stream(), g, part, N, F, HW, per);
  hipLaunchKernelGGL(bias_grad_final_kernel, dim3((F + 255) / 256), dim3(256), 0, stream(), part, db, F, S);
  ttrt_free(part);
  return launched();
}

int tt_k_maxpool_fwd(const float *x, float *y, int N, int C, int H, int W, int ph, int pw, int sh,
                     int sw, int Ho, int Wo) {
  const long total = (long)N * C * Ho * Wo;
  if (total <= 0) return 0;
  TT_LAUNCH_I(maxpool_fwd_kernel, total, x, y, N, C, H, W, ph, pw, sh, sw, Ho, Wo);
  return launched();
}

int tt_k_maxpool_bwd(const float *x, const float *g, float *dx, int N, int C, int H, int W, int ph,
                     int pw, int sh, int sw, int Ho, int Wo) {
  const long total = (long)N * C * H * W;
  if (total <= 0) return 0;
  if (ph == sh && pw == sw) {
    const long nwin = (long)N * C * Ho * Wo;
    TT_LAUNCH_I(maxpool_bwd_tiled_kernel, nwin, x, g, dx, N, C, H, W, ph, pw, Ho, Wo);
    const int hcov = Ho * ph, wcov = Wo * pw;
    if (hcov < H || wcov < W)
      TT_LAUNCH_I(pool_uncovered_zero_kernel, total, dx, N, C, H, W, hcov, wcov);
  } else {
    TT_LAUNCH_I(maxpool_bwd_gather_kernel, total, x, g, dx, N, C, H, W, ph, pw, sh, sw, Ho, Wo);
  }
  return launched();
}

int tt_k_avgpool_fwd(const float *x, float *y, int N, int C, int H, int W, int ph, int pw, int sh,
                     int sw, int Ho, int Wo) {
  const long total = (long)N * C * Ho * Wo;
  if (total <= 0) return 0;
  const float norm = 1.0f / (float)(ph * pw);
  TT_LAUNCH_I(avgpool_fwd_kernel, total, x, y, N, C, H, W, ph, pw, sh, sw, Ho, Wo, norm);
  return launched();
}

int tt_k_avgpool_bwd(const float *g, float *dx, int N, int C, int H, int W, int ph, int pw, int sh,
                     int sw, int Ho, int Wo) {
  const long total = (long)N * C * H * W;
  if (total <= 0) return 0;
  const float norm = 1.0f / (float)(ph * pw);
  TT_LAUNCH_I(avgpool_bwd_kernel, total, g, dx, N, C, H, W, ph, pw, sh, sw, Ho, Wo, norm);
  return launched();
}

}  // extern "C"
