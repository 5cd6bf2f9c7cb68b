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

// col2im, one pixel (n, ci, h, w) per lane with consecutive lanes on
// consecutive pixels, so every tap's reads are contiguous across the wave.
// The taps are summed kh then kw ascending from +0.0f, the reference's
// scatter order, with no atomics.  S1 specialises stride 1 (no division per
// tap); I is the index type.
template <typename I, bool S1>
__global__ void __launch_bounds__(256)
col2im_px_kernel(const float *__restrict__ col, float *__restrict__ x, int N, int C, int H, int W,
                 int HH, int WW, int sh, int sw, int ph, int pw, int Ho, int Wo) {
  const I total = (I)N * C * H * W;
  const long HoWo = (long)Ho * Wo, Ncol = (long)N * HoWo;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I q = i / (I)W;
    const int w = (int)(i - q * (I)W);
    const I plane = q / (I)H;
    const int h = (int)(q - plane * (I)H);
    const I n = plane / (I)C;
    const int ci = (int)(plane - n * (I)C);
    const float *cb = col + (long)n * HoWo + (long)ci * HH * WW * Ncol;
    float acc = 0.0f;
    for (int kh = 0; kh < HH; kh++) {
      int ho = h + ph - kh;
      if constexpr (S1) {
        if (ho < 0 || ho >= Ho) continue;
      } else {
        if (ho < 0 || ho % sh) continue;
        ho /= sh;
        if (ho >= Ho) continue;
      }
      for (int kw = 0; kw < WW; kw++) {
        int wo = w + pw - kw;
        if constexpr (S1) {
          if (wo < 0 || wo >= Wo) continue;
        } else {
          if (wo < 0 || wo % sw) continue;
          wo /= sw;
          if (wo >= Wo) continue;
        }
        acc += cb[(long)(kh * WW + kw) * Ncol + (long)ho * Wo + wo];
      }
    }
    x[i] = acc;
  }
}

// col2im staged through LDS, one workgroup per (image n, channel ci) plane:
// the plane's taps*Ho*Wo column entries (row c = ci*taps + t, columns
// n*Ho*Wo ..) are read once with 16-byte loads, then each lane gathers its
// pixels from LDS in the same order as col2im_px_kernel (kh then kw
// ascending from +0.0f), so the two are bit-identical.  VEC: a lane owns 4
// consecutive pixels of a row (W % 4 == 0) and stores them with one 16-byte
// store.  Requires Ho*Wo % 4 == 0 and a 16-byte aligned column matrix.
template <bool S1, bool VEC>
__global__ void __launch_bounds__(256)
col2im_lds_kernel(const float *__restrict__ col, float *__restrict__ x, int N, int C, int H, int W,
                  int HH, int WW, int sh, int sw, int ph, int pw, int Ho, int Wo) {
  extern __shared__ float cs[];
  const int n = blockIdx.x / C, ci = blockIdx.x - n * C;
  const int HoWo = Ho * Wo, taps = HH * WW;
  const long Ncol = (long)N * HoWo;
  const float *src = col + (long)ci * taps * Ncol + (long)n * HoWo;
  const int q4 = HoWo / 4;
  for (int i = threadIdx.x; i < taps * q4; i += 256) {
    const int t = i / q4, q = i - t * q4;
    *reinterpret_cast<float4 *>(cs + t * HoWo + 4 * q) =
        *reinterpret_cast<const float4 *>(src + (long)t * Ncol + 4 * q);
  }
  __syncthreads();
  float *dst = x + (long)blockIdx.x * H * W;
  constexpr int PX = VEC ? 4 : 1;
  for (int i = threadIdx.x * PX; i < H * W; i += 256 * PX) {
    const int h = i / W, w0 = i - h * W;
    float acc[PX];
#pragma unroll
    for (int j = 0; j < PX; j++) acc[j] = 0.0f;
    for (int kh = 0; kh < HH; kh++) {
      int ho = h + ph - kh;
      if constexpr (S1) {
        if (ho < 0 || ho >= Ho) continue;
      } else {
        if (ho < 0 || ho % sh) continue;
        ho /= sh;
        if (ho >= Ho) continue;
      }
      const float *rowp = cs + kh * WW * HoWo + ho * Wo;
      for (int kw = 0; kw < WW; kw++) {
#pragma unroll
        for (int j = 0; j < PX; j++) {
          int wo = w0 + j + pw - kw;
          if constexpr (S1) {
            if (wo < 0 || wo >= Wo) continue;
          } else {
            if (wo < 0 || wo % sw) continue;
            wo /= sw;
            if (wo >= Wo) continue;
          }
          acc[j] += rowp[kw * HoWo + wo];
        }
      }
    }
    if constexpr (VEC)
      *reinterpret_cast<float4 *>(dst + i) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    else
      dst[i] = acc[0];
  }
}

// im2col with one workgroup per (kernel tap c, 1024 consecutive columns p):
// row c of the column matrix is contiguous in p, each lane writes 4 columns
// with one 16-byte store, c comes from the grid and a lane divides only by
// Ho*Wo and Wo.  Requires Ncol % 4 == 0.
__global__ void __launch_bounds__(256)
im2col_rows_kernel(const float *__restrict__ x, float *__restrict__ col, int N, int C, int H,
                   int W, int HH, int WW, int sh, int sw, int ph, int pw, int Ho, int Wo) {
  const int c = blockIdx.y;
  const int kw = c % WW, kh = (c / WW) % HH, ci = c / (HH * WW);
  const unsigned HoWo = (unsigned)(Ho * Wo);
  const unsigned Ncol = (unsigned)N * HoWo;
  const unsigned p0 = (blockIdx.x * 256u + threadIdx.x) * 4u;
  if (p0 >= Ncol) return;
  unsigned n = p0 / HoWo;
  const unsigned rem = p0 - n * HoWo;
  int ho = (int)(rem / (unsigned)Wo), wo = (int)(rem - (unsigned)ho * Wo);
  float v[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int hi = ho * sh - ph + kh, wi = wo * sw - pw + kw;
    v[j] = (hi >= 0 && hi < H && wi >= 0 && wi < W)
               ? x[(((long)n * C + ci) * H + hi) * (long)W + wi] : 0.0f;
    if (++wo == Wo) { wo = 0; if (++ho == Ho) { ho = 0; ++n; } }
  }
  *reinterpret_cast<float4 *>(col + (long)c * Ncol + p0) = make_float4(v[0], v[1], v[2], v[3]);
}

// im2col staged through LDS: one workgroup per (image n, channel ci) plane
// reads the H x W plane once (16-byte loads), then writes the HH*WW column
// rows it feeds, c = ci*HH*WW + kh*WW + kw, from LDS with 16-byte stores.
// A lane owns the same 4 consecutive outputs (ho, wo..wo+3) of every tap.
// Requires Wo % 4 == 0 (outputs of a lane stay in one row, stores aligned).
// With ones_row, the channel-0 workgroup of image n also writes image n's
// part of the extra (C*HH*WW)-th row of ones.
__global__ void __launch_bounds__(256)
im2col_lds_kernel(const float *__restrict__ x, float *__restrict__ col, int N, int C, int H,
                  int W, int HH, int WW, int sh, int sw, int ph, int pw, int Ho, int Wo,
                  int ones_row) {
  extern __shared__ float plane[];
  const int n = blockIdx.x / C, ci = blockIdx.x - (blockIdx.x / C) * C;
  const int HWi = H * W;
  const float *src = x + (long)blockIdx.x * HWi;
  if ((W & 3) == 0 && (((uintptr_t)src & 15) == 0)) {
    for (int i = threadIdx.x * 4; i < HWi; i += 1024)
      *reinterpret_cast<float4 *>(plane + i) = *reinterpret_cast<const float4 *>(src + i);
  } else {
    for (int i = threadIdx.x; i < HWi; i += 256) plane[i] = src[i];
  }
  __syncthreads();
  const int HoWo = Ho * Wo;
  const long Ncol = (long)N * HoWo;
  const int taps = HH * WW;
  float *dst0 = col + (long)ci * taps * Ncol + (long)n * HoWo;
  for (int o = threadIdx.x * 4; o < HoWo; o += 1024) {
    const int ho = o / Wo, wo = o - (o / Wo) * Wo;
    for (int kh = 0; kh < HH; kh++) {
      const int hi = ho * sh - ph + kh;
      const bool hok = hi >= 0 && hi < H;
      for (int kw = 0; kw < WW; kw++) {
        float v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int wi = (wo + j) * sw - pw + kw;
          v[j] = (hok && wi >= 0 && wi < W) ? plane[hi * W + wi] : 0.0f;
        }
        *reinterpret_cast<float4 *>(dst0 + (long)(kh * WW + kw) * Ncol + o) =
            make_float4(v[0], v[1], v[2], v[3]);
      }
    }
    if (ones_row && ci == 0)
      *reinterpret_cast<float4 *>(col + (long)C * taps * Ncol + (long)n * HoWo + o) =
          make_float4(1.0f, 1.0f, 1.0f, 1.0f);
  }
}

// 2x2 / stride-2 max pool, two outputs per lane: two 16-byte loads (rows 2ho
// and 2ho+1, columns 4q..4q+3) and one 8-byte store.  Requires W % 4 == 0.
template <typename I>
__global__ void maxpool2x2_fwd_kernel(const float *__restrict__ x, float *__restrict__ y, int H,
                                      int W, int Ho, int Wo, I total) {
  const int Wq = Wo / 2;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I r = i / Wq;  // (nc, ho) row index
    const int q = (int)(i - r * Wq);
    const I nc = r / Ho;
    const int ho = (int)(r - nc * Ho);
    const float *xp = x + ((long)nc * H + 2 * ho) * W + 4 * q;
    const float4 a = *reinterpret_cast<const float4 *>(xp);
    const float4 b = *reinterpret_cast<const float4 *>(xp + W);
    float m0 = -INFINITY, m1 = -INFINITY;
    if (a.x > m0) m0 = a.x; if (a.y > m0) m0 = a.y; if (b.x > m0) m0 = b.x; if (b.y > m0) m0 = b.y;
    if (a.z > m1) m1 = a.z; if (a.w > m1) m1 = a.w; if (b.z > m1) m1 = b.z; if (b.w > m1) m1 = b.w;
    *reinterpret_cast<float2 *>(y + (long)r * Wo + 2 * q) = make_float2(m0, m1);
  }
}

// matching backward: recompute each window's first strict maximum, write
// 0.0f + g there and +0.0f elsewhere (rows below 2*Ho are zeroed separately)
__device__ __forceinline__ void argmax4(float v0, float v1, float v2, float v3, int &am) {
  float m = -INFINITY;
  am = 0;
  if (v0 > m) { m = v0; am = 0; }
  if (v1 > m) { m = v1; am = 1; }
  if (v2 > m) { m = v2; am = 2; }
  if (v3 > m) { m = v3; am = 3; }
}

// dxr of the 2x2 pool + relu backward from the windows' codes (bits 0-1 the
// argmax, bits 2-5 the relu mask; pool_code in conv.hip): a thread takes two
// windows, as maxpool2x2_bwd_kernel, and writes the same values -- the
// incoming gradient (+0 added, as there) where the argmax is and the relu
// value is > 0, +0 elsewhere.
template <typename I>
__global__ void maxpool2x2_code_bwd_kernel(const unsigned char *__restrict__ codes,
                                           const float *__restrict__ g, float *__restrict__ dxr,
                                           int H, int W, int Ho, int Wo, I total) {
  const int Wq = Wo / 2;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I r = i / Wq;
    const int q = (int)(i - r * Wq);
    const I nc = r / Ho;
    const int ho = (int)(r - nc * Ho);
    const long off = ((long)nc * H + 2 * ho) * W + 4 * q;
    const unsigned c2 = *reinterpret_cast<const unsigned short *>(codes + (long)r * Wo + 2 * q);
    const float2 gv = *reinterpret_cast<const float2 *>(g + (long)r * Wo + 2 * q);
    const float g0 = 0.0f + gv.x, g1 = 0.0f + gv.y;
    const unsigned c0 = c2 & 0xff, c1 = c2 >> 8;
    auto at = [](unsigned c, unsigned k, float v) {
      return ((c & 3) == k && ((c >> (2 + k)) & 1)) ? v : 0.0f;
    };
    *reinterpret_cast<float4 *>(dxr + off) = make_float4(at(c0, 0, g0), at(c0, 1, g0), at(c1, 0, g1), at(c1, 1, g1));
    *reinterpret_cast<float4 *>(dxr + off + W) = make_float4(at(c0, 2, g0), at(c0, 3, g0), at(c1, 2, g1), at(c1, 3, g1));
  }
}

// RELU: x is the output of a relu whose only consumer is this pool; dxr =
// relu backward of dx (dx where x > 0, else +0.0f) is written in the same
// pass (x > 0 exactly when the relu's input is > 0); dx may then be null,
// and only dxr is written.  PRE: x is the relu's input instead (its relu,
// x > 0 ? x : +0, is taken on load: the same values, so the same argmax).
template <typename I, bool RELU = false, bool PRE = false>
__global__ void maxpool2x2_bwd_kernel(const float *__restrict__ x, const float *__restrict__ g,
                                      float *__restrict__ dx, int H, int W, int Ho, int Wo,
                                      I total, float *__restrict__ dxr = nullptr) {
  const int Wq = Wo / 2;
  const I stride = (I)gridDim.x * blockDim.x;
  for (I i = (I)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const I r = i / Wq;
    const int q = (int)(i - r * Wq);
    const I nc = r / Ho;
    const int ho = (int)(r - nc * Ho);
    const long off = ((long)nc * H + 2 * ho) * W + 4 * q;
    float4 a = *reinterpret_cast<const float4 *>(x + off);
    float4 b = *reinterpret_cast<const float4 *>(x + off + W);
    if constexpr (PRE) {
      a = make_float4(a.x > 0.0f ? a.x : 0.0f, a.y > 0.0f ? a.y : 0.0f, a.z > 0.0f ? a.z : 0.0f,
                      a.w > 0.0f ? a.w : 0.0f);
      b = make_float4(b.x > 0.0f ? b.x : 0.0f, b.y > 0.0f ? b.y : 0.0f, b.z > 0.0f ? b.z : 0.0f,
                      b.w > 0.0f ? b.w : 0.0f);
    }
    const float2 gv = *reinterpret_cast<const float2 *>(g + (long)r * Wo + 2 * q);
    int am0, am1;
    argmax4(a.x, a.y, b.x, b.y, am0);
    argmax4(a.z, a.w, b.z, b.w, am1);
    const float g0 = 0.0f + gv.x, g1 = 0.0f + gv.y;
    float4 top = make_float4(am0 == 0 ? g0 : 0.0f, am0 == 1 ? g0 : 0.0f, am1 == 0 ? g1 : 0.0f, am1 == 1 ? g1 : 0.0f);
    float4 bot = make_float4(am0 == 2 ? g0 : 0.0f, am0 == 3 ? g0 : 0.0f, am1 == 2 ? g1 : 0.0f, am1 == 3 ? g1 : 0.0f);
    if (!RELU || dx) {
      *reinterpret_cast<float4 *>(dx + off) = top;
      *reinterpret_cast<float4 *>(dx + off + W) = bot;
    }
    if constexpr (RELU) {
      const float4 rt = make_float4(a.x > 0.0f ? top.x : 0.0f, a.y > 0.0f ? top.y : 0.0f,
                                    a.z > 0.0f ? top.z : 0.0f, a.w > 0.0f ? top.w : 0.0f);
      const float4 rb = make_float4(b.x > 0.0f ? bot.x : 0.0f, b.y > 0.0f ? bot.y : 0.0f,
                                    b.z > 0.0f ? bot.z : 0.0f, b.w > 0.0f ? bot.w : 0.0f);
      *reinterpret_cast<float4 *>(dxr + off) = rt;
      *reinterpret_cast<float4 *>(dxr + off + W) = rb;
    }
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

// LDS-staged im2col: the input plane must fit in 64 KB of LDS and the
// column rows must be 16-byte aligned.
static bool im2col_lds_fits(int N, int C, int H, int W, int Wo, const float *col) {
  return Wo % 4 == 0 && (long)H * W <= 16384 && (long)N * C < (1L << 31) &&
         (((uintptr_t)col & 15) == 0);
}

static int im2col_lds(const float *x, float *col, int N, int C, int H, int W, int HH, int WW,
                      int sh, int sw, int ph, int pw, int Ho, int Wo, int ones) {
  hipLaunchKernelGGL(im2col_lds_kernel, dim3((unsigned)((long)N * C)), dim3(256),
                     sizeof(float) * (size_t)H * W, stream(), x, col, N, C, H, W, HH, WW, sh, sw, ph,
                     pw, Ho, Wo, ones);
  return launched();
}

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
  const long Kc = (long)C * HH * WW;
  if (im2col_lds_fits(N, C, H, W, Wo, col))
    return im2col_lds(x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, 0);
  if (Ncol % 4 == 0 && Kc <= 65535 && Ncol < (1L << 32) - 4096 && (((uintptr_t)col & 15) == 0)) {
    hipLaunchKernelGGL(im2col_rows_kernel, dim3((unsigned)((Ncol / 4 + 255) / 256), (unsigned)Kc),
                       dim3(256), 0, stream(), x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
    return launched();
  }
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

int tt_k_im2col_ones(const float *x, float *col, int N, int C, int H, int W, int HH, int WW,
                     int sh, int sw, int ph, int pw, int Ho, int Wo) {
  if (im2col_lds_fits(N, C, H, W, Wo, col))
    return im2col_lds(x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, 1);
  const int rc = tt_k_im2col(x, col, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
  if (rc) return rc;
  const long Ncol = (long)N * Ho * Wo;
  return tt_k_fill(col + (long)C * HH * WW * Ncol, Ncol, 1.0f);
}

int tt_k_col2im(const float *col, float *x, int N, int C, int H, int W, int HH, int WW, int sh,
                int sw, int ph, int pw, int Ho, int Wo) {
  const long total = (long)N * C * H * W;
  if (total <= 0) return 0;
  const bool s1 = sh == 1 && sw == 1;
  const long HoWo = (long)Ho * Wo;
  const size_t lds = sizeof(float) * (size_t)HH * WW * HoWo;
  if (HoWo % 4 == 0 && lds <= 65536 && (long)N * C < (1L << 31) && ((uintptr_t)col & 15) == 0) {
    const dim3 g((unsigned)((long)N * C)), b(256);
    const bool vec = W % 4 == 0 && ((uintptr_t)x & 15) == 0;
    if (s1 && vec) hipLaunchKernelGGL((col2im_lds_kernel<true, true>), g, b, lds, stream(), col, x, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
    else if (s1)   hipLaunchKernelGGL((col2im_lds_kernel<true, false>), g, b, lds, stream(), col, x, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
    else if (vec)  hipLaunchKernelGGL((col2im_lds_kernel<false, true>), g, b, lds, stream(), col, x, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
    else           hipLaunchKernelGGL((col2im_lds_kernel<false, false>), g, b, lds, stream(), col, x, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
    return launched();
  }
  const dim3 g(blocks_for(total)), b(256);
  if (total < (1L << 31)) {
    if (s1) hipLaunchKernelGGL((col2im_px_kernel<unsigned, true>), g, b, 0, stream(), col, x, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
    else    hipLaunchKernelGGL((col2im_px_kernel<unsigned, false>), g, b, 0, stream(), col, x, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
  } else {
    if (s1) hipLaunchKernelGGL((col2im_px_kernel<unsigned long, true>), g, b, 0, stream(), col, x, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
    else    hipLaunchKernelGGL((col2im_px_kernel<unsigned long, false>), g, b, 0, stream(), col, x, N, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo);
  }
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
  if (ph == 2 && pw == 2 && sh == 2 && sw == 2 && W % 4 == 0 && (((uintptr_t)x & 15) == 0) &&
      (((uintptr_t)y & 7) == 0)) {
    const long pairs = total / 2;  // Wo = W/2 is even
    if (pairs < (1L << 31))
      hipLaunchKernelGGL(maxpool2x2_fwd_kernel<unsigned>, dim3(blocks_for(pairs)), dim3(256), 0, stream(), x, y, H, W, Ho, Wo, (unsigned)pairs);
    else
      hipLaunchKernelGGL(maxpool2x2_fwd_kernel<unsigned long>, dim3(blocks_for(pairs)), dim3(256), 0, stream(), x, y, H, W, Ho, Wo, (unsigned long)pairs);
    return launched();
  }
  TT_LAUNCH_I(maxpool_fwd_kernel, total, x, y, N, C, H, W, ph, pw, sh, sw, Ho, Wo);
  return launched();
}

// 2x2 / stride-2 max pool backward fused with the backward of the relu that
// produced its input: dx = pool backward (as tt_k_maxpool_bwd), dxr = dx
// where x > 0 else +0.0f.  -1 when the shape or alignment does not fit the
// 2x2 kernel (the caller then runs the two backwards separately).
}  // extern "C"

namespace {
template <bool PRE>
int maxpool2x2_relu_bwd(const float *x, const float *g, float *dx, float *dxr, int N, int C,
                        int H, int W, int Ho, int Wo) {
  const long total = (long)N * C * H * W;
  if (total <= 0) return 0;
  if (W % 4 != 0 || Ho != H / 2 || Wo != W / 2 || (((uintptr_t)x & 15) != 0) ||
      (((uintptr_t)dx & 15) != 0) || !dxr || (((uintptr_t)dxr & 15) != 0) ||
      (((uintptr_t)g & 7) != 0))
    return -1;
  const long pairs = (long)N * C * Ho * Wo / 2;
  if (pairs < (1L << 31))
    hipLaunchKernelGGL((maxpool2x2_bwd_kernel<unsigned, true, PRE>), dim3(blocks_for(pairs)), dim3(256),
                       0, stream(), x, g, dx, H, W, Ho, Wo, (unsigned)pairs, dxr);
  else
    hipLaunchKernelGGL((maxpool2x2_bwd_kernel<unsigned long, true, PRE>), dim3(blocks_for(pairs)),
                       dim3(256), 0, stream(), x, g, dx, H, W, Ho, Wo, (unsigned long)pairs, dxr);
  if (2 * Ho < H) {
    if (dx) TT_LAUNCH_I(pool_uncovered_zero_kernel, total, dx, N, C, H, W, 2 * Ho, 2 * Wo);
    TT_LAUNCH_I(pool_uncovered_zero_kernel, total, dxr, N, C, H, W, 2 * Ho, 2 * Wo);
  }
  return launched();
}

}  // namespace

extern "C" {

int tt_k_maxpool2x2_relu_bwd(const float *x, const float *g, float *dx, float *dxr, int N, int C,
                             int H, int W, int Ho, int Wo) {
  return maxpool2x2_relu_bwd<false>(x, g, dx, dxr, N, C, H, W, Ho, Wo);
}

int tt_k_maxpool2x2_prerelu_bwd(const float *xpre, const float *g, float *dx, float *dxr, int N,
                                int C, int H, int W, int Ho, int Wo) {
  return maxpool2x2_relu_bwd<true>(xpre, g, dx, dxr, N, C, H, W, Ho, Wo);
}

int tt_k_maxpool2x2_code_relu_bwd(const unsigned char *codes, const float *g, float *dxr, int N,
                                  int C, int H, int W, int Ho, int Wo) {
  const long pairs = (long)N * C * Ho * Wo / 2;
  if (pairs <= 0) return 0;
  if (W % 4 != 0 || H != 2 * Ho || W != 2 * Wo || !codes || !g || !dxr ||
      (((uintptr_t)codes & 1) != 0) || (((uintptr_t)dxr & 15) != 0) || (((uintptr_t)g & 7) != 0))
    return -1;
  if (pairs < (1L << 31))
    hipLaunchKernelGGL(maxpool2x2_code_bwd_kernel<unsigned>, dim3(blocks_for(pairs)), dim3(256), 0,
                       stream(), codes, g, dxr, H, W, Ho, Wo, (unsigned)pairs);
  else
    hipLaunchKernelGGL(maxpool2x2_code_bwd_kernel<unsigned long>, dim3(blocks_for(pairs)),
                       dim3(256), 0, stream(), codes, g, dxr, H, W, Ho, Wo, (unsigned long)pairs);
  return launched();
}

int tt_k_maxpool_bwd(const float *x, const float *g, float *dx, int N, int C, int H, int W, int ph,
                     int pw, int sh, int sw, int Ho, int Wo) {
  const long total = (long)N * C * H * W;
  if (total <= 0) return 0;
  if (ph == 2 && pw == 2 && sh == 2 && sw == 2 && W % 4 == 0 && (((uintptr_t)x & 15) == 0) &&
      (((uintptr_t)dx & 15) == 0) && (((uintptr_t)g & 7) == 0)) {
    const long pairs = (long)N * C * Ho * Wo / 2;
    if (pairs < (1L << 31))
      hipLaunchKernelGGL(maxpool2x2_bwd_kernel<unsigned>, dim3(blocks_for(pairs)), dim3(256), 0, stream(), x, g, dx, H, W, Ho, Wo, (unsigned)pairs);
    else
      hipLaunchKernelGGL(maxpool2x2_bwd_kernel<unsigned long>, dim3(blocks_for(pairs)), dim3(256), 0, stream(), x, g, dx, H, W, Ho, Wo, (unsigned long)pairs);
    if (2 * Ho < H)
      TT_LAUNCH_I(pool_uncovered_zero_kernel, total, dx, N, C, H, W, 2 * Ho, 2 * Wo);
  } else if (ph == sh && pw == sw) {
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
