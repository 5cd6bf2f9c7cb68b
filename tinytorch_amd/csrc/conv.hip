// Direct convolution on the matrix cores with the image staged in LDS
// (gfx950).  Replaces, for convolutions whose per-image row slab fits in LDS,
// the reference's im2col + GEMM sequence behind tt_conv2d / ag_conv2d:
//
//   forward  out = W * im2col(x) + bias, NCHW     reference src/ops_spatial.c:71-127
//   dW, db   dW = Gperm * im2col(x)^T, db = sum g reference src/autograd.c:456-513
//   dX       col2im(W^T * Gperm), stride 1         reference src/autograd.c:515-539,406-434
//
// The im2col matrix is never written.  A workgroup copies the input rows its
// output pixels need (all channels, R rows of W floats each, rows outside the
// image as zeros) from HBM into LDS once, and the MFMA operand for im2col
// element (k, p), k = (c*HH + kh)*WW + kw, p = ho*Wo + wo, is read from LDS at
//     koff[k] + pix[p],  koff = (c*R + kh)*W + kw - pw,  pix = (ho-ho0)*sh*W + wo*sw
// and replaced by 0 when the column wo*sw + kw - pw falls outside [0, W) --
// the horizontal zero padding is applied on read, so each channel's rows are
// one contiguous block of x and are staged with 16-byte direct global->LDS
// loads.  Every staged element feeds up to HH*WW im2col entries: HBM sees the
// input about once per workgroup instead of an HH*WW-fold im2col matrix being
// written and read back.
//
//   forward / dX: v_mfma_f32_32x32x2_f32, A = weights (32 output channels,
//     LDS [k][f], 32 floats a row), B = the slab.  Lane l feeds A[l%32][l/32]
//     and B[l/32][l%32]; accumulator r of lane l holds row 8(r/4) + 4(l/32) +
//     r%4, column l%32.  Each wave owns PB blocks of 32 consecutive output
//     pixels.  Taps past K read a zero plane after the slab, so no operand is
//     ever 0 * (input value) for a tap that does not exist.
//   dX of a stride-1 convolution is the forward convolution of the output
//     gradient with the kernel flipped in (kh, kw) and channels swapped,
//     padding HH-1-ph: the flip is applied while staging the weights.
//   dW: v_mfma_f32_16x16x4_f32, A = the output gradient (16 filters x 4
//     pixels, staged in LDS), B = the slab (4 pixels x 16 taps).  Lane l
//     feeds A[l%16][l/16], B[l/16][l%16]; accumulator r holds row 4(l/16)+r,
//     column l%16.  The sum over a workgroup's pixels goes to a partial
//     (F x (K+1), last column = the bias gradient summed on the VALU), and a
//     second kernel adds the partials in index order: deterministic, no
//     atomics.
//
// Staging: activations and output gradients with direct loads
// (global_load_lds_dwordx4 when rows are 16-byte aligned, else _dword);
// weights through registers (coalesced reads of the weight tensor, transposed
// LDS writes).  Measured on MI355X, linear 16-byte direct loads fill LDS about
// 10x faster than per-lane scattered 4-byte ones.
#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>
#include <stdlib.h>
#include "tt_rt.h"

#include "probe.h"
TT_PROBE_DEFINE(conv)

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

inline hipStream_t stream() { return (hipStream_t)ttrt_stream(); }

constexpr int NT = 256;                    // threads per workgroup (4 waves)
constexpr long LDS_MAX = 160L * 1024;      // bytes of LDS per workgroup on gfx950
constexpr int GUARD = 64;                  // floats before the slab (reads at -pw are masked)

// Convolution geometry as the kernels see it: input C x H x W, kernel
// HH x WW, stride, padding, output Ho x Wo, F output channels, K = C*HH*WW.
struct Geo {
  int C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, F, K;
};

// Slab of one workgroup: output pixels [p0, p1) of image n cover output rows
// ho0..; input rows ho0*sh-ph .. +R-1 are staged as R rows of W floats per
// channel, then a zero plane of R*W floats.
struct Slab {
  int ho0, R;
};

__device__ __forceinline__ Slab slab_of(const Geo &g, int p0, int p1) {
  Slab s;
  s.ho0 = p0 / g.Wo;
  const int ho1 = (p1 - 1) / g.Wo;
  s.R = (ho1 - s.ho0) * g.sh + g.HH;
  return s;
}

// n / d for 0 <= n < 2^24, 0 < d < 2^16 through the float reciprocal, with
// one correction step each way (the estimate is within 1 of the quotient).
__device__ __forceinline__ int fdiv(int n, int d, float rcp) {
  int q = (int)((float)n * rcp);
  const int r = n - q * d;
  q += (r >= d) - (r < 0);
  return q;
}

// Every padding element of a staged operand is loaded from here.
__device__ __attribute__((aligned(16))) float g_zero_src[4];

// Direct loads: lane i's 4 (or 16) bytes from `src` go to LDS at lds_wave +
// 4i (16i); M0 holds the wave-uniform LDS byte address.  Nothing lands in
// registers, so a wave issues all of its staging loads back to back and the
// kernel waits for them once (vmcnt(0) and a barrier).
__device__ __forceinline__ void dma_dword(const float *src, const float *lds_wave) {
  const unsigned addr = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_wave);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off"
               :
               : "s"(addr), "v"(src)
               : "memory", "m0");
}

__device__ __forceinline__ void dma_dwordx4(const float *src, const float *lds_wave) {
  const unsigned addr = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds_wave);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(addr), "v"(src)
               : "memory", "m0");
}

__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

inline __host__ __device__ int round_up(int v, int m) { return (v + m - 1) / m * m; }

// Copy T floats into LDS at dst, viewed as blocks of B floats: element j of
// block b is src[b * bstride + j] when b < nb and jlo <= j < jhi, else 0.
// VEC: 16-byte loads (B, bstride, jlo, jhi multiples of 4, src 16-byte
// aligned); dst is then filled in whole 256-float runs.  NTH threads take part.
template <bool VEC, int NTH = NT>
__device__ __forceinline__ void stage_blocks(float *dst, const float *__restrict__ src, int T,
                                             int B, int nb, long bstride, int jlo, int jhi) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const float rcpB = 1.0f / (float)B;
  constexpr int E = VEC ? 4 : 1;   // floats per lane per load
  for (int base = wave * 64 * E; base < T; base += NTH * E) {
    const int i = base + lane * E;
    const int b = fdiv(i, B, rcpB), j = i - b * B;
    const bool ok = i < T && b < nb && j >= jlo && j < jhi;
    const float *p = ok ? src + b * bstride + j : g_zero_src;
    if constexpr (VEC) dma_dwordx4(p, dst + base);
    else dma_dword(p, dst + base);
  }
}

// Channel stride of the slab in LDS: R rows of W floats plus 4 floats of
// padding.  The pad moves consecutive channels to other banks: the 32 taps
// of a weight-gradient operand read (3 to 4 channels of 3x3 taps) would
// otherwise fall on a handful of banks whenever R*W is a multiple of 32
// (16-way conflicts at W = 16); with it, 4-way at worst.
__host__ __device__ inline int slab_cs(int R, int W) { return R * W + 4; }

// Slab of image n: channel blocks of CS floats (rows hs..hs+R-1 of x, those
// outside [0, H) as zeros, then the pad), then the zero plane.
template <bool VEC, int NTH = NT>
__device__ __forceinline__ void stage_slab(float *xs, const float *__restrict__ x, const Geo &g,
                                           const Slab &s, int n) {
  const int hs = s.ho0 * g.sh - g.ph;
  const int CS = slab_cs(s.R, g.W);
  const int rlo = hs < 0 ? -hs : 0;
  const int rhi = g.H - hs < s.R ? g.H - hs : s.R;
  const float *xn = x + (long)n * g.C * g.H * g.W + (long)hs * g.W;
  stage_blocks<VEC, NTH>(xs, xn, (g.C + 1) * CS, CS, g.C, (long)g.H * g.W, rlo * g.W, rhi * g.W);
}

// Gapped slab (weight gradient, 16-byte staging): every row of W floats sits
// in a slot of W + G floats behind G zeros, G a multiple of 4 covering the
// left padding and the right overhang of the widest tap, so a tap read past
// either end of a row lands in a gap and reads zero -- no mask per read.
// Channel stride R*(W+G) + 4, then a zero plane.  The DMA still fills LDS in
// whole 16-byte runs: a lane whose chunk falls in a gap loads the zero source.
__host__ __device__ inline int gslab_gap(const Geo &g) {
  const int ro = (g.Wo - 1) * g.sw - g.pw + g.WW - g.W;  // right overhang
  int need = g.pw > ro ? g.pw : ro;
  if (need < 1) need = 1;
  return round_up(need, 4);
}
__host__ __device__ inline int gslab_rw(const Geo &g) { return g.W + gslab_gap(g); }
__host__ __device__ inline int gslab_cs(int R, const Geo &g) { return R * gslab_rw(g) + 4; }

template <int NTH = NT>
__device__ __forceinline__ void stage_gslab(float *xs, const float *__restrict__ x, const Geo &g,
                                            const Slab &s, int n) {
  const int hs = s.ho0 * g.sh - g.ph;
  const int G = gslab_gap(g), RW = g.W + G;
  const int CS = gslab_cs(s.R, g);
  const int T = (g.C + 1) * CS;
  const float rcpC = 1.0f / (float)CS, rcpR = 1.0f / (float)RW;
  const float *xn = x + (long)n * g.C * g.H * g.W;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  for (int base = wave * 256; base < T; base += NTH * 4) {
    const int i = base + lane * 4;
    const int c = fdiv(i, CS, rcpC), rem = i - c * CS;
    const int slot = fdiv(rem, RW, rcpR), j = rem - slot * RW;
    const int row = hs + slot;
    const bool ok = i < T && c < g.C && slot < s.R && j >= G && row >= 0 && row < g.H;
    const float *p = ok ? xn + ((long)c * g.H + row) * g.W + (j - G) : g_zero_src;
    dma_dwordx4(p, xs + base);
  }
}

// output pixel p -> (LDS offset of its first tap's row start inside the
// gapped slab, wo*sw): rows of gslab_rw floats, data behind the gap
__device__ __forceinline__ int2 gslab_pixel(const Geo &g, const Slab &s, int p) {
  const int ho = fdiv(p, g.Wo, 1.0f / (float)g.Wo), wo = p - ho * g.Wo;
  return make_int2((ho - s.ho0) * g.sh * gslab_rw(g) + wo * g.sw + gslab_gap(g), wo * g.sw);
}

// tap k of the gapped slab -> LDS offset (taps past K -> the zero plane)
__device__ __forceinline__ int gslab_tap(const Geo &g, const Slab &s, int k) {
  const int CS = gslab_cs(s.R, g), RW = gslab_rw(g);
  if (k >= g.K) return g.C * CS;
  const int taps = g.HH * g.WW;
  const int c = fdiv(k, taps, 1.0f / (float)taps), t = k - c * taps;
  const int kh = fdiv(t, g.WW, 1.0f / (float)g.WW), kw = t - kh * g.WW;
  return c * CS + kh * RW + gslab_gap(g) + kw - g.pw;
}

// im2col row k -> (LDS offset of the tap inside the slab, kw - pw, offset of
// the flipped tap in the FLIP weight layout); taps past K -> the zero plane,
// never masked (their weight offset is 0: a finite weight times zero).
__device__ __forceinline__ int4 tap_entry(const Geo &g, const Slab &s, int k) {
  const int CS = slab_cs(s.R, g.W);
  if (k >= g.K) return make_int4(g.C * CS, 0, 0, 0);
  const int taps = g.HH * g.WW;
  const int c = fdiv(k, taps, 1.0f / (float)taps), t = k - c * taps;
  const int kh = fdiv(t, g.WW, 1.0f / (float)g.WW), kw = t - kh * g.WW;
  return make_int4(c * CS + kh * g.W + kw - g.pw, kw - g.pw, c * 32 * taps + taps - 1 - t, 0);
}

// output pixel p -> (LDS offset inside the slab, wo*sw)
__device__ __forceinline__ int2 pixel_entry(const Geo &g, const Slab &s, int p) {
  const int ho = fdiv(p, g.Wo, 1.0f / (float)g.Wo), wo = p - ho * g.Wo;
  return make_int2((ho - s.ho0) * g.sh * g.W + wo * g.sw, wo * g.sw);
}

// B operand: slab element at tap + pixel, 0 in the horizontal padding
__device__ __forceinline__ float slab_read(const float *xs, int4 tap, int2 pix, int W) {
  const float v = xs[tap.x + pix.x];
  return (unsigned)(pix.y + tap.y) < (unsigned)W ? v : 0.0f;
}

// Row stride of the forward weights in LDS: whole 16-byte reads, and
// 8 lanes reading rows f..f+7 at one k cover all 32 banks (stride = 4 mod 32).
__host__ __device__ inline int wrow_stride(int Kp) { return round_up(Kp, 32) + 4; }

// Weights of one block of 32 output channels into LDS with direct loads.
//   forward: ws[f][KST] = W[f0+f][0..K) (zeros past K and past F): rows of
//     the weight tensor, so each row is one contiguous copy;
//   FLIP (the dX convolution; w is the forward kernel, C_in x F_out x HH x
//     WW in this geometry's terms): ws[fi][c][t] = w[fi][f0+c][t] for c < 32
//     (zeros past F), the tensor's own order; the tap flip is applied when
//     the operand is read (tap_entry's .z).
template <bool FLIP, bool VEC>
__device__ __forceinline__ void stage_weights(float *ws, const float *__restrict__ w,
                                              const Geo &g, int f0, int Kp) {
  const int nf = g.F - f0 < 32 ? g.F - f0 : 32;
  const int taps = g.HH * g.WW;
  if constexpr (FLIP)
    stage_blocks<VEC>(ws, w + (long)f0 * taps, g.C * 32 * taps, 32 * taps, g.C,
                      (long)g.F * taps, 0, nf * taps);
  else
    stage_blocks<VEC>(ws, w + (long)f0 * g.K, 32 * wrow_stride(Kp), wrow_stride(Kp), nf,
                      g.K, 0, g.K);
}

// ---- forward (and stride-1 dX with FLIP) ----
//
// Grid: x = image * chunks + chunk (chunks of 128*PB output pixels), y =
// block of 32 output channels.
template <int PB, bool FLIP, bool VEC>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 2)))
conv_fwd_lds_kernel(const float *__restrict__ x, const float *__restrict__ w,
                    const float *__restrict__ bias, float *__restrict__ out,
                    float *__restrict__ rout, float *__restrict__ /*pout: 3x3 kernel only*/,
                    float *__restrict__ /*cout*/, float *__restrict__ /*dout*/,
                    unsigned char *__restrict__ /*aout*/, Geo g, int chunks) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  constexpr int CHUNK = 128 * PB;
  const int n = blockIdx.x / chunks, chunk = blockIdx.x - n * chunks;
  const int P = g.Ho * g.Wo;
  const int p0 = chunk * CHUNK;
  const int p1 = min(p0 + CHUNK, P);
  const int f0 = blockIdx.y * 32;
  const int Kp = (g.K + 7) & ~7;  // whole groups of 4 k-steps per lane half
  const int Kh = Kp >> 1;         // lane half h takes k = h*Kh + step
  const int KST = wrow_stride(Kp);
  const int taps = g.HH * g.WW;
  const Slab s = slab_of(g, p0, p1);

  float *ws = smem;                                  // forward: 32 x KST; FLIP: C x 32 x taps
  int4 *tab = (int4 *)(ws + (FLIP ? round_up(g.K * 32, 256) : round_up(32 * KST, 256)));
  float *bs = (float *)(tab + Kp);                   // 32 (+pad): bias of the block
  float *xs = bs + 64 + GUARD;                       // (C+1) x R x W (whole 16-byte loads)

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  stage_slab<VEC>(xs, x, g, s, n);
  stage_weights<FLIP, VEC>(ws, w, g, f0, Kp);
  for (int k = tid; k < Kp; k += NT) tab[k] = tap_entry(g, s, k);
  if (tid < 32) bs[tid] = (bias && f0 + tid < g.F) ? bias[f0 + tid] : 0.0f;
  dma_wait();
  __syncthreads();

  const int l32 = lane & 31, half = lane >> 5;
  int2 pix[PB];
#pragma unroll
  for (int j = 0; j < PB; j++) {
    const int p = p0 + (wave * PB + j) * 32 + l32;
    pix[j] = p < p1 ? pixel_entry(g, s, p) : make_int2(0, -(1 << 20));  // masked
  }
  f32x16 acc[PB];
#pragma unroll
  for (int j = 0; j < PB; j++)
    for (int r = 0; r < 16; r++) acc[j][r] = 0.0f;

  // Software pipeline over groups of U = 4 k-steps: while the MFMAs of group
  // i run, the operands of group i+1 and the tap entries of group i+2 are
  // read from LDS, so no MFMA waits on an LDS round trip.  Lane half h
  // covers k = h*Kh + step (A and B agree on the order, so the sum is the
  // same); the forward weights of 4 steps are one 16-byte read.
  constexpr int U = 4;
  const float *wa = FLIP ? ws + l32 * taps : ws + l32 * KST + half * Kh;
  const int4 *tb = tab + half * Kh;
  const int groups = Kh / U;
  float a_c[U], b_c[U][PB];
  int4 t_c[U], t_n[U];
#pragma unroll
  for (int u = 0; u < U; u++) t_c[u] = tb[u];
  if constexpr (FLIP) {
#pragma unroll
    for (int u = 0; u < U; u++) a_c[u] = wa[t_c[u].z];
  } else {
    const float4 a4 = *(const float4 *)wa;
    a_c[0] = a4.x; a_c[1] = a4.y; a_c[2] = a4.z; a_c[3] = a4.w;
  }
#pragma unroll
  for (int u = 0; u < U; u++)
#pragma unroll
    for (int j = 0; j < PB; j++) b_c[u][j] = slab_read(xs, t_c[u], pix[j], g.W);
  {
    const int g1 = groups > 1 ? 1 : 0;
#pragma unroll
    for (int u = 0; u < U; u++) t_n[u] = tb[g1 * U + u];
  }
  for (int gi = 0; gi < groups; gi++) {
    const int g1 = gi + 1 < groups ? gi + 1 : gi;
    const int g2 = gi + 2 < groups ? gi + 2 : g1;
    float a_n[U], b_n[U][PB];
    int4 t_nn[U];
    if constexpr (FLIP) {
#pragma unroll
      for (int u = 0; u < U; u++) a_n[u] = wa[t_n[u].z];
    } else {
      const float4 a4 = *(const float4 *)(wa + g1 * U);
      a_n[0] = a4.x; a_n[1] = a4.y; a_n[2] = a4.z; a_n[3] = a4.w;
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
#pragma unroll
      for (int j = 0; j < PB; j++) b_n[u][j] = slab_read(xs, t_n[u], pix[j], g.W);
      t_nn[u] = tb[g2 * U + u];
    }
#pragma unroll
    for (int u = 0; u < U; u++)
#pragma unroll
      for (int j = 0; j < PB; j++)
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a_c[u], b_c[u][j], acc[j], 0, 0, 0);
#pragma unroll
    for (int u = 0; u < U; u++) {
      a_c[u] = a_n[u];
      t_n[u] = t_nn[u];
#pragma unroll
      for (int j = 0; j < PB; j++) b_c[u][j] = b_n[u][j];
    }
  }

  float bv[16];  // bias of this lane's 16 rows (zeros when there is none)
#pragma unroll
  for (int r = 0; r < 16; r++) bv[r] = bs[8 * (r >> 2) + 4 * half + (r & 3)];
  float *on = out + (long)n * g.F * P;
  // rout: the relu of the output as well (x > 0 ? x : +0, NaN -> +0)
  float *rn = rout ? rout + (long)n * g.F * P : nullptr;
  // one unrolled store loop per form (a branch on rn inside it defeats the unroll)
  auto store = [&](auto relu) {
#pragma unroll
    for (int j = 0; j < PB; j++) {
      const int p = p0 + (wave * PB + j) * 32 + l32;
      if (p >= p1) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int f = f0 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (f < g.F) {
          const float v = acc[j][r] + bv[r];
          on[(long)f * P + p] = v;
          if constexpr (decltype(relu)::value) rn[(long)f * P + p] = v > 0.0f ? v : 0.0f;
        }
      }
    }
  };
  if (rn) store(std::true_type{});
  else store(std::false_type{});
}

// A 2x2 pool window of relu values (>= +0, never NaN) at top-left, top-right,
// bottom-left, bottom-right: returns its max, and its code -- bits 0-1 the
// first position holding the max in that order (the order the pool backward
// scans: maxpool2x2_bwd_kernel), bits 2-5 which of the four are > 0 (the
// relu backward's mask).  Bit for bit, the pool backward and the relu
// backward after it need nothing else (maxpool2x2_code_bwd_kernel).
__device__ __forceinline__ float pool_code(float tl, float tr, float bl, float br,
                                           unsigned &code) {
  float m = tl;
  unsigned am = 0;
  if (tr > m) { m = tr; am = 1; }
  if (bl > m) { m = bl; am = 2; }
  if (br > m) { m = br; am = 3; }
  code = am | (tl > 0.0f ? 4u : 0u) | (tr > 0.0f ? 8u : 0u) | (bl > 0.0f ? 16u : 0u) |
         (br > 0.0f ? 32u : 0u);
  return m;
}

// ---- forward / dX for KH x KW kernels known at compile time ----
//
// Lane half h of the 32x32x2 MFMA takes input channels [h*CH2, (h+1)*CH2)
// (CH2 = ceil(C/2); an odd C borrows the zero plane as channel C), so both
// halves use the same tap (kh, kw) at every step: the tap is a loop
// constant, the slab address is a per-lane base (advanced once per channel)
// plus an immediate, and the horizontal padding is one of KW lane masks
// computed once.  The main loop reads no tables and does almost no VALU
// work.  Weights as in the generic kernel (forward rows of KST floats, FLIP
// in the tensor's order).
//
// KS = 2: eight waves, the second four taking the upper half of the channel
// steps of the same pixels; their sums are added in LDS (the waves of a
// workgroup that fills a CU's LDS then share each SIMD two ways).
template <int PB, bool FLIP, bool VEC, int KH, int KW, int KS = 1>
__global__ void __launch_bounds__(NT * KS) __attribute__((amdgpu_waves_per_eu(1, 2)))
conv_fwd_k_kernel(const float *__restrict__ x, const float *__restrict__ w,
                  const float *__restrict__ bias, float *__restrict__ out,
                  float *__restrict__ rout, float *__restrict__ pout, float *__restrict__ cout,
                  float *__restrict__ dout, unsigned char *__restrict__ aout, Geo g, int chunks) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  constexpr int CHUNK = 128 * PB, TAPS = KH * KW;
  const int n = blockIdx.x / chunks, chunk = blockIdx.x - n * chunks;
  const int P = g.Ho * g.Wo;
  const int p0 = chunk * CHUNK;
  const int p1 = min(p0 + CHUNK, P);
  const int f0 = blockIdx.y * 32;
  const int CH2 = (g.C + 1) >> 1;
  const int KST = wrow_stride(2 * CH2 * TAPS);
  const Slab s = slab_of(g, p0, p1);
  // 16-byte staging: the gapped slab (reads past a row end hit zeros, no
  // masks); otherwise rows of W floats and a select per read
  const int RW = VEC ? gslab_cs(s.R, g) : slab_cs(s.R, g.W);  // channel stride of the slab
  const int RS = VEC ? gslab_rw(g) : g.W;                     // row stride of the slab
  const int nf = g.F - f0 < 32 ? g.F - f0 : 32;

  float *ws = smem;  // forward: 32 x KST; FLIP: 2*CH2 x 32 x TAPS
  float *bs = ws + (FLIP ? round_up(2 * CH2 * 32 * TAPS, 256) : round_up(32 * KST, 256));
  float *xs = bs + 64 + GUARD;                       // (C+1) x R x W

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int pw4 = wave & 3, grp = wave >> 2;  // pixel blocks, channel-step group
  constexpr int NTH = NT * KS;
  if constexpr (VEC) stage_gslab<NTH>(xs, x, g, s, n);
  else stage_slab<VEC, NTH>(xs, x, g, s, n);
  {
    if constexpr (FLIP)
      stage_blocks<VEC, NTH>(ws, w + (long)f0 * TAPS, 2 * CH2 * 32 * TAPS, 32 * TAPS, g.C,
                        (long)g.F * TAPS, 0, nf * TAPS);
    else if (VEC && g.K % 4 == 0)
      stage_blocks<true, NTH>(ws, w + (long)f0 * g.K, 32 * KST, KST, nf, g.K, 0, g.K);
    else  // rows of K floats not 16-byte aligned (K % 4 != 0): 4-byte loads
      stage_blocks<false, NTH>(ws, w + (long)f0 * g.K, 32 * KST, KST, nf, g.K, 0, g.K);
  }
  if (tid < 32) bs[tid] = (bias && f0 + tid < g.F) ? bias[f0 + tid] : 0.0f;
  dma_wait();
  __syncthreads();

  const int l32 = lane & 31, half = lane >> 5;
  const int hoff = half * CH2 * RW - g.pw;
  int bj[PB];
  bool mk[PB][KW];
#pragma unroll
  for (int j = 0; j < PB; j++) {
    const int p = p0 + (pw4 * PB + j) * 32 + l32;
    // past the chunk: every tap masked (gapped: any in-slab pixel, the
    // output is not stored)
    int2 e = make_int2(VEC ? g.pw : 0, -(1 << 20));
    if (p < p1) e = VEC ? gslab_pixel(g, s, p) : pixel_entry(g, s, p);
    bj[j] = e.x + hoff;
#pragma unroll
    for (int kw = 0; kw < KW; kw++) mk[j][kw] = (unsigned)(e.y + kw - g.pw) < (unsigned)g.W;
  }
  f32x16 acc[PB];
#pragma unroll
  for (int j = 0; j < PB; j++)
    for (int r = 0; r < 16; r++) acc[j][r] = 0.0f;

  const float *wa = FLIP ? ws + l32 * TAPS + half * CH2 * 32 * TAPS
                         : ws + l32 * KST + half * CH2 * TAPS;
  constexpr int WSTEP_FLIP = 32 * TAPS;
  // this wave's channel steps [cs0, cs1): all of them, or one half each
  // (KS = 2 needs CH2 even)
  const int cs0 = grp * (CH2 / KS), cs1 = cs0 + CH2 / KS;
  const int steps = cs1 - cs0;
  // operands of channel c+1 are read before the MFMAs of channel c
  auto load = [&](int c, float (&a)[TAPS], float (&b)[TAPS][PB]) {
    const float *wc = wa + c * (FLIP ? WSTEP_FLIP : TAPS);
    const int cb = c * RW;
#pragma unroll
    for (int t = 0; t < TAPS; t++) a[t] = FLIP ? wc[TAPS - 1 - t] : wc[t];
#pragma unroll
    for (int j = 0; j < PB; j++)
#pragma unroll
      for (int kh = 0; kh < KH; kh++) {
        const float *row = xs + bj[j] + cb + kh * RS;
#pragma unroll
        for (int kw = 0; kw < KW; kw++) b[kh * KW + kw][j] = row[kw];  // raw: masked at use
      }
  };
  auto mfmas = [&](const float (&a)[TAPS], const float (&b)[TAPS][PB]) {
#pragma unroll
    for (int t = 0; t < TAPS; t++)
#pragma unroll
      for (int j = 0; j < PB; j++) {
        const float bm = VEC || mk[j][t % KW] ? b[t][j] : 0.0f;
        acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t], bm, acc[j], 0, 0, 0);
      }
  };
  if (!FLIP && steps % 4 == 0 && cs0 % 4 == 0) {
    // Forward weights of four channels at a time: 4*TAPS floats per lane as
    // 16-byte reads (row stride KST = 4 mod 32: eight lanes cover all banks,
    // where single-float reads of 32 rows fall on 8 banks), a quad ahead.
    // The slab operands alternate two sets a channel ahead as below.
    constexpr int NV = TAPS;  // 16-byte vectors per quad (4 * TAPS floats)
    const int q0 = cs0 / 4, quads = cs1 / 4;
    auto loadw = [&](int q, f32x4 (&wv)[NV]) {
      const f32x4 *p = (const f32x4 *)(wa + q * 4 * TAPS);
#pragma unroll
      for (int i = 0; i < NV; i++) wv[i] = p[i];
    };
    auto loadb = [&](int c, float (&b)[TAPS][PB]) {
      const int cb = c * RW;
#pragma unroll
      for (int j = 0; j < PB; j++)
#pragma unroll
        for (int kh = 0; kh < KH; kh++) {
          const float *row = xs + bj[j] + cb + kh * RS;
#pragma unroll
          for (int kw = 0; kw < KW; kw++) b[kh * KW + kw][j] = row[kw];
        }
    };
    auto mfq = [&](const f32x4 (&wv)[NV], const int cc, const float (&b)[TAPS][PB]) {
#pragma unroll
      for (int t = 0; t < TAPS; t++)
#pragma unroll
        for (int j = 0; j < PB; j++) {
          const int e = cc * TAPS + t;
          const float bm = VEC || mk[j][t % KW] ? b[t][j] : 0.0f;
          acc[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(wv[e >> 2][e & 3], bm, acc[j], 0, 0, 0);
        }
    };
    f32x4 w0[NV], w1[NV];
    float b0[TAPS][PB], b1[TAPS][PB];
    loadw(q0, w0);
    loadb(cs0, b0);
    for (int q = q0; q < quads; q += 2) {
      const int c = 4 * q;
      const int cl = cs1 - 1;
      loadw(q + 1 < quads ? q + 1 : q, w1);
      loadb(c + 1, b1);
      __builtin_amdgcn_sched_barrier(0);
      mfq(w0, 0, b0);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 2, b0);
      __builtin_amdgcn_sched_barrier(0);
      mfq(w0, 1, b1);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 3, b1);
      __builtin_amdgcn_sched_barrier(0);
      mfq(w0, 2, b0);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 4 < cl ? c + 4 : cl, b0);
      __builtin_amdgcn_sched_barrier(0);
      mfq(w0, 3, b1);
      __builtin_amdgcn_sched_barrier(0);
      if (q + 1 >= quads) break;
      loadw(q + 2 < quads ? q + 2 : q + 1, w0);
      loadb(c + 5, b1);
      __builtin_amdgcn_sched_barrier(0);
      mfq(w1, 0, b0);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 6, b0);
      __builtin_amdgcn_sched_barrier(0);
      mfq(w1, 1, b1);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 7, b1);
      __builtin_amdgcn_sched_barrier(0);
      mfq(w1, 2, b0);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 8 < cl ? c + 8 : cl, b0);
      __builtin_amdgcn_sched_barrier(0);
      mfq(w1, 3, b1);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
    // two operand sets in turn: a channel's operands are read a whole channel
    // before its MFMAs (a read past the last channel re-reads the last one)
    float a0[TAPS], b0[TAPS][PB], a1[TAPS], b1[TAPS][PB];
    if (steps > 0) load(cs0, a0, b0);
    int c = cs0;
    for (; c + 1 < cs1; c += 2) {
      load(c + 1, a1, b1);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      load(c + 2 < cs1 ? c + 2 : c + 1, a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a1, b1);
      __builtin_amdgcn_sched_barrier(0);
    }
    if (c < cs1) mfmas(a0, b0);
  }

  float bv[16];
#pragma unroll
  for (int r = 0; r < 16; r++) bv[r] = bs[8 * (r >> 2) + 4 * half + (r & 3)];
  if constexpr (KS == 2) {
    // the upper group's sums through LDS (every wave is past its last read
    // of the operands at the first barrier), added in a fixed order
    float *red = smem + pw4 * (PB * 16 * 64) + lane;
    __syncthreads();
    if (grp == 1) {
#pragma unroll
      for (int j = 0; j < PB; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) red[(j * 16 + r) * 64] = acc[j][r];
    }
    __syncthreads();
    if (grp == 1) return;
#pragma unroll
    for (int j = 0; j < PB; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[j][r] += red[(j * 16 + r) * 64];
  }

  float *on = out + (long)n * g.F * P;
  // rout: the relu of the output as well (x > 0 ? x : +0, NaN -> +0)
  float *rn = rout ? rout + (long)n * g.F * P : nullptr;
  // one unrolled store loop per form (a branch on rn inside it defeats the unroll)
  auto store = [&](auto relu) {
#pragma unroll
    for (int j = 0; j < PB; j++) {
      const int p = p0 + (pw4 * PB + j) * 32 + l32;
      if (p >= p1) continue;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int f = f0 + 8 * (r >> 2) + 4 * half + (r & 3);
        if (f < g.F) {
          const float v = acc[j][r] + bv[r];
          on[(long)f * P + p] = v;
          if constexpr (decltype(relu)::value) rn[(long)f * P + p] = v > 0.0f ? v : 0.0f;
        }
      }
    }
  };
  if (pout) {
    // relu and the 2x2 / stride-2 max pool of it as well (pout, N x F x
    // Ho/2 x Wo/2; the host checks that Ho and Wo are even, chunks start on
    // even rows and a row pair is either inside one 32-pixel block
    // (32 % Wo == 0, 32 / Wo even) or two consecutive blocks (Wo == 32, PB
    // even)).  The relu values are >= +0 and never NaN, so their max does
    // not depend on the order of the comparisons: the pool's output bit for
    // bit.  Every lane takes part in the shuffles; stores are masked.  cout /
    // dout (optional): the pool output once more (a flattening reshape's copy,
    // the same layout) and padded -- rows of F*Ho*Wo/4 + 1 floats per image,
    // the last one 1 (a padones after the reshape).
    float o[PB][16];
#pragma unroll
    for (int j = 0; j < PB; j++) {
      const int p = p0 + (pw4 * PB + j) * 32 + l32;
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int f = f0 + 8 * (r >> 2) + 4 * half + (r & 3);
        const float v = acc[j][r] + bv[r];
        o[j][r] = v > 0.0f ? v : 0.0f;
        if (f < g.F && p < p1) {
          on[(long)f * P + p] = v;
          if (rn) rn[(long)f * P + p] = o[j][r];
        }
      }
    }
    const int P4 = P >> 2, Wo2 = g.Wo >> 1;
    float *pn = pout + (long)n * g.F * P4;
    float *cn = cout ? cout + (long)n * g.F * P4 : nullptr;
    const long drow = (long)g.F * P4 + 1;
    float *dn = dout ? dout + (long)n * drow : nullptr;
    if (dn && blockIdx.y == 0 && chunk == 0 && tid == 0) dn[drow - 1] = 1.0f;
    auto put = [&](long o, float m) {
      pn[o] = m;
      if (cn) cn[o] = m;
      if (dn) dn[o] = m;
    };
    // aout (optional): each window's code (pool_code), N x F x Ho/2 x Wo/2 bytes
    unsigned char *an = aout ? aout + (long)n * g.F * P4 : nullptr;
    if (g.Wo == 32) {  // rows 2i, 2i+1 are blocks j, j+1
#pragma unroll
      for (int j = 0; j + 1 < PB; j += 2) {
        const int pj = p0 + (pw4 * PB + j) * 32;
        const int prow = pj >> 6;
        const bool lead = (l32 & 1) == 0 && pj < p1;
        if (an) {
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const float a = o[j][r], b = o[j + 1][r];
            const float a1 = __shfl_xor(a, 1, 64), b1 = __shfl_xor(b, 1, 64);
            unsigned code;
            const float m = pool_code(a, a1, b, b1, code);
            const int f = f0 + 8 * (r >> 2) + 4 * half + (r & 3);
            const long po = (long)f * P4 + prow * Wo2 + (l32 >> 1);
            if (lead && f < g.F) {
              put(po, m);
              an[po] = (unsigned char)code;
            }
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const float m0 = fmaxf(o[j][r], o[j + 1][r]);
            const float m = fmaxf(m0, __shfl_xor(m0, 1, 64));
            const int f = f0 + 8 * (r >> 2) + 4 * half + (r & 3);
            if (lead && f < g.F) put((long)f * P4 + prow * Wo2 + (l32 >> 1), m);
          }
        }
      }
    } else {  // rows 2i, 2i+1 are lanes l and l ^ Wo of one block
#pragma unroll
      for (int j = 0; j < PB; j++) {
        const int p = p0 + (pw4 * PB + j) * 32 + l32;
        const int row = p / g.Wo, col = p - row * g.Wo;
        const bool lead = (col & 1) == 0 && (row & 1) == 0 && p < p1;
        if (an) {
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const float a = o[j][r];
            const float a1 = __shfl_xor(a, 1, 64), b = __shfl_xor(a, g.Wo, 64);
            const float b1 = __shfl_xor(a, g.Wo ^ 1, 64);
            unsigned code;
            const float m = pool_code(a, a1, b, b1, code);
            const int f = f0 + 8 * (r >> 2) + 4 * half + (r & 3);
            const long po = (long)f * P4 + (row >> 1) * Wo2 + (col >> 1);
            if (lead && f < g.F) {
              put(po, m);
              an[po] = (unsigned char)code;
            }
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const float m0 = fmaxf(o[j][r], __shfl_xor(o[j][r], 1, 64));
            const float m = fmaxf(m0, __shfl_xor(m0, g.Wo, 64));
            const int f = f0 + 8 * (r >> 2) + 4 * half + (r & 3);
            if (lead && f < g.F) put((long)f * P4 + (row >> 1) * Wo2 + (col >> 1), m);
          }
        }
      }
    }
  } else if (rn) {
    store(std::true_type{});
  } else {
    store(std::false_type{});
  }
}

// ---- weight gradient partials ----
//
// Grid: x = image * chunks + chunk (chunk = CH output pixels), y = block of
// FB filters (FB = 16 * FS).  Waves: KS of them split the chunk's pixels
// (4-pixel steps, interleaved), 4/KS groups split the FS x JB grid of 16x16
// output blocks as (FS/MF) x (JB/JW) rectangles of MF x JW blocks.  Partial
// z = blockIdx.x gets part[z][f][k] (k < K) and part[z][f][K] = sum of g.
template <int MF, int JW, int KS, bool VEC, bool ROWS>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 2)))
conv_dw_lds_kernel(const float *__restrict__ gr, const float *__restrict__ x,
                   float *__restrict__ part, Geo g, int chunks, int CH, int FS) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int n = blockIdx.x / chunks, chunk = blockIdx.x - n * chunks;
  const int P = g.Ho * g.Wo;
  const int p0 = chunk * CH;
  const int p1 = min(p0 + CH, P);
  const int np = p1 - p0;
  const int npp = (np + 3) & ~3;
  const int GS = ((npp + 31) & ~31) + 4;   // g row stride: 16 rows x 4 pixels hit distinct banks
  const int FB = 16 * FS;
  const int f0 = blockIdx.y * FB;
  const int JB16 = ((g.K + 15) >> 4) << 4;
  const Slab s = slab_of(g, p0, p1);

  float *gs = smem;                                    // FB x GS (whole 16-byte loads)
  int2 *pixt = (int2 *)(gs + round_up(FB * GS, 256));  // npp pixel entries
  int4 *ktab = (int4 *)(pixt + npp);                   // JB16 tap entries
  float *xs = (float *)(ktab + JB16) + GUARD;          // (C+1) x R x W

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const float *gn = gr + (long)n * g.F * P + (long)f0 * P + p0;
  const int nf = g.F - f0 < FB ? g.F - f0 : FB;
  stage_blocks<VEC>(gs, gn, FB * GS, GS, nf, P, 0, np);
  stage_slab<VEC>(xs, x, g, s, n);
  for (int q = tid; q < npp; q += NT)
    pixt[q] = q < np ? pixel_entry(g, s, p0 + q) : make_int2(0, -(1 << 20));  // masked
  for (int k = tid; k < JB16; k += NT) ktab[k] = tap_entry(g, s, k);
  dma_wait();
  __syncthreads();

  // bias gradient partial: TPR consecutive lanes per filter row
  {
    const int TPR = NT / FB;
    const int f = tid / TPR, sub = tid - f * TPR;
    float sum = 0.0f;
    for (int q = sub; q < np; q += TPR) sum += gs[f * GS + q];
    for (int o = 1; o < TPR; o <<= 1) sum += __shfl_xor(sum, o, 64);
    const int fo = f0 + f;
    if (sub == 0 && fo < g.F) part[((long)blockIdx.x * g.F + fo) * (g.K + 1) + g.K] = sum;
  }

  const int JB = (g.K + 15) >> 4;
  const int ks = wave % KS, grp = wave / KS;
  const int fgroups = FS / MF;
  const int fs0 = (grp % fgroups) * MF, jb0 = (grp / fgroups) * JW;
  const int l16 = lane & 15, q4 = lane >> 4;

  int4 kof[JW];
#pragma unroll
  for (int jw = 0; jw < JW; jw++) {
    const int k = (jb0 + jw) * 16 + l16;
    kof[jw] = k < JB16 ? ktab[k] : make_int4(g.C * slab_cs(s.R, g.W), 0, 0, 0);  // past JB: zero plane
  }

  f32x4 acc[MF][JW];
#pragma unroll
  for (int m = 0; m < MF; m++)
#pragma unroll
    for (int jw = 0; jw < JW; jw++) acc[m][jw] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

  const bool active = jb0 < JB;   // wave-uniform
  if constexpr (ROWS) {
    // Whole output rows (Wo a multiple of 16, chunk = whole rows): wave ks
    // takes rows ks, ks+KS, ...; a row is walked in 16-pixel segments of 4
    // steps whose pixel offsets are immediates.  Lane (tap l16, pixel q4):
    // slab column of step s in a segment at wo0 = (wo0 + 4s + q4)*sw + kw - pw.
    if (active) {
      const int rows = np / g.Wo;
      int cq[JW], bb[JW];
#pragma unroll
      for (int jw = 0; jw < JW; jw++) {
        cq[jw] = q4 * g.sw + kof[jw].y;
        bb[jw] = kof[jw].x + q4 * g.sw;
      }
      const float *ga = gs + (fs0 * 16 + l16) * GS + q4;
      for (int r = ks; r < rows; r += KS) {
        const int pr = r * g.sh * g.W;   // chunk rows start at s.ho0
        for (int wo0 = 0; wo0 < g.Wo; wo0 += 16) {
          const int qb = r * g.Wo + wo0;
          const int pb = pr + wo0 * g.sw;
#pragma unroll
          for (int st = 0; st < 4; st++) {
            float a[MF];
#pragma unroll
            for (int m = 0; m < MF; m++) a[m] = ga[m * 16 * GS + qb + 4 * st];
#pragma unroll
            for (int jw = 0; jw < JW; jw++) {
              const float v = xs[bb[jw] + pb + 4 * st * g.sw];
              const bool ok = (unsigned)(cq[jw] + (wo0 + 4 * st) * g.sw) < (unsigned)g.W;
              const float b = ok ? v : 0.0f;
#pragma unroll
              for (int m = 0; m < MF; m++)
                acc[m][jw] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[m], b, acc[m][jw], 0, 0, 0);
            }
          }
        }
      }
    }
  } else {
  const int nst = npp >> 2;
  const int T = active && nst > ks ? (nst - ks + KS - 1) / KS : 0;
  if (T > 0) {
    // step t covers pixels (ks + t*KS)*4 .. +3 of the chunk
    const float *ga = gs + (fs0 * 16 + l16) * GS + q4;
#pragma unroll 2
    for (int t = 0; t < T; t++) {
      const int st = ks + t * KS;
      const int2 px = pixt[st * 4 + q4];
      float a[MF];
#pragma unroll
      for (int m = 0; m < MF; m++) a[m] = ga[m * 16 * GS + st * 4];
#pragma unroll
      for (int jw = 0; jw < JW; jw++) {
        const float b = slab_read(xs, kof[jw], px, g.W);
#pragma unroll
        for (int m = 0; m < MF; m++)
          acc[m][jw] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[m], b, acc[m][jw], 0, 0, 0);
      }
    }
  }
  }

  if constexpr (KS > 1) {
    // the KS pixel-split waves of a group add their accumulators in order
    __syncthreads();  // every wave is done reading the slab: reuse it
    float *red = xs;
    constexpr int PER = MF * JW * 4;
    if (ks > 0) {
#pragma unroll
      for (int m = 0; m < MF; m++)
#pragma unroll
        for (int jw = 0; jw < JW; jw++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            red[(((grp * (KS - 1) + ks - 1) * PER) + (m * JW + jw) * 4 + r) * 64 + lane] =
                acc[m][jw][r];
    }
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int o = 1; o < KS; o++)
#pragma unroll
      for (int m = 0; m < MF; m++)
#pragma unroll
        for (int jw = 0; jw < JW; jw++)
#pragma unroll
          for (int r = 0; r < 4; r++)
            acc[m][jw][r] +=
                red[(((grp * (KS - 1) + o - 1) * PER) + (m * JW + jw) * 4 + r) * 64 + lane];
  }
  if (jb0 >= JB) return;

  float *pz = part + (long)blockIdx.x * g.F * (g.K + 1);
#pragma unroll
  for (int jw = 0; jw < JW; jw++) {
    const int k = (jb0 + jw) * 16 + l16;
    if (k >= g.K) continue;
#pragma unroll
    for (int m = 0; m < MF; m++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int f = f0 + (fs0 + m) * 16 + 4 * q4 + r;
        if (f < g.F) pz[(long)f * (g.K + 1) + k] = acc[m][jw][r];
      }
  }
}

// ---- weight gradient partials on 32x32x2 MFMAs (even Wo, whole rows) ----
//
// Block (32 filters) x (32 taps) per MFMA, two output pixels per step: lane
// l feeds A[f = l%32][pixel h = l/32] = g and B[pixel h][tap l%32] = the
// slab; accumulator r holds filter 8(r/4) + 4h + r%4, tap l%32.  Grid: x =
// image * chunks + chunk (chunk = whole output rows), y = block of 32
// filters.  Waves: 4/KS groups take JW tap blocks each, the KS waves of a
// group take rows ks, ks+KS, ...; each row is walked two pixels a step with
// the pixel offsets as immediates (4 steps unrolled).  Measured on gfx950
// the 32x32x2 form runs ~20% faster than 16x16x4.
template <int JW, int KS, bool VEC>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 2)))
conv_dw32_kernel(const float *__restrict__ gr, const float *__restrict__ x,
                 float *__restrict__ part, Geo g, int chunks, int CH) {
  extern __shared__ __attribute__((aligned(16))) float smem[];
  constexpr int FB = 32;
  const int n = blockIdx.x / chunks, chunk = blockIdx.x - n * chunks;
  const int P = g.Ho * g.Wo;
  const int p0 = chunk * CH;
  const int p1 = min(p0 + CH, P);
  const int np = p1 - p0;
  const int GS = ((np + 31) & ~31) + 4;
  const int f0 = blockIdx.y * FB;
  const int JB = (g.K + 31) >> 5;                  // 32-tap blocks
  const Slab s = slab_of(g, p0, p1);

  float *gs = smem;                                       // FB x GS
  int4 *ktab = (int4 *)(gs + round_up(FB * GS, 256));     // 32*JB tap entries
  float *xs = (float *)(ktab + 32 * JB) + GUARD;          // (C+1) x R x W

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const float *gn = gr + (long)n * g.F * P + (long)f0 * P + p0;
  const int nf = g.F - f0 < FB ? g.F - f0 : FB;
  stage_blocks<VEC>(gs, gn, FB * GS, GS, nf, P, 0, np);
  // 16-byte staging: the gapped slab (no masks in the loop)
  if constexpr (VEC) {
    stage_gslab(xs, x, g, s, n);
    for (int k = tid; k < 32 * JB; k += NT) ktab[k] = make_int4(gslab_tap(g, s, k), 0, 0, 0);
  } else {
    stage_slab<VEC>(xs, x, g, s, n);
    for (int k = tid; k < 32 * JB; k += NT) ktab[k] = tap_entry(g, s, k);
  }
  dma_wait();
  __syncthreads();

  // this workgroup's partial: JB blocks of 16 x 64 accumulators (the MFMA
  // register layout, so every store is 256 contiguous bytes), then the 32
  // bias sums
  float *pz = part + ((long)blockIdx.x * gridDim.y + blockIdx.y) * (JB * 1024 + 32);
  {  // bias gradient partial: 8 consecutive lanes per filter row
    const int f = tid >> 3, sub = tid & 7;
    float sum = 0.0f;
    for (int q = sub; q < np; q += 8) sum += gs[f * GS + q];
    for (int o = 1; o < 8; o <<= 1) sum += __shfl_xor(sum, o, 64);
    if (sub == 0) pz[JB * 1024 + f] = sum;
  }

  const int ks = wave % KS, grp = wave / KS;
  const int jb0 = grp * JW;
  const int l32 = lane & 31, h = lane >> 5;
  int bb[JW], cq[JW];
#pragma unroll
  for (int jw = 0; jw < JW; jw++) {
    const int k = (jb0 + jw) * 32 + l32;
    const int zplane = g.C * (VEC ? gslab_cs(s.R, g) : slab_cs(s.R, g.W));
    const int4 t = k < 32 * JB ? ktab[k] : make_int4(zplane, 0, 0, 0);
    bb[jw] = t.x + h * g.sw;      // slab offset of (tap, pixel h) at the row start
    cq[jw] = t.y + h * g.sw;      // its column relative to wo*sw
  }
  f32x16 acc[JW];
#pragma unroll
  for (int jw = 0; jw < JW; jw++)
    for (int r = 0; r < 16; r++) acc[jw][r] = 0.0f;

  if (jb0 < JB) {
    // this wave's steps: rows ks, ks+KS, ... of the chunk, Wo/2 steps a row;
    // the operands of step t+1 are read before the MFMAs of step t
    const int rows = np / g.Wo;
    const int half_w = g.Wo >> 1;
    const int T = rows > ks ? ((rows - ks + KS - 1) / KS) * half_w : 0;
    const float *ga = gs + l32 * GS + h;
    // (scalar) offsets of the current step: g column qa, slab offset xo,
    // column col; a step adds 2 pixels, a row end jumps KS rows ahead
    const int RS = VEC ? gslab_rw(g) : g.W;  // slab row stride
    const int qstep_row = KS * g.Wo - 2 * half_w, xstep_row = KS * g.sh * RS - 2 * half_w * g.sw;
    auto load = [&](int qa, int xo, float &a, float (&b)[JW]) {  // raw: masked at use
      a = ga[qa];
#pragma unroll
      for (int jw = 0; jw < JW; jw++) b[jw] = xs[bb[jw] + xo];
    };
    auto advance = [&](int &qa_, int &xo_, int &st_) {
      qa_ += 2;
      xo_ += 2 * g.sw;
      if (++st_ == half_w) { st_ = 0; qa_ += qstep_row; xo_ += xstep_row; }
    };
    auto mfmas = [&](float a, const float (&b)[JW], int st_) {
      const int col = 2 * st_ * g.sw;
#pragma unroll
      for (int jw = 0; jw < JW; jw++) {
        const float bm = VEC || (unsigned)(cq[jw] + col) < (unsigned)g.W ? b[jw] : 0.0f;
        acc[jw] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, bm, acc[jw], 0, 0, 0);
      }
    };
    // two operand sets in turn: a step's operands are read a whole step
    // before its MFMAs (a read past the last step re-reads the last one)
    int qa = ks * g.Wo, xo = ks * g.sh * RS, st = 0;
    float a0 = 0.0f, b0[JW], a1, b1[JW];
    if (T > 0) load(qa, xo, a0, b0);
    int t = 0;
    for (; t + 1 < T; t += 2) {
      int qa1 = qa, xo1 = xo, st1 = st;
      advance(qa1, xo1, st1);
      load(qa1, xo1, a1, b1);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a0, b0, st);
      __builtin_amdgcn_sched_barrier(0);
      int qa2 = qa1, xo2 = xo1, st2 = st1;
      advance(qa2, xo2, st2);
      const bool more = t + 2 < T;
      load(more ? qa2 : qa1, more ? xo2 : xo1, a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a1, b1, st1);
      __builtin_amdgcn_sched_barrier(0);
      qa = qa2;
      xo = xo2;
      st = st2;
    }
    if (t < T) mfmas(a0, b0, st);
  }

  if constexpr (KS > 1) {
    // the KS row-split waves of a group add their accumulators in order
    __syncthreads();  // operands no longer read: reuse the whole LDS
    float *red = smem;
    constexpr int PER = JW * 16;
    if (ks > 0) {
#pragma unroll
      for (int jw = 0; jw < JW; jw++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          red[((grp * (KS - 1) + ks - 1) * PER + jw * 16 + r) * 64 + lane] = acc[jw][r];
    }
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int o = 1; o < KS; o++)
#pragma unroll
      for (int jw = 0; jw < JW; jw++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          acc[jw][r] += red[((grp * (KS - 1) + o - 1) * PER + jw * 16 + r) * 64 + lane];
  }
  if (jb0 >= JB) return;
#pragma unroll
  for (int jw = 0; jw < JW; jw++) {
    if (jb0 + jw >= JB) break;
#pragma unroll
    for (int r = 0; r < 16; r++) pz[((jb0 + jw) * 16 + r) * 64 + lane] = acc[jw][r];
  }
}

// Sum of the dw32 partials.  A workgroup takes XL consecutive groups of 4
// partial elements (16-byte loads) x ZL lanes: lane ty adds partials z = ty,
// ty+ZL, ... in order, lane 0 adds the ZL sums in order, and writes the
// gradient entries the elements hold: block jb, accumulator r, lane l ->
// filter fb*32 + 8(r/4) + 4(l/32) + r%4, tap jb*32 + l%32; the last 32 of a
// block -> bias.  Partials are JB*1024 + 32 floats (a multiple of 4).
template <int ZL>
__global__ void __launch_bounds__(NT)
conv_dw32_reduce_kernel(const float *__restrict__ part, float *__restrict__ dw,
                        float *__restrict__ db, int Z, int FBLK, int JB, int F, int K) {
  constexpr int XL = NT / ZL;
  __shared__ f32x4 sums[ZL][XL];
  const int tx = threadIdx.x % XL, ty = threadIdx.x / XL;
  const int S = JB * 1024 + 32;
  const long total4 = (long)FBLK * S / 4;
  const long e4 = (long)blockIdx.x * XL + tx;
  f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
  if (e4 < total4) {
    const f32x4 *p = (const f32x4 *)part + e4;
#pragma unroll 8
    for (int z = ty; z < Z; z += ZL) sum += p[(long)z * total4];
  }
  sums[ty][tx] = sum;
  __syncthreads();
  if (ty != 0 || e4 >= total4) return;
  for (int j = 1; j < ZL; j++) sum += sums[j][tx];
#pragma unroll
  for (int u = 0; u < 4; u++) {
    const long e = e4 * 4 + u;
    const int fb = (int)(e / S), i = (int)(e - (long)fb * S);
    if (i >= JB * 1024) {
      const int f = fb * 32 + (i - JB * 1024);
      if (db && f < F) db[f] = sum[u];
      continue;
    }
    const int jb = i >> 10, r = (i >> 6) & 15, l = i & 63;
    const int f = fb * 32 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    const int k = jb * 32 + (l & 31);
    if (f < F && k < K) dw[(long)f * K + k] = sum[u];
  }
}

// ---- weight gradient, one workgroup per (output rows of one image, taps, filters) ----
//
// Workgroup (u, ts, fb) computes the dW contribution of unit u (RC output
// rows of one image) for filters [32 fb, 32 fb + 32) and the taps of tap
// set ts (NTGW groups of TG blocks of 32 taps).  It stages the unit's output
// gradient rows (32 filters) and the input rows they need (the channels of
// the tap set, gapped slab) once, with 16-byte direct loads.  Wave w takes
// tap group w / 4 of the set and the rows pq, pq + 4, ... (pq = w % 4) of
// the unit, so the 4 SIMDs of a CU get equal shares and g and x are read
// once per workgroup.  (Staging in two phases, the first phase's MFMAs
// running while the second's loads are in flight, measured slower: the
// loads of all workgroups are bandwidth-bound together.)
// The 4 waves of a tap group add their accumulators through LDS
// ((0 + 2) + (1 + 3)) and wave pq = 0 writes the unit's partial block, which
// conv_dwt_reduce_kernel sums over the units in unit order.  MFMA operands
// as conv_dw32_kernel: lane l feeds A[f = l%32][pixel h = l/32] = g and
// B[pixel h][tap l%32] = the gapped slab; accumulator r of block jb holds
// filter 8(r/4) + 4h + r%4, tap 32 jb + l%32.  The bias gradient is summed
// on the VALU from the same A operands (first group of the first tap set).
constexpr int DWT_NPQ = 4;  // waves sharing a tap group (pixel quarters)
constexpr int DWT_UB = 8;   // pooled-gradient items a lane decodes per batch
constexpr int DWT_UPL = 16;  // units of partials a reduction lane adds (at most; 4, 8 slower)

// CODE: gr is the gradient of a 2x2 / stride-2 max pool of the relu of this
// convolution's output (N x F x Ho/2 x Wo/2) and codes its windows' codes
// (pool_code): the output gradient rows are decoded into LDS as the pool +
// relu backward would have written them (maxpool2x2_code_bwd_kernel), so
// that gradient is never stored.  Needs even RC (or one unit per image),
// even Ho and Wo % 8 == 0.
// The workgroup (u, ts, fb) of nu units; every thread of a workgroup of
// 64 * DWT_NPQ * NTGW calls it.
template <int TG, int NTGW, bool CODE = false>
__device__ __forceinline__ void conv_dwt_block(const float *__restrict__ gr,
                                               const float *__restrict__ x,
                                               float *__restrict__ part, const Geo &g, int RC,
                                               int nch, int GS, int CS, int RW, int jbp,
                                               const unsigned char *__restrict__ codes, int u,
                                               int ts, int fb, int nu) {
  constexpr int NTH = 64 * DWT_NPQ * NTGW;
  constexpr int SLOT = TG * 1024 + 64;  // one wave's accumulators and bias in LDS
  extern __shared__ __attribute__((aligned(16))) float smem[];
  const int n = u / nch, ho0 = (u - n * nch) * RC;
  const int rows = min(g.Ho, ho0 + RC) - ho0;
  const int P = g.Ho * g.Wo;
  const int f0 = fb * 32;
  const int nf = g.F - f0 < 32 ? g.F - f0 : 32;
  const int taps = g.HH * g.WW;
  const int kts = ts * NTGW * TG * 32;  // first tap of the set
  const int c0 = kts / taps;
  const int c1 = min(g.C, (min(g.K, kts + NTGW * TG * 32) + taps - 1) / taps);
  const int nc = c1 - c0;
  const int G = RW - g.W;  // zeros before each row's W floats (rows of RW)
  const int R = (rows - 1) * g.sh + g.HH;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tgw = wave / DWT_NPQ, pq = wave - tgw * DWT_NPQ;
  const int l32 = lane & 31, h = lane >> 5;
  const float *gs = smem;
  const float *xs = smem + round_up(32 * GS, 256);

  // stage the gapped slab of channels [c0, c1) and a zero plane, then g
  {
    const int hs = ho0 * g.sh - g.ph;
    const int T = (nc + 1) * CS;
    const float rcpC = 1.0f / (float)CS, rcpR = 1.0f / (float)RW;
    const float *xn = x + ((long)n * g.C + c0) * g.H * g.W;
    if (((RW | CS | G) & 3) == 0) {  // whole 16-byte runs
      for (int base = wave * 256; base < T; base += NTH * 4) {
        const int i = base + lane * 4;
        const int c = fdiv(i, CS, rcpC), rem = i - c * CS;
        const int slot = fdiv(rem, RW, rcpR), j = rem - slot * RW;
        const int row = hs + slot;
        const bool ok = i < T && c < nc && slot < R && j >= G && row >= 0 && row < g.H;
        dma_dwordx4(ok ? xn + ((long)c * g.H + row) * g.W + (j - G) : g_zero_src,
                    xs + base);
      }
    } else {  // a layout of odd strides: element by element
      for (int base = wave * 64; base < T; base += NTH) {
        const int i = base + lane;
        const int c = fdiv(i, CS, rcpC), rem = i - c * CS;
        const int slot = fdiv(rem, RW, rcpR), j = rem - slot * RW;
        const int row = hs + slot;
        const bool ok = i < T && c < nc && slot < R && j >= G && row >= 0 && row < g.H;
        dma_dword(ok ? xn + ((long)c * g.H + row) * g.W + (j - G) : g_zero_src, xs + base);
      }
    }
  }
  // stage g rows (32 x GS) -- after the slab's DMA is issued, so a decode
  // (CODE) waits on its own loads while the slab is in flight
  if constexpr (CODE) {
    // four pixels of one row a lane: two pool windows (a 2-byte code pair,
    // a float2 of the pooled gradient), written with one 16-byte LDS store;
    // DWT_UB items a lane at a time, all their loads issued (unconditional,
    // out-of-range items read window 0) before any is decoded
    const int Ho2 = g.Ho >> 1, Wo2 = g.Wo >> 1, RWo = rows * g.Wo;
    const int q4 = GS >> 2, T4 = 32 * q4;
    const float rcpQ = 1.0f / (float)q4, rcpW = 1.0f / (float)(g.Wo >> 2);
    const long wbase = ((long)(n * g.F + f0) * Ho2 + (ho0 >> 1)) * Wo2;
    for (int base = tid; base < T4; base += NTH * DWT_UB) {
      unsigned c2[DWT_UB], kk[DWT_UB];
      float2 gv[DWT_UB];
      bool ok[DWT_UB];
#pragma unroll
      for (int u = 0; u < DWT_UB; u++) {
        const int i = base + u * NTH;
        const int b = fdiv(i, q4, rcpQ), j = (i - b * q4) * 4;
        ok[u] = i < T4 && b < nf && j < RWo;
        const int hr = fdiv(j >> 2, g.Wo >> 2, rcpW);  // row within the unit
        const int wo = j - hr * g.Wo;
        const long w2 = ok[u] ? wbase + ((long)b * Ho2 + (hr >> 1)) * Wo2 + (wo >> 1) : 0;
        kk[u] = ((ho0 + hr) & 1) * 2;
        c2[u] = *reinterpret_cast<const unsigned short *>(codes + w2);
        gv[u] = *reinterpret_cast<const float2 *>(gr + w2);
      }
#pragma unroll
      for (int u = 0; u < DWT_UB; u++) {
        const int i = base + u * NTH;
        if (i >= T4) break;
        const float g0 = 0.0f + gv[u].x, g1 = 0.0f + gv[u].y;
        const unsigned k = kk[u], ca = c2[u] & 0xff, cb = c2[u] >> 8;
        auto at = [](unsigned c, unsigned kq, float val) {
          return ((c & 3) == kq && ((c >> (2 + kq)) & 1)) ? val : 0.0f;
        };
        const float4 v = ok[u] ? make_float4(at(ca, k, g0), at(ca, k + 1, g0), at(cb, k, g1),
                                             at(cb, k + 1, g1))
                               : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        *reinterpret_cast<float4 *>(smem + i * 4) = v;
      }
    }
  } else {
    stage_blocks<true, NTH>(smem, gr + (long)n * g.F * P + (long)f0 * P + (long)ho0 * g.Wo,
                            32 * GS, GS, nf, P, 0, rows * g.Wo);
  }

  // this lane's tap offsets inside the slab (taps past K: the zero plane)
  const int kt0 = kts + tgw * TG * 32;
  int bb[TG];
#pragma unroll
  for (int jw = 0; jw < TG; jw++) {
    const int k = kt0 + jw * 32 + l32;
    int off = nc * CS;
    if (k < g.K) {
      const int c = k / taps - c0, t = k % taps;
      const int kh = t / g.WW, kw = t - kh * g.WW;
      off = c * CS + kh * RW + G + kw - g.pw;
    }
    bb[jw] = off;
  }
  f32x16 acc[TG];
#pragma unroll
  for (int jw = 0; jw < TG; jw++)
#pragma unroll
    for (int r = 0; r < 16; r++) acc[jw][r] = 0.0f;
  float bsum = 0.0f;
  dma_wait();
  __syncthreads();
  TT_PROBE(1, 5);

  // items (row, quad): rows pq, pq+4, ... of the unit; lane half h takes
  // the pixels [h*Wo/2, h*Wo/2 + Wo/2) of a row, four at a time: one 16-byte
  // read of g (rows of GS = 4 mod 32 floats: eight lanes of a read cover the
  // 32 banks) feeds four MFMA steps.  Two operand sets in turn: the next
  // item's operands are read into one while the current item's MFMAs use
  // the other (no register copies in the loop).
  const int half_w = g.Wo >> 1;
  const int quads = half_w >> 2;
  const int xh = h * half_w * g.sw;
  const int xstep = DWT_NPQ * g.sh * RW - quads * 4 * g.sw;  // next row, first quad
  const int gstep = DWT_NPQ * g.Wo - quads * 4;
  const int nrow = kt0 < g.K && rows > pq ? (rows - pq + DWT_NPQ - 1) / DWT_NPQ : 0;
  const int nit = nrow * quads;
  const float *ga = gs + l32 * GS + h * half_w;
  {
    int go = pq * g.Wo, xo = pq * g.sh * RW + xh;  // item offsets into g and the slab
    int qd = 0, left = nit;
    // step to the next item (the last item stays put, so a read past the
    // end re-reads it)
    auto advance = [&]() {
      if (--left <= 0) return;
      if (++qd == quads) {
        qd = 0;
        go += gstep + 4;
        xo += xstep + 4 * g.sw;
      } else {
        go += 4;
        xo += 4 * g.sw;
      }
    };
    auto load = [&](f32x4 &a4, float (&bv)[4][TG]) {
      a4 = *(const f32x4 *)(ga + go);
#pragma unroll
      for (int e = 0; e < 4; e++)
#pragma unroll
        for (int jw = 0; jw < TG; jw++) bv[e][jw] = xs[bb[jw] + xo + e * g.sw];
    };
    auto mfmas = [&](const f32x4 &a4, const float (&bv)[4][TG]) {
#pragma unroll
      for (int e = 0; e < 4; e++)
#pragma unroll
        for (int jw = 0; jw < TG; jw++)
          acc[jw] = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[e], bv[e][jw], acc[jw], 0, 0, 0);
      bsum += (a4[0] + a4[1]) + (a4[2] + a4[3]);
    };
    f32x4 a0, a1;
    float b0[4][TG], b1[4][TG];
    if (nit > 0) load(a0, b0);
#pragma unroll 1
    for (int it = 0; it < nit; it += 2) {
      advance();
      load(a1, b1);  // item it+1 (or it again)
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      if (it + 1 >= nit) break;
      advance();
      load(a0, b0);  // item it+2
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a1, b1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  bsum += __shfl_xor(bsum, 32, 64);  // both halves of filter l32
  TT_PROBE(1, 6);

  // add the DWT_NPQ waves of each tap group: (0 + 2) + (1 + 3), through LDS
#pragma unroll
  for (int s = DWT_NPQ / 2; s >= 1; s >>= 1) {
    __syncthreads();
    if (pq >= s && pq < 2 * s) {
      float *d = smem + (tgw * s + pq - s) * SLOT;
#pragma unroll
      for (int jw = 0; jw < TG; jw++)
#pragma unroll
        for (int r = 0; r < 16; r++) d[(jw * 16 + r) * 64 + lane] = acc[jw][r];
      d[TG * 1024 + lane] = bsum;
    }
    __syncthreads();
    if (pq < s) {
      const float *d = smem + (tgw * s + pq) * SLOT;
#pragma unroll
      for (int jw = 0; jw < TG; jw++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[jw][r] += d[(jw * 16 + r) * 64 + lane];
      bsum += d[TG * 1024 + lane];
    }
  }
  if (pq != 0) return;
  float *pz = part + ((long)fb * nu + u) * ((long)jbp * 1024 + 32);
  const int jb0 = (ts * NTGW + tgw) * TG;
#pragma unroll
  for (int jw = 0; jw < TG; jw++)
#pragma unroll
    for (int r = 0; r < 16; r++) pz[((jb0 + jw) * 16 + r) * 64 + lane] = acc[jw][r];
  if (ts == 0 && tgw == 0 && lane < 32) pz[jbp * 1024 + lane] = bsum;
}

template <int TG, int NTGW, bool CODE = false>
__global__ void __launch_bounds__(64 * DWT_NPQ * NTGW)
conv_dwt_kernel(const float *__restrict__ gr, const float *__restrict__ x,
                float *__restrict__ part, Geo g, int RC, int nch, int GS, int CS, int RW,
                int jbp, const unsigned char *__restrict__ codes) {
  conv_dwt_block<TG, NTGW, CODE>(gr, x, part, g, RC, nch, GS, CS, RW, jbp, codes, blockIdx.x,
                                 blockIdx.y, blockIdx.z, gridDim.x);
}

// dW / db from the dwt partials: each lane owns 4 consecutive elements of a
// filter block's partial (16-byte loads; a wave's loads cover whole 1 KB
// runs) and adds the units z, z+ZL, ... in order, 8 loads in flight; the ZL
// lanes of an element are then added in lane order.
// One workgroup's share of the reduction: block blk of the columns (dw or
// db NULL: that output is not written).
// wdw / wdb (optional): the weights and bias dw / db are the gradients of;
// each gets the SGD step w -= lr * g from the value just stored (the same
// arithmetic as sgd_multi_kernel, without contraction).
template <int ZL>
__device__ __forceinline__ void dwt_reduce_block(int blk, f32x4 *sums,
                                                 const float *__restrict__ part,
                                                 float *__restrict__ dw, float *__restrict__ db,
                                                 int nu, int nfb, int jbp, int F, int K,
                                                 float *__restrict__ wdw = nullptr,
                                                 float *__restrict__ wdb = nullptr,
                                                 float lr = 0.0f) {
  constexpr int XL = NT / ZL;  // 4-element columns per workgroup
  const int S4 = (jbp * 1024 + 32) / 4;
  const int tx = threadIdx.x % XL, ty = threadIdx.x / XL;
  const long e4 = (long)blk * XL + tx;
  const bool in = e4 < (long)nfb * S4;
  const long ec = in ? e4 : 0;
  const int fb = (int)(ec / S4), i4 = (int)(ec - (long)fb * S4);
  const f32x4 *p = (const f32x4 *)part + (long)fb * nu * S4 + i4;
  // the weights the step changes, loaded before the partials (loaded after
  // the sum, they cost one more memory round trip before the stores)
  const int i = i4 * 4;
  const bool isb = i >= jbp * 1024;
  const int jb = i >> 10, r = (i >> 6) & 15, l = i & 63;
  const int f = fb * 32 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
  const int k = jb * 32 + (l & 31);
  float wpre[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (ty == 0 && in) {
    if (isb) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int fe = fb * 32 + (i + e - jbp * 1024);
        if (wdb && fe < F) wpre[e] = wdb[fe];
      }
    } else if (wdw && f < F) {
#pragma unroll
      for (int e = 0; e < 4; e++)
        if (k + e < K) wpre[e] = wdw[(long)f * K + k + e];
    }
  }
  f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int q0 = ty; q0 < nu; q0 += 8 * ZL) {
    f32x4 t[8];
#pragma unroll
    for (int k = 0; k < 8; k++) t[k] = p[(long)min(q0 + k * ZL, nu - 1) * S4];
#pragma unroll
    for (int k = 0; k < 8; k++)
      if (q0 + k * ZL < nu) v += t[k];
  }
  sums[ty * XL + tx] = v;
  __syncthreads();
  if (ty != 0 || !in) return;
  for (int z = 1; z < ZL; z++) v += sums[z * XL + tx];
  if (isb) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int fe = fb * 32 + (i + e - jbp * 1024);
      if (db && fe < F) db[fe] = v[e];
      if (wdb && fe < F) wdb[fe] = wpre[e] - lr * v[e];
    }
    return;
  }
  if (f >= F || !dw) return;
#pragma unroll
  for (int e = 0; e < 4; e++)
    if (k + e < K) {
      dw[(long)f * K + k + e] = v[e];
      if (wdw) wdw[(long)f * K + k + e] = wpre[e] - lr * v[e];
    }
}

template <int ZL>
__global__ void __launch_bounds__(NT)
conv_dwt_reduce_kernel(const float *__restrict__ part, float *__restrict__ dw,
                       float *__restrict__ db, int nu, int nfb, int jbp, int F, int K) {
  __shared__ f32x4 sums[NT];
  dwt_reduce_block<ZL>(blockIdx.x, sums, part, dw, db, nu, nfb, jbp, F, K);
}

// Up to DWT_JOBS deferred reductions in one launch: blocks [start[q],
// start[q+1]) take job q, each exactly as its own conv_dwt_reduce_kernel.
constexpr int DWT_JOBS = 4;
struct DwtJobs {
  TTDwtJob j[DWT_JOBS];
  int start[DWT_JOBS + 1];
  int n;
};
__global__ void __launch_bounds__(NT) conv_dwt_reduce_multi_kernel(DwtJobs js) {
  __shared__ f32x4 sums[NT];
  int q = 0;
  while (q + 1 < js.n && (int)blockIdx.x >= js.start[q + 1]) q++;
  const TTDwtJob &j = js.j[q];
  const int blk = blockIdx.x - js.start[q];
  switch (j.zl) {
#define TT_DJ(ZL_)                                                                         \
  case ZL_:                                                                                \
    dwt_reduce_block<ZL_>(blk, sums, j.part, j.dw, j.db, j.nu, j.nfb, j.jbp, j.F, j.K);    \
    break;
    TT_DJ(1) TT_DJ(2) TT_DJ(4) TT_DJ(8) TT_DJ(16) TT_DJ(32) TT_DJ(64)
#undef TT_DJ
  }
}

// dw[f][k] = sum_z part[z][f][k] (k < K), db[f] = sum_z part[z][f][K]; ZL
// lanes per output each add every ZL-th partial in order, then lane 0 adds
// the ZL sums in order.
template <int ZL>
__global__ void __launch_bounds__(NT)
conv_dw_reduce_kernel(const float *__restrict__ part, float *__restrict__ dw,
                      float *__restrict__ db, int Z, int F, int K) {
  constexpr int XL = NT / ZL;
  __shared__ float sums[ZL][XL];
  const int tx = threadIdx.x % XL, ty = threadIdx.x / XL;
  const int total = F * (K + 1);
  const int idx = blockIdx.x * XL + tx;
  float s = 0.0f;
  if (idx < total)
    for (int z = ty; z < Z; z += ZL) s += part[(long)z * total + idx];
  sums[ty][tx] = s;
  __syncthreads();
  if (ty != 0 || idx >= total) return;
  for (int j = 1; j < ZL; j++) s += sums[j][tx];
  const int f = idx / (K + 1), k = idx - f * (K + 1);
  if (k < K) dw[(long)f * K + k] = s;
  else if (db) db[f] = s;
}

// ---- host-side planning ----

bool geo_ok(long N, long C, long H, long W, long F, long HH, long WW, long sh, long sw, long ph,
            long pw, long Ho, long Wo) {
  if (N <= 0 || C <= 0 || H <= 0 || W <= 0 || F <= 0 || HH <= 0 || WW <= 0 || sh <= 0 ||
      sw <= 0 || ph < 0 || pw < 0 || Ho <= 0 || Wo <= 0)
    return false;
  if (Ho != (H + 2 * ph - HH) / sh + 1 || Wo != (W + 2 * pw - WW) / sw + 1) return false;
  const long lim = 0x7fffffffL;
  // pixel and tap indices go through a float-reciprocal division (< 2^24);
  // reads at column -pw stay inside the guard before the slab
  return N * C * H * W < lim && N * F * Ho * Wo < lim && C * HH * WW < 65536 &&
         Ho * Wo < (1L << 24) && N < 65536L * 16 && pw < GUARD;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Most output rows a run of L consecutive pixels can touch.
inline int rows_spanned(int L, int Wo) { return (L + Wo - 2) / Wo + 1; }

// LDS floats of the slab for L consecutive output pixels, rounded to whole
// 256-float runs of 16-byte loads (LDS_MAX / 4 + 1 when it cannot fit)
inline long slab_floats(const Geo &g, int L) {
  const long R = (long)(rows_spanned(L, g.Wo) - 1) * g.sh + g.HH;
  const long f = (long)(g.C + 1) * (R * g.W + 4);
  if (f > LDS_MAX / 4) return LDS_MAX / 4 + 1;
  return round_up((int)f, 256);
}

// TT_FAIL_DIRECT_CONV=1 (environment, read once): every launch of the direct
// forward / dX kernels reports a launch failure although the planner covers
// the shape, so the callers' fallbacks can be tested.
bool fail_direct() {
  static int v = -1;
  if (v < 0) {
    const char *e = getenv("TT_FAIL_DIRECT_CONV");
    v = (e && *e && *e != '0') ? 1 : 0;
  }
  return v == 1;
}

// Kernels that take more than 64 KB of dynamic LDS need the limit raised
// once per function (the runtime call is slow enough to show up per launch).
bool allow_big_lds(const void *fn) {
  static const void *done[32];
  static int ndone = 0;
  for (int i = 0; i < ndone; i++)
    if (done[i] == fn) return true;
  if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)LDS_MAX) !=
      hipSuccess)
    return false;
  if (ndone < 32) done[ndone++] = fn;
  return true;
}

struct FwdPlan {
  int pb = 0, chunks = 0, ks = 1;
  size_t lds = 0;
};

inline bool is_k3(const Geo &g) { return g.HH == 3 && g.WW == 3; }

FwdPlan plan_fwd(const Geo &g, int N, bool flip) {
  FwdPlan best;
  const int P = g.Ho * g.Wo;
  const int Kp = (g.K + 7) & ~7;
  const int fblocks = (g.F + 31) / 32;
  const int K2 = 2 * ((g.C + 1) / 2) * g.HH * g.WW;  // 3x3 kernel: channels padded to even
  for (int pb = 2; pb >= 1; pb--) {
    const int chunk = 128 * pb;
    const int chunks = (P + chunk - 1) / chunk;
    long sf = slab_floats(g, chunk < P ? chunk : P);
    if (is_k3(g) && g.W % 4 == 0) {  // 16-byte staging takes the gapped slab (larger)
      const long R = (long)(rows_spanned(chunk < P ? chunk : P, g.Wo) - 1) * g.sh + g.HH;
      const long gx = round_up((int)min((long)(g.C + 1) * (R * gslab_rw(g) + 4), (long)LDS_MAX), 256);
      if (gx > sf) sf = gx;
    }
    long wsz, tabsz;
    if (is_k3(g)) {
      wsz = flip ? round_up(K2 * 32, 256) : round_up(32 * wrow_stride(K2), 256);
      tabsz = 0;
    } else {
      wsz = flip ? round_up(g.K * 32, 256) : round_up(32 * wrow_stride(Kp), 256);
      tabsz = 4L * Kp;
    }
    const long lds = 4L * (wsz + tabsz + 64 + GUARD + sf);
    if (lds > LDS_MAX) continue;
    best.pb = pb;
    best.chunks = chunks;
    best.lds = (size_t)lds;
    // the wider chunk amortises the slab halo; take it while the grid still
    // gives every CU two workgroups
    if ((long)N * chunks * fblocks >= 512) break;
  }
  // a workgroup that takes more than half the LDS runs alone on its CU: the
  // 3x3 kernel then splits the channel steps over eight waves (two per SIMD)
  // and adds the halves through LDS (PB x 16 KB, reusing the operands' space)
  if (best.pb && is_k3(g) && ((g.C + 1) / 2) % 2 == 0 && best.lds > (size_t)LDS_MAX / 2 &&
      best.lds >= (size_t)best.pb * 16384)
    best.ks = 2;
  return best;
}

// The 3x3 forward kernel can also write the 2x2 / stride-2 max pool of its
// relu: even Ho and Wo, chunks starting on even rows, and a row pair inside one
// 32-pixel block (32 % Wo == 0, 32 / Wo even) or two consecutive blocks
// (Wo == 32, two blocks per wave).
bool pool_fusable(const Geo &g, const FwdPlan &pl) {
  const int chunk = 128 * pl.pb;
  if (!is_k3(g) || g.Ho % 2 || g.Wo % 2 || chunk % (2 * g.Wo)) return false;
  if (g.Wo == 32) return pl.pb % 2 == 0;
  return g.Wo < 32 && 32 % g.Wo == 0 && (32 / g.Wo) % 2 == 0;
}

template <int PB, bool FLIP, bool VEC>
int launch_fwd(const float *x, const float *w, const float *bias, float *out, float *rout,
               float *pout, float *cout, float *dout, unsigned char *aout, const Geo &g, int N,
               const FwdPlan &pl) {
  auto kern = !is_k3(g)     ? conv_fwd_lds_kernel<PB, FLIP, VEC>
              : pl.ks == 2 ? conv_fwd_k_kernel<PB, FLIP, VEC, 3, 3, 2>
                           : conv_fwd_k_kernel<PB, FLIP, VEC, 3, 3, 1>;
  if (pl.lds > 64 * 1024 && !allow_big_lds((const void *)kern)) return -1;
  const dim3 grid((unsigned)(N * pl.chunks), (unsigned)((g.F + 31) / 32));
  hipLaunchKernelGGL(kern, grid, dim3(NT * pl.ks), pl.lds, stream(), x, w, bias, out, rout, pout,
                     cout, dout, aout, g, pl.chunks);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

template <bool FLIP>
int run_fwd(const float *x, const float *w, const float *bias, float *out, const Geo &g, int N,
            bool dry, float *rout = nullptr, float *pout = nullptr, float *cout = nullptr,
            float *dout = nullptr, unsigned char *aout = nullptr) {
  const FwdPlan pl = plan_fwd(g, N, FLIP);
  if (!pl.pb) return -1;
  if (pout && !(!FLIP && pool_fusable(g, pl))) return -1;
  if ((cout || dout || aout) && !pout) return -1;
  if (dry) return 0;
  if (fail_direct()) return -3;
  // 16-byte loads: 4-aligned rows of x and of the weight blocks (the 3x3
  // forward kernel stages weight rows that are not 16-byte aligned with
  // 4-byte loads whatever VEC is)
  const int taps = g.HH * g.WW;
  bool wok;  // the weights can be staged under this VEC choice
  if (is_k3(g) && !FLIP) wok = g.K % 4 != 0 || aligned16(w);  // else 4-byte loads
  else wok = aligned16(w) && (FLIP ? (g.F * taps) % 4 == 0 && ((g.F % 32) * taps) % 4 == 0 &&
                                         (32 * taps) % 4 == 0
                                   : g.K % 4 == 0);
  const bool vec = g.W % 4 == 0 && aligned16(x) && wok;
  if (pl.pb == 2)
    return vec ? launch_fwd<2, FLIP, true>(x, w, bias, out, rout, pout, cout, dout, aout, g, N, pl)
               : launch_fwd<2, FLIP, false>(x, w, bias, out, rout, pout, cout, dout, aout, g, N,
                                            pl);
  return vec ? launch_fwd<1, FLIP, true>(x, w, bias, out, rout, pout, cout, dout, aout, g, N, pl)
             : launch_fwd<1, FLIP, false>(x, w, bias, out, rout, pout, cout, dout, aout, g, N, pl);
}

// dW kernel variants: (MF, JW, KS) with FS = filters/16 per workgroup.
//   V0 (1, 9, 1): FS = 1 -> 1 x 4 groups, K <= 576
//   V1 (2, 2, 4): FS = 2, one group, K <= 32, waves split the pixels
//   V2 (1, 4, 2): FS = 2, 2 x 1 groups, K <= 64, pairs of waves split the pixels
//   V3 (1, 9, 2): FS = 1, 1 x 2 groups, K <= 288, pairs of waves split the pixels
struct DwPlan {
  int var = -1, fs = 0, ch = 0, chunks = 0;
  size_t lds = 0;
};

// 32x32x2 dW variants (JW, KS): 4/KS groups of JW 32-tap blocks.
//   W0 (1, 4): K <= 32      W1 (2, 2): K <= 128
//   W2 (5, 2): K <= 320     W3 (9, 1): K <= 1152
DwPlan plan_dw32(const Geo &g, int N) {
  DwPlan pl;
  const int JB = (g.K + 31) / 32;
  const int P = g.Ho * g.Wo;
  if (g.Wo % 2 != 0) return pl;
  int groups;
  if (JB <= 1) { pl.var = 10; groups = 1; }
  else if (JB <= 4) { pl.var = 11; groups = 2; }
  else if (JB <= 10) { pl.var = 12; groups = 2; }
  else if (JB <= 36) { pl.var = 13; groups = 4; }
  else return pl;
  (void)groups;
  const int fblocks = (g.F + 31) / 32;
  // whole rows per chunk: whole images, halved while the grid gives a CU
  // fewer than two workgroups and the partials stay small (each halving
  // doubles the partial traffic)
  int rows = g.Ho;
  while (rows > 1 && (long)N * ((g.Ho + rows - 1) / rows) * fblocks < 512 &&
         (long)N * ((g.Ho + rows / 2 - 1) / (rows / 2)) * g.F * (g.K + 1) * 4 <= (8L << 20))
    rows = (rows + 1) / 2;
  for (;; rows = (rows + 1) / 2) {
    const int ch = rows * g.Wo;
    const int GS = ((ch + 31) & ~31) + 4;
    const int JWv = pl.var == 10 ? 1 : pl.var == 11 ? 2 : pl.var == 12 ? 5 : 9;
    const int KSv = pl.var == 10 ? 4 : pl.var == 13 ? 1 : 2;
    const long red = (long)(4 / KSv) * (KSv - 1) * JWv * 16 * 64;
    long xs = slab_floats(g, ch < P ? ch : P);
    if (g.W % 4 == 0) {  // 16-byte staging takes the gapped slab (larger)
      const long R = (long)(rows_spanned(ch < P ? ch : P, g.Wo) - 1) * g.sh + g.HH;
      const long gx = round_up((int)min((long)(g.C + 1) * (R * gslab_rw(g) + 4), (long)LDS_MAX), 256);
      if (gx > xs) xs = gx;
    }
    const long main = round_up(32 * GS, 256) + 4L * 32 * JB + GUARD + xs;
    const long lds = 4L * (main > red ? main : red);
    if (lds <= LDS_MAX) {
      pl.ch = ch;
      pl.chunks = (P + ch - 1) / ch;
      pl.fs = 2;
      pl.lds = (size_t)lds;
      return pl;
    }
    if (rows == 1) break;
  }
  pl.var = -1;
  return pl;
}

DwPlan plan_dw(const Geo &g, int N) {
  DwPlan pl = plan_dw32(g, N);
  if (pl.var >= 0) return pl;
  const int JB = (g.K + 15) / 16;
  const int P = g.Ho * g.Wo;
  if (JB <= 2) { pl.var = 1; pl.fs = 2; }
  else if (JB <= 4) { pl.var = 2; pl.fs = 2; }
  else if (JB <= 18) { pl.var = 3; pl.fs = 1; }
  else if (JB <= 36) { pl.var = 0; pl.fs = 1; }
  else return pl;
  const int fblocks = (g.F + 16 * pl.fs - 1) / (16 * pl.fs);
  // pixels per workgroup: whole images down to 64-pixel chunks, until the
  // grid gives every CU two workgroups (one wave per SIMD leaves the LDS
  // latency of each step exposed); more chunks mean more partial traffic
  int ch = (P + 3) & ~3;
  while (ch > 64 && (long)N * ((P + ch - 1) / ch) * fblocks < 512) ch = ((ch / 2) + 3) & ~3;
  for (;; ch = ((ch / 2) + 3) & ~3) {
    const int npp = (ch + 3) & ~3;
    const int GS = ((npp + 31) & ~31) + 4;
    // the pixel-split variants add their waves' accumulators through a buffer
    // that reuses the slab: groups * (KS-1) * MF*JW*4 floats per lane
    const long red = pl.var == 1   ? 1L * 3 * 2 * 2 * 4 * 64
                     : pl.var == 2 ? 2L * 1 * 1 * 4 * 4 * 64
                     : pl.var == 3 ? 2L * 1 * 1 * 9 * 4 * 64
                                   : 0;
    long xs = slab_floats(g, ch < P ? ch : P);
    if (xs < red) xs = red;
    const long lds =
        4L * (round_up(16 * pl.fs * GS, 256) + 2L * npp + 4L * JB * 16 + GUARD + xs);
    if (lds <= LDS_MAX) {
      pl.ch = ch;
      pl.chunks = (P + ch - 1) / ch;
      pl.lds = (size_t)lds;
      return pl;
    }
    if (ch <= 4) break;
  }
  pl.var = -1;
  return pl;
}

template <int MF, int JW, int KS, bool VEC>
int launch_dw(const float *gr, const float *x, float *part, const Geo &g, int N, const DwPlan &pl) {
  // whole-row walk when rows are whole 16-pixel segments and chunks whole rows
  const bool rows = g.Wo % 16 == 0 && pl.ch % g.Wo == 0;
  auto kern = rows ? conv_dw_lds_kernel<MF, JW, KS, VEC, true>
                   : conv_dw_lds_kernel<MF, JW, KS, VEC, false>;
  if (pl.lds > 64 * 1024 && !allow_big_lds((const void *)kern)) return -1;
  const dim3 grid((unsigned)(N * pl.chunks), (unsigned)((g.F + 16 * pl.fs - 1) / (16 * pl.fs)));
  hipLaunchKernelGGL(kern, grid, dim3(NT), pl.lds, stream(), gr, x, part, g, pl.chunks, pl.ch,
                     pl.fs);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

template <int JW, int KS, bool VEC>
int launch_dw32(const float *gr, const float *x, float *part, const Geo &g, int N,
                const DwPlan &pl) {
  auto kern = conv_dw32_kernel<JW, KS, VEC>;
  if (pl.lds > 64 * 1024 && !allow_big_lds((const void *)kern)) return -1;
  const dim3 grid((unsigned)(N * pl.chunks), (unsigned)((g.F + 31) / 32));
  hipLaunchKernelGGL(kern, grid, dim3(NT), pl.lds, stream(), gr, x, part, g, pl.chunks, pl.ch);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

template <bool VEC>
int launch_dw_var(const float *gr, const float *x, float *part, const Geo &g, int N,
                  const DwPlan &pl) {
  switch (pl.var) {
    case 10: return launch_dw32<1, 4, VEC>(gr, x, part, g, N, pl);
    case 11: return launch_dw32<2, 2, VEC>(gr, x, part, g, N, pl);
    case 12: return launch_dw32<5, 2, VEC>(gr, x, part, g, N, pl);
    case 13: return launch_dw32<9, 1, VEC>(gr, x, part, g, N, pl);
    case 0: return launch_dw<1, 9, 1, VEC>(gr, x, part, g, N, pl);
    case 1: return launch_dw<2, 2, 4, VEC>(gr, x, part, g, N, pl);
    case 2: return launch_dw<1, 4, 2, VEC>(gr, x, part, g, N, pl);
    default: return launch_dw<1, 9, 2, VEC>(gr, x, part, g, N, pl);
  }
}

int g_dwt = 1;  // tiled weight gradient enabled (tth_conv_dwt)

// ---- dwt planning ----
struct DwtPlan {
  int tg = 0, ntgw = 0, nts = 0, nfb = 0, rc = 0, nch = 0, units = 0, gs = 0, cs = 0, rw = 0,
      jbp = 0;
  size_t lds = 0;
};

// Layout of the dwt slab: rows of rw floats (the row's W floats behind rw - W
// zeros, at least the padding and the widest tap's overhang), channels cs
// floats apart, chosen so that the 32 taps of an MFMA operand read fall on
// as few shared banks as possible (32 banks of 4 bytes, a half-wave at a
// time) among the layouts 16-byte loads can stage (rows, gap and channel
// stride multiples of 4); only if none exists, element-by-element staging.
// With 3x3 taps a conflict-free layout exists only with rows of 3 mod 32
// floats (a channel's 9 taps on 9 consecutive banks) and channels 9-11 or
// 21-23 mod 32 apart, which 16-byte loads cannot fill: the best staged by
// them reads 2-way.
void dwt_layout_search(const Geo &g, int R, int TG, int &rw_out, int &cs_out) {
  const int taps = g.HH * g.WW;
  const int ro = (g.Wo - 1) * g.sw - g.pw + g.WW - g.W;  // right overhang
  int need = g.pw > ro ? g.pw : ro;
  if (need < 1) need = 1;
  long best_key = 1L << 50;
  for (int rw = g.W + need; rw < g.W + need + 32; rw++) {
    for (int pad = 0; pad < 32; pad++) {
      const int cs = R * rw + pad;
      const bool vec = ((rw | cs | (rw - g.W)) & 3) == 0;
      int worst = 0;
      for (int jb = 0; jb < (g.K + 31) / 32 && jb < 64; jb++) {
        const int k0 = (jb / TG) * TG * 32, c0 = k0 / taps;
        int cnt[32] = {0};
        for (int l = 0; l < 32; l++) {
          const int k = jb * 32 + l;
          if (k >= g.K) break;
          const int c = k / taps - c0, t = k % taps, kh = t / g.WW, kw = t % g.WW;
          const int b = ((c * cs + kh * rw + kw) % 32 + 32) % 32;
          if (++cnt[b] > worst) worst = cnt[b];
        }
      }
      // 16-byte staging first (element-by-element staging measured slower
      // than the 2-way conflicts it removes: conv2's weight gradient 17 ->
      // 23 us), then the fewest conflicts, then the smaller slab
      const long key = (vec ? 0 : (1L << 40)) + ((long)worst << 32) + cs;
      if (key < best_key) {
        best_key = key;
        rw_out = rw;
        cs_out = cs;
      }
    }
  }
}

// dwt_layout_search, remembered per geometry (the plan is made on every
// backward pass; the search takes about a millisecond)
void dwt_layout(const Geo &g, int R, int TG, int &rw, int &cs) {
  struct Entry {
    int key[10], rw, cs;
  };
  static Entry cache[32];
  static int n = 0, next = 0;  // entries held, the one to replace next
  const int key[10] = {g.W, g.Wo, g.WW, g.HH, g.sw, g.pw, g.K, g.C, R, TG};
  for (int i = 0; i < n; i++) {
    bool same = true;
    for (int k = 0; k < 10; k++) same &= cache[i].key[k] == key[k];
    if (same) {
      rw = cache[i].rw;
      cs = cache[i].cs;
      return;
    }
  }
  dwt_layout_search(g, R, TG, rw, cs);
  Entry &e = cache[next];
  next = (next + 1) % 32;
  if (n < 32) n++;
  for (int k = 0; k < 10; k++) e.key[k] = key[k];
  e.rw = rw;
  e.cs = cs;
}

// The tiled weight gradient covers 16-byte staged (W % 4 == 0) convolutions
// with Wo % 8 == 0.  Tap blocks of 32 go in groups of TG <= 3 (one wave's
// accumulators), up to 4 groups per workgroup (16 waves); the unit is the
// largest number of output rows whose staging fits the LDS while the grid
// still has about 2048 waves (8 per SIMD) to spread.
DwtPlan plan_dwt(const Geo &g, int N) {
  DwtPlan pl;
  if (g.W % 4 != 0 || g.Wo % 8 != 0) return pl;
  const int JB = (g.K + 31) / 32;
  const int TG = JB < 3 ? JB : 3;
  const int NTG = (JB + TG - 1) / TG;
  const int nts = (NTG + 3) / 4, ntgw = (NTG + nts - 1) / nts;
  const int taps = g.HH * g.WW;
  const int ncmax = min(g.C, (ntgw * TG * 32 + taps - 1) / taps + 1);  // channels a set spans
  const int nfb = (g.F + 31) / 32;
  const int nw = DWT_NPQ * ntgw;
  const long red = 4L * ntgw * (DWT_NPQ / 2) * (TG * 1024 + 64);
  for (int rc = g.Ho;; rc = (rc + 1) / 2) {
    const int R = (rc - 1) * g.sh + g.HH;
    int rw = 0, cs = 0;
    dwt_layout(g, R, TG, rw, cs);
    const int gs = ((rc * g.Wo + 31) & ~31) + 4;
    const long stage = 4L * (round_up(32 * gs, 256) + round_up((ncmax + 1) * cs, 256));
    const long lds = stage > red ? stage : red;
    const int nch = (g.Ho + rc - 1) / rc;
    const long waves = (long)N * nch * nts * nfb * nw;
    if (lds > LDS_MAX || (waves < 2048 && rc > DWT_NPQ)) {
      if (rc == 1) break;
      continue;
    }
    if ((long)N * nch > 0x7fffffffL) break;
    pl.tg = TG;
    pl.ntgw = ntgw;
    pl.nts = nts;
    pl.nfb = nfb;
    pl.rc = rc;
    pl.nch = nch;
    pl.units = N * nch;
    pl.gs = gs;
    pl.cs = cs;
    pl.rw = rw;
    pl.jbp = nts * ntgw * TG;
    pl.lds = (size_t)lds;
    return pl;
  }
  pl.tg = 0;
  return pl;
}

// defer: the reduction is not launched but described there (its partials
// then belong to the job)
template <int TG, int NTGW, bool CODE = false>
int launch_dwt(const float *gr, const float *x, float *dw, float *db, const Geo &g,
               const DwtPlan &pl, const unsigned char *codes = nullptr,
               TTDwtJob *defer = nullptr) {
  auto kern = conv_dwt_kernel<TG, NTGW, CODE>;
  if (pl.lds > 64 * 1024 && !allow_big_lds((const void *)kern)) return -1;
  const long S = (long)pl.jbp * 1024 + 32;
  float *part = (float *)ttrt_alloc(sizeof(float) * (size_t)(S * pl.units * pl.nfb));
  if (!part) return -2;
  hipLaunchKernelGGL(kern, dim3((unsigned)pl.units, (unsigned)pl.nts, (unsigned)pl.nfb),
                     dim3(64 * DWT_NPQ * NTGW), pl.lds, stream(), gr, x, part, g, pl.rc, pl.nch,
                     pl.gs, pl.cs, pl.rw, pl.jbp, codes);
  int rc = hipGetLastError() == hipSuccess ? 0 : -3;
  if (rc == 0) {
    const long cols = (long)pl.nfb * (S / 4);
    // lanes per element: about 16 units each
    int zl = 1;
    while (zl < 64 && zl * DWT_UPL < pl.units) zl *= 2;
    if (defer) {
      *defer = TTDwtJob{part, dw, db, pl.units, pl.nfb, pl.jbp, g.F, g.K, zl,
                        (int)((cols + NT / zl - 1) / (NT / zl))};
      return 0;
    }
#define TT_DWR(ZL_)                                                                          \
  case ZL_:                                                                                  \
    hipLaunchKernelGGL(conv_dwt_reduce_kernel<ZL_>,                                          \
                       dim3((unsigned)((cols + NT / ZL_ - 1) / (NT / ZL_))), dim3(NT), 0,    \
                       stream(), part, dw, db, pl.units, pl.nfb, pl.jbp, g.F, g.K);          \
    break;
    switch (zl) {
      TT_DWR(1) TT_DWR(2) TT_DWR(4) TT_DWR(8) TT_DWR(16) TT_DWR(32) TT_DWR(64)
    }
#undef TT_DWR
    rc = hipGetLastError() == hipSuccess ? 0 : -3;
  }
  ttrt_free(part);  // stream-ordered: the kernels above run before any reuse
  return rc;
}

template <bool CODE>
int launch_dwt_plan(const float *gr, const float *x, float *dw, float *db, const Geo &g,
                    const DwtPlan &pl, const unsigned char *codes = nullptr,
                    TTDwtJob *defer = nullptr) {
  if (pl.tg == 1) return launch_dwt<1, 1, CODE>(gr, x, dw, db, g, pl, codes, defer);
  if (pl.tg == 2) return launch_dwt<2, 1, CODE>(gr, x, dw, db, g, pl, codes, defer);
  if (pl.tg != 3) return -1;
  switch (pl.ntgw) {
    case 1: return launch_dwt<3, 1, CODE>(gr, x, dw, db, g, pl, codes, defer);
    case 2: return launch_dwt<3, 2, CODE>(gr, x, dw, db, g, pl, codes, defer);
    case 3: return launch_dwt<3, 3, CODE>(gr, x, dw, db, g, pl, codes, defer);
    case 4: return launch_dwt<3, 4, CODE>(gr, x, dw, db, g, pl, codes, defer);
  }
  return -1;
}

// ---- two convolutions in one launch ----
//
// conv(3x3, pad 1) -> relu -> 2x2 max pool -> conv(3x3, pad 1) -> relu -> 2x2
// max pool for 32x32 images of C1 <= 4 channels, 32 then 64 filters (the
// CNN's feature extractor), one workgroup of eight waves per image half: the
// first convolution's pooled output never leaves the CU between the two.
//
//   staging (one wait): the image rows the half needs (20 rows: the 16 rows
//     of the second convolution's 8 output rows, its one-row halo, and the
//     first convolution's own halo) as a gapped slab, both filter banks, both
//     biases, all with direct global->LDS loads.  The first filter bank is
//     written k-major ([k][f]) by choosing each lane's source; the second
//     (74 KB) is still in flight while the first convolution runs.
//   MFMA operands swapped against conv_fwd_k_kernel: A = the image (32
//     pixels), B = the filters, so lane l (filter l % 32) gets 16 pixels in
//     its accumulators -- 4 consecutive rows 8(r/4) + 4h + r%4, chosen to be
//     the top-left, top-right, bottom-left and bottom-right pixels of one
//     pool window.  Bias, relu, pool and the window's code then need no lane
//     exchange, and every lane does one pool per window instead of one per
//     pixel.  Each output is the same k sequence of the same products as in
//     conv_fwd_k_kernel (lane half h takes channels [h*CH2, (h+1)*CH2), taps
//     in order), so the values are bit for bit those of that kernel.
//   phase A: the first convolution's 18 output rows (9 pooled rows: 8 owned
//     plus one halo row) as 18 blocks of 8 windows (a row pair's left or
//     right half) dealt round robin to the waves; the pooled rows go to an
//     LDS slab laid out for the second convolution, the owned rows' codes to
//     an LDS tile.
//   phase B: the second convolution on that slab: wave w takes a 4x8 pixel
//     patch (w % 4, 8 windows) and 32 filters (w / 4).
//   LDS banks: a half-wave's 32 operand reads hit 32 different banks (slab
//     rows 48 floats apart for phase A's 2x16 pixels, 24 apart for phase B's
//     4x8: two or four disjoint runs mod 32); the pooled values are written
//     with an odd (or 9-dword) stride per filter.
//   The pooled outputs and codes of both convolutions are gathered in LDS and
//     written as whole 16-byte runs: pool1 (N x 32 x 16 x 16) and its codes
//     before phase B (they drain under its MFMAs), pool2 (N x 64 x 8 x 8),
//     its flattened copy, its padded copy (rows of 4097, last one 1) and its
//     codes at the end.  The convolutions' own outputs are not written; snap1
//     / snap2 (optional) get the filters and biases as they were read (w1 |
//     b1, w2 | b2), from which a later launch can recompute them.
namespace chain {
constexpr int NTH = 512;
constexpr int W1 = 32, F1 = 32;                   // first convolution: 32x32 -> 32 filters
constexpr int W2 = 16, F2 = 64;                   // second: 16x16 (pool1) -> 64 filters
constexpr int G1 = 16, RS1 = W1 + G1, R1 = 20, CS1 = R1 * RS1 + 4;  // image slab
constexpr int G2 = 8, RS2 = W2 + G2, R2 = 10, CS2 = R2 * RS2 + 5;   // pool1 slab (odd stride)
constexpr int KST2 = 292;                         // wrow_stride(F1 * 9)
constexpr int PT = 33, CT = 36;                   // pool2 tile strides (floats, bytes)
constexpr int C1T = 132;                          // pool1 codes tile stride (bytes)
constexpr int O_WS2 = 0;                          // F2 x KST2
constexpr int O_WS1 = O_WS2 + F2 * KST2;          // [k][f], 36 x 32
constexpr int O_B = O_WS1 + 36 * 32;              // bias1 (32), bias2 (64)
constexpr int O_X1 = O_B + 128;                   // image slab, 4 planes (then pool2 tiles)
constexpr int X1_SZ = 4096;
constexpr int O_X2 = O_X1 + X1_SZ;                // pool1 slab, F1 planes
constexpr int O_C1 = O_X2 + F1 * CS2 + 4;         // pool1 codes tile, F1 x C1T bytes
constexpr int LDS_FLOATS = O_C1 + F1 * C1T / 4;
static_assert(4 * CS1 <= X1_SZ && F2 * PT + F2 * CT / 4 <= X1_SZ, "image slab area");
static_assert(O_X1 % 64 == 0 && O_X2 % 4 == 0 && (F1 * CS2) % 4 == 0, "alignment");
static_assert(LDS_FLOATS * 4 <= LDS_MAX, "LDS");
}  // namespace chain

template <int CH2, int FCN>
__global__ void __launch_bounds__(chain::NTH)
conv_chain_fwd_kernel(const float *__restrict__ x, const float *__restrict__ w1,
                      const float *__restrict__ b1, const float *__restrict__ w2,
                      const float *__restrict__ b2, float *__restrict__ pool1,
                      unsigned char *__restrict__ codes1, float *__restrict__ pool2,
                      float *__restrict__ copy2, float *__restrict__ pad2,
                      unsigned char *__restrict__ codes2, float *__restrict__ snap1,
                      float *__restrict__ snap2, const float *__restrict__ fcw,
                      float *__restrict__ fcpart, int C1) {
  using namespace chain;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float *ws2 = smem + O_WS2, *ws1 = smem + O_WS1, *bs = smem + O_B;
  float *xs1 = smem + O_X1, *xs2 = smem + O_X2;
  unsigned char *c1t = (unsigned char *)(smem + O_C1);
  const int n = blockIdx.x >> 1, hf = blockIdx.x & 1;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, half = lane >> 5;
  const int K1 = C1 * 9;
  const int qlo = hf ? 7 : 0;           // first pooled row of phase A
  const int iy0 = 2 * qlo - 1;          // image row of slab row 0
  TT_PROBE(0, 0);

  // ---- staging: image slab, filter bank 1 (k-major), biases, then bank 2 ----
  {
    const float *xn = x + (long)n * C1 * 1024;
    constexpr int T1 = 2 * CH2 * CS1;
    for (int base = wave * 256; base < T1; base += NTH * 4) {
      const int i = base + lane * 4;
      const int c = i / CS1, rem = i - c * CS1;
      const int slot = rem / RS1, j = rem - slot * RS1;
      const int row = iy0 + slot;
      const bool ok = i < T1 && c < C1 && slot < R1 && j >= G1 && row >= 0 && row < 32;
      dma_dwordx4(ok ? xn + (c * 32 + row) * 32 + (j - G1) : g_zero_src, xs1 + base);
    }
    for (int base = wave * 64; base < 2 * CH2 * 9 * 32; base += NTH) {
      const int d = base + lane, k = d >> 5, f = d & 31;
      dma_dword(k < K1 ? w1 + f * K1 + k : g_zero_src, ws1 + base);
    }
    if (wave < 2) {
      const int d = wave * 64 + lane;
      const float *p = d < 32 ? (b1 ? b1 + d : g_zero_src)
                              : d < 96 ? (b2 ? b2 + d - 32 : g_zero_src) : g_zero_src;
      dma_dword(p, bs + wave * 64);
    }
    stage_blocks<true, NTH>(ws2, w2, F2 * KST2, KST2, F2, F1 * 9, 0, F1 * 9);
    // zeros under the pool1 slab (its gaps, pads and out-of-image rows)
    const f32x4 z = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = tid; i < F1 * CS2 / 4; i += NTH) reinterpret_cast<f32x4 *>(xs2)[i] = z;
  }
  // the filters and biases as read, for a later recomputation of the
  // convolutions' outputs (snap1 = w1 | b1, snap2 = w2 | b2): a slice per
  // workgroup
  if (snap1) {
    const int T1s = 32 * K1 + 32, T = T1s + F2 * F1 * 9 + F2;
    const int per = (T + gridDim.x - 1) / gridDim.x;
    const int end = min(T, (int)(blockIdx.x + 1) * per);
    for (int i = blockIdx.x * per + tid; i < end; i += NTH) {
      if (i < 32 * K1) snap1[i] = w1[i];
      else if (i < T1s) snap1[i] = b1 ? b1[i - 32 * K1] : 0.0f;
      else if (i < T1s + F2 * F1 * 9) snap2[i - T1s] = w2[i - T1s];
      else snap2[i - T1s] = b2 ? b2[i - T1s - F2 * F1 * 9] : 0.0f;
    }
  }
  // every wave issued at least 9 loads of bank 2 after the rest
  asm volatile("s_waitcnt vmcnt(9)" ::: "memory");
  __syncthreads();
  TT_PROBE(0, 1);

  // ---- phase A: first convolution, bias, relu, pool, codes ----
  {
    const float *wa = ws1 + half * CH2 * 9 * 32 + l32;
    const float bias = bs[l32];
    const int win = l32 >> 2, dy = (l32 >> 1) & 1, dx = l32 & 1;
    bool first = true;
    // 18 blocks (9 row pairs x 2 column halves of 8 windows), round robin
    for (int blk = wave; blk < 18; blk += 8) {
      const int i = blk >> 1, j = blk & 1;
      const int bj = (2 * i + dy) * RS1 + 2 * (8 * j + win) + dx + G1 - 1 + half * CH2 * CS1;
      f32x16 acc;
      for (int r = 0; r < 16; r++) acc[r] = 0.0f;
      auto load = [&](int c, float (&a)[9], float (&b)[9]) {
#pragma unroll
        for (int t = 0; t < 9; t++) a[t] = wa[(c * 9 + t) * 32];
#pragma unroll
        for (int kh = 0; kh < 3; kh++)
#pragma unroll
          for (int kw = 0; kw < 3; kw++) b[kh * 3 + kw] = xs1[bj + c * CS1 + kh * RS1 + kw];
      };
      auto mfmas = [&](const float (&a)[9], const float (&b)[9]) {
#pragma unroll
        for (int t = 0; t < 9; t++)
          acc = __builtin_amdgcn_mfma_f32_32x32x2f32(b[t], a[t], acc, 0, 0, 0);
      };
      float a0[9], bb0[9], a1[9], bb1[9];
      load(0, a0, bb0);
      int c = 0;
      for (; c + 1 < CH2; c += 2) {
        load(c + 1, a1, bb1);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(a0, bb0);
        __builtin_amdgcn_sched_barrier(0);
        load(c + 2 < CH2 ? c + 2 : c + 1, a0, bb0);
        __builtin_amdgcn_sched_barrier(0);
        mfmas(a1, bb1);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (c < CH2) mfmas(a0, bb0);
      if (first) dma_wait();  // bank 2 landed (before any store counts against vmcnt)
      first = false;

      const int q = qlo + i;                  // pooled row
      const bool own = q >= 8 * hf && q < 8 * hf + 8;
      const int srow = q - 8 * hf + 1;        // its row in the pool1 slab
      float *dst = xs2 + l32 * CS2 + srow * RS2 + G2;
      unsigned char *cdst = c1t + l32 * C1T + (q - 8 * hf) * 16;
#pragma unroll
      for (int qq = 0; qq < 4; qq++) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float v = acc[4 * qq + e] + bias;
          o[e] = v > 0.0f ? v : 0.0f;
        }
        unsigned code;
        const float m = pool_code(o[0], o[1], o[2], o[3], code);
        const int pc = 8 * j + 2 * qq + half;
        dst[pc] = m;
        if (own) cdst[pc] = (unsigned char)code;
      }
    }
  }
  __syncthreads();
  TT_PROBE(0, 2);

  // ---- pool1 and its codes (owned rows) from LDS, drained under phase B ----
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int idx = tid + k * NTH, f = idx >> 5, r8 = (idx >> 2) & 7, c4 = idx & 3;
    const float *s = xs2 + f * CS2 + (r8 + 1) * RS2 + G2 + 4 * c4;
    const f32x4 v = {s[0], s[1], s[2], s[3]};
    *reinterpret_cast<f32x4 *>(pool1 + (((long)n * F1 + f) * 16 + 8 * hf + r8) * 16 + 4 * c4) = v;
  }
  if (tid < 256) {
    const int f = tid >> 3, r8 = tid & 7;
    const unsigned *s = reinterpret_cast<const unsigned *>(c1t + f * C1T + r8 * 16);
    const uint4 v = {s[0], s[1], s[2], s[3]};
    *reinterpret_cast<uint4 *>(codes1 + ((long)n * F1 + f) * 256 + 128 * hf + 16 * r8) = v;
  }

  // the classifier rows of this thread's four pool2 features (FCN classes
  // each), loaded now and used after phase B
  float fw[FCN > 0 ? 4 * FCN : 1];
  if constexpr (FCN > 0) {
    const float *wr = fcw + (long)((tid >> 3) * 64 + 32 * hf + 4 * (tid & 7)) * FCN;
#pragma unroll
    for (int i = 0; i < 4 * FCN; i++) fw[i] = wr[i];
  }

  // ---- phase B: second convolution on the pool1 slab ----
  const int pb = wave & 3, fb = wave >> 2;
  f32x16 acc;
  for (int r = 0; r < 16; r++) acc[r] = 0.0f;
  {
    const int win = l32 >> 2, dy = (l32 >> 1) & 1, dx = l32 & 1;
    const int hol = 4 * (pb >> 1) + 2 * (win >> 2) + dy, wo = 8 * (pb & 1) + 2 * (win & 3) + dx;
    const int bj = hol * RS2 + wo + G2 - 1 + half * 16 * CS2;
    const float *wa = ws2 + (32 * fb + l32) * KST2 + half * 16 * 9;
    auto loadw = [&](int q, f32x4 (&wv)[9]) {
      const f32x4 *p = (const f32x4 *)(wa + q * 36);
#pragma unroll
      for (int i = 0; i < 9; i++) wv[i] = p[i];
    };
    auto loadb = [&](int c, float (&b)[9]) {
#pragma unroll
      for (int kh = 0; kh < 3; kh++)
#pragma unroll
        for (int kw = 0; kw < 3; kw++) b[kh * 3 + kw] = xs2[bj + c * CS2 + kh * RS2 + kw];
    };
    auto mfq = [&](const f32x4 (&wv)[9], const int cc, const float (&b)[9]) {
#pragma unroll
      for (int t = 0; t < 9; t++) {
        const int e = cc * 9 + t;
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(b[t], wv[e >> 2][e & 3], acc, 0, 0, 0);
      }
    };
    f32x4 wq0[9], wq1[9];
    float bb0[9], bb1[9];
    loadw(0, wq0);
    loadb(0, bb0);
    for (int q = 0; q < 4; q += 2) {
      const int c = 4 * q;
      loadw(q + 1, wq1);
      loadb(c + 1, bb1);
      __builtin_amdgcn_sched_barrier(0);
      mfq(wq0, 0, bb0);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 2, bb0);
      __builtin_amdgcn_sched_barrier(0);
      mfq(wq0, 1, bb1);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 3, bb1);
      __builtin_amdgcn_sched_barrier(0);
      mfq(wq0, 2, bb0);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 4, bb0);
      __builtin_amdgcn_sched_barrier(0);
      mfq(wq0, 3, bb1);
      __builtin_amdgcn_sched_barrier(0);
      loadw(q + 2 < 4 ? q + 2 : q + 1, wq0);
      loadb(c + 5, bb1);
      __builtin_amdgcn_sched_barrier(0);
      mfq(wq1, 0, bb0);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 6, bb0);
      __builtin_amdgcn_sched_barrier(0);
      mfq(wq1, 1, bb1);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 7, bb1);
      __builtin_amdgcn_sched_barrier(0);
      mfq(wq1, 2, bb0);
      __builtin_amdgcn_sched_barrier(0);
      loadb(c + 8 < 16 ? c + 8 : 15, bb0);
      __builtin_amdgcn_sched_barrier(0);
      mfq(wq1, 3, bb1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();  // every wave is past phase A's slab: the pool2 tiles reuse it
  TT_PROBE(0, 3);

  // ---- bias, relu, pool, codes of the second convolution ----
  float *pt = xs1;                                      // F2 x PT pooled values
  unsigned char *ct = (unsigned char *)(xs1 + F2 * PT);  // F2 x CT codes
  {
    const int f = 32 * fb + l32;
    const float bias = bs[32 + f];
#pragma unroll
    for (int qq = 0; qq < 4; qq++) {
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float v = acc[4 * qq + e] + bias;
        o[e] = v > 0.0f ? v : 0.0f;
      }
      unsigned code;
      const float m = pool_code(o[0], o[1], o[2], o[3], code);
      const int wi = 2 * qq + half;
      const int po = (2 * (pb >> 1) + (wi >> 2)) * 8 + 4 * (pb & 1) + (wi & 3);
      pt[f * PT + po] = m;
      ct[f * CT + po] = (unsigned char)code;
    }
  }
  __syncthreads();
  {
    const int f = tid >> 3, k = tid & 7;
    const float *s = pt + f * PT + 4 * k;
    const f32x4 v = {s[0], s[1], s[2], s[3]};
    const long o = ((long)n * F2 + f) * 64 + 32 * hf + 4 * k;
    *reinterpret_cast<f32x4 *>(pool2 + o) = v;
    if (copy2) *reinterpret_cast<f32x4 *>(copy2 + o) = v;
    if (pad2) {
      float *d = pad2 + (long)n * (F2 * 64 + 1) + f * 64 + 32 * hf + 4 * k;
      d[0] = v[0];
      d[1] = v[1];
      d[2] = v[2];
      d[3] = v[3];
      if (hf == 0 && tid == 0) pad2[(long)n * (F2 * 64 + 1) + F2 * 64] = 1.0f;
    }
    if (tid < 128) {
      const unsigned *cs = reinterpret_cast<const unsigned *>(ct + (tid >> 1) * CT + 16 * (tid & 1));
      const uint4 cv = {cs[0], cs[1], cs[2], cs[3]};
      *reinterpret_cast<uint4 *>(codes2 + ((long)n * F2 + (tid >> 1)) * 64 + 32 * hf +
                                 16 * (tid & 1)) = cv;
    }
    if constexpr (FCN > 0) {
      // the classifier's partial logits over this half's 2048 features
      // (the flattened pool2 row times the weights' rows, the bias left to
      // the reduction): fused multiply-adds over the thread's 4 features,
      // then the 512 threads' pieces of class j added in a fixed order --
      // 32 threads a class, thread l the pieces l, l + 32, ... in order (on
      // 32 banks), then a tree
      float *red = ws2;  // the second filter bank is no longer read
#pragma unroll
      for (int j = 0; j < FCN; j++) {
        float a = v[0] * fw[j];
        a = __builtin_fmaf(v[1], fw[FCN + j], a);
        a = __builtin_fmaf(v[2], fw[2 * FCN + j], a);
        a = __builtin_fmaf(v[3], fw[3 * FCN + j], a);
        red[j * NTH + tid] = a;
      }
      __syncthreads();
      const int j = tid >> 5, l = tid & 31;
      float a = 0.0f;
      if (j < FCN) {
#pragma unroll
        for (int i = 0; i < 16; i++) a += red[j * NTH + i * 32 + l];
      }
#pragma unroll
      for (int m = 16; m >= 1; m >>= 1) a += __shfl_xor(a, m, 32);
      if (j < FCN && l == 0) fcpart[((long)hf * gridDim.x / 2 + n) * FCN + j] = a;
    }
  }
  TT_PROBE(0, 4);
}

// ---- the middle of the two-convolution chain's backward in one launch ----
//
// For the chain of conv_chain_fwd_kernel: from the second convolution's
// output gradient dc2 (N x 64 x 16 x 16), its input gradient dx2 (the first
// pool's gradient, N x 32 x 16 x 16), then -- without writing or re-reading
// it -- the first pool + relu backward decoded from the pool codes and the
// first convolution's weight gradient partials (dw1 | db1 per unit of 8
// output rows, exactly the partial blocks conv_dwt_kernel<1, 1, true> writes,
// for the same deferred reduction).  One workgroup of eight waves per image
// half:
//   staging: dc2's rows (the half and a one-row halo each side, gapped rows
//     of 24 floats), the second filter bank in its own order (the FLIP
//     layout of conv_fwd_k_kernel), the image rows of the half plus halo and
//     the first pool's codes, all with direct loads and one wait;
//   phase 1: dx2 as conv_fwd_k_kernel<1, FLIP, VEC, 3, 3, 2> computes it
//     (waves 4-7 take the upper half of the channel steps and their sums are
//     added to waves 0-3's in LDS), on 4x8 pixel patches (a half-wave's
//     operand reads on 32 different banks); the same MFMA sequence per
//     output, so the same bits;
//   phase 2: waves 0-3 store dx2 and write the first convolution's output
//     gradient into LDS from each pool window's code (the pool + relu
//     backward: the window's gradient at its first argmax when that relu
//     value is > 0, else zero);
//   phase 3: the weight gradient of two units of 8 rows, four waves a unit,
//     as conv_dwt_kernel<1, 1, true> (the same items, MFMA order, LDS sum
//     (0 + 2) + (1 + 3) and bias sum), one partial block a unit.
namespace chainb {
constexpr int NTH = 512;
constexpr int G2 = 8, RS2 = 16 + G2, R2 = 10, CS2 = R2 * RS2 + 4;   // dc2 slab
// image slab: rows of 35 floats (3 zeros, 32 values), channels 630 floats
// apart: the 27 taps of a weight-gradient operand read on 27 different banks
// (a channel's 9 taps on 9 consecutive banks, channels 22 mod 32 apart);
// staged element by element
constexpr int GX = 3, RWX = 32 + GX, RX = 18, CSX = RX * RWX;
constexpr int GS = 260;                  // g1 tile: per filter, 8 rows x 32 + 4
constexpr int SLOT = 1024 + 64;          // one wave's dW accumulators and bias sum
constexpr int O_W = 0;                   // filter bank 2, then the g1 tiles of both units
constexpr int W_SZ = 64 * 32 * 9;
constexpr int O_D = O_W + W_SZ;          // dc2 slab, then the partial sums
constexpr int O_X = O_D + 64 * CS2;      // image slab (4 planes)
constexpr int X_SZ = 2816;
constexpr int O_C = O_X + X_SZ;          // pool codes, 32 x 128 bytes
constexpr int LDS_FLOATS = O_C + 1024;
static_assert(2 * 32 * GS <= W_SZ && 4 * CSX + 64 <= X_SZ && X_SZ % 256 == 0, "regions");
static_assert((64 * CS2) % 256 == 0 && 2 * 2 * SLOT <= 64 * CS2, "dc2 slab");
static_assert(LDS_FLOATS * 4 <= LDS_MAX, "LDS");
}  // namespace chainb

// Workgroup blk (image blk / 2, half blk % 2); the first 512 threads.
__device__ __forceinline__ void conv_chain_bwd_block(const float *__restrict__ dc2,
                                                     const float *__restrict__ w2,
                                                     const unsigned char *__restrict__ codes1,
                                                     const float *__restrict__ x,
                                                     float *__restrict__ dx2,
                                                     float *__restrict__ part, int C1, int blk) {
  using namespace chainb;
  extern __shared__ __attribute__((aligned(16))) float smem[];
  float *ws = smem + O_W, *ds = smem + O_D, *xs = smem + O_X;
  const unsigned char *c1t = (const unsigned char *)(smem + O_C);
  const int n = blk >> 1, hf = blk & 1;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, half = lane >> 5;

  // ---- staging ----
  {
    const float *gn = dc2 + (long)n * 64 * 256;
    for (int base = wave * 256; base < 64 * CS2; base += NTH * 4) {
      const int i = base + lane * 4;
      const int c = i / CS2, rem = i - c * CS2;
      const int slot = rem / RS2, j = rem - slot * RS2;
      const int row = 8 * hf - 1 + slot;
      const bool ok = slot < R2 && j >= G2 && row >= 0 && row < 16;
      dma_dwordx4(ok ? gn + (c * 16 + row) * 16 + (j - G2) : g_zero_src, ds + base);
    }
    for (int base = wave * 256; base < W_SZ; base += NTH * 4)
      dma_dwordx4(w2 + base + lane * 4, ws + base);
    const float *xn = x + (long)n * C1 * 1024;
    for (int base = wave * 64; base < 4 * CSX; base += NTH) {
      const int i = base + lane;
      const int c = i / CSX, rem = i - c * CSX;
      const int slot = rem / RWX, j = rem - slot * RWX;
      const int row = 16 * hf - 1 + slot;
      const bool ok = c < C1 && slot < RX && j >= GX && row >= 0 && row < 32;
      dma_dword(ok ? xn + (c * 32 + row) * 32 + (j - GX) : g_zero_src, xs + base);
    }
    if (wave < 4) {
      const int i = wave * 1024 + lane * 16;  // byte of the 32 x 128 tile
      dma_dwordx4((const float *)(codes1 + ((long)n * 32 + (i >> 7)) * 256 + 128 * hf + (i & 127)),
                  smem + O_C + wave * 256);
    }
  }
  dma_wait();
  __syncthreads();
  TT_PROBE(1, 1);

  // ---- phase 1: dx2 (the flipped-kernel convolution of dc2) ----
  const int pb = wave & 3, grp = wave >> 2;
  const int r4 = l32 >> 3, c8 = l32 & 7;
  const int hol = 4 * (pb >> 1) + r4, wo = 8 * (pb & 1) + c8;  // pixel in the half
  f32x16 acc;
  for (int r = 0; r < 16; r++) acc[r] = 0.0f;
  {
    const int bj = hol * RS2 + wo + G2 - 1 + half * 32 * CS2;
    const float *wa = ws + l32 * 9 + half * 32 * 32 * 9;
    auto load = [&](int c, float (&a)[9], float (&b)[9]) {
      const float *wc = wa + c * 32 * 9;
#pragma unroll
      for (int t = 0; t < 9; t++) a[t] = wc[8 - t];
#pragma unroll
      for (int kh = 0; kh < 3; kh++)
#pragma unroll
        for (int kw = 0; kw < 3; kw++) b[kh * 3 + kw] = ds[bj + c * CS2 + kh * RS2 + kw];
    };
    auto mfmas = [&](const float (&a)[9], const float (&b)[9]) {
#pragma unroll
      for (int t = 0; t < 9; t++)
        acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[t], b[t], acc, 0, 0, 0);
    };
    const int cs0 = grp * 16, cs1 = cs0 + 16;
    float a0[9], b0[9], a1[9], b1[9];
    load(cs0, a0, b0);
    for (int c = cs0; c < cs1; c += 2) {
      load(c + 1, a1, b1);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      load(c + 2 < cs1 ? c + 2 : c + 1, a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a1, b1);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // the upper channel group's sums through LDS, added in a fixed order
  {
    float *red = ds + pb * 1024 + lane;
    __syncthreads();
    if (grp == 1) {
#pragma unroll
      for (int r = 0; r < 16; r++) red[r * 64] = acc[r];
    }
    __syncthreads();
    if (grp == 0) {
#pragma unroll
      for (int r = 0; r < 16; r++) acc[r] += red[r * 64];
    }
  }

  TT_PROBE(1, 2);
  // ---- phase 2: dx2, and the first convolution's output gradient in LDS ----
  if (grp == 0) {
    const int pr = 8 * hf + hol;
    float *g1 = ws + (hol >> 2) * 32 * GS + ((2 * hol) & 7) * 32 + 2 * wo;
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int c = 8 * (r >> 2) + 4 * half + (r & 3);
      const float v = acc[r] + 0.0f;  // the dX kernel's (zero) bias
      dx2[(((long)n * 32 + c) * 16 + pr) * 16 + wo] = v;
      const unsigned code = c1t[c * 128 + hol * 16 + wo];
      const float gv = 0.0f + v;
      auto at = [&](unsigned kq) {
        return ((code & 3) == kq && ((code >> (2 + kq)) & 1)) ? gv : 0.0f;
      };
      float *d = g1 + c * GS;
      *reinterpret_cast<float2 *>(d) = make_float2(at(0), at(1));
      *reinterpret_cast<float2 *>(d + 32) = make_float2(at(2), at(3));
    }
  }
  __syncthreads();

  TT_PROBE(1, 3);
  // ---- phase 3: the first convolution's weight gradient, two units ----
  {
    const int uu = wave >> 2, pq = wave & 3;
    const int K1 = C1 * 9;
    int bb = C1 * CSX;  // taps past K: the zero plane
    if (l32 < K1) {
      const int c = l32 / 9, t = l32 - c * 9, kh = t / 3, kw = t - kh * 3;
      bb = c * CSX + kh * RWX + GX + kw - 1;
    }
    f32x16 dacc;
    for (int r = 0; r < 16; r++) dacc[r] = 0.0f;
    float bsum = 0.0f;
    const float *ga = ws + uu * 32 * GS + l32 * GS + half * 16;
    constexpr int quads = 4;
    constexpr int xstep = 4 * RWX - quads * 4, gstep = 4 * 32 - quads * 4;
    int go = pq * 32, xo = pq * RWX + half * 16 + uu * 8 * RWX;
    int qd = 0, left = 8;
    auto advance = [&]() {
      if (--left <= 0) return;
      if (++qd == quads) {
        qd = 0;
        go += gstep + 4;
        xo += xstep + 4;
      } else {
        go += 4;
        xo += 4;
      }
    };
    auto load = [&](f32x4 &a4, float (&bv)[4]) {
      a4 = *(const f32x4 *)(ga + go);
#pragma unroll
      for (int e = 0; e < 4; e++) bv[e] = xs[bb + xo + e];
    };
    auto mfmas = [&](const f32x4 &a4, const float (&bv)[4]) {
#pragma unroll
      for (int e = 0; e < 4; e++)
        dacc = __builtin_amdgcn_mfma_f32_32x32x2f32(a4[e], bv[e], dacc, 0, 0, 0);
      bsum += (a4[0] + a4[1]) + (a4[2] + a4[3]);
    };
    f32x4 a0, a1;
    float b0[4], b1[4];
    load(a0, b0);
#pragma unroll 1
    for (int it = 0; it < 8; it += 2) {
      advance();
      load(a1, b1);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      advance();
      load(a0, b0);
      __builtin_amdgcn_sched_barrier(0);
      mfmas(a1, b1);
      __builtin_amdgcn_sched_barrier(0);
    }
    bsum += __shfl_xor(bsum, 32, 64);  // both halves of filter l32
    // the four waves of a unit: (0 + 2) + (1 + 3), through LDS
#pragma unroll
    for (int s = 2; s >= 1; s >>= 1) {
      __syncthreads();
      if (pq >= s && pq < 2 * s) {
        float *d = ds + (uu * 2 + pq - s) * SLOT;
#pragma unroll
        for (int r = 0; r < 16; r++) d[r * 64 + lane] = dacc[r];
        d[1024 + lane] = bsum;
      }
      __syncthreads();
      if (pq < s) {
        const float *d = ds + (uu * 2 + pq) * SLOT;
#pragma unroll
        for (int r = 0; r < 16; r++) dacc[r] += d[r * 64 + lane];
        bsum += d[1024 + lane];
      }
    }
    if (pq == 0) {
      float *pz = part + ((long)n * 4 + 2 * hf + uu) * (1024 + 32);
#pragma unroll
      for (int r = 0; r < 16; r++) pz[r * 64 + lane] = dacc[r];
      if (lane < 32) pz[1024 + lane] = bsum;
    }
  }
}

__global__ void __launch_bounds__(chainb::NTH)
conv_chain_bwd_kernel(const float *__restrict__ dc2, const float *__restrict__ w2,
                      const unsigned char *__restrict__ codes1, const float *__restrict__ x,
                      float *__restrict__ dx2, float *__restrict__ part, int C1) {
  conv_chain_bwd_block(dc2, w2, codes1, x, dx2, part, C1, blockIdx.x);
}

// The same and the second convolution's weight gradient (conv_dwt_kernel<3,
// 3>, independent of it) in one grid: workgroups [0, 2N) the chain's
// backward middle, the rest the weight-gradient workgroups (unit, filter
// block), so the second set starts on each CU as the first one leaves it --
// no launch boundary between them.  768 threads (the weight gradient's 12
// waves); the chain's workgroups use the first 512.
__global__ void __launch_bounds__(64 * DWT_NPQ * 3)
conv_chain_bwd_dw2_kernel(const float *__restrict__ dc2, const float *__restrict__ w2,
                          const unsigned char *__restrict__ codes1, const float *__restrict__ x,
                          float *__restrict__ dx2, float *__restrict__ part1, int C1,
                          const float *__restrict__ x2, float *__restrict__ part2, Geo g2,
                          int RC, int nch, int GS, int CS, int RW, int jbp, int nu2,
                          int nchain) {
  TT_PROBE(1, 0);
  if ((int)blockIdx.x < nchain) {
    if (threadIdx.x >= chainb::NTH) return;
    conv_chain_bwd_block(dc2, w2, codes1, x, dx2, part1, C1, blockIdx.x);
    TT_PROBE(1, 15);
    return;
  }
  const int b = blockIdx.x - nchain;
  conv_dwt_block<3, 3, false>(dc2, x2, part2, g2, RC, nch, GS, CS, RW, jbp, nullptr, b % nu2,
                              0, b / nu2, nu2);
  TT_PROBE(1, 15);
}

int g_lds_conv = 1;  // tth_conv_lds

}  // namespace

extern "C" int tth_conv_dwt(int on) {
  const int prev = g_dwt;
  if (on >= 0) g_dwt = on ? 1 : 0;
  return prev;
}

extern "C" int tth_conv_lds(int on) {
  const int prev = g_lds_conv;
  if (on >= 0) g_lds_conv = on ? 1 : 0;
  return prev;
}

// Which LDS-staged kernels cover this convolution: bit 0 forward, bit 1
// weight gradient, bit 2 input gradient.  0 when switched off.
extern "C" int tt_k_conv2d_lds_plan(int N, int C, int H, int W, int F, int HH, int WW, int sh,
                                    int sw, int ph, int pw, int Ho, int Wo) {
  if (!g_lds_conv || !geo_ok(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo)) return 0;
  int bits = 0;
  const Geo g{C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, F, C * HH * WW};
  if (run_fwd<false>(nullptr, nullptr, nullptr, nullptr, g, N, true) == 0) bits |= 1;
  if (plan_dw(g, N).var >= 0) bits |= 2;
  if (sh == 1 && sw == 1 && ph <= HH - 1 && pw <= WW - 1) {
    const Geo gx{F, Ho, Wo, HH, WW, 1, 1, HH - 1 - ph, WW - 1 - pw, H, W, C, F * HH * WW};
    if (run_fwd<true>(nullptr, nullptr, nullptr, nullptr, gx, N, true) == 0) bits |= 4;
  }
  return bits;
}

// out (N,F,Ho,Wo) = conv(x, w) + bias (bias may be NULL).  -1: not covered.
extern "C" int tt_k_conv2d_fwd_lds(const float *x, const float *w, const float *bias, float *out,
                                   int N, int C, int H, int W, int F, int HH, int WW, int sh,
                                   int sw, int ph, int pw, int Ho, int Wo) {
  if (!x || !w || !out || !geo_ok(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo)) return -1;
  const Geo g{C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, F, C * HH * WW};
  return run_fwd<false>(x, w, bias, out, g, N, false);
}

// The same convolution with its relu: out as above and rout = relu(out)
// from the same values in one launch (bit-identical to tt_k_conv2d_fwd_lds
// followed by tt_k_relu_fwd).  -1: not covered.
extern "C" int tt_k_conv2d_relu_fwd_lds(const float *x, const float *w, const float *bias,
                                        float *out, float *rout, int N, int C, int H, int W,
                                        int F, int HH, int WW, int sh, int sw, int ph, int pw,
                                        int Ho, int Wo) {
  if (!x || !w || !out || !rout || out == rout ||
      !geo_ok(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo))
    return -1;
  const Geo g{C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, F, C * HH * WW};
  return run_fwd<false>(x, w, bias, out, g, N, false, rout);
}

// The same convolution with its relu and the 2x2 / stride-2 max pool of the
// relu: out, rout as above and pout (N x F x Ho/2 x Wo/2) in one launch
// (bit-identical to tt_k_conv2d_relu_fwd_lds followed by the max pool);
// cout / dout (optional): the pool output flattened per image, as a copy and
// padded with a last column of ones (a reshape and a padones after it);
// rout may be NULL (the relu is then only pooled, not stored); codes
// (optional): one byte per pool window for tt_k_maxpool2x2_code_relu_bwd.
// -1: not covered (see pool_fusable).
extern "C" int tt_k_conv2d_relu_pool_fwd_lds(const float *x, const float *w, const float *bias,
                                             float *out, float *rout, float *pout, float *cout,
                                             float *dout, unsigned char *codes, int N, int C,
                                             int H, int W, int F, int HH, int WW, int sh, int sw,
                                             int ph, int pw, int Ho, int Wo) {
  if (!x || !w || !out || !pout || out == rout ||
      !geo_ok(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo))
    return -1;
  const Geo g{C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, F, C * HH * WW};
  return run_fwd<false>(x, w, bias, out, g, N, false, rout, pout, cout, dout, codes);
}

// dw (F, C*HH*WW) and, when db is given, db (F) from the output gradient g
// (N,F,Ho,Wo) and the input x.  -1: not covered; -2: out of memory.
extern "C" int tt_k_conv2d_dw_lds(const float *gr, const float *x, float *dw, float *db, int N,
                                  int C, int H, int W, int F, int HH, int WW, int sh, int sw,
                                  int ph, int pw, int Ho, int Wo) {
  if (!gr || !x || !dw || !geo_ok(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo)) return -1;
  const Geo g{C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, F, C * HH * WW};
  if (g_dwt && aligned16(x) && aligned16(gr)) {
    const DwtPlan tp = plan_dwt(g, N);
    if (tp.tg) return launch_dwt_plan<false>(gr, x, dw, db, g, tp);
  }
  const DwPlan pl = plan_dw(g, N);
  if (pl.var < 0) return -1;
  const long Z = (long)N * pl.chunks;
  const bool d32 = pl.var >= 10;
  const int FBLK = (F + 31) / 32, JB32 = (g.K + 31) / 32;
  const long total = d32 ? (long)FBLK * (JB32 * 1024 + 32) : (long)F * (g.K + 1);
  if (Z * total >= 0x7fffffffL) return -1;
  float *part = (float *)ttrt_alloc(sizeof(float) * (size_t)(Z * total));
  if (!part) return -2;
  // 16-byte loads need 4-aligned rows of x and of the output gradient
  const int P = Ho * Wo;
  const bool vec = W % 4 == 0 && P % 4 == 0 && aligned16(x) && aligned16(gr);
  int rc = vec ? launch_dw_var<true>(gr, x, part, g, N, pl)
               : launch_dw_var<false>(gr, x, part, g, N, pl);
  if (rc == 0) {
    // lanes per output: enough workgroups to spread the partial reads
    // (the dw32 reduction reads 4 floats a lane and keeps at least 8
    // partials per lane: measured faster than more lanes with fewer loads)
    int zl = 1;
    const long units = d32 ? total / 4 : total;
    while (zl < 32 && zl < Z && units * zl * 2 <= 2048L * NT && (!d32 || zl * 16 <= Z)) zl *= 2;
#define TT_RED(ZL_)                                                                       \
  if (d32)                                                                                \
    hipLaunchKernelGGL(conv_dw32_reduce_kernel<ZL_>,                                      \
                       dim3((unsigned)((total / 4 + NT / ZL_ - 1) / (NT / ZL_))), dim3(NT), \
                       0, stream(), part, dw, db, (int)Z, FBLK, JB32, F, g.K);            \
  else                                                                                    \
    hipLaunchKernelGGL(conv_dw_reduce_kernel<ZL_>,                                        \
                       dim3((unsigned)((total + NT / ZL_ - 1) / (NT / ZL_))), dim3(NT), 0, \
                       stream(), part, dw, db, (int)Z, F, g.K)
    switch (zl) {
      case 1: TT_RED(1); break;
      case 2: TT_RED(2); break;
      case 4: TT_RED(4); break;
      case 8: TT_RED(8); break;
      case 16: TT_RED(16); break;
      default: TT_RED(32); break;
    }
#undef TT_RED
    rc = hipGetLastError() == hipSuccess ? 0 : -3;
  }
  ttrt_free(part);  // stream-ordered: the kernels above run before any reuse
  return rc;
}

// dw / db as tt_k_conv2d_dw_lds from the gradient gp of the 2x2 / stride-2
// max pool of the relu of this convolution's output and the pool windows'
// codes (tt_k_conv2d_relu_pool_fwd_lds): the output gradient is decoded
// while it is staged, never stored (bit for bit tt_k_maxpool2x2_code_relu_bwd
// followed by tt_k_conv2d_dw_lds on its result).  dw == NULL: only reports
// whether the shape is covered (0) or not (-1).
extern "C" int tt_k_conv2d_dw_lds_pooled(const float *gp, const unsigned char *codes,
                                         const float *x, float *dw, float *db, int N, int C,
                                         int H, int W, int F, int HH, int WW, int sh, int sw,
                                         int ph, int pw, int Ho, int Wo) {
  if (!geo_ok(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo) || Ho % 2 || Wo % 2 || !g_dwt)
    return -1;
  const Geo g{C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, F, C * HH * WW};
  const DwtPlan tp = plan_dwt(g, N);
  if (!tp.tg || (tp.rc % 2 && tp.nch > 1)) return -1;
  if (!dw) return 0;
  if (!gp || !codes || !x || !aligned16(x) || ((uintptr_t)gp & 7) || ((uintptr_t)codes & 1))
    return -1;
  return launch_dwt_plan<true>(gp, x, dw, db, g, tp, codes);
}

// dx (N,C,H,W) of a stride-1 convolution from the output gradient g
// (N,F,Ho,Wo) and the weights w (F,C,HH,WW).  -1: not covered.
extern "C" int tt_k_conv2d_dx_lds(const float *gr, const float *w, float *dx, int N, int C, int H,
                                  int W, int F, int HH, int WW, int sh, int sw, int ph, int pw,
                                  int Ho, int Wo) {
  if (!gr || !w || !dx || !geo_ok(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo)) return -1;
  if (sh != 1 || sw != 1 || ph > HH - 1 || pw > WW - 1) return -1;
  const Geo gx{F, Ho, Wo, HH, WW, 1, 1, HH - 1 - ph, WW - 1 - pw, H, W, C, F * HH * WW};
  return run_fwd<true>(gr, w, nullptr, dx, gx, N, false);
}

extern "C" int ttk_conv2d_dwt_defer(const float *gr, const unsigned char *codes, const float *x,
                                    float *dw, float *db, const int q[13], TTDwtJob *job) {
  const int N = q[0], C = q[1], H = q[2], W = q[3], F = q[4], HH = q[5], WW = q[6], sh = q[7],
            sw = q[8], ph = q[9], pw = q[10], Ho = q[11], Wo = q[12];
  if (!gr || !x || !dw || !job || !g_dwt || !geo_ok(N, C, H, W, F, HH, WW, sh, sw, ph, pw, Ho, Wo))
    return -1;
  const Geo g{C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, F, C * HH * WW};
  const DwtPlan tp = plan_dwt(g, N);
  if (!tp.tg || !aligned16(x)) return -1;
  if (codes) {
    if (Ho % 2 || Wo % 2 || (tp.rc % 2 && tp.nch > 1) || ((uintptr_t)gr & 7) ||
        ((uintptr_t)codes & 1))
      return -1;
    return launch_dwt_plan<true>(gr, x, dw, db, g, tp, codes, job);
  }
  if (!aligned16(gr)) return -1;
  return launch_dwt_plan<false>(gr, x, dw, db, g, tp, nullptr, job);
}

extern "C" int ttk_dwt_reduce_jobs(const TTDwtJob *jobs, int n) {
  int rc = 0;
  for (int b = 0; b < n; b += DWT_JOBS) {
    DwtJobs js{};
    js.n = n - b < DWT_JOBS ? n - b : DWT_JOBS;
    long tot = 0;
    for (int q = 0; q < js.n; q++) {
      js.j[q] = jobs[b + q];
      js.start[q] = (int)tot;
      tot += jobs[b + q].nblk;
    }
    js.start[js.n] = (int)tot;
    if (tot > 0) {
      hipLaunchKernelGGL(conv_dwt_reduce_multi_kernel, dim3((unsigned)tot), dim3(NT), 0,
                         stream(), js);
      if (hipGetLastError() != hipSuccess) rc = -3;
    }
    for (int q = 0; q < js.n; q++) ttrt_free(js.j[q].part);  // stream-ordered
  }
  return rc;
}

// The pending reductions of an SGD step's gradients and the step itself in
// one launch: blocks [0, start[n]) reduce job q (writing its dw / db and
// stepping wdw[q] / wdb[q] when given), the rest step the plain tensors
// (a thread an element).
struct DwtSgd {
  TTDwtJob j[DWT_JOBS];
  float *wdw[DWT_JOBS], *wdb[DWT_JOBS];
  int start[DWT_JOBS + 1];
  int n;
  float *pw[TT_SGD_MAX];
  const float *pg[TT_SGD_MAX];
  long pn[TT_SGD_MAX];
  long pstart[TT_SGD_MAX + 1];
  int np;
  float lr;
};
__global__ void __launch_bounds__(NT) conv_dwt_reduce_sgd_kernel(DwtSgd js) {
  __shared__ f32x4 sums[NT];
  const int bx = blockIdx.x;
  if (bx >= js.start[js.n]) {
    const long b = bx - js.start[js.n];
    int t = 0;
    while (t + 1 < js.np && b >= js.pstart[t + 1]) t++;
    const long i = (b - js.pstart[t]) * NT + threadIdx.x;
    if (i < js.pn[t]) js.pw[t][i] -= js.lr * js.pg[t][i];
    return;
  }
  int q = 0;
  while (q + 1 < js.n && bx >= js.start[q + 1]) q++;
  const TTDwtJob &j = js.j[q];
  const int blk = bx - js.start[q];
  switch (j.zl) {
#define TT_DJ(ZL_)                                                                         \
  case ZL_:                                                                                \
    dwt_reduce_block<ZL_>(blk, sums, j.part, j.dw, j.db, j.nu, j.nfb, j.jbp, j.F, j.K,     \
                          js.wdw[q], js.wdb[q], js.lr);                                    \
    break;
    TT_DJ(1) TT_DJ(2) TT_DJ(4) TT_DJ(8) TT_DJ(16) TT_DJ(32) TT_DJ(64)
#undef TT_DJ
  }
}

extern "C" int ttk_dwt_reduce_sgd(const TTDwtJob *jobs, float *const *wdw, float *const *wdb,
                                  int nj, float *const *pw, const float *const *pg,
                                  const long *pn, int np, float lr) {
  if (nj < 1 || nj > DWT_JOBS || np < 0 || np > TT_SGD_MAX) return 1;
  DwtSgd js{};
  js.n = nj;
  js.np = np;
  js.lr = lr;
  long tot = 0;
  for (int q = 0; q < nj; q++) {
    js.j[q] = jobs[q];
    js.wdw[q] = wdw[q];
    js.wdb[q] = wdb[q];
    js.start[q] = (int)tot;
    tot += jobs[q].nblk;
  }
  js.start[nj] = (int)tot;
  long ptot = 0;
  for (int t = 0; t < np; t++) {
    js.pw[t] = pw[t];
    js.pg[t] = pg[t];
    js.pn[t] = pn[t];
    js.pstart[t] = ptot;
    ptot += (pn[t] + NT - 1) / NT;
  }
  js.pstart[np] = ptot;
  if (tot + ptot > 0x7fffffffL) return 1;
  if (tot + ptot > 0)
    hipLaunchKernelGGL(conv_dwt_reduce_sgd_kernel, dim3((unsigned)(tot + ptot)), dim3(NT), 0,
                       stream(), js);
  const int rc = hipGetLastError() == hipSuccess ? 0 : -3;
  for (int q = 0; q < nj; q++) ttrt_free(js.j[q].part);  // stream-ordered
  return rc;
}

extern "C" void ttk_dwt_job_drop(TTDwtJob *job) {
  if (!job) return;
  ttrt_free(job->part);
  job->part = nullptr;
}

// The CNN feature extractor's two convolutions in one launch (see
// conv_chain_fwd_kernel): x (N x C1 x 32 x 32, C1 <= 4), w1 (32 x C1 x 3 x 3),
// w2 (64 x 32 x 3 x 3), biases optional; pad 1, stride 1, relu, 2x2 / stride-2
// max pools.  Writes pool1 (N x 32 x 16 x 16) and codes1, pool2 (N x 64 x 8 x
// 8) and codes2 (one byte per pool window, as tt_k_conv2d_relu_pool_fwd_lds),
// and, when given, copy2 (pool2 again), pad2 (N x 4097: pool2 flattened, then
// 1) and snap1 / snap2 (both or neither: 32*C1*9 + 32 and 18432 + 64 floats,
// w1 | b1 and w2 | b2 as read, zeros for a NULL bias).  Every value bit for
// bit that of two tt_k_conv2d_relu_pool_fwd_lds launches.  fcpart (optional,
// fcn == 10): the partial logits of a classifier fcw (4096 x 10 rows, bias
// not included) over each image half's 2048 pool2 features, fcpart[h][n][j]
// for h = 0, 1.  -1: shape or alignment not covered (nothing launched).
extern "C" int tt_k_conv2d_chain_fwd(const float *x, const float *w1, const float *b1,
                                     const float *w2, const float *b2, float *pool1,
                                     unsigned char *codes1, float *pool2, float *copy2,
                                     float *pad2, unsigned char *codes2, float *snap1,
                                     float *snap2, const float *fcw, int fcn, float *fcpart,
                                     int N, int C1, int H, int W, int F1, int F2) {
  if (!x || !w1 || !w2 || !pool1 || !codes1 || !pool2 || !codes2 || N <= 0 || N > 65535 ||
      C1 < 1 || C1 > 4 || H != 32 || W != 32 || F1 != chain::F1 || F2 != chain::F2 ||
      !snap1 != !snap2)
    return -1;
  if (!aligned16(x) || !aligned16(w2) || !aligned16(pool1) || !aligned16(pool2) ||
      ((uintptr_t)codes1 & 15) || ((uintptr_t)codes2 & 15) || (copy2 && !aligned16(copy2)))
    return -1;
  if (fail_direct()) return -3;
  if (fcpart && (fcn != 10 || !fcw)) return -1;
  auto kern = fcpart ? (C1 > 2 ? conv_chain_fwd_kernel<2, 10> : conv_chain_fwd_kernel<1, 10>)
                     : (C1 > 2 ? conv_chain_fwd_kernel<2, 0> : conv_chain_fwd_kernel<1, 0>);
  constexpr size_t lds = sizeof(float) * chain::LDS_FLOATS;
  if (!allow_big_lds((const void *)kern)) return -1;
  hipLaunchKernelGGL(kern, dim3((unsigned)(2 * N)), dim3(chain::NTH), lds, stream(), x, w1, b1, w2,
                     b2, pool1, codes1, pool2, copy2, pad2, codes2, snap1, snap2, fcw, fcpart, C1);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// The middle of the two-convolution chain's backward (conv_chain_bwd_kernel):
// dx2 (N x 32 x 16 x 16) = the input gradient of the second convolution (w2
// 64 x 32 x 3 x 3, pad 1) from its output gradient dc2 (N x 64 x 16 x 16),
// bit for bit tt_k_conv2d_dx_lds; then the first convolution's (x N x C1 x
// 32 x 32, C1 <= 3, 32 filters, 3x3, pad 1) weight and bias gradient from
// dx2 through the 2x2 pool + relu backward of codes1, as the deferred
// reduction *job (the partials tt_k_conv2d_dw_lds_pooled would reduce, the
// same values).  -1: not covered (nothing launched); < -1: error.
extern "C" int ttk_conv2d_chain_bwd(const float *dc2, const float *w2, const unsigned char *codes1,
                                    const float *x, float *dx2, float *dw1, float *db1, int N,
                                    int C1, TTDwtJob *job, const float *x2, float *dw2,
                                    float *db2, TTDwtJob *job2) {
  if (!dc2 || !w2 || !codes1 || !x || !dx2 || !dw1 || !job || !g_dwt || N <= 0 ||
      N > 16383 || C1 < 1 || C1 > 3)
    return -1;
  if (!aligned16(dc2) || !aligned16(w2) || !aligned16(x) || ((uintptr_t)codes1 & 15)) return -1;
  // the partials must be those of the plan tt_k_conv2d_dw_lds_pooled takes
  const Geo g1{C1, 32, 32, 3, 3, 1, 1, 1, 1, 32, 32, 32, C1 * 9};
  const DwtPlan tp = plan_dwt(g1, N);
  if (tp.tg != 1 || tp.ntgw != 1 || tp.nts != 1 || tp.nfb != 1 || tp.rc != 8 || tp.jbp != 1)
    return -1;
  // the second convolution's weight gradient in the same grid: its plan must
  // be the 3 x 3 tap-group kernel over whole images
  const Geo g2{32, 16, 16, 3, 3, 1, 1, 1, 1, 16, 16, 64, 288};
  DwtPlan t2;
  if (dw2) {
    if (!x2 || !job2 || !aligned16(x2)) return -1;
    t2 = plan_dwt(g2, N);
    if (t2.tg != 3 || t2.ntgw != 3 || t2.nts != 1 || t2.lds > sizeof(float) * chainb::LDS_FLOATS)
      return -1;
  }
  if (fail_direct()) return -3;
  constexpr size_t lds = sizeof(float) * chainb::LDS_FLOATS;
  const void *kern = dw2 ? (const void *)conv_chain_bwd_dw2_kernel : (const void *)conv_chain_bwd_kernel;
  if (!allow_big_lds(kern)) return -1;
  const long S = 1024 + 32;
  float *part = (float *)ttrt_alloc(sizeof(float) * (size_t)(S * tp.units));
  if (!part) return -2;
  float *part2 = nullptr;
  const long S2 = dw2 ? (long)t2.jbp * 1024 + 32 : 0;
  if (dw2 && !(part2 = (float *)ttrt_alloc(sizeof(float) * (size_t)(S2 * t2.units * t2.nfb)))) {
    ttrt_free(part);
    return -2;
  }
  if (dw2)
    hipLaunchKernelGGL(conv_chain_bwd_dw2_kernel, dim3((unsigned)(2 * N + t2.units * t2.nfb)),
                       dim3(64 * DWT_NPQ * 3), lds, stream(), dc2, w2, codes1, x, dx2, part, C1,
                       x2, part2, g2, t2.rc, t2.nch, t2.gs, t2.cs, t2.rw, t2.jbp, t2.units,
                       2 * N);
  else
    hipLaunchKernelGGL(conv_chain_bwd_kernel, dim3((unsigned)(2 * N)), dim3(chainb::NTH), lds,
                       stream(), dc2, w2, codes1, x, dx2, part, C1);
  if (hipGetLastError() != hipSuccess) {
    ttrt_free(part);
    ttrt_free(part2);
    return -3;
  }
  if (dw2) {
    const long cols2 = (long)t2.nfb * (S2 / 4);
    int zl2 = 1;
    while (zl2 < 64 && zl2 * DWT_UPL < t2.units) zl2 *= 2;
    *job2 = TTDwtJob{part2, dw2, db2, t2.units, t2.nfb, t2.jbp, 64, 288, zl2,
                     (int)((cols2 + NT / zl2 - 1) / (NT / zl2))};
  }
  const long cols = S / 4;
  int zl = 1;
  while (zl < 64 && zl * DWT_UPL < tp.units) zl *= 2;
  *job = TTDwtJob{part, dw1, db1, tp.units, 1, 1, 32, C1 * 9, zl,
                  (int)((cols + NT / zl - 1) / (NT / zl))};
  return 0;
}

// ttk_conv2d_chain_bwd with the reductions run at once: dw1 / db1 (and dw2 /
// db2) written.
extern "C" int tt_k_conv2d_chain_bwd(const float *dc2, const float *w2,
                                     const unsigned char *codes1, const float *x, float *dx2,
                                     float *dw1, float *db1, const float *x2, float *dw2,
                                     float *db2, int N, int C1) {
  TTDwtJob job[2];
  const int rc = ttk_conv2d_chain_bwd(dc2, w2, codes1, x, dx2, dw1, db1, N, C1, &job[0], x2, dw2,
                                      db2, &job[1]);
  if (rc != 0) return rc;
  return ttk_dwt_reduce_jobs(job, dw2 ? 2 : 1);
}
