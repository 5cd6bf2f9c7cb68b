// fp32 GEMM on the CDNA4 matrix cores (gfx950).
//
// Replaces, behind the same C ABI:
//   tt_sgemm_rowmajor      reference src/gemm.c:569-641  (C = A*B, NN)
//   matmul_nt              reference src/autograd.c:66-84 (dA = dC * B^T)
//   matmul_tn              reference src/autograd.c:87-103 (dB = A^T * dC)
//   conv forward GEMM      reference src/ops_spatial.c:96-121 (W*col, +bias, NCHW permute)
//   sgemm_A_Bt_local       reference src/autograd.c:439-454 (conv dW = Gperm * col^T)
//   conv dX GEMM           reference src/autograd.c:515-539 (dcol = W^T * Gperm)
//
// Design
//   * v_mfma_f32_32x32x2_f32: one instruction multiplies a 32x2 by a 2x32
//     fp32 block (2048 FMA, 16 passes).  Lane l feeds A[l%32][l/32] and
//     B[l/32][l%32]; it receives D rows 8*(r/4) + 4*(l/32) + r%4, column l%32,
//     in accumulator r = 0..15.
//   * K is consumed 8 at a time per lane half: lane half g = l/32 holds the
//     four k values kk+4g .. kk+4g+3 of each operand, so four MFMAs cover k
//     kk..kk+7 (instruction s sums k = kk+s and kk+4+s).  With k-contiguous
//     LDS rows that is one ds_read_b128 per 32-row block.
//   * 256 threads = 4 waves in a 2x2 grid; wave tile (BM/2)x(BN/2) made of
//     (BM/64)x(BN/64) 32x32 MFMA blocks whose accumulators stay in registers.
//   * Global -> register prefetch of tile k+1 overlaps the MFMAs on tile k;
//     LDS is double buffered so one barrier per K tile suffices.
//   * LDS padding: k-contiguous rows are BK+4 floats (16-byte row skew, the
//     b128 reads of 16 consecutive rows hit disjoint banks); m/n-contiguous
//     rows are BM+8 floats (lane halves reading rows k and k+4 land 32 banks
//     apart).
//   * Out-of-range rows/cols/k are zero-filled in LDS, so any M, N, K works
//     (the ragged 1000x1003x997 case); stores are predicated.
//   * Tiles are remapped XCD-aware: the dispatcher deals workgroups round
//     robin over the 8 XCDs, so consecutive logical tiles are gathered onto
//     one XCD (shared L2) and grouped GROUP_M tile-rows at a time.
//   * Split-K for small-MN / huge-K shapes (conv dW has K = N*Ho*Wo): each
//     split writes a partial tile to a workspace and a second kernel sums the
//     splits in a fixed order (deterministic, no atomics).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include "tt_rt.h"
#include "probe.h"
TT_PROBE_DEFINE(gemm)

namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int NT = 256;      // threads per workgroup
constexpr int GROUP_M = 8;   // tile-row grouping for L2 reuse

// Epilogues: plain row-major store; conv forward (bias[row] added, column p
// stored to out[p / HW][row][p % HW]); conv dW with its bias gradient (the
// last of N columns holds sum_p g[row][p] against a row of ones appended to
// the im2col matrix: it is written to db[row] = ((float *)bias)[row], the
// first N-1 columns to C with leading dimension ldc).
enum { EPI_STORE = 0, EPI_BIAS_NCHW = 1, EPI_DW_BIAS = 2 };

// Operand addressing.  The "contiguous" index of an operand is k for a
// k-contiguous A or B^T layout, or m / n for an m/n-contiguous layout.  A
// permuted operand splits its contiguous index i into (i / hw, i % hw) and
// addresses  p[row*ld + (i/hw)*img + i%hw]  -- an NCHW gradient read as the
// F x (N*Ho*Wo) matrix without materialising the permute.
struct Opnd {
  const float *p;
  long ld;
  long img;
  int hw;
};

// Implicit im2col operand: element (kc, p) of the (C*HH*WW [+1]) x
// (N*Ho*Wo) im2col matrix of the NCHW tensor x -- x[n][c][ho*sh-ph+kh]
// [wo*sw-pw+kw] or 0 in the padding, with kc = (c*HH + kh)*WW + kw and
// p = (n*Ho + ho)*Wo + wo (the reference layout, src/ops_spatial.c:48-67),
// and, when `ones`, a last row kc = Kc of ones.  The GEMM reads it straight
// from x: no im2col matrix is written or read.  Element offsets fit in 32
// bits (checked at launch).
struct I2C {
  const float *x;
  int C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, Kc, ones;
};

// Per-kc entry of the workgroup's LDS table: .x = c*H*W + kh*W + kw, .y =
// kh << 16 | kw, or a negative .y for a row of ones / an empty row.
constexpr int I2C_ONES = -1, I2C_EMPTY = -2;
constexpr int I2C_TAB = 1024;  // k entries per workgroup (forward / dX form)

__device__ __forceinline__ int2 i2c_entry(const I2C &cv, int kc, int lim) {
  if (kc >= lim) return make_int2(0, I2C_EMPTY);
  if (kc >= cv.Kc) return make_int2(0, cv.ones ? I2C_ONES : I2C_EMPTY);
  const unsigned taps = (unsigned)(cv.HH * cv.WW);
  const unsigned c = (unsigned)kc / taps;
  const unsigned r = (unsigned)kc - c * taps;
  const unsigned kh = r / (unsigned)cv.WW;
  const unsigned kw = r - kh * (unsigned)cv.WW;
  return make_int2((int)(c * (unsigned)(cv.H * cv.W) + kh * (unsigned)cv.W + kw),
                   (int)((kh << 16) | kw));
}

// Origin of output pixel p: offset of x[n][0][hi0][wi0] and (hi0, wi0); a
// pixel at or past `lim` gets an origin that no tap can bring in range.
struct I2CPix {
  int base, hi0, wi0;
};

__device__ __forceinline__ I2CPix i2c_pixel(const I2C &cv, long p, long lim) {
  I2CPix o{0, -(1 << 30), 0};
  if (p >= lim) return o;
  const unsigned hw = (unsigned)(cv.Ho * cv.Wo);
  const unsigned n = (unsigned)p / hw;
  const unsigned r = (unsigned)p - n * hw;
  const unsigned ho = r / (unsigned)cv.Wo;
  const unsigned wo = r - ho * (unsigned)cv.Wo;
  o.hi0 = (int)ho * cv.sh - cv.ph;
  o.wi0 = (int)wo * cv.sw - cv.pw;
  o.base = (int)(n * (unsigned)(cv.C * cv.H * cv.W)) + o.hi0 * cv.W + o.wi0;
  return o;
}

// Branch-free: the load is always issued (from x[0] when the tap falls in
// the padding) and the value selected afterwards.  A load under a divergent
// branch makes the compiler wait for it before the branches rejoin, which
// serialises every element's memory latency.
__device__ __forceinline__ float i2c_value(const I2C &cv, const I2CPix &px, int2 en) {
  const int hi = px.hi0 + (en.y >> 16);
  const int wi = px.wi0 + (en.y & 0xffff);
  const bool inb = en.y >= 0 && (unsigned)hi < (unsigned)cv.H && (unsigned)wi < (unsigned)cv.W;
  const float v = cv.x[inb ? px.base + en.x : 0];
  const float other = (en.y == I2C_ONES && px.hi0 > -(1 << 29)) ? 1.0f : 0.0f;
  return inb ? v : other;
}

// Contiguous indices are below 2^31 (checked at launch), so the permuted
// split uses 32-bit unsigned division -- 64-bit division is a long software
// sequence on the GPU.
template <bool PERM>
__device__ __forceinline__ long cidx(const Opnd &o, long i) {
  if constexpr (PERM) {
    const unsigned ui = (unsigned)i, hw = (unsigned)o.hw;
    const unsigned q = ui / hw;
    return (long)q * o.img + (long)(ui - q * hw);
  } else {
    return i;
  }
}

// Load 4 consecutive contiguous-index elements (i0 % 4 == 0) of stored row
// `row`, zero-filling what lies outside [0, rows) x [0, ext).
template <bool PERM, bool VEC>
__device__ __forceinline__ float4 load4(const Opnd &o, long row, long rows, long i0, long ext) {
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (row >= rows) return v;
  const float *base = o.p + row * o.ld;
  if (VEC && i0 + 3 < ext) {
    v = *reinterpret_cast<const float4 *>(base + cidx<PERM>(o, i0));
  } else {
    if (i0 + 0 < ext) v.x = base[cidx<PERM>(o, i0 + 0)];
    if (i0 + 1 < ext) v.y = base[cidx<PERM>(o, i0 + 1)];
    if (i0 + 2 < ext) v.z = base[cidx<PERM>(o, i0 + 2)];
    if (i0 + 3 < ext) v.w = base[cidx<PERM>(o, i0 + 3)];
  }
  return v;
}

// W consecutive floats from LDS (16/8/4-byte aligned) into t[0..W-1]
template <int W>
__device__ __forceinline__ void ldsvec(float *t, const float *p) {
  if constexpr (W == 4) {
    const float4 v = *reinterpret_cast<const float4 *>(p);
    t[0] = v.x; t[1] = v.y; t[2] = v.z; t[3] = v.w;
  } else if constexpr (W == 2) {
    const float2 v = *reinterpret_cast<const float2 *>(p);
    t[0] = v.x; t[1] = v.y;
  } else {
    t[0] = p[0];
  }
}

template <int W>
__device__ __forceinline__ void stvec(float *p, const float *v) {
  if constexpr (W == 4) {
    *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
  } else if constexpr (W == 2) {
    *reinterpret_cast<float2 *>(p) = make_float2(v[0], v[1]);
  } else {
    p[0] = v[0];
  }
}

template <int BM, int BN, int BK, int WM, bool A_KC, bool A_PERM, bool B_NC, bool B_PERM,
          bool VEC, int EPI>
struct Cfg {
  static constexpr int WN = 4 / WM;             // wave grid WM x WN
  static constexpr int MI = BM / (32 * WM);     // 32x32 blocks per wave along m
  static constexpr int NI = BN / (32 * WN);     // ... along n
  static constexpr int A_ROWS = A_KC ? BM : BK; // stored rows of the LDS A tile
  static constexpr int A_LD = A_KC ? BK + 4 : BM + 8;
  static constexpr int B_ROWS = B_NC ? BK : BN;
  static constexpr int B_LD = B_NC ? BN + 8 : BK + 4;
  static constexpr int A_SZ = A_ROWS * A_LD;
  static constexpr int B_SZ = B_ROWS * B_LD;
  static constexpr int STAGE = A_SZ + B_SZ;
  static constexpr int A_V4 = BM * BK / 4 / NT;  // float4 loads per thread
  static constexpr int B_V4 = BN * BK / 4 / NT;
  static_assert(A_V4 >= 1 && B_V4 >= 1, "tile too small for 256 threads");
  static_assert(MI >= 1 && NI >= 1 && BM % (32 * WM) == 0 && BN % (32 * WN) == 0 && BK % 8 == 0,
                "tile shape");
  static_assert(MI == 1 || MI == 2 || MI == 4, "MI must be 1, 2 or 4");
  static_assert(NI == 1 || NI == 2 || NI == 4, "NI must be 1, 2 or 4");
};

template <int BM, int BN, int BK, int WM, bool A_KC, bool A_PERM, bool B_NC, bool B_PERM,
          bool VEC, int EPI, bool B_I2C>
__device__ __forceinline__ void gemm_body(float *smem, int M, int N, int K, const Opnd &A,
                                          const Opnd &B, float *__restrict__ C, long ldc,
                                          long split_stride, int kchunk,
                                          const float *__restrict__ bias, int HW, bool cvec,
                                          const I2C &cv) {
  using G = Cfg<BM, BN, BK, WM, A_KC, A_PERM, B_NC, B_PERM, VEC, EPI>;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  const int l32 = lane & 31;
  const int g = lane >> 5;

  // ---- XCD-aware tile mapping ----
  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = (N + BN - 1) / BN;
  const int ntiles = tiles_m * tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int group = GROUP_M * tiles_n;
  const int first_m = (pid / group) * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (pid % group) % gsz;
  const int tn = (pid % group) / gsz;
  const long m0 = (long)tm * BM;
  const long n0 = (long)tn * BN;

  const int kbeg = blockIdx.z * kchunk;
  const int kend = min(K, kbeg + kchunk);
  const int nk = (kend - kbeg + BK - 1) / BK;
  C += (long)blockIdx.z * split_stride;

  const int wm = (wave / G::WN) * (BM / WM);
  const int wn = (wave % G::WN) * (BN / G::WN);

  f32x16 acc[G::MI][G::NI];
#pragma unroll
  for (int i = 0; i < G::MI; i++)
#pragma unroll
    for (int j = 0; j < G::NI; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  float4 ra[G::A_V4], rb[G::B_V4];

  // ---- implicit im2col B: LDS table of kc decompositions, pixel origins ----
  // Forward / dX form (B_NC): the table covers this split's k range; each
  // thread owns one column p (fixed) and 4*B_V4 rows.  dW form (!B_NC): the
  // table covers the tile's BN rows kc; each thread owns one k column
  // (p = k0 + tid % BK, decomposed per K tile) and 4*B_V4 rows.
  static_assert(!B_I2C || (B_NC ? NT % BN == 0 : BN % 32 == 0), "I2C tile shape");
  constexpr int I2C_RSTEP = B_NC ? (NT / BN) * 4 : (NT / BK) * 4;  // row step between v
  int2 *tab = reinterpret_cast<int2 *>(smem + 2 * G::STAGE);
  const int i2c_c = B_NC ? tid % BN : tid % BK;        // owned column in the LDS tile
  const int i2c_r = B_NC ? (tid / BN) * 4 : (tid / BK) * 4;  // first owned row
  I2CPix px{0, -(1 << 30), 0};
  if constexpr (B_I2C) {
    if constexpr (B_NC) {
      for (int i = tid; i < nk * BK; i += NT) tab[i] = i2c_entry(cv, kbeg + i, kend);
      px = i2c_pixel(cv, n0 + i2c_c, N);
    } else {
      for (int i = tid; i < BN; i += NT) tab[i] = i2c_entry(cv, (int)n0 + i, N);
    }
    __syncthreads();
  }
  auto i2c_load = [&](int kt, float4 *xb) {
    if constexpr (B_I2C) {
      if constexpr (!B_NC) px = i2c_pixel(cv, kbeg + (long)kt * BK + i2c_c, kend);
      // all table entries first (one LDS wait), then every load
      int4 en[G::B_V4][2];
#pragma unroll
      for (int v = 0; v < G::B_V4; v++) {
        const int r = i2c_r + v * I2C_RSTEP;
        const int4 *tp = reinterpret_cast<const int4 *>(tab + (B_NC ? kt * BK + r : r));
        en[v][0] = tp[0];
        en[v][1] = tp[1];
      }
#pragma unroll
      for (int v = 0; v < G::B_V4; v++) {
        xb[v] = make_float4(i2c_value(cv, px, make_int2(en[v][0].x, en[v][0].y)),
                            i2c_value(cv, px, make_int2(en[v][0].z, en[v][0].w)),
                            i2c_value(cv, px, make_int2(en[v][1].x, en[v][1].y)),
                            i2c_value(cv, px, make_int2(en[v][1].z, en[v][1].w)));
      }
    }
  };

  // Interior tiles of unpermuted, 16-byte aligned operands take a branch-free
  // path: per-thread element offsets are fixed for the whole K loop and
  // advance by a uniform stride per K tile.  Edge tiles and permuted
  // operands use the bounds-checked loads.
  // A permuted operand (an NCHW gradient read as F x N*Ho*Wo) is 16 bytes
  // contiguous per float4 when hw % 4 == 0, which VEC guarantees: its fixed
  // part is precomputed, its K-dependent split (one 32-bit division per
  // float4) is done per K tile.
  constexpr bool FAST_OK = VEC;
  const bool interior = FAST_OK && (m0 + BM <= M) && (n0 + BN <= N);
  long aoff[G::A_V4], boff[G::B_V4];
  int acol[G::A_V4];
  if constexpr (FAST_OK) {
#pragma unroll
    for (int v = 0; v < G::A_V4; v++) {
      const int q = tid + v * NT;
      if constexpr (A_KC) {
        const int r = q / (BK / 4), c = (q % (BK / 4)) * 4;
        acol[v] = c;
        aoff[v] = A_PERM ? (m0 + r) * A.ld : (m0 + r) * A.ld + kbeg + c;
      } else {
        const int r = q / (BM / 4), c = (q % (BM / 4)) * 4;
        acol[v] = c;
        aoff[v] = (long)(kbeg + r) * A.ld + m0 + c;
      }
    }
#pragma unroll
    for (int v = 0; v < G::B_V4; v++) {
      const int q = tid + v * NT;
      if constexpr (B_I2C) {
        boff[v] = 0;
      } else if constexpr (B_NC) {
        const int r = q / (BN / 4), c = (q % (BN / 4)) * 4;
        boff[v] = (long)(kbeg + r) * B.ld + cidx<B_PERM>(B, n0 + c);
      } else {
        const int r = q / (BK / 4), c = (q % (BK / 4)) * 4;
        boff[v] = (n0 + r) * B.ld + kbeg + c;
      }
    }
  }

  auto gload = [&](int kt, float4 *xa, float4 *xb) {
    const long k0 = kbeg + (long)kt * BK;
    if (FAST_OK && interior && k0 + BK <= kend) {
      const long astep = A_KC ? (long)kt * BK : (long)kt * BK * A.ld;
      const long bstep = B_NC ? (long)kt * BK * B.ld : (long)kt * BK;
#pragma unroll
      for (int v = 0; v < G::A_V4; v++) {
        if constexpr (A_PERM)
          xa[v] = *reinterpret_cast<const float4 *>(A.p + aoff[v] + cidx<true>(A, k0 + acol[v]));
        else
          xa[v] = *reinterpret_cast<const float4 *>(A.p + aoff[v] + astep);
      }
      if constexpr (B_I2C) {
        i2c_load(kt, xb);
      } else {
#pragma unroll
        for (int v = 0; v < G::B_V4; v++)
          xb[v] = *reinterpret_cast<const float4 *>(B.p + boff[v] + bstep);
      }
      return;
    }
#pragma unroll
    for (int v = 0; v < G::A_V4; v++) {
      const int q = tid + v * NT;
      if constexpr (A_KC) {  // stored row = m, contiguous = k
        const int r = q / (BK / 4), c = (q % (BK / 4)) * 4;
        xa[v] = load4<A_PERM, VEC>(A, m0 + r, M, k0 + c, kend);
      } else {               // stored row = k, contiguous = m
        const int r = q / (BM / 4), c = (q % (BM / 4)) * 4;
        xa[v] = load4<false, VEC>(A, k0 + r, kend, m0 + c, M);
      }
    }
    if constexpr (B_I2C) {
      i2c_load(kt, xb);
      return;
    }
#pragma unroll
    for (int v = 0; v < G::B_V4; v++) {
      const int q = tid + v * NT;
      if constexpr (B_NC) {  // stored row = k, contiguous = n
        const int r = q / (BN / 4), c = (q % (BN / 4)) * 4;
        xb[v] = load4<B_PERM, VEC>(B, k0 + r, kend, n0 + c, N);
      } else {               // stored row = n, contiguous = k
        const int r = q / (BK / 4), c = (q % (BK / 4)) * 4;
        xb[v] = load4<false, VEC>(B, n0 + r, N, k0 + c, kend);
      }
    }
  };

  auto sstore = [&](int buf, const float4 *xa, const float4 *xb) {
    float *sA = smem + buf * G::STAGE;
    float *sB = sA + G::A_SZ;
#pragma unroll
    for (int v = 0; v < G::A_V4; v++) {
      const int q = tid + v * NT;
      int r, c;
      if constexpr (A_KC) { r = q / (BK / 4); c = (q % (BK / 4)) * 4; }
      else                { r = q / (BM / 4); c = (q % (BM / 4)) * 4; }
      *reinterpret_cast<float4 *>(sA + r * G::A_LD + c) = xa[v];
    }
    if constexpr (B_I2C) {
      // one column, four consecutive rows per v: scalar LDS writes
#pragma unroll
      for (int v = 0; v < G::B_V4; v++) {
        float *d = sB + (i2c_r + v * I2C_RSTEP) * G::B_LD + i2c_c;
        d[0] = xb[v].x;
        d[G::B_LD] = xb[v].y;
        d[2 * G::B_LD] = xb[v].z;
        d[3 * G::B_LD] = xb[v].w;
      }
      return;
    }
#pragma unroll
    for (int v = 0; v < G::B_V4; v++) {
      const int q = tid + v * NT;
      int r, c;
      if constexpr (B_NC) { r = q / (BN / 4); c = (q % (BN / 4)) * 4; }
      else                { r = q / (BK / 4); c = (q % (BK / 4)) * 4; }
      *reinterpret_cast<float4 *>(sB + r * G::B_LD + c) = xb[v];
    }
  };

  // Operand fragments.  A k-contiguous operand is read as one float4 of 4 k
  // per 32-row block.  An m- (n-) contiguous operand is read as one vector of
  // MI (NI) consecutive m (n) per k: lane l32 then feeds row/column l32 of
  // block i (j) with element MI*l32 + i (NI*l32 + j), i.e. the blocks are
  // interleaved in m (n) and the epilogue maps them back.
  auto compute = [&](int buf) {
    const float *sA = smem + buf * G::STAGE;
    const float *sB = sA + G::A_SZ;
#pragma unroll
    for (int kk = 0; kk < BK; kk += 8) {
      float a[G::MI][4], b[G::NI][4];
      if constexpr (A_KC) {
#pragma unroll
        for (int i = 0; i < G::MI; i++) {
          const float4 t = *reinterpret_cast<const float4 *>(sA + (wm + 32 * i + l32) * G::A_LD + kk + 4 * g);
          a[i][0] = t.x; a[i][1] = t.y; a[i][2] = t.z; a[i][3] = t.w;
        }
      } else {
#pragma unroll
        for (int s = 0; s < 4; s++) {
          float t[G::MI];
          ldsvec<G::MI>(t, sA + (kk + 4 * g + s) * G::A_LD + wm + G::MI * l32);
#pragma unroll
          for (int i = 0; i < G::MI; i++) a[i][s] = t[i];
        }
      }
      if constexpr (B_NC) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
          float t[G::NI];
          ldsvec<G::NI>(t, sB + (kk + 4 * g + s) * G::B_LD + wn + G::NI * l32);
#pragma unroll
          for (int j = 0; j < G::NI; j++) b[j][s] = t[j];
        }
      } else {
#pragma unroll
        for (int j = 0; j < G::NI; j++) {
          const float4 t = *reinterpret_cast<const float4 *>(sB + (wn + 32 * j + l32) * G::B_LD + kk + 4 * g);
          b[j][0] = t.x; b[j][1] = t.y; b[j][2] = t.z; b[j][3] = t.w;
        }
      }
#pragma unroll
      for (int s = 0; s < 4; s++)
#pragma unroll
        for (int i = 0; i < G::MI; i++)
#pragma unroll
          for (int j = 0; j < G::NI; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
    }
  };

  if (nk > 0) {
    gload(0, ra, rb);
    sstore(0, ra, rb);
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
      const bool more = kt + 1 < nk;
      if (more) gload(kt + 1, ra, rb);
      compute(kt & 1);
      if (more) sstore((kt + 1) & 1, ra, rb);
      __syncthreads();
    }
  }

  // ---- epilogue ----
  // block i row rho (acc r: rho = 8*(r/4) + 4*g + r%4) is m = wm + 32*i + rho
  // (k-contiguous A) or wm + MI*rho + i (interleaved A); block j column l32
  // is n = wn + 32*j + l32 or wn + NI*l32 + j (interleaved B).  With
  // interleaved B a lane owns NI adjacent columns and stores them as one
  // vector.  Everything that depends only on the column (the NCHW split of
  // the conv epilogue) is computed once per lane, outside the row loops.
  constexpr int NC = B_NC ? 1 : G::NI;  // column groups per lane
  constexpr int NW = B_NC ? G::NI : 1;  // adjacent columns per group
  long cbase[NC];     // element offset of the group's first column, row 0
  long cstride;       // offset between consecutive rows
  bool cok[NC], cvok[NC];
  if constexpr (EPI == EPI_BIAS_NCHW) cstride = HW;
  else cstride = ldc;
#pragma unroll
  for (int j = 0; j < NC; j++) {
    const long col = n0 + wn + (B_NC ? G::NI * l32 : 32 * j + l32);
    cok[j] = col < N;
    cvok[j] = cvec && col + NW <= N;
    if constexpr (EPI == EPI_BIAS_NCHW) {
      const unsigned q = (unsigned)col / (unsigned)HW;
      const unsigned hw = (unsigned)col - q * (unsigned)HW;
      cbase[j] = (long)q * M * HW + hw;
      cvok[j] = cvok[j] && hw + NW <= (unsigned)HW;
    } else {
      cbase[j] = col;
    }
  }
#pragma unroll
  for (int i = 0; i < G::MI; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int rho = 8 * (r >> 2) + 4 * g + (r & 3);
      const long row = m0 + (A_KC ? wm + 32 * i + rho : wm + G::MI * rho + i);
      if (row >= M) continue;
      const float bv = (EPI == EPI_BIAS_NCHW && bias) ? bias[row] : 0.f;
#pragma unroll
      for (int j = 0; j < NC; j++) {
        if (!cok[j]) continue;
        float v[NW];
#pragma unroll
        for (int w = 0; w < NW; w++) v[w] = acc[i][B_NC ? w : j][r] + bv;
        const long col = n0 + wn + (B_NC ? G::NI * l32 : 32 * j + l32);
        if constexpr (EPI == EPI_DW_BIAS) {
#pragma unroll
          for (int w = 0; w < NW; w++) {
            if (col + w < N - 1) C[row * ldc + col + w] = v[w];
            else if (col + w == N - 1) const_cast<float *>(bias)[row] = v[w];
          }
        } else if (cvok[j]) {
          stvec<NW>(C + row * cstride + cbase[j], v);
        } else if constexpr (EPI == EPI_STORE) {
#pragma unroll
          for (int w = 0; w < NW; w++)
            if (col + w < N) C[row * ldc + col + w] = v[w];
        } else {
#pragma unroll
          for (int w = 0; w < NW; w++) {
            const long cc = col + w;
            if (cc >= N) continue;
            const unsigned q = (unsigned)cc / (unsigned)HW;
            C[((long)q * M + row) * HW + ((unsigned)cc - q * (unsigned)HW)] = v[w];
          }
        }
      }
    }
}

template <int BM, int BN, int BK, int WM, bool A_KC, bool A_PERM, bool B_NC, bool B_PERM,
          bool VEC, int EPI, bool B_I2C>
__global__ void __launch_bounds__(NT)
gemm_mfma_kernel(int M, int N, int K, Opnd A, Opnd B, float *__restrict__ C, long ldc,
                 long split_stride, int kchunk, const float *__restrict__ bias, int HW,
                 bool cvec, I2C cv) {
  using G = Cfg<BM, BN, BK, WM, A_KC, A_PERM, B_NC, B_PERM, VEC, EPI>;
  // implicit im2col adds its int2 table (2 floats per entry)
  constexpr int TAB = B_I2C ? 2 * (B_NC ? I2C_TAB : BN) : 0;
  __shared__ __attribute__((aligned(16))) float smem[2 * G::STAGE + TAB];
  gemm_body<BM, BN, BK, WM, A_KC, A_PERM, B_NC, B_PERM, VEC, EPI, B_I2C>(
      smem, M, N, K, A, B, C, ldc, split_stride, kchunk, bias, HW, cvec, cv);
}

// The 256x256 tile keeps 256 fp32 accumulators per lane: one wave per SIMD,
// the whole register file.
template <int BM, int BN, int BK, int WM, bool A_KC, bool A_PERM, bool B_NC, bool B_PERM,
          bool VEC, int EPI>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_mfma_big_kernel(int M, int N, int K, Opnd A, Opnd B, float *__restrict__ C, long ldc,
                     long split_stride, int kchunk, const float *__restrict__ bias, int HW,
                     bool cvec) {
  using G = Cfg<BM, BN, BK, WM, A_KC, A_PERM, B_NC, B_PERM, VEC, EPI>;
  __shared__ __attribute__((aligned(16))) float smem[2 * G::STAGE];
  gemm_body<BM, BN, BK, WM, A_KC, A_PERM, B_NC, B_PERM, VEC, EPI, false>(
      smem, M, N, K, A, B, C, ldc, split_stride, kchunk, bias, HW, cvec, I2C{});
}

// Deterministic split-K reduction: out = sum_{z=0..S-1} ws[z] (+ epilogue).
// A workgroup is XL outputs x ZL split-lanes (XL*ZL = 256): lane ty adds
// z = ty, ty+ZL, ... in order, then lane ty == 0 adds the ZL lane sums in
// order.  Small outputs with many splits (conv dW, K = N*Ho*Wo) use wide ZL
// so that hundreds of waves share the reduction.
template <int EPI, int ZL>
__global__ void __launch_bounds__(256)
splitk_reduce_kernel(const float *__restrict__ ws, float *__restrict__ C, int M, int N, int S,
                     long ldc, const float *__restrict__ bias, int HW) {
  constexpr int XL = 256 / ZL;
  __shared__ float part[ZL][XL];
  const int tx = threadIdx.x % XL, ty = threadIdx.x / XL;
  const long total = (long)M * N;
  const long idx = (long)blockIdx.x * XL + tx;
  float s = 0.f;
  if (idx < total) {
#pragma unroll 4
    for (int z = ty; z < S; z += ZL) s += ws[z * total + idx];
  }
  part[ty][tx] = s;
  __syncthreads();
  if (ty != 0 || idx >= total) return;
  for (int j = 1; j < ZL; j++) s += part[j][tx];
  const unsigned row = (unsigned)(idx / N), col = (unsigned)(idx - (long)row * N);
  if constexpr (EPI == EPI_STORE) {
    C[(long)row * ldc + col] = s;
  } else if constexpr (EPI == EPI_DW_BIAS) {
    if ((int)col < N - 1) C[(long)row * ldc + col] = s;
    else const_cast<float *>(bias)[row] = s;
  } else {
    const unsigned q = col / (unsigned)HW;
    C[((long)q * M + row) * HW + (col - q * (unsigned)HW)] = s + (bias ? bias[row] : 0.f);
  }
}

// The split-K reduction of a row-major C = A*B (ldc = N) with the relu +
// padones that follow it in an MLP layer fused in: R = relu(C) and
// P = [R, 1] (M x (N+1)) as well as C, the values relu_padones_rows_kernel
// writes from C.
struct ReluPadEx {
  float *r, *p;         // may be null (the bias-only form)
  const float *bias;    // row added to every output row, or null
};

template <int ZL>
__device__ __forceinline__ float reduce_one(const float *__restrict__ ws, int S, long total,
                                            long idx, int ty, float (*part)[256 / ZL], int tx) {
  float s = 0.f;
  if (idx < total) {
#pragma unroll 4
    for (int z = ty; z < S; z += ZL) s += ws[z * total + idx];
  }
  part[ty][tx] = s;
  __syncthreads();
  if (ty == 0)
    for (int j = 1; j < ZL; j++) s += part[j][tx];
  return s;
}

template <int ZL>
__global__ void __launch_bounds__(256)
splitk_reduce_relu_pad_kernel(const float *__restrict__ ws, float *__restrict__ C, int M, int N,
                              int S, ReluPadEx ex) {
  constexpr int XL = 256 / ZL;
  __shared__ float part[ZL][XL];
  const int tx = threadIdx.x % XL, ty = threadIdx.x / XL;
  const long total = (long)M * N;
  const long idx = (long)blockIdx.x * XL + tx;
  const float s = reduce_one<ZL>(ws, S, total, idx, ty, part, tx);
  if (ty != 0 || idx >= total) return;
  const unsigned row = (unsigned)(idx / N), col = (unsigned)(idx - (long)row * N);
  const float v = ex.bias ? s + ex.bias[col] : s;
  const float o = v > 0.0f ? v : 0.0f;
  C[idx] = v;
  if (ex.r) ex.r[idx] = o;
  if (ex.p) {
    float *pr = ex.p + (long)row * (N + 1);
    pr[col] = o;
    if ((int)col == N - 1) pr[N] = 1.0f;
  }
}

// ---- 256x256 tile with direct global->LDS loads ----
// gfx950's global_load_lds_dwordx4 moves 16 bytes per lane from global memory
// straight into LDS (lane i of a wave writes bytes [16i, 16i+16) after the
// wave-uniform LDS address), so the next K tile needs no staging registers:
// the 64 VGPRs the register-staged kernel spends on it go to fragment
// buffers, and the ds_write pass disappears.  Operand layouts in LDS:
//   m/n-contiguous (NN's B, TN's A; rows k of 256 floats): one wave load
//     fills one padded row, fragments read as 4 consecutive m/n per lane
//     (interleaved blocks, as in the register-staged kernel);
//   k-contiguous (NN's A, NT's B; rows m/n of 32 k, unpadded 128-byte rows):
//     a wave load fills 8 rows, and 16-byte chunk c of row R sits in slot
//     c ^ ((R >> 1) & 7), so the fragment reads (32 rows at one chunk per
//     half-wave) spread over all banks; each lane loads the global chunk
//     that belongs in its slot.
// Interior-only: the host uses it when M and N are multiples of 256, the K
// range of every split a multiple of 32, and all rows 16-byte aligned.
constexpr int D_BM = 256, D_BN = 256, D_BK = 32;
constexpr int D_KC_LD = D_BK;        // k-contiguous rows (swizzled)
constexpr int D_NC_LD = D_BN + 8;    // m/n-contiguous rows (padded)
constexpr int D_KC_SZ = D_BM * D_KC_LD;
constexpr int D_NC_SZ = D_BK * D_NC_LD;

// One wave-wide direct load.  Issued from inline assembly on purpose: the
// compiler's own LDS-DMA builtin makes it assume the DMA may alias every
// later LDS read, and it then waits for the next tile's loads before the
// current tile's fragment reads, serialising the pipeline.  Here the kernel
// orders them itself: s_waitcnt vmcnt(0) + barrier before a tile is read.
// M0 holds the wave-uniform LDS byte address of lane 0's 16 bytes.
__device__ __forceinline__ void g2lds16(const float *src, const float *lds) {
  const unsigned addr = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(addr), "v"(src)
               : "memory", "m0");
}

__device__ __forceinline__ void wait_vm_all() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Per-lane sources and wave-uniform destinations of one operand's 8 wave
// loads per K tile.  KC: rows r = wave*64 + 8j + lane/8 of 32 k (swizzled);
// NC: rows k = wave*8 + j of 256 floats.
template <bool KC>
struct DirectOperand {
  const float *src[KC ? 8 : 1];
  long ld;
  __device__ __forceinline__ void init(const float *p, long ld_, long r0, int kbeg, int wave,
                                       int lane) {
    ld = ld_;
    if constexpr (KC) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int R = wave * 64 + 8 * j + (lane >> 3);
        const int c = (lane & 7) ^ ((R >> 1) & 7);
        src[j] = p + (r0 + R) * ld + kbeg + 4 * c;
      }
    } else {
      src[0] = p + (long)(kbeg + wave * 8) * ld + r0 + 4 * lane;
    }
  }
  __device__ __forceinline__ void issue(int kt, float *lds, int wave) const {
    issue_part<0, 8>(kt, lds, wave);
  }
  // loads J0 .. J0+NJ-1 of the 8
  template <int J0, int NJ>
  __device__ __forceinline__ void issue_part(int kt, float *lds, int wave) const {
    const long k = (long)kt * D_BK;
#pragma unroll
    for (int j = J0; j < J0 + NJ; j++) {
      if constexpr (KC) g2lds16(src[j] + k, lds + (wave * 64 + 8 * j) * D_KC_LD);
      else g2lds16(src[0] + (k + j) * ld, lds + (wave * 8 + j) * D_NC_LD);
    }
  }
  // fragment v[x][s] (x = 32-row block, s = k within the 8-step) for rows
  // base + 32x + l32 (KC) or m/n base + 4*l32 + x (NC, interleaved)
  __device__ __forceinline__ static void frag(const float *lds, int base, int kk, int l32, int g,
                                              float (*v)[4]) {
    if constexpr (KC) {
#pragma unroll
      for (int x = 0; x < 4; x++) {
        const int R = base + 32 * x + l32;
        const int slot = ((kk >> 2) + g) ^ ((R >> 1) & 7);
        const float4 t = *reinterpret_cast<const float4 *>(lds + R * D_KC_LD + 4 * slot);
        v[x][0] = t.x; v[x][1] = t.y; v[x][2] = t.z; v[x][3] = t.w;
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const float4 t =
            *reinterpret_cast<const float4 *>(lds + (kk + 4 * g + s) * D_NC_LD + base + 4 * l32);
        v[0][s] = t.x; v[1][s] = t.y; v[2][s] = t.z; v[3][s] = t.w;
      }
    }
  }
};

template <bool A_KC, bool B_NC>
__global__ void __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(1, 1)))
gemm_direct_kernel(int M, int N, int K, const float *__restrict__ A, long lda,
                   const float *__restrict__ B, long ldb, float *__restrict__ C, long ldc,
                   long split_stride, int kchunk) {
  constexpr int A_SZ = A_KC ? D_KC_SZ : D_NC_SZ;
  constexpr int B_SZ = B_NC ? D_NC_SZ : D_KC_SZ;
  constexpr int STAGE = A_SZ + B_SZ;
  __shared__ __attribute__((aligned(16))) float smem[2 * STAGE];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: LDS addresses in SGPRs
  const int l32 = lane & 31;
  const int g = lane >> 5;

  const int tiles_m = M / D_BM, tiles_n = N / D_BN;
  const int ntiles = tiles_m * tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int group = GROUP_M * tiles_n;
  const int first_m = (pid / group) * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (pid % group) % gsz;
  const int tn = (pid % group) / gsz;
  const long m0 = (long)tm * D_BM;
  const long n0 = (long)tn * D_BN;
  const int kbeg = blockIdx.z * kchunk;
  const int nk = (min(K, kbeg + kchunk) - kbeg) / D_BK;
  C += (long)blockIdx.z * split_stride;

  const int wm = (wave >> 1) * 128;
  const int wn = (wave & 1) * 128;

  // A k-contiguous: rows m of A (M x K); else rows k of A (K x M).
  // B m/n-contiguous: rows k of B (K x N); else rows n of B (N x K).
  DirectOperand<A_KC> opa;
  DirectOperand<!B_NC> opb;
  opa.init(A, lda, m0, kbeg, wave, lane);
  opb.init(B, ldb, n0, kbeg, wave, lane);

  f32x16 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  // The fragments of step kk+8 are read while the MFMAs of step kk run.
  // mid(c), c = 0..3, runs after the c-th group of 16 MFMAs of the tile's
  // first step: the next tile's loads go out a quarter at a time, each chunk
  // in the shadow of queued MFMAs, instead of as one block the matrix pipe
  // waits through.  After the third step the wave waits for those loads and
  // meets the others at the barrier (the next tile is then complete in LDS
  // and this tile's last fragments are already in registers), so the last
  // step's MFMAs cover the reads of the next tile's first fragments.
  float a[2][4][4], b[2][4][4];
  auto compute = [&](int buf, bool more, auto mid) {
    const float *sA = smem + buf * STAGE;
    const float *sB = sA + A_SZ;
    const float *nA = smem + (buf ^ 1) * STAGE;
    const float *nB = nA + A_SZ;
#pragma unroll
    for (int q = 0; q < D_BK / 8; q++) {
      const bool last = q + 1 == D_BK / 8;
      if (!last) {
        DirectOperand<A_KC>::frag(sA, wm, 8 * (q + 1), l32, g, a[(q + 1) & 1]);
        DirectOperand<!B_NC>::frag(sB, wn, 8 * (q + 1), l32, g, b[(q + 1) & 1]);
      } else if (more) {
        DirectOperand<A_KC>::frag(nA, wm, 0, l32, g, a[0]);
        DirectOperand<!B_NC>::frag(nB, wn, 0, l32, g, b[0]);
      }
#pragma unroll
      for (int s = 0; s < 4; s++) {
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q & 1][i][s], b[q & 1][j][s],
                                                             acc[i][j], 0, 0, 0);
        // Schedule (the compiler otherwise sinks each fragment read to just
        // before its first MFMA and waits on it): the step's first group
        // carries the 8 reads for the following step, one per 2 MFMAs.
        if (s == 0) {
#pragma unroll
          for (int r = 0; r < 8; r++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
            __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);  // MFMA
          }
        } else {
          __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);
        }
        if (q == 0) {
          __builtin_amdgcn_sched_barrier(0);
          mid(s);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      if (q + 2 == D_BK / 8) {
        __builtin_amdgcn_sched_barrier(0);
        wait_vm_all();
        __syncthreads();
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };

  if (nk > 0) {
    opa.issue(0, smem, wave);
    opb.issue(0, smem + A_SZ, wave);
    wait_vm_all();
    __syncthreads();
    DirectOperand<A_KC>::frag(smem, wm, 0, l32, g, a[0]);
    DirectOperand<!B_NC>::frag(smem + A_SZ, wn, 0, l32, g, b[0]);
    for (int kt = 0; kt < nk; kt++) {
      float *nb = smem + ((kt + 1) & 1) * STAGE;
      const bool more = kt + 1 < nk;
      compute(kt & 1, more, [&](int c) {
        if (!more) return;
        if (c == 0) opa.template issue_part<0, 4>(kt + 1, nb, wave);
        else if (c == 1) opa.template issue_part<4, 4>(kt + 1, nb, wave);
        else if (c == 2) opb.template issue_part<0, 4>(kt + 1, nb + A_SZ, wave);
        else opb.template issue_part<4, 4>(kt + 1, nb + A_SZ, wave);
      });
    }
  }

  // epilogue: block i row rho (acc r: rho = 8*(r/4) + 4*g + r%4) is
  // m = wm + 32i + rho (k-contiguous A) or wm + 4*rho + i (interleaved A);
  // block j column l32 is n = wn + 4*l32 + j (interleaved B: one float4 per
  // row) or wn + 32j + l32.
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int rho = 8 * (r >> 2) + 4 * g + (r & 3);
      const long row = m0 + (A_KC ? wm + 32 * i + rho : wm + 4 * rho + i);
      float *crow = C + row * ldc + n0 + wn;
      // streaming stores: C is not read again by this kernel
      if constexpr (B_NC) {
        typedef float f32x4v __attribute__((ext_vector_type(4)));
        const f32x4v v = {acc[i][0][r], acc[i][1][r], acc[i][2][r], acc[i][3][r]};
        __builtin_nontemporal_store(v, reinterpret_cast<f32x4v *>(crow + 4 * l32));
      } else {
#pragma unroll
        for (int j = 0; j < 4; j++) __builtin_nontemporal_store(acc[i][j][r], crow + 32 * j + l32);
      }
    }
}

// ---- 64x64 tile with direct loads, a deep LDS pipeline and in-workgroup split-K ----
// For GEMMs too small to give every CU a 256x256 tile (1024^3 has 16 of
// them).  A 64x64 tile per CU needs four times the loads per MFMA of the
// 256x256 tile, so the kernel keeps several K tiles of loads in flight
// (global->LDS DMA, no staging registers) and splits each K tile over its NW
// waves: wave w multiplies the whole 64x64 tile over its BK/NW k of the tile
// with four independent 32x32 accumulators, and the NW wave sums are added in
// LDS at the end in wave order (deterministic).  With NW = 8 two waves share
// each SIMD, so one wave's MFMAs run while the other issues its loads.
// Operands are 16-byte aligned with leading dimensions and contiguous extents
// multiples of 4; any M, N, K otherwise.
// LDS layouts (per stage):
//   k-contiguous operand: 64 rows of BK k, 16-byte chunk c of row R in slot
//     c ^ swz(R) (the b128 fragment reads of 32 rows at one chunk spread
//     over all banks);
//   m/n-contiguous operand: BK rows k of 64 floats; fragments are read as
//     float2, so block x of a wave holds m/n = 2*l32 + x (interleaved).
constexpr int M_T = 64;

__device__ __attribute__((aligned(16))) float g_gemm_zero[4];

// DMA with a wave-uniform base address in SGPRs and a per-lane 32-bit byte
// offset: the K loop advances only the scalar base, so issuing a tile's
// loads takes no vector instructions (vector ALU work between MFMAs stalls
// the matrix pipe).
__device__ __forceinline__ void g2lds16s(const float *sbase, unsigned voff, const float *lds) {
  const unsigned addr = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2"
               :
               : "s"(addr), "v"(voff), "s"(sbase)
               : "memory", "m0");
}

// The 4-byte forms: lane l's float goes to M0 + 4l.  A source needs only
// 4-byte alignment, so rows of any length are read in place.
__device__ __forceinline__ void g2lds4s(const float *sbase, unsigned voff, const float *lds) {
  const unsigned addr = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, %2"
               :
               : "s"(addr), "v"(voff), "s"(sbase)
               : "memory", "m0");
}
__device__ __forceinline__ void g2lds4(const float *src, const float *lds) {
  const unsigned addr = __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)lds);
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off"
               :
               : "s"(addr), "v"(src)
               : "memory", "m0");
}

// s_waitcnt vmcnt(N) for a compile-time N (capped at the counter's 63)
template <int N>
__device__ __forceinline__ void wait_vm() {
  constexpr int n = N > 63 ? 63 : N;
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(n) : "memory");
}

// One operand's loads.  x4 form (DW false): 16 bytes a lane, a load fills
// 256 floats of LDS.  DW form: 4 bytes a lane, a load fills 64 floats; the
// same LDS layout, element by element, so any row length and alignment is
// read in place (no aligned copy).  KC: rows r0+R of a row-major (rows x K)
// matrix, BK k per tile.  NC: rows k of a row-major (K x cols) matrix,
// columns r0 .. r0+63.  lim = rows (KC) or the columns that may be read (NC:
// x4 form a multiple of 4, at least cols; DW form cols).  Rows / columns past
// lim load row / column lim-1 (x4 NC: the 4 columns from lim-4) instead (they
// only feed outputs that are not stored), so a tile's loads need no range
// test; only k past the end of the K range (the last tile) must read zeros.
// Each lane keeps the byte offset of its element in every load relative to
// the tile origin (row r0 at k0 for KC, row k0 at column r0 for NC); the host
// keeps these below 2^32 (64 rows of the leading dimension).
template <bool KC, int BK, int NW, int T = M_T, int KSL = NW, bool DW = false>
struct MidOperand {
  // T: the tile's extent in this operand (rows for KC, columns for NC);
  // KSL: waves sharing one K tile (its k slices)
  static constexpr int CPR = BK / 4;               // 16-byte chunks per KC row
  static constexpr int LF = DW ? 64 : 256;         // floats of LDS per load
  static constexpr int NL = T * BK / (LF * NW);    // loads per wave per tile
  static_assert(NL >= 1 && NL * LF * NW == T * BK, "tile too small for the waves");
  // 16-byte chunk swizzle of KC rows: a fragment read of 16 lanes (rows R..
  // R+15 of one chunk) touches every bank once (8-k rows: rows 8 apart would
  // share banks, so their two chunks swap)
  __device__ __forceinline__ static int swz(int R) {
    return BK == 8 ? (R >> 3) & 1 : BK == 32 ? (R >> 1) & 7 : R & 15;
  }
  unsigned voff[NL];
  const float *p;
  long ld, r0;
  int wave, lane;
  // the tile float that load j's lane fills, as (x4 load q4, its lane l4,
  // float e of the lane's 16 bytes)
  __device__ __forceinline__ void pos(int j, int &q4, int &l4, int &e) const {
    const int f = (wave * NL + j) * LF + (DW ? lane : 4 * lane);
    q4 = f >> 8;
    l4 = (f & 255) >> 2;
    e = f & 3;
  }
  __device__ __forceinline__ void init(const float *p_, long ld_, long r0_, int lim, int wave_,
                                       int lane_) {
    p = p_;
    ld = ld_;
    r0 = r0_;
    wave = wave_;
    lane = lane_;
#pragma unroll
    for (int j = 0; j < NL; j++) {
      int q4, l4, e;
      pos(j, q4, l4, e);
      long off;  // element offset from the tile origin
      if constexpr (KC) {
        const int R = q4 * (256 / BK) + l4 / CPR;
        off = (min(r0 + R, (long)lim - 1) - r0) * ld + koff(j);
      } else {
        const long c = DW ? min(r0 + 4 * (l4 % (T / 4)) + e, (long)lim - 1)
                          : min(r0 + 4 * (l4 % (T / 4)), (long)lim - 4);
        off = (long)koff(j) * ld + (c - r0);
      }
      voff[j] = (unsigned)(off * 4);
    }
  }
  // k of load j's lane relative to the tile's first k (NC: an x4 load fills
  // 256/T rows k of T floats)
  __device__ __forceinline__ int koff(int j) const {
    int q4, l4, e;
    pos(j, q4, l4, e);
    if constexpr (KC) {
      const int R = q4 * (256 / BK) + l4 / CPR;
      return 4 * ((l4 % CPR) ^ swz(R)) + e;
    } else {
      return q4 * (256 / T) + l4 / (T / 4);
    }
  }
  // LDS float offset of load j's first lane
  __device__ __forceinline__ int dst(int j) const { return (wave * NL + j) * LF; }
  // tile origin for the tile starting at absolute k = k0 (wave-uniform; made
  // scalar explicitly, as the DMA takes it in SGPRs)
  __device__ __forceinline__ const float *origin(int k0) const {
    const float *o = KC ? p + r0 * ld + k0 : p + (long)k0 * ld + r0;
    const uintptr_t u = (uintptr_t)o;
    const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)u);
    const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(u >> 32));
    return reinterpret_cast<const float *>(((uintptr_t)hi << 32) | lo);
  }
  __device__ __forceinline__ void issue(int j, const float *org, float *lds) const {
    if constexpr (DW) g2lds4s(org, voff[j], lds + dst(j));
    else g2lds16s(org, voff[j], lds + dst(j));
  }
  // the last tile: k >= kend reads zeros
  __device__ __forceinline__ void issue_tail(int j, const float *org, int k0, int kend,
                                             float *lds) const {
    const float *sp =
        (k0 + koff(j) < kend)
            ? reinterpret_cast<const float *>(reinterpret_cast<const char *>(org) + voff[j])
            : g_gemm_zero;
    if constexpr (DW) g2lds4(sp, lds + dst(j));
    else g2lds16(sp, lds + dst(j));
  }
  // fragments of k slice ks, sub-slice h (8 k): v[x][s] for
  // k = ks*BK/KSL + 8h + 4g + s and row base + 32x + l32 (KC) or m/n
  // base + 2*l32 + x (NC)
  __device__ __forceinline__ static void frag(const float *lds, int ks, int base, int h, int l32,
                                              int g, float (*v)[4]) {
    if constexpr (KC) {
#pragma unroll
      for (int x = 0; x < 2; x++) {
        const int R = base + 32 * x + l32;
        const int slot = (ks * (BK / (4 * KSL)) + 2 * h + g) ^ swz(R);
        const float4 t = *reinterpret_cast<const float4 *>(lds + R * BK + 4 * slot);
        v[x][0] = t.x; v[x][1] = t.y; v[x][2] = t.z; v[x][3] = t.w;
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; s++) {
        const float2 t = *reinterpret_cast<const float2 *>(
            lds + (ks * (BK / KSL) + 8 * h + 4 * g + s) * T + base + 2 * l32);
        v[0][s] = t.x; v[1][s] = t.y;
      }
    }
  }
};

// ROWS: rows of A per tile (64, or 256 for tall operands with few columns:
// four 64-row blocks share each tile of B); NWK: waves per K tile.  Wave w
// owns row block w / NWK and k slice w % NWK.  PRIV (one row block, BK = 8 NW):
// each wave loads only its own 8-k slice of every tile into a ring of its own,
// so no wave reads what another loaded and the K loop has no barrier (each
// wave waits only for its own loads); the same products summed in the same
// order as the shared ring.
template <bool A_KC, bool B_NC, int BK, int S, int NW, int ROWS = M_T, int NWK = NW,
          bool DW = false, bool PRIV = false>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW / 4, 2)))
gemm_mid_kernel(int M, int N, int K, const float *__restrict__ A, long lda,
                const float *__restrict__ B, long ldb, float *__restrict__ C, long ldc,
                long split_stride, int kchunk, bool cvec, int alim, int blim) {
  TT_PROBE(0, 0);
  static_assert(S >= 3, "the pipeline needs three stages");
  constexpr int NTH = 64 * NW;
  static_assert(ROWS % M_T == 0 && NW == (ROWS / M_T) * NWK, "waves = row blocks x k slices");
  static_assert(!PRIV || (ROWS == M_T && NWK == NW && BK == 8 * NW), "private slices: 8 k a wave");
  // a private ring holds one wave's operands: tiles of 8 k, loaded by that wave alone
  constexpr int OBK = PRIV ? 8 : BK, OW = PRIV ? 1 : NW, OKS = PRIV ? 1 : NWK;
  constexpr int OPA = ROWS * OBK, OPB = M_T * OBK;  // floats per operand per stage
  constexpr int STAGE = OPA + OPB;
  constexpr int PIPE = S * STAGE * (PRIV ? NW : 1), RED = NW * M_T * M_T;
  static_assert(!PRIV || S * STAGE == M_T * M_T, "a wave's sums fill its own ring");
  constexpr int KSUB = OBK / (8 * OKS);  // 8-k sub-slices per wave per tile
  static_assert(KSUB >= 1, "tile too shallow for the waves");
  __shared__ __attribute__((aligned(16))) float smem[PIPE > RED ? PIPE : RED];
  using OA = MidOperand<A_KC, OBK, OW, ROWS, OKS, DW>;
  using OB = MidOperand<!B_NC, OBK, OW, M_T, OKS, DW>;
  constexpr int NL = OA::NL + OB::NL;  // loads per wave per tile
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int g = lane >> 5;
  const int rb = wave / NWK, ks = wave % NWK;  // row block, k slice

  const int tiles_m = (M + ROWS - 1) / ROWS, tiles_n = (N + M_T - 1) / M_T;
  const int ntiles = tiles_m * tiles_n;
  int pid = blockIdx.x;
  if ((ntiles & 7) == 0) pid = (pid & 7) * (ntiles >> 3) + (pid >> 3);
  const int group = GROUP_M * tiles_n;
  const int first_m = (pid / group) * GROUP_M;
  const int gsz = min(tiles_m - first_m, GROUP_M);
  const int tm = first_m + (pid % group) % gsz;
  const int tn = (pid % group) / gsz;
  const long m0 = (long)tm * ROWS;
  const long n0 = (long)tn * M_T;
  const int kbeg = blockIdx.z * kchunk;
  const int kend = min(K, kbeg + kchunk);
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
  C += (long)blockIdx.z * split_stride;

  OA opa;
  OB opb;
  // A k-contiguous: rows m of A (M x K); else rows k of A (K x M), columns m.
  // B m/n-contiguous: rows k of B (K x N); else rows n of B (N x K).
  // (alim / blim: the rows of a KC operand, the readable columns of an NC one)
  opa.init(A, lda, m0, alim, PRIV ? 0 : wave, lane);
  opb.init(B, ldb, n0, blim, PRIV ? 0 : wave, lane);
  // the wave's ring and the k of its slice in a tile (private ring)
  float *const ring = PRIV ? smem + wave * (S * STAGE) : smem;
  const int kw = PRIV ? 8 * wave : 0;
  const int fks = PRIV ? 0 : ks;

#ifdef TT_PHASE_PROBE
  long long waited = 0;
#endif
  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  // loads J0 .. J0+NJ-1 of the NL of tile kt (A's first, then B's)
  auto issue_part = [&](int kt, int j0, int nj) {
    float *st = ring + (kt % S) * STAGE;
    const int k0 = kbeg + kt * BK + kw;
    const float *oa = opa.origin(k0), *ob = opb.origin(k0);
    if (k0 + OBK <= kend) {
#pragma unroll
      for (int j = 0; j < NL; j++) {
        if (j < j0 || j >= j0 + nj) continue;
        if (j < OA::NL) opa.issue(j, oa, st);
        else opb.issue(j - OA::NL, ob, st + OPA);
      }
    } else {
#pragma unroll
      for (int j = 0; j < NL; j++) {
        if (j < j0 || j >= j0 + nj) continue;
        if (j < OA::NL) opa.issue_tail(j, oa, k0, kend, st);
        else opb.issue_tail(j - OA::NL, ob, k0, kend, st + OPA);
      }
    }
  };
  auto frags = [&](int kt, float (*a)[2][4], float (*b)[2][4]) {
    const float *st = ring + (kt % S) * STAGE;
#pragma unroll
    for (int h = 0; h < KSUB; h++) {
      OA::frag(st, fks, rb * M_T, h, l32, g, a[h]);
      OB::frag(st + OPA, fks, 0, h, l32, g, b[h]);
    }
  };
  auto mfma4 = [&](float (*ca)[2][4], float (*cb)[2][4], int h, int s) {
#pragma unroll
    for (int x = 0; x < 2; x++)
#pragma unroll
      for (int y = 0; y < 2; y++)
        acc[x][y] = __builtin_amdgcn_mfma_f32_32x32x2f32(ca[h][x][s], cb[h][y][s], acc[x][y], 0, 0, 0);
  };
  // Tile kt: wait for tile kt+1 (tiles up to kt+S-2 are issued; S-3 may stay
  // in flight, all of them near the end) and meet the other waves; read tile
  // kt+1's fragments (they land under the MFMAs), then the MFMAs on the
  // current fragments in groups of 4, each group followed by an equal share
  // of the loads of tile kt+S-1 (into the stage tile kt-1 left, which every
  // wave finished reading before the previous barrier).  The barrier and the
  // reads are unconditional (on the last tile they read a stale stage nobody
  // uses): under a branch the compiler's wait-count merge makes the MFMAs
  // wait for the new reads instead of only for the previous tile's.
  auto step = [&](int kt, float (*ca)[2][4], float (*cb)[2][4], float (*na)[2][4],
                  float (*nb)[2][4]) {
#ifdef TT_PHASE_PROBE
    const long long tw0 = __builtin_amdgcn_s_memtime();
#endif
    if (kt + S - 2 < nk) wait_vm<NL *(S - 3)>();
    else wait_vm<0>();
#ifdef TT_PHASE_PROBE
    asm volatile("s_nop 0" ::: "memory");
    waited += __builtin_amdgcn_s_memtime() - tw0;
#endif
    if constexpr (!PRIV) __syncthreads();
    __builtin_amdgcn_sched_barrier(0);
    frags(kt + 1, na, nb);
    __builtin_amdgcn_sched_barrier(0);
    const bool more = kt + S - 1 < nk;
    constexpr int G = 4 * KSUB;  // groups of 4 MFMAs
    constexpr int PER = (NL + G - 1) / G;
#pragma unroll
    for (int q = 0; q < G; q++) {
      mfma4(ca, cb, q / 4, q % 4);
      __builtin_amdgcn_sched_barrier(0);
      if (more && q * PER < NL) issue_part(kt + S - 1, q * PER, PER);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  if (nk > 0) {
    for (int t = 0; t < S - 1 && t < nk; t++) issue_part(t, 0, NL);
    if (nk >= S - 1) wait_vm<NL *(S - 2)>();
    else wait_vm<0>();
    if constexpr (!PRIV) __syncthreads();
    TT_PROBE(0, 1);
    float a0[KSUB][2][4], b0[KSUB][2][4], a1[KSUB][2][4], b1[KSUB][2][4];
    frags(0, a0, b0);
#ifdef TT_PHASE_PROBE
    const long long tl0 = __builtin_amdgcn_s_memtime();
#endif
    for (int kt = 0; kt < nk; kt += 2) {
      step(kt, a0, b0, a1, b1);
      if (kt + 1 < nk) step(kt + 1, a1, b1, a0, b0);
    }
#ifdef TT_PHASE_PROBE
    if ((tid & 63) == 0 && blockIdx.x < 1024 && wave < 8) {
      // kernel slots 2 and 3: each wave's cycles waiting for its loads, and in its K loop
      tt_probe_ts[(2 * 1024 + blockIdx.x) * 16 + wave] = waited;
      tt_probe_ts[(3 * 1024 + blockIdx.x) * 16 + wave] = __builtin_amdgcn_s_memtime() - tl0;
    }
#endif
  }

  // wave sums -> LDS, 64x64 floats a wave (acc r of block (x, y): row
  // 8*(r/4) + 4g + r%4 of the block), then each thread adds the NWK k-slice
  // sums of its outputs in order.  A private ring takes its own wave's sums
  // as soon as that wave's K loop ends (its loads have all landed), so the
  // waves that finish first write theirs while the others still compute;
  // the shared ring is free once every wave is past its K loop.  With B
  // k-contiguous a lane's two stores are 32 columns apart and the two
  // half-waves write rows 4 (8) apart: the row's 32-column halves swap on
  // those rows so the 64 lanes hit 64 banks.
  TT_PROBE(0, 2);
  if (wave < 8) TT_PROBE_WAVE(0, 6 + wave);
  if constexpr (!PRIV) __syncthreads();
  auto swz = [](int m) { return B_NC ? 0 : 32 * ((A_KC ? m >> 2 : m >> 3) & 1); };
  float *red = smem + wave * (M_T * M_T);
#pragma unroll
  for (int x = 0; x < 2; x++)
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const int i = 8 * (r >> 2) + 4 * g + (r & 3);
      const int m = A_KC ? 32 * x + i : 2 * i + x;
      if constexpr (B_NC) {
        *reinterpret_cast<float2 *>(red + m * M_T + 2 * l32) = make_float2(acc[x][0][r], acc[x][1][r]);
      } else {
        red[m * M_T + (l32 ^ swz(m))] = acc[x][0][r];
        red[m * M_T + ((32 + l32) ^ swz(m))] = acc[x][1][r];
      }
    }
  TT_PROBE(0, 3);
  __syncthreads();
  TT_PROBE(0, 4);
#pragma unroll
  for (int f0 = 0; f0 < ROWS * M_T / 4; f0 += NTH) {
    const int f = f0 + tid;  // float4 index: row f / 16, columns 4 * (f % 16) ..
    const int mr = f >> 4, n = 4 * (f & 15);
    const int fb = mr / M_T, m = mr - fb * M_T;  // row block, row in it
    const long row = m0 + mr;
    if (row >= M) continue;
    const float *rb0 = smem + (fb * NWK) * (M_T * M_T) + m * M_T + (n ^ swz(m));
    float4 v = *reinterpret_cast<const float4 *>(rb0);
#pragma unroll
    for (int w = 1; w < NWK; w++) {
      const float4 t = *reinterpret_cast<const float4 *>(rb0 + w * (M_T * M_T));
      v.x += t.x; v.y += t.y; v.z += t.z; v.w += t.w;
    }
    float *crow = C + row * ldc;
    const long col = n0 + n;
    if (cvec && col + 3 < N) {
      *reinterpret_cast<float4 *>(crow + col) = v;
    } else {
      if (col < N) crow[col] = v.x;
      if (col + 1 < N) crow[col + 1] = v.y;
      if (col + 2 < N) crow[col + 2] = v.z;
      if (col + 3 < N) crow[col + 3] = v.w;
    }
  }
  TT_PROBE(0, 5);
}

inline hipStream_t stream() { return (hipStream_t)ttrt_stream(); }

// Workspace of a GEMM call (split-K partials, aligned operand copies).  By
// default it comes from the caching allocator; inside tt_k_gemm_noalloc it is
// carved out of the static device array `scratch` (bump allocation, nothing
// returned until the call ends).  Every path requests all of its workspace
// before its first launch, so a request the scratch cannot hold fails with
// nothing enqueued.
struct WsArena {
  char *base;
  size_t cap, used;
};
WsArena *g_arena = nullptr;

float *ws_alloc(size_t bytes) {
  if (!g_arena) return (float *)ttrt_alloc(bytes);
  const size_t b = (bytes + 255) / 256 * 256;
  if (g_arena->used + b > g_arena->cap) return nullptr;
  float *p = (float *)(g_arena->base + g_arena->used);
  g_arena->used += b;
  return p;
}

void ws_free(void *p) {
  if (!g_arena) ttrt_free(p);
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// Tile configurations (BM x BN, wave grid WM x 4/WM).
// (the K64 tiles take 64 k per LDS stage: half the K iterations and twice
// the loads in flight per iteration, for latency-bound skinny GEMMs)
enum Tile { T128x128 = 0, T128x64, T64x64, T32x256, T64x256, T256x256, T256x128, T64x128,
            T32x128, T64x64K64, T32x128K64, NTILE };
constexpr int TILE_BM[NTILE] = {128, 128, 64, 32, 64, 256, 256, 64, 32, 64, 32};
constexpr int TILE_BN[NTILE] = {128, 64, 64, 256, 256, 256, 128, 128, 128, 64, 128};
constexpr int TILE_BK[NTILE] = {32, 32, 32, 32, 32, 32, 32, 32, 32, 64, 64};

// tuning override (tth_gemm_config): -1 = automatic
int g_force_tile = -1, g_force_splits = -1;
int g_direct = 1;  // direct-to-LDS 256x256 kernel enabled (tth_gemm_direct)
int g_mid = 1;     // 64x64 direct-load kernel for plain GEMMs (tth_gemm_mid; 2: shared k tiles)
int g_mid_force = 0;  // every plain GEMM of small size takes it too (tth_gemm_mid_force)
int g_small = 1;   // 32x32 register kernel for small plain GEMMs (tth_gemm_small)
int g_t16 = 1;     // 16x16 forward kernel for GEMMs below a full 32x32 grid (tth_gemm_t16)

struct Plan {
  int tile, splits, kchunk;
};

inline long ntiles(int t, int M, int N) {
  return (long)((M + TILE_BM[t] - 1) / TILE_BM[t]) * ((N + TILE_BN[t] - 1) / TILE_BN[t]);
}

// Pick a tile that wastes little of the output and a split count so that the
// launch covers the 256 CUs.  tth_gemm_config() forces a choice (tuning).
// fraction of the padded tile grid that holds real output
inline double fill(int t, int M, int N) {
  const double pm = (double)((M + TILE_BM[t] - 1) / TILE_BM[t]) * TILE_BM[t];
  const double pn = (double)((N + TILE_BN[t] - 1) / TILE_BN[t]) * TILE_BN[t];
  return (double)M * N / (pm * pn);
}

Plan plan(int M, int N, int K) {
  const int CUS = 256;
  Plan p{T64x64, 1, K};
  // Largest tile that still gives every CU a workgroup and wastes little of
  // itself on padding; otherwise the small tile that fits the output best
  // (F x N*Ho*Wo conv shapes have M = 32 or 64).
  const int big[] = {T256x256, T256x128, T128x128};
  int chosen = -1;
  for (int t : big)
    if (ntiles(t, M, N) >= CUS && fill(t, M, N) >= 0.87) { chosen = t; break; }
  if (chosen < 0) {
    // small tiles: the best output fill first; among tiles within 2 % of it,
    // the one with the most workgroups.  These GEMMs are bound by memory
    // latency, which several workgroups per CU hide better than one larger
    // one (measured: 2 x 64x64 per CU beat 1 x 64x128 on the conv GEMMs).
    const int small[] = {T128x64, T64x64, T32x256, T64x256, T64x128, T32x128};
    auto allowed = [&](int t) {
      if (t == T128x64 && (N > 64 || ntiles(t, M, N) < CUS)) return false;
      if ((t == T32x256 || t == T32x128) && M > 32) return false;
      if ((t == T64x256 || t == T64x128) && M > 64) return false;
      return true;
    };
    double best = -1.0;
    for (int t : small)
      if (allowed(t)) best = fmax(best, fill(t, M, N));
    long most = -1;
    for (int t : small) {
      if (!allowed(t) || fill(t, M, N) < best - 0.02) continue;
      const long nt = ntiles(t, M, N);
      if (nt > most) { most = nt; chosen = t; }
    }
  }
  p.tile = chosen;
  if (g_force_tile >= 0 && g_force_tile < NTILE) p.tile = g_force_tile;
  const long tiles = ntiles(p.tile, M, N);
  // Split K (deterministically reduced afterwards) until the grid fills the
  // CUs: each K tile of a small GEMM is latency-bound, so parallelism over K
  // beats a long serial K loop.  Long reductions (conv dW, K = N*Ho*Wo) may
  // go to ~4 workgroups per CU while each split keeps >= 256 k.
  int s = 1;
  while (s < 256 && tiles * s * 2 <= CUS && (long)K / (s * 2) >= 32) s *= 2;
  if (tiles < CUS)
    while (s < 256 && tiles * s * 2 <= 4L * CUS && (long)K / (s * 2) >= 256) s *= 2;
  if (g_force_splits >= 1) s = g_force_splits;
  int kc = (K + s - 1) / s;
  const int bk = TILE_BK[p.tile];
  kc = (kc + bk - 1) / bk * bk;
  p.kchunk = kc;
  p.splits = (K + kc - 1) / kc;
  return p;
}

template <int BM, int BN, int BK, int WM, bool A_KC, bool A_PERM, bool B_NC, bool B_PERM,
          bool VEC, int EPI, bool B_I2C>
void launch_tile(int M, int N, int K, const Opnd &A, const Opnd &B, float *C, long ldc,
                 long split_stride, int splits, int kchunk, const float *bias, int HW,
                 const I2C &cv) {
  const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
  dim3 grid(tiles, 1, splits);
  // vector epilogue stores need 16-byte aligned rows (NCHW: HW a multiple of 4)
  const bool cvec = aligned16(C) && (EPI == EPI_STORE ? (ldc % 4 == 0) : (HW % 4 == 0));
  if constexpr (BM * BN >= 256 * 256) {
    static_assert(!B_I2C, "implicit im2col is not built for the 256x256 tile");
    hipLaunchKernelGGL((gemm_mfma_big_kernel<BM, BN, BK, WM, A_KC, A_PERM, B_NC, B_PERM, VEC, EPI>),
                       grid, dim3(NT), 0, stream(), M, N, K, A, B, C, ldc, split_stride, kchunk,
                       bias, HW, cvec);
  } else {
    hipLaunchKernelGGL(
        (gemm_mfma_kernel<BM, BN, BK, WM, A_KC, A_PERM, B_NC, B_PERM, VEC, EPI, B_I2C>), grid,
        dim3(NT), 0, stream(), M, N, K, A, B, C, ldc, split_stride, kchunk, bias, HW, cvec, cv);
  }
}

// The epilogue that tt_k_gemm_relu_pad asks of the split-K reduction writing
// its C; `applied` tells it whether the GEMM took a split-K path (else it
// launches the epilogue on its own).
enum { HOOK_RELU_PAD = 1, HOOK_CE = 2 };
struct RedHook {
  int kind;
  const float *C;
  ReluPadEx rp;
  const TTCeHook *ce;  // HOOK_CE: the softmax-CE that follows (rp.bias is the bias)
  int applied;         // 1: the epilogue ran in the reduction; 2: the CE too
};
RedHook *g_red_hook = nullptr;

int reduce_hooked(const float *ws, int M, int N, int S) {
  RedHook &h = *g_red_hook;
  float *C = const_cast<float *>(h.C);
  const long total = (long)M * N;
  int zl = 1;
  while (zl < 32 && zl < S && (total * zl * 2) <= 2048L * 256) zl *= 2;
  if (zl < 4 && S >= 4) zl = 4;
  if (h.kind == HOOK_CE) {
    const int rc = ttk_reduce_ce(ws, C, M, N, S, zl, h.ce);
    if (rc < 0) return rc;
    if (rc == 0) {
      h.applied = 2;
      return 0;
    }
  }
#define TT_HK(ZL_)                                                                            \
  case ZL_:                                                                                   \
    hipLaunchKernelGGL((splitk_reduce_relu_pad_kernel<ZL_>),                                  \
                       dim3((unsigned)((total + 256 / ZL_ - 1) / (256 / ZL_))), dim3(256), 0,  \
                       stream(), ws, C, M, N, S, h.rp);                                       \
    break;
  switch (zl) {
    TT_HK(1) TT_HK(2) TT_HK(4) TT_HK(8) TT_HK(16)
    default: TT_HK(32)
  }
#undef TT_HK
  if (hipGetLastError() != hipSuccess) return -3;
  h.applied = 1;
  return 0;
}

// Sum the S partial products of a split-K launch into C (+ epilogue).
template <int EPI>
int reduce_splits(const float *ws, float *C, int M, int N, int S, long ldc, const float *bias,
                  int HW) {
  const long total = (long)M * N;
  if constexpr (EPI == EPI_STORE) {
    if (g_red_hook && g_red_hook->C == C && ldc == N) return reduce_hooked(ws, M, N, S);
  }
  // widen the split-lanes until ~2048 workgroups share the reduction (at
  // most 32 lanes, at most S): each lane's loads are independent, so more
  // lanes means more loads in flight for the few outputs of a conv dW
  int zl = 1;
  while (zl < 32 && zl < S && (total * zl * 2) <= 2048L * 256) zl *= 2;
  if (zl < 4 && S >= 4) zl = 4;
#define TT_RED(ZL_)                                                                            \
  hipLaunchKernelGGL((splitk_reduce_kernel<EPI, ZL_>), dim3((unsigned)((total + 256 / ZL_ - 1) / \
                                                                      (256 / ZL_))),            \
                     dim3(256), 0, stream(), ws, C, M, N, S, ldc, bias, HW)
  switch (zl) {
    case 1: TT_RED(1); break;
    case 2: TT_RED(2); break;
    case 4: TT_RED(4); break;
    case 8: TT_RED(8); break;
    case 16: TT_RED(16); break;
    default: TT_RED(32); break;
  }
#undef TT_RED
  return hipGetLastError() != hipSuccess ? -3 : 0;
}

// dst (rows x ldp, ldp a multiple of 4) = src (rows x cols, leading dimension
// ld) with columns cols .. ldp-1 zero: a 16-byte aligned copy of an operand
// whose rows are not.
// Small plain GEMM: one 32x32 tile of C per workgroup, its K range split over
// SW waves, each multiplying its k slice with operands loaded straight into
// registers (no LDS staging, no split-K workspace); the wave sums are added
// through LDS in wave order (deterministic).  Lane l of v_mfma_f32_32x32x2
// feeds A[l%32][k] and B[k][l%32]; lane half h takes k = 4h..4h+3 of each
// 8-k group, one per MFMA, so the four MFMAs of a group cover its 8 k.
// Loads run a chunk of SG groups ahead of the MFMAs (two register sets).
// VA / VB: the operand is k-contiguous with 16-byte aligned rows, so a lane
// reads its 4 k as one 16-byte load.  Rows / columns past the matrix load
// the last valid one (their outputs are not stored); k past the slice loads
// zeros.
// waves per small-GEMM workgroup (measured: 4 beats 8 and 2 on the MLP step's
// 32x32 tiles, 0.0554 -> 0.0537 ms; two workgroups then share a CU)
constexpr int SW = 4;
constexpr int SG = 4;  // 8-k groups per pipelined chunk
// Where a small-GEMM tile's outputs go: C (ldc), and for the dA of a
// matmul whose input is a padones (of a relu output R), also the padones
// input's gradient d1 = C[:, :-1] and d2 = d1 masked by R > 0 (d2 = d1
// without R); d1 / d2 are (M x (N-1)) row-major.
// w - lr * g with the product rounded on its own (this file is compiled with
// contraction; the empty asm hides the product from the multiply-add
// combiner), as the SGD kernels compute it
__device__ __forceinline__ float sgd_sub(float w, float lr, float g) {
  float p = lr * g;
  asm volatile("" : "+v"(p));
  return w - p;
}

struct SmallOut {
  float *C;
  long ldc;
  float *d1, *d2;
  const float *R;
  // forward epilogue (C = A * B + bias row): bias[n] added to every row;
  // relu = relu(C) and pad = [relu, 1] (M x (N+1)) when given
  const float *bias = nullptr;
  float *relu = nullptr, *pad = nullptr;
  // row ones_m of op(A) is all ones instead of A's (A, m-contiguous, then
  // has ones_m columns: the padones column [X, 1] of a matrix X)
  int ones_m = -1;
  // C is a gradient: the weights wsgd (laid out as C) get the SGD step
  // w -= lr * C from the stored value (multiply rounded on its own, as the
  // SGD kernel computes it)
  float *wsgd = nullptr;
  float lr = 0.0f;
};

// PK: the probe slot set of the calling kernel (phase-probe builds only)
template <bool A_KC, bool B_NC, bool VA, bool VB, int PK = 1>
__device__ __forceinline__ void small_tile(int M, int N, int K, const float *__restrict__ A,
                                           long lda, const float *__restrict__ B, long ldb,
                                           const SmallOut &out, int kc, int bx, int by,
                                           float *red) {
  TT_PROBE(PK, 0);
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  const int m0 = by * 32, n0 = bx * 32;
  const bool one = m0 + l32 == out.ones_m;
  const int mr = min(m0 + l32, out.ones_m >= 0 ? out.ones_m - 1 : M - 1);
  const int nr = min(n0 + l32, N - 1);
  // this lane's A row / B column: element k at base + k * step
  const float *ap = A_KC ? A + (long)mr * lda : A + mr;
  const long as = A_KC ? 1 : lda;
  const float *bp = B_NC ? B + nr : B + (long)nr * ldb;
  const long bs = B_NC ? ldb : 1;
  const int k0 = w * kc, k1 = min(K, k0 + kc);
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; r++) acc[r] = 0.0f;
  auto load = [&](int kb, float (&a)[SG][4], float (&b)[SG][4]) {
#pragma unroll
    for (int g = 0; g < SG; g++) {
      const int kq = kb + 8 * g + 4 * h;
      if (VA && kq + 3 < k1) {
        const float4 v = *(const float4 *)(ap + kq);
        a[g][0] = v.x; a[g][1] = v.y; a[g][2] = v.z; a[g][3] = v.w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++) a[g][i] = kq + i < k1 ? ap[(long)(kq + i) * as] : 0.0f;
      }
      if (!A_KC && one) {
#pragma unroll
        for (int i = 0; i < 4; i++) a[g][i] = kq + i < k1 ? 1.0f : 0.0f;
      }
      if (VB && kq + 3 < k1) {
        const float4 v = *(const float4 *)(bp + kq);
        b[g][0] = v.x; b[g][1] = v.y; b[g][2] = v.z; b[g][3] = v.w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++) b[g][i] = kq + i < k1 ? bp[(long)(kq + i) * bs] : 0.0f;
      }
    }
  };
  auto mfmas = [&](const float (&a)[SG][4], const float (&b)[SG][4]) {
#pragma unroll
    for (int g = 0; g < SG; g++)
#pragma unroll
      for (int i = 0; i < 4; i++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[g][i], b[g][i], acc, 0, 0, 0);
  };
  // the epilogue: thread e (of 64 SW) takes outputs e + 64 SW j of the tile
  // (row / 32, column % 32: stores of consecutive columns); their relu
  // outputs, weights to step and bias are loaded before the K loop, clamped
  // to the matrix, so that they arrive with the first operands (loaded after
  // the wave sums, they cost one more memory round trip before the stores)
  constexpr int EPT = 32 * 32 / (64 * SW);  // outputs a thread
  const int ecol = threadIdx.x & 31, erow0 = threadIdx.x >> 5;
  const int ne = min(n0 + ecol, N - 1);
  float rv[EPT], wv[EPT];
  if (out.R) {
    const int nc = ne < N - 1 ? ne : (N > 1 ? N - 2 : 0);
#pragma unroll
    for (int j = 0; j < EPT; j++)
      rv[j] = out.R[(long)min(m0 + erow0 + 8 * j, M - 1) * (N - 1) + nc];
  }
  if (out.wsgd) {
#pragma unroll
    for (int j = 0; j < EPT; j++)
      wv[j] = out.wsgd[(long)min(m0 + erow0 + 8 * j, M - 1) * out.ldc + ne];
  }
  const float bn = out.bias ? out.bias[ne] : 0.0f;
  constexpr int CK = 8 * SG;  // k per chunk
  float a0[SG][4], b0[SG][4], a1[SG][4], b1[SG][4];
  if (k0 < k1) load(k0, a0, b0);
  for (int kb = k0; kb < k1; kb += 2 * CK) {
    const bool more = kb + CK < k1;
    if (more) load(kb + CK, a1, b1);
    mfmas(a0, b0);
    if (!more) break;
    if (kb + 2 * CK < k1) load(kb + 2 * CK, a0, b0);
    mfmas(a1, b1);
  }
  // every wave's sums to LDS (acc r of lane (l32, h): row 8 (r / 4) + 4 h +
  // r % 4, column l32); each thread then adds the SW wave sums of its
  // outputs in wave order
  TT_PROBE(PK, 1);
#pragma unroll
  for (int r = 0; r < 16; r++) red[(w * 16 + r) * 64 + lane] = acc[r];
  __syncthreads();
  TT_PROBE(PK, 2);
  const bool pad = out.d1 || out.d2;
  const int n = n0 + ecol;
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const int row = erow0 + 8 * j;
    const int src = (4 * (row >> 3) + (row & 3)) * 64 + 32 * ((row >> 2) & 1) + ecol;
    float v = red[src];
#pragma unroll
    for (int o = 1; o < SW; o++) v += red[o * 16 * 64 + src];
    const int m = m0 + row;
    if (m >= M || n >= N) continue;
    if (out.bias) {  // forward: C = acc + bias[n], and its relu / padded relu
      v = v + bn;
      out.C[(long)m * out.ldc + n] = v;
      const float o = v > 0.0f ? v : 0.0f;
      if (out.relu) out.relu[(long)m * N + n] = o;
      if (out.pad) {
        float *pr = out.pad + (long)m * (N + 1);
        pr[n] = o;
        if (n == N - 1) pr[N] = 1.0f;
      }
      continue;
    }
    out.C[(long)m * out.ldc + n] = v;
    if (out.wsgd) out.wsgd[(long)m * out.ldc + n] = sgd_sub(wv[j], out.lr, v);
    if (pad && n < N - 1) {
      const long o = (long)m * (N - 1) + n;
      if (out.d1) out.d1[o] = v;
      if (out.d2) out.d2[o] = out.R ? (rv[j] > 0.0f ? v : 0.0f) : v;
    }
  }
  TT_PROBE(PK, 3);
}

template <bool A_KC, bool B_NC, bool VA, bool VB>
__global__ void __launch_bounds__(64 * SW)
gemm_small_kernel(int M, int N, int K, const float *__restrict__ A, long lda,
                  const float *__restrict__ B, long ldb, float *__restrict__ C, long ldc, int kc,
                  int ones_m) {
  __shared__ float red[SW * 16 * 64];
  SmallOut out{C, ldc, nullptr, nullptr, nullptr};
  out.ones_m = ones_m;
  small_tile<A_KC, B_NC, VA, VB>(M, N, K, A, lda, B, ldb, out, kc, blockIdx.x, blockIdx.y, red);
}

// The weight gradients [X, 1]^T G of up to two tt_k_gemm_tn_padones jobs and
// an SGD step in one launch: workgroups [0, J.j[0].gblocks) are job 0's
// tiles (gx across), the next J.j[1].gblocks job 1's, each also stepping its
// tile of the job's wsgd; the rest step the plain tensors of P, a thread an
// element (sgd_sub, as sgd_multi_kernel).
struct SgdPlain {
  float *w[TT_SGD_MAX];
  const float *g[TT_SGD_MAX];
  long n[TT_SGD_MAX];
  long start[TT_SGD_MAX + 1];
  int np;
  float lr;
};
struct TnJob {
  int M, N, K, kc, ones_m, gx, gblocks;
  const float *A, *B;
  float *C, *wsgd;
};
struct TnJobs {
  TnJob j[2];
  int nj;
};
__global__ void __launch_bounds__(64 * SW)
gemm_tn_padones_sgd_kernel(TnJobs J, SgdPlain P) {
  __shared__ float red[SW * 16 * 64];
  int b = blockIdx.x;
  for (int q = 0; q < J.nj; q++) {
    const TnJob &t = J.j[q];
    if (b < t.gblocks) {
      SmallOut out{t.C, t.N, nullptr, nullptr, nullptr};
      out.ones_m = t.ones_m;
      out.wsgd = t.wsgd;
      out.lr = P.lr;
      small_tile<false, true, false, false>(t.M, t.N, t.K, t.A, t.ones_m, t.B, t.N, out, t.kc,
                                            b % t.gx, b / t.gx, red);
      return;
    }
    b -= t.gblocks;
  }
  int k = 0;
  while (k + 1 < P.np && b >= P.start[k + 1]) k++;
  const long i = (b - P.start[k]) * (64 * SW) + threadIdx.x;
  if (i < P.n[k]) P.w[k][i] = sgd_sub(P.w[k][i], P.lr, P.g[k][i]);
}

// The same tiles with a forward epilogue (SmallOut::bias / relu / pad).
template <bool VA, bool VB>
__global__ void __launch_bounds__(64 * SW)
gemm_small_epi_kernel(int M, int N, int K, const float *__restrict__ A, long lda,
                      const float *__restrict__ B, long ldb, SmallOut out, int kc) {
  __shared__ float red[SW * 16 * 64];
  small_tile<true, true, VA, VB>(M, N, K, A, lda, B, ldb, out, kc, blockIdx.x, blockIdx.y, red);
}

// C = A * B + bias (and relu / padded relu) on 16x16 tiles for GEMMs too
// small to fill the chip with 32x32 tiles (the MLP's hidden layers: 256 x
// 512 x 784, 256 x 256 x 512).  A row-major M x K (rows 16-byte aligned,
// K % 4 == 0), B row-major K x N.  Eight waves split K into equal slices of
// NCH 16-k chunks; a wave issues all of its slice's loads at once (NCH x 8
// registers a lane) so it waits for one round trip, not one per chunk, then
// runs 4 * NCH 16x16x4 MFMAs; the wave sums are added in LDS in wave order.
// (Four waves a workgroup measured slower, sixteen no faster.)  TN column
// blocks of 16 per workgroup share the A fragments.
// Lane l (r = l % 16, q = l / 16) loads A[m0 + r][kb + 4q .. 4q+3] and
// B[kb + 4q + i][n0 + r]; MFMA i of a chunk then sums k = kb + 4q + i over
// q.  Loads past the matrix are clamped to it and their values zeroed.
typedef float f32x4t __attribute__((ext_vector_type(4)));
constexpr int T16W = 8;  // waves per workgroup
template <int NCH, int TN>
__global__ void __launch_bounds__(64 * T16W)
gemm_t16_epi_kernel(int M, int N, int K, const float *__restrict__ A,
                    const float *__restrict__ B, SmallOut out, int kc) {
  __shared__ float red[T16W * 4 * TN * 64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int m0 = blockIdx.y * 16, n0 = blockIdx.x * 16 * TN;
  const int mr = min(m0 + r, M - 1);
  const int k0 = w * kc, k1 = min(K, k0 + kc);
  const float *__restrict__ ap = A + (long)mr * K;
  // the epilogue: thread e < 256 TN takes output row e / (16 TN), column e %
  // (16 TN) of the tile; its bias is loaded with the operands (a load issued
  // after the wave sums is one more memory round trip before the stores)
  const int erow = threadIdx.x / (16 * TN), ecol = threadIdx.x % (16 * TN);
  const float bn = out.bias[min(n0 + ecol, N - 1)];
  float4 av[NCH];
  float bv[NCH][TN][4];
#pragma unroll
  for (int c = 0; c < NCH; c++) {
    const int kq = k0 + 16 * c + 4 * q;
    av[c] = *reinterpret_cast<const float4 *>(ap + min(kq, K - 4));
#pragma unroll
    for (int t = 0; t < TN; t++) {
      const float *__restrict__ bp = B + min(n0 + 16 * t + r, N - 1);
#pragma unroll
      for (int i = 0; i < 4; i++) bv[c][t][i] = bp[(long)min(kq + i, K - 1) * N];
    }
  }
  f32x4t acc[TN];
#pragma unroll
  for (int t = 0; t < TN; t++) acc[t] = f32x4t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < NCH; c++) {
    const int kq = k0 + 16 * c + 4 * q;
    const float a4[4] = {av[c].x, av[c].y, av[c].z, av[c].w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const bool in = kq + i < k1;
#pragma unroll
      for (int t = 0; t < TN; t++)
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(in ? a4[i] : 0.0f, in ? bv[c][t][i] : 0.0f,
                                                      acc[t], 0, 0, 0);
    }
  }
  // every wave's sums to LDS; then each thread adds the eight wave sums of
  // its output in wave order and stores it (the stores spread over the
  // workgroup instead of one wave)
#pragma unroll
  for (int t = 0; t < TN; t++)
#pragma unroll
    for (int i = 0; i < 4; i++) red[((w * TN + t) * 4 + i) * 64 + lane] = acc[t][i];
  __syncthreads();
  if (threadIdx.x >= 256 * TN) return;
  const int t = ecol >> 4, i = erow & 3;
  const int src = (t * 4 + i) * 64 + 16 * (erow >> 2) + (ecol & 15);
  float v = red[src];
#pragma unroll
  for (int o = 1; o < T16W; o++) v += red[o * TN * 4 * 64 + src];
  const int m = m0 + erow, n = n0 + ecol;
  if (m >= M || n >= N) return;
  v += bn;
  out.C[(long)m * out.ldc + n] = v;
  const float o = v > 0.0f ? v : 0.0f;
  if (out.relu) out.relu[(long)m * N + n] = o;
  if (out.pad) {
    float *pr = out.pad + (long)m * (N + 1);
    pr[n] = o;
    if (n == N - 1) pr[N] = 1.0f;
  }
}

// Partial products of a skinny GEMM (N <= 16 columns, a long K: the CNN
// classifier's 128 x 4096 -> 10) for split-K: workgroup (tile_n, tile_m, z)
// multiplies its 16x16 tile over k slice z on the same eight-wave scheme and
// stores the tile's valid part to ws[z] (M x N), for reduce_splits.  A
// row-major (lda, rows 16-byte aligned, lda % 4 == 0, K % 4 == 0), B
// row-major (ldb).
template <int NCH>
__global__ void __launch_bounds__(64 * T16W)
gemm_t16_split_kernel(int M, int N, int K, const float *__restrict__ A, long lda,
                      const float *__restrict__ B, long ldb, float *__restrict__ ws,
                      int kslice) {
  __shared__ float red[(T16W - 1) * 4 * 64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int m0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
  const int mr = min(m0 + r, M - 1), nr = min(n0 + r, N - 1);
  const int ks = blockIdx.z * kslice, ke = min(K, ks + kslice);
  const int k0 = ks + w * 16 * NCH, k1 = min(ke, k0 + 16 * NCH);
  const float *__restrict__ ap = A + (long)mr * lda;
  const float *__restrict__ bp = B + nr;
  float4 av[NCH];
  float bv[NCH][4];
#pragma unroll
  for (int c = 0; c < NCH; c++) {
    const int kq = k0 + 16 * c + 4 * q;
    av[c] = *reinterpret_cast<const float4 *>(ap + min(kq, K - 4));
#pragma unroll
    for (int i = 0; i < 4; i++) bv[c][i] = bp[(long)min(kq + i, K - 1) * ldb];
  }
  f32x4t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int c = 0; c < NCH; c++) {
    const int kq = k0 + 16 * c + 4 * q;
    const float a4[4] = {av[c].x, av[c].y, av[c].z, av[c].w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const bool in = kq + i < k1;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(in ? a4[i] : 0.0f, in ? bv[c][i] : 0.0f, acc, 0,
                                                 0, 0);
    }
  }
  if (w > 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) red[((w - 1) * 4 + i) * 64 + lane] = acc[i];
  }
  __syncthreads();
  if (w > 0) return;
#pragma unroll
  for (int o = 0; o < T16W - 1; o++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] += red[(o * 4 + i) * 64 + lane];
  const int n = n0 + r;
  if (n >= N) return;
  float *wz = ws + (long)blockIdx.z * M * N;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int m = m0 + 4 * q + i;
    if (m < M) wz[(long)m * N + n] = acc[i];
  }
}

// The 16x16-tile forward when it applies: 0 launched, 1 not covered, < 0
// launch error.  Taken for at least 256 tiles (one a CU) and at most 1024,
// K <= 1024.
int run_t16(int M, int N, int K, const float *A, const float *B, const SmallOut &out) {
  const long tiles = (long)((M + 15) / 16) * ((N + 15) / 16);
  if (!g_t16 || K < 16 || K % 4 || !aligned16(A) || tiles < 256 || tiles > 1024 ||
      K > 1024 || (M + 15) / 16 > 65535)
    return 1;
  static_assert(T16W == 8, "K <= 1024 is at most 8 chunks of 16 k a wave");
  const int nch = (K + 16 * T16W - 1) / (16 * T16W);  // 16-k chunks a wave
  const int kc = 16 * nch;
  // two column blocks a workgroup (16x32 tiles, each A fragment feeding two
  // MFMAs) while that still leaves 256 workgroups (the MLP's 256x512x784:
  // step 0.0463 -> 0.0453 ms); at 256 tiles the halved grid is slower
  const int tn = tiles >= 512 ? 2 : 1;
  const dim3 grid((unsigned)((N + 16 * tn - 1) / (16 * tn)), (unsigned)((M + 15) / 16));
#define TT_T16(NCH_)                                                                          \
  if (tn == 2)                                                                                \
    hipLaunchKernelGGL((gemm_t16_epi_kernel<NCH_, 2>), grid, dim3(64 * T16W), 0, stream(), M, N, \
                       K, A, B, out, kc);                                                     \
  else                                                                                        \
    hipLaunchKernelGGL((gemm_t16_epi_kernel<NCH_, 1>), grid, dim3(64 * T16W), 0, stream(), M, N, \
                       K, A, B, out, kc)
  switch (nch) {
    case 1: TT_T16(1); break;
    case 2: TT_T16(2); break;
    case 3: TT_T16(3); break;
    case 4: TT_T16(4); break;
    case 5: TT_T16(5); break;
    case 6: TT_T16(6); break;
    case 7: TT_T16(7); break;
    default: TT_T16(8); break;  // K <= 1024: at most 8 chunks a wave
  }
#undef TT_T16
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// Both gradients of a matmul C = A * B in one launch of small-GEMM tiles:
// dA = G * B^T (the tiles of tt_k_gemm(M, K, N, G, N, 0, B, N, 1, ...)) in
// workgroups [0, nba), dB = A^T * G (tt_k_gemm(K, N, M, A, K, 1, G, N, 0, ...))
// after them; each tile is computed exactly as its own launch computes it.
struct SmallJob {
  int M, N, K;
  const float *A;
  long lda;
  const float *B;
  long ldb;
  SmallOut out;
  int kc, nbx;
};

template <bool VDA>
__global__ void __launch_bounds__(64 * SW)
gemm_small_pair_kernel(SmallJob da, SmallJob db, int nba) {
  __shared__ float red[SW * 16 * 64];
  const int i = blockIdx.x;
  if (i < nba)
    small_tile<true, false, VDA, VDA, 2>(da.M, da.N, da.K, da.A, da.lda, da.B, da.ldb, da.out,
                                         da.kc, i % da.nbx, i / da.nbx, red);
  else
    small_tile<false, true, false, false, 2>(db.M, db.N, db.K, db.A, db.lda, db.B, db.ldb, db.out,
                                             db.kc, (i - nba) % db.nbx, (i - nba) / db.nbx, red);
}

// small_ok: below the 64x64 kernel's range (2MNK < 2^29) with at least 128
// tiles to spread -- 256 unless K <= 512 (a long K on half the CUs measured
// slower than the split-K kernel: 256x512x784 16.2 vs 10.6 us) -- and
// every k-contiguous operand 16-byte aligned (rows read
// by 32 lanes one float at a time bound the address path: measured slower
// than the split-K register kernel).
template <bool A_KC, bool B_NC>
bool small_ok(int M, int N, int K, const Opnd &A, const Opnd &B) {
  const long tiles = (long)((M + 31) / 32) * ((N + 31) / 32);
  const bool va = !A_KC || (aligned16(A.p) && A.ld % 4 == 0);
  const bool vb = B_NC || (aligned16(B.p) && B.ld % 4 == 0);
  return g_small && K > 0 && 2.0 * M * N * K < (double)(1L << 29) && tiles >= 128 &&
         (tiles >= 256 || K <= 512) && (M + 31) / 32 <= 65535 && va && vb;
}

template <bool A_KC, bool B_NC>
int run_small(int M, int N, int K, const Opnd &A, const Opnd &B, float *C, long ldc) {
  const int kc = ((K + SW - 1) / SW + 7) / 8 * 8;
  const dim3 grid((unsigned)((N + 31) / 32), (unsigned)((M + 31) / 32));
  // 16-byte loads of a k-contiguous operand whose rows are 16-byte aligned
  const bool va = A_KC && aligned16(A.p) && A.ld % 4 == 0;
  const bool vb = !B_NC && aligned16(B.p) && B.ld % 4 == 0;
#define TT_SMALL(VA_, VB_)                                                                      \
  hipLaunchKernelGGL((gemm_small_kernel<A_KC, B_NC, VA_, VB_>), grid, dim3(64 * SW), 0, stream(), \
                     M, N, K, A.p, A.ld, B.p, B.ld, C, ldc, kc, -1)
  if (va && vb) TT_SMALL(A_KC, !B_NC);
  else if (va) TT_SMALL(A_KC, false);
  else if (vb) TT_SMALL(false, !B_NC);
  else TT_SMALL(false, false);
#undef TT_SMALL
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// Plain GEMM on 64x64 tiles (gemm_mid_kernel), split over K until the grid
// covers the CUs.  Operands 16-byte aligned, leading dimensions multiples of
// 4 (and at most 2^22), K % 4 == 0 for k-contiguous operands, M / N % 4 == 0
// for m/n-contiguous ones (mid_ok).
template <bool A_KC, bool B_NC>
bool mid_ok(int M, int N, int K, const Opnd &A, const Opnd &B, bool vec) {
  const bool kc_ops = A_KC || !B_NC;
  // below ~0.5 GFLOP the per-launch cost of the deep pipeline and the wave
  // sums outweighs its faster K loop (measured: 512^3 and the MLP GEMMs are
  // faster on the register-staged 64x64 kernel)
  return g_mid && vec && (g_mid_force || 2.0 * M * N * K >= (double)(1L << 29)) &&
         A.ld <= (1L << 22) && B.ld <= (1L << 22) && (!kc_ops || K % 4 == 0) &&
         (A_KC || M % 4 == 0) && (!B_NC || N % 4 == 0);
}

// Split-K count of the 64x64 kernel: split until the grid covers the CUs;
// a split's k range is a whole number of 64-k tiles (the 32-k kernel takes
// the same ranges).  *kc_out receives the k range of one split.
int mid_splits(int M, int N, int K, int *kc_out) {
  const int CUS = 256;
  const long tiles = (long)((M + M_T - 1) / M_T) * ((N + M_T - 1) / M_T);
  int s = 1;
  while (s < 64 && tiles * s * 2 <= CUS && K / (s * 2) >= 128) s *= 2;
  if (g_force_splits >= 1) s = g_force_splits;
  int kc = ((K + s - 1) / s + 63) / 64 * 64;
  if (kc < 64) kc = 64;
  *kc_out = kc;
  return K > 0 ? (K + kc - 1) / kc : 1;
}

// DW: 4-byte loads (operands of any alignment and row length, read in place).
template <bool A_KC, bool B_NC, bool DW = false>
int run_mid(int M, int N, int K, const Opnd &A, const Opnd &B, float *C, long ldc) {
  const int CUS = 256;
  const long tiles = (long)((M + M_T - 1) / M_T) * ((N + M_T - 1) / M_T);
  int kc;
  const int splits = mid_splits(M, N, K, &kc);
  float *target = C;
  long tld = ldc;
  float *ws = nullptr;
  if (splits > 1) {
    ws = ws_alloc(sizeof(float) * (size_t)M * N * splits);
    if (!ws) return -2;
    target = ws;
    tld = N;
  }
  const bool cvec = aligned16(target) && tld % 4 == 0;
  const dim3 grid((unsigned)tiles, 1, splits);
  const long sstride = (long)M * N;
  // at most one workgroup per CU: 8 waves (two per SIMD), a ring of 4
  // stages of 8 k per wave (128 KB of LDS); more: 4 waves, 4 stages of 8 k
  // per wave (64 KB), two workgroups per CU.  g_mid 2: the rings shared by
  // the waves (64-k stages, 4 of them, and 32-k stages, 5 of them)
  const int alim = M, blim = N;
  const long tiles256 = (long)((M + 255) / 256) * ((N + M_T - 1) / M_T);
  if (N <= M_T && splits == 1 && tiles256 >= CUS)
    // tall: 256-row tiles, the 64 columns of B loaded once for four row blocks
    hipLaunchKernelGGL((gemm_mid_kernel<A_KC, B_NC, 32, 4, 8, 256, 2, DW>),
                       dim3((unsigned)tiles256), dim3(512), 0, stream(), M, N, K, A.p, A.ld, B.p,
                       B.ld, target, tld, sstride, kc, cvec, alim, blim);
  else if (tiles * splits <= CUS && g_mid != 2)
    hipLaunchKernelGGL((gemm_mid_kernel<A_KC, B_NC, 64, 4, 8, M_T, 8, DW, true>), grid, dim3(512),
                       0, stream(), M, N, K, A.p, A.ld, B.p, B.ld, target, tld, sstride, kc, cvec,
                       alim, blim);
  else if (tiles * splits <= CUS)
    hipLaunchKernelGGL((gemm_mid_kernel<A_KC, B_NC, 64, 4, 8, M_T, 8, DW>), grid, dim3(512), 0,
                       stream(), M, N, K, A.p, A.ld, B.p, B.ld, target, tld, sstride, kc, cvec,
                       alim, blim);
  else if (g_mid != 2)
    hipLaunchKernelGGL((gemm_mid_kernel<A_KC, B_NC, 32, 4, 4, M_T, 4, DW, true>), grid, dim3(256),
                       0, stream(), M, N, K, A.p, A.ld, B.p, B.ld, target, tld, sstride, kc, cvec,
                       alim, blim);
  else
    hipLaunchKernelGGL((gemm_mid_kernel<A_KC, B_NC, 32, 5, 4, M_T, 4, DW>), grid, dim3(256), 0,
                       stream(), M, N, K, A.p, A.ld, B.p, B.ld, target, tld, sstride, kc, cvec,
                       alim, blim);
  const bool own = ws != nullptr;
  if (hipGetLastError() != hipSuccess) { if (own) ws_free(ws); return -3; }
  if (ws) {
    const int rc = reduce_splits<EPI_STORE>(ws, C, M, N, splits, ldc, nullptr, 1);
    if (own) ws_free(ws);
    if (rc) return rc;
  }
  return 0;
}

template <bool A_KC, bool A_PERM, bool B_NC, bool B_PERM, int EPI, bool B_I2C = false>
int run(int M, int N, int K, Opnd A, Opnd B, float *C, long ldc, const float *bias, int HW,
        bool vec, const I2C &cv = I2C{}) {
  if (M <= 0 || N <= 0) return 0;
  // K == 0 runs no K tiles: the epilogue stores zeros (plus bias)
  Plan p = plan(M, N, K > 0 ? K : 1);
  if constexpr (!A_PERM && !B_PERM && !B_I2C && EPI == EPI_STORE) {
    if (p.tile != T256x256 && p.tile != T256x128 && p.tile != T128x128 && g_force_tile < 0) {
      if (!g_mid_force && small_ok<A_KC, B_NC>(M, N, K, A, B))
        return run_small<A_KC, B_NC>(M, N, K, A, B, C, ldc);
      if (mid_ok<A_KC, B_NC>(M, N, K, A, B, vec)) return run_mid<A_KC, B_NC>(M, N, K, A, B, C, ldc);
      // operands that are not 16-byte aligned (ragged leading dimensions,
      // K % 4 != 0 with k-contiguous rows): the same kernel with 4-byte loads
      if (g_mid && (g_mid_force || 2.0 * M * N * K >= 1e9) && A.ld <= (1L << 22) &&
          B.ld <= (1L << 22))
        return run_mid<A_KC, B_NC, true>(M, N, K, A, B, C, ldc);
    }
  }
  if constexpr (A_KC && B_NC && !A_PERM && !B_PERM && !B_I2C) {
    // skinny outputs over a long K: 16x16 tiles split over K (partials of
    // eight-wave workgroups), then the usual reduction and epilogue
    const long tiles = (long)((M + 15) / 16) * ((N + 15) / 16);
    if (g_t16 && g_force_tile < 0 && N <= 16 && K >= 2048 && K % 4 == 0 && A.ld % 4 == 0 &&
        aligned16(A.p) && tiles <= 128 && (M + 15) / 16 <= 65535) {
      int S = (int)(256 / tiles);
      if (S > (K + 127) / 128) S = (K + 127) / 128;
      const int kslice = ((K + S - 1) / S + 127) / 128 * 128;
      S = (K + kslice - 1) / kslice;
      const int nch = kslice / 128;
      if (nch <= 16) {
        float *ws = ws_alloc(sizeof(float) * (size_t)M * N * S);
        if (!ws) return -2;
        const dim3 grid((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16), (unsigned)S);
#define TT_T16S(NCH_)                                                                         \
  hipLaunchKernelGGL((gemm_t16_split_kernel<NCH_>), grid, dim3(64 * T16W), 0, stream(), M, N, K, \
                     A.p, A.ld, B.p, B.ld, ws, kslice)
        switch (nch) {
          case 1: TT_T16S(1); break;
          case 2: TT_T16S(2); break;
          case 3: TT_T16S(3); break;
          case 4: TT_T16S(4); break;
          case 5: case 6: TT_T16S(6); break;
          case 7: case 8: TT_T16S(8); break;
          default: TT_T16S(16); break;
        }
#undef TT_T16S
        if (hipGetLastError() != hipSuccess) { ws_free(ws); return -3; }
        const int rc = reduce_splits<EPI>(ws, C, M, N, S, ldc, bias, HW);
        ws_free(ws);
        return rc;
      }
    }
  }
  if constexpr (B_I2C) {
    // no 256-wide big tile; a split's k range must fit the LDS kc table
    if (p.tile == T256x256 || p.tile == T256x128) p.tile = T128x128;
    if (B_NC && p.kchunk > I2C_TAB) {
      const int s = (K + I2C_TAB - 1) / I2C_TAB;
      const int bk = TILE_BK[p.tile];
      p.kchunk = ((K + s - 1) / s + bk - 1) / bk * bk;
      p.splits = (K + p.kchunk - 1) / p.kchunk;
    }
  }
  float *target = C;
  long tgt_ld = ldc;
  float *ws = nullptr;
  int epi_direct = 1;
  if (p.splits > 1) {
    ws = ws_alloc(sizeof(float) * (size_t)M * N * p.splits);
    if (!ws) return -2;
    target = ws;
    tgt_ld = N;
    epi_direct = 0;
  }
  const long sstride = (long)M * N;
#define TT_LAUNCH(BM_, BN_, BK_, WM_, VEC_, EPI_)                                             \
  launch_tile<BM_, BN_, BK_, WM_, A_KC, A_PERM, B_NC, B_PERM, VEC_, EPI_, B_I2C>(             \
      M, N, K, A, B, target, tgt_ld, sstride, p.splits, p.kchunk, bias, HW, cv)
#define TT_VECK(BM_, BN_, BK_, WM_, EPI_)                 \
  if (vec) TT_LAUNCH(BM_, BN_, BK_, WM_, true, EPI_);      \
  else TT_LAUNCH(BM_, BN_, BK_, WM_, false, EPI_);
#define TT_VEC(BM_, BN_, WM_, EPI_) TT_VECK(BM_, BN_, 32, WM_, EPI_)
#define TT_SHAPES(EPI_)                                     \
  switch (p.tile) {                                         \
    case T128x128: TT_VEC(128, 128, 2, EPI_) break;         \
    case T128x64:  TT_VEC(128, 64, 2, EPI_) break;          \
    case T64x64:   TT_VEC(64, 64, 2, EPI_) break;           \
    case T32x256:  TT_VEC(32, 256, 1, EPI_) break;          \
    case T64x256:  TT_VEC(64, 256, 1, EPI_) break;          \
    case T64x128:  TT_VEC(64, 128, 1, EPI_) break;          \
    case T32x128:  TT_VEC(32, 128, 1, EPI_) break;          \
    case T64x64K64:  TT_VECK(64, 64, 64, 2, EPI_) break;    \
    case T32x128K64: TT_VECK(32, 128, 64, 1, EPI_) break;   \
    case T256x256: if constexpr (!B_I2C) { TT_VEC(256, 256, 2, EPI_) } break; \
    default:       if constexpr (!B_I2C) { TT_VEC(256, 128, 2, EPI_) } break; \
  }
  bool done = false;
  if constexpr (!A_PERM && !B_PERM && !B_I2C && EPI == EPI_STORE) {
    // plain GEMM on whole 256x256 tiles: the direct-to-LDS kernel
    if (g_direct && p.tile == T256x256 && vec && M % D_BM == 0 && N % D_BN == 0 &&
        K % D_BK == 0 && p.kchunk % D_BK == 0 && aligned16(target) && tgt_ld % 4 == 0) {
      const dim3 grid((M / D_BM) * (N / D_BN), 1, p.splits);
      hipLaunchKernelGGL((gemm_direct_kernel<A_KC, B_NC>), grid, dim3(NT), 0, stream(), M, N, K,
                         A.p, A.ld, B.p, B.ld, target, tgt_ld, sstride, p.kchunk);
      done = true;
    }
  }
  if (done) {
  } else if (epi_direct) { TT_SHAPES(EPI) } else { TT_SHAPES(EPI_STORE) }
#undef TT_SHAPES
#undef TT_VEC
#undef TT_VECK
#undef TT_LAUNCH
  if (hipGetLastError() != hipSuccess) { if (ws) ws_free(ws); return -3; }
  if (ws) {
    const int rc = reduce_splits<EPI>(ws, C, M, N, p.splits, ldc, bias, HW);
    ws_free(ws);
    if (rc) return rc;
  }
  return 0;
}

}  // namespace

extern "C" int tth_gemm_direct(int on) {
  g_direct = on ? 1 : 0;
  return 0;
}

extern "C" int tth_gemm_mid(int on) {
  g_mid = on == 2 ? 2 : on ? 1 : 0;
  return 0;
}

extern "C" int tth_gemm_mid_force(int on) {
  g_mid_force = on ? 1 : 0;
  return 0;
}

extern "C" int tth_gemm_small(int on) {
  g_small = on ? 1 : 0;
  return 0;
}

extern "C" int tth_gemm_t16(int on) {
  g_t16 = on ? 1 : 0;
  return 0;
}

extern "C" int tth_gemm_config(int tile, int splits) {
  if (tile >= NTILE || splits > 1024) return -1;
  g_force_tile = tile;
  g_force_splits = splits;
  return 0;
}

extern "C" int tt_k_gemm(int M, int N, int K, const float *A, int lda, int transA,
                         const float *B, int ldb, int transB, float *C, int ldc) {
  if (M < 0 || N < 0 || K < 0 || !A || !B || !C) return -1;
  Opnd a{A, lda, 0, 1}, b{B, ldb, 0, 1};
  const bool vec = aligned16(A) && aligned16(B) && (lda % 4 == 0) && (ldb % 4 == 0);
  if (!transA && !transB) return run<true, false, true, false, EPI_STORE>(M, N, K, a, b, C, ldc, nullptr, 1, vec);
  if (!transA && transB)  return run<true, false, false, false, EPI_STORE>(M, N, K, a, b, C, ldc, nullptr, 1, vec);
  if (transA && !transB)  return run<false, false, true, false, EPI_STORE>(M, N, K, a, b, C, ldc, nullptr, 1, vec);
  return run<false, false, false, false, EPI_STORE>(M, N, K, a, b, C, ldc, nullptr, 1, vec);
}

// C = A * B (row-major, contiguous) and the relu + padones that follow it:
// R = relu(C), P = [R, 1].  Fused into the split-K reduction when the GEMM
// takes a split-K path, else a separate pass; the same values either way.
extern "C" int tt_k_gemm_relu_pad(int M, int N, int K, const float *A, const float *B, float *C,
                                  float *R, float *P) {
  if (M <= 0 || N <= 0 || K < 0 || !A || !B || !C || !R || !P) return -1;
  RedHook h{};
  h.kind = HOOK_RELU_PAD;
  h.C = C;
  h.rp = ReluPadEx{R, P, nullptr};
  g_red_hook = &h;
  const int rc = tt_k_gemm(M, N, K, A, K, 0, B, N, 0, C, N);
  g_red_hook = nullptr;
  if (rc) return rc;
  return h.applied ? 0 : tt_k_relu_padones_fwd(C, R, P, M, N);
}

// Both gradients of C = A * B (A M x K, B K x N, row-major) in one launch,
// when tt_k_gemm would compute each of them with its small-GEMM kernel:
// the same tiles, so the same values as two tt_k_gemm calls.  d1 / d2: the
// padones (and relu) backward fused into dA's stores, as in tt_k_head_bwd.
// -1: not covered (nothing launched).
extern "C" int tt_k_matmul_bwd_small(const float *A, int M, int K, const float *B, int N,
                                     const float *G, float *dB, float *dA, float *d1, float *d2,
                                     const float *R) {
  if (M <= 0 || K <= 0 || N <= 0 || !A || !B || !G || !dA || !dB || ((d1 || d2) && K < 2) ||
      g_force_tile >= 0)
    return -1;
  const Opnd g{G, N, 0, 1}, b{B, N, 0, 1}, a{A, K, 0, 1};
  auto big = [](const Plan &p) {
    return p.tile == T256x256 || p.tile == T256x128 || p.tile == T128x128;
  };
  // run()'s choice for dA = G * B^T (M, K, N) and dB = A^T * G (K, N, M)
  if (big(plan(M, K, N)) || big(plan(K, N, M)) || !small_ok<true, false>(M, K, N, g, b) ||
      !small_ok<false, true>(K, N, M, a, g))
    return -1;
  SmallJob da{M, K, N, G, N, B, N, SmallOut{dA, K, d1, d2, R}, ((N + SW - 1) / SW + 7) / 8 * 8,
              (K + 31) / 32};
  SmallJob db{K, N, M, A, K, G, N, SmallOut{dB, N, nullptr, nullptr, nullptr},
              ((M + SW - 1) / SW + 7) / 8 * 8, (N + 31) / 32};
  const long nba = (long)da.nbx * ((M + 31) / 32), nbb = (long)db.nbx * ((K + 31) / 32);
  if (nba + nbb > 0x7fffffffL) return -1;
  // 16-byte loads of G's and B's k-contiguous rows (the loads only, not the values)
  const bool vec = aligned16(G) && aligned16(B) && N % 4 == 0;
  if (vec)
    hipLaunchKernelGGL(gemm_small_pair_kernel<true>, dim3((unsigned)(nba + nbb)), dim3(64 * SW), 0,
                       stream(), da, db, (int)nba);
  else
    hipLaunchKernelGGL(gemm_small_pair_kernel<false>, dim3((unsigned)(nba + nbb)), dim3(64 * SW),
                       0, stream(), da, db, (int)nba);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// dW = [X, 1]^T * G ((Kx + 1) x N; X rows x Kx, G rows x N, row-major and
// contiguous): the weight gradient of a matmul whose input is padones(X),
// without the padded copy -- row Kx of the product is the column sums of G,
// taken by the same MFMA tiles from a row of ones.  Bit for bit
// tt_k_gemm(Kx + 1, N, rows, [X, 1], Kx + 1, 1, G, N, 0, dW, N), on the
// shapes where that call takes the small-GEMM tiles; -1 elsewhere (nothing
// launched).
extern "C" int tt_k_gemm_tn_padones(int rows, int Kx, int N, const float *X, const float *G,
                                    float *dW) {
  if (rows <= 0 || Kx <= 0 || N <= 0 || g_force_tile >= 0) return -1;
  const int M = Kx + 1;
  const Opnd a{X, Kx, 0, 1}, g{G, N, 0, 1};
  const Plan p = plan(M, N, rows);
  if (p.tile == T256x256 || p.tile == T256x128 || p.tile == T128x128 ||
      !small_ok<false, true>(M, N, rows, a, g) || (M + 31) / 32 > 65535)
    return -1;
  if (!dW) return 0;  // only asked whether the shape is covered
  if (!X || !G) return -1;
  const int kc = ((rows + SW - 1) / SW + 7) / 8 * 8;
  const dim3 grid((unsigned)((N + 31) / 32), (unsigned)((M + 31) / 32));
  hipLaunchKernelGGL((gemm_small_kernel<false, true, false, false>), grid, dim3(64 * SW), 0,
                     stream(), M, N, rows, X, (long)Kx, G, (long)N, dW, (long)N, kc, Kx);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// tt_k_gemm_tn_padones on any shape its tiles can index, also where the
// planner would pick another kernel (few tiles: a classifier's 257 x 10
// weight gradient) -- for a gradient computed inside another launch or
// materialised on its own after all.  NULL dW: only asks.
extern "C" int ttk_gemm_tn_padones_any(int rows, int Kx, int N, const float *X, const float *G,
                                       float *dW) {
  if (rows <= 0 || Kx <= 0 || N <= 0 || (Kx + 1 + 31) / 32 > 65535) return -1;
  if (!dW) return 0;
  if (!X || !G) return -1;
  const int M = Kx + 1;
  const int kc = ((rows + SW - 1) / SW + 7) / 8 * 8;
  const dim3 grid((unsigned)((N + 31) / 32), (unsigned)((M + 31) / 32));
  hipLaunchKernelGGL((gemm_small_kernel<false, true, false, false>), grid, dim3(64 * SW), 0,
                     stream(), M, N, rows, X, (long)Kx, G, (long)N, dW, (long)N, kc, Kx);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// Up to two tt_k_gemm_tn_padones jobs, each with the SGD step wsgd -= lr *
// dW, plus the plain steps pw -= lr * pg, in one launch.  1: not covered,
// nothing launched.
extern "C" int ttk_gemm_tn_padones_sgd_jobs(const TTTnSgdJob *jobs, int nj, float lr,
                                            float *const *pw, const float *const *pg,
                                            const long *pn, int np) {
  if (nj < 1 || nj > 2 || np < 0 || np > TT_SGD_MAX) return 1;
  TnJobs J{};
  J.nj = nj;
  long gtot = 0;
  for (int q = 0; q < nj; q++) {
    const TTTnSgdJob &a = jobs[q];
    if (!a.X || !a.G || !a.dW || !a.wsgd ||
        ttk_gemm_tn_padones_any(a.rows, a.Kx, a.N, nullptr, nullptr, nullptr) != 0)
      return 1;
    TnJob &t = J.j[q];
    t.M = a.Kx + 1;
    t.N = a.N;
    t.K = a.rows;
    t.kc = ((a.rows + SW - 1) / SW + 7) / 8 * 8;
    t.ones_m = a.Kx;
    t.gx = (a.N + 31) / 32;
    t.gblocks = t.gx * ((t.M + 31) / 32);
    t.A = a.X;
    t.B = a.G;
    t.C = a.dW;
    t.wsgd = a.wsgd;
    gtot += t.gblocks;
  }
  SgdPlain P{};
  P.np = np;
  P.lr = lr;
  long tot = 0;
  for (int t = 0; t < np; t++) {
    P.w[t] = pw[t];
    P.g[t] = pg[t];
    P.n[t] = pn[t];
    P.start[t] = tot;
    tot += (pn[t] + 64 * SW - 1) / (64 * SW);
  }
  P.start[np] = tot;
  if (gtot + tot > 0x7fffffffL) return 1;
  hipLaunchKernelGGL(gemm_tn_padones_sgd_kernel, dim3((unsigned)(gtot + tot)), dim3(64 * SW), 0,
                     stream(), J, P);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

extern "C" int ttk_gemm_tn_padones_sgd(int rows, int Kx, int N, const float *X, const float *G,
                                       float *dW, float *wsgd, float lr, float *const *pw,
                                       const float *const *pg, const long *pn, int np) {
  const TTTnSgdJob j{rows, Kx, N, X, G, dW, wsgd};
  return ttk_gemm_tn_padones_sgd_jobs(&j, 1, lr, pw, pg, pn, np);
}

// C = A * B + bias (A M x K, B K x N row-major and contiguous; bias a row of
// N added to every row of C), optionally with R = relu(C) and P = [R, 1]:
// the matmul of a padones output computed from the padones input (its
// aligned rows) and the weights' last row.  Small GEMMs store the epilogue
// from their tiles, split-K GEMMs from their reduction, the rest in a pass
// after the GEMM.
extern "C" int tt_k_gemm_bias_relu_pad(int M, int N, int K, const float *A, const float *B,
                                       const float *bias, float *C, float *R, float *P) {
  if (M <= 0 || N <= 0 || K < 0 || !A || !B || !bias || !C || (!R && P) || (R && !P))
    return -1;
  if (g_force_tile < 0) {  // skinny outputs (a classifier): a workgroup per row
    const int rr = ttk_gemm_rows(A, B, bias, C, R, P, M, N, K, nullptr);
    if (rr != 1) return rr;
  }
  if (g_force_tile < 0) {  // 16x16 tiles below a full grid of 32x32 ones
    SmallOut out{C, N, nullptr, nullptr, nullptr};
    out.bias = bias;
    out.relu = R;
    out.pad = P;
    const int rt = run_t16(M, N, K, A, B, out);
    if (rt != 1) return rt;
  }
  const Opnd a{A, K, 0, 1}, b{B, N, 0, 1};
  auto big = [](const Plan &p) {
    return p.tile == T256x256 || p.tile == T256x128 || p.tile == T128x128;
  };
  if (K > 0 && g_force_tile < 0 && !big(plan(M, N, K)) && small_ok<true, true>(M, N, K, a, b)) {
    const int kc = ((K + SW - 1) / SW + 7) / 8 * 8;
    const dim3 grid((unsigned)((N + 31) / 32), (unsigned)((M + 31) / 32));
    SmallOut out{C, N, nullptr, nullptr, nullptr};
    out.bias = bias;
    out.relu = R;
    out.pad = P;
    if (aligned16(A) && K % 4 == 0)
      hipLaunchKernelGGL((gemm_small_epi_kernel<true, false>), grid, dim3(64 * SW), 0, stream(),
                         M, N, K, A, (long)K, B, (long)N, out, kc);
    else
      hipLaunchKernelGGL((gemm_small_epi_kernel<false, false>), grid, dim3(64 * SW), 0, stream(),
                         M, N, K, A, (long)K, B, (long)N, out, kc);
    return hipGetLastError() == hipSuccess ? 0 : -3;
  }
  RedHook h{};
  h.kind = HOOK_RELU_PAD;
  h.C = C;
  h.rp = ReluPadEx{R, P, bias};
  g_red_hook = &h;
  const int rc = tt_k_gemm(M, N, K, A, K, 0, B, N, 0, C, N);
  g_red_hook = nullptr;
  if (rc) return rc;
  return h.applied ? 0 : ttk_bias_relu_pad(C, bias, R, P, M, N);
}

// C = A * B + bias as tt_k_gemm_bias_relu_pad (C only) and, when the GEMM
// takes a split-K path, the softmax-CE of C's rows in its reduction
// (ttk_reduce_ce: probs, seed, rowloss).  0: all written; 1: only C (the
// caller runs the softmax-CE); < 0: error.
extern "C" int tt_k_gemm_bias_ce(int M, int N, int K, const float *A, const float *B,
                                 const float *bias, float *C, const int32_t *host_labels,
                                 float *probs, float *seed, float *rowloss, float scale) {
  if (M <= 0 || N <= 0 || K < 0 || !A || !B || !bias || !C || !host_labels || !probs || !seed ||
      !rowloss)
    return -1;
  const Opnd a{A, K, 0, 1}, b{B, N, 0, 1};
  const TTCeHook ce{bias, host_labels, probs, seed, rowloss, scale};
  if (g_force_tile < 0) {  // skinny outputs: a workgroup per row, the CE in its epilogue
    const int rr = ttk_gemm_rows(A, B, bias, C, nullptr, nullptr, M, N, K, &ce);
    if (rr != 1) return rr;
    // too many rows for the CE's labels: the logits as tt_k_gemm_bias_relu_pad
    // forms them, the CE the caller's
    const int rc = ttk_gemm_rows(A, B, bias, C, nullptr, nullptr, M, N, K, nullptr);
    if (rc != 1) return rc ? rc : 1;
  }
  auto big = [](const Plan &p) {
    return p.tile == T256x256 || p.tile == T256x128 || p.tile == T128x128;
  };
  if (K > 0 && g_force_tile < 0 && !big(plan(M, N, K)) && small_ok<true, true>(M, N, K, a, b)) {
    const int rc = tt_k_gemm_bias_relu_pad(M, N, K, A, B, bias, C, nullptr, nullptr);
    return rc ? rc : 1;
  }
  RedHook h{};
  h.kind = HOOK_CE;
  h.C = C;
  h.rp = ReluPadEx{nullptr, nullptr, bias};
  h.ce = &ce;
  g_red_hook = &h;
  const int rc = tt_k_gemm(M, N, K, A, K, 0, B, N, 0, C, N);
  g_red_hook = nullptr;
  if (rc) return rc;
  if (h.applied == 2) return 0;
  if (h.applied == 1) return 1;
  const int rb = ttk_bias_relu_pad(C, bias, nullptr, nullptr, M, N);
  return rb ? rb : 1;
}

// ---- the GEMM without allocation (tt_k_gemm_noalloc) ----
// Its workspace lives in this fixed device array; each GPU holds its own copy
// for the life of the process.  In host code the name `scratch` is only a
// stand-in for the device symbol: its device address is looked up once per
// device (ttg_scratch_setup, called from the runtime's initialisation) and
// only that address is handed to kernels.
static __device__ __align__(256) char scratch[TT_GEMM_SCRATCH_BYTES];
namespace {
constexpr int MAX_DEV = 64;
char *g_scratch_dev[MAX_DEV];  // device address of `scratch`, per device
}  // namespace

extern "C" int ttg_scratch_setup(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return -1;
  if (g_scratch_dev[dev]) return 0;
  void *ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
    (void)hipGetLastError();
    return -1;
  }
  g_scratch_dev[dev] = (char *)ptr;
  return 0;
}

extern "C" int tt_k_gemm_noalloc(int M, int N, int K, const float *A, int lda, int transA,
                                 const float *B, int ldb, int transB, float *C, int ldc) {
  if (M < 0 || N < 0 || K < 0 || !A || !B || !C) return -1;
  if (ttrt_init() != 0) return -3;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEV) return -3;
  if (!g_scratch_dev[dev] && ttg_scratch_setup() != 0) return -3;
  WsArena arena{g_scratch_dev[dev], (size_t)TT_GEMM_SCRATCH_BYTES, 0};
  g_arena = &arena;
  int rc = tt_k_gemm(M, N, K, A, lda, transA, B, ldb, transB, C, ldc);
  g_arena = nullptr;
  if (rc == -2) {  // the workspace this shape needs exceeds the scratch: nothing was launched
    ttrt_set_error(TT_E_SCRATCH);
    rc = TT_E_SCRATCH;
  }
  return rc;
}

extern "C" int tt_k_conv_fwd(int F, int Kc, long Ncol, int HW, const float *W, const float *col,
                             const float *bias, float *out) {
  if (F <= 0 || Kc <= 0 || Ncol <= 0 || HW <= 0 || Ncol > 0x7fffffffL) return -1;
  Opnd a{W, Kc, 0, 1}, b{col, Ncol, 0, 1};
  const bool vec = aligned16(W) && aligned16(col) && (Kc % 4 == 0) && (Ncol % 4 == 0);
  return run<true, false, true, false, EPI_BIAS_NCHW>(F, (int)Ncol, Kc, a, b, out, 0, bias, HW, vec);
}

extern "C" int tt_k_conv_dw(int F, int Kc, long Ncol, int HW, const float *g, const float *col,
                            float *dW) {
  if (F <= 0 || Kc <= 0 || Ncol <= 0 || HW <= 0 || Ncol > 0x7fffffffL) return -1;
  // A = Gperm (m = f, k = p, permuted k), B = col^T (B stored Kc x Ncol = N x K)
  Opnd a{g, HW, (long)F * HW, HW}, b{col, Ncol, 0, 1};
  const bool vec = aligned16(g) && aligned16(col) && (HW % 4 == 0) && (Ncol % 4 == 0);
  return run<true, true, false, false, EPI_STORE>(F, Kc, (int)Ncol, a, b, dW, Kc, nullptr, 1, vec);
}

extern "C" int tt_k_conv_dw_bias(int F, int Kc, long Ncol, int HW, const float *g,
                                 const float *col1, float *dW, float *db) {
  if (F <= 0 || Kc <= 0 || Ncol <= 0 || HW <= 0 || Ncol > 0x7fffffffL || !db) return -1;
  // B = [col; ones]^T: Kc + 1 stored rows of Ncol
  Opnd a{g, HW, (long)F * HW, HW}, b{col1, Ncol, 0, 1};
  const bool vec = aligned16(g) && aligned16(col1) && (HW % 4 == 0) && (Ncol % 4 == 0);
  return run<true, true, false, false, EPI_DW_BIAS>(F, Kc + 1, (int)Ncol, a, b, dW, Kc, db, 1, vec);
}

extern "C" int tt_k_conv_dcol(int F, int Kc, long Ncol, int HW, const float *W, const float *g,
                              float *dcol) {
  if (F <= 0 || Kc <= 0 || Ncol <= 0 || HW <= 0 || Ncol > 0x7fffffffL) return -1;
  // A = W^T (A stored F x Kc = K x M), B = Gperm (k = f, n = p, permuted n)
  Opnd a{W, Kc, 0, 1}, b{g, HW, (long)F * HW, HW};
  const bool vec = aligned16(W) && aligned16(g) && (Kc % 4 == 0) && (HW % 4 == 0);
  return run<false, false, true, true, EPI_STORE>(Kc, (int)Ncol, F, a, b, dcol, Ncol, nullptr, 1, vec);
}

// ---- implicit-GEMM convolution (im2col folded into the B operand) ----

namespace {

// Kernel taps of the transposed convolution: wt[c][(f*HH + kh)*WW + kw] =
// w[f][c][HH-1-kh][WW-1-kw] (C x F*HH*WW, k-contiguous rows).
__global__ void conv_flip_weights_kernel(const float *__restrict__ w, float *__restrict__ wt, int F,
                                         int C, int HH, int WW) {
  const int taps = HH * WW;
  const long total = (long)F * C * taps;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long)gridDim.x * blockDim.x) {
    const int t = (int)(i % taps);
    const long fc = i / taps;
    const int c = (int)(fc % C), f = (int)(fc / C);
    const int kh = t / WW, kw = t - kh * WW;
    wt[((long)c * F + f) * taps + (HH - 1 - kh) * WW + (WW - 1 - kw)] = w[i];
  }
}

bool i2c_fits(long xnumel, long ncol) { return xnumel < 0x7fffffffL && ncol < 0x7fffffffL; }

}  // namespace

// out = conv(x, w) + bias in NCHW: the conv forward GEMM W (F x Kc) times the
// implicit im2col of x (reference src/ops_spatial.c:71-127).
extern "C" int tt_k_conv2d_fwd_implicit(const float *x, const float *w, const float *bias,
                                        float *out, int N, int C, int H, int W, int F, int HH,
                                        int WW, int sh, int sw, int ph, int pw, int Ho, int Wo) {
  if (!x || !w || !out || N <= 0 || C <= 0 || F <= 0 || HH <= 0 || WW <= 0 || Ho <= 0 || Wo <= 0)
    return -1;
  const long ncol = (long)N * Ho * Wo;
  const long kc = (long)C * HH * WW;
  if (!i2c_fits((long)N * C * H * W, ncol) || kc > 0x7fffffffL) return -1;
  I2C cv{x, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, (int)kc, 0};
  Opnd a{w, kc, 0, 1}, b{nullptr, 0, 0, 1};
  const bool vec = aligned16(w) && kc % 4 == 0;
  return run<true, false, true, false, EPI_BIAS_NCHW, true>(F, (int)ncol, (int)kc, a, b, out, 0,
                                                            bias, Ho * Wo, vec, cv);
}

// dW (F x Kc) = Gperm (F x N*Ho*Wo) times the implicit im2col of x,
// transposed; with db, the ones row gives db in the same GEMM (reference
// src/autograd.c:467-513).
extern "C" int tt_k_conv2d_dw_implicit(const float *g, const float *x, float *dw, float *db,
                                       int N, int C, int H, int W, int F, int HH, int WW, int sh,
                                       int sw, int ph, int pw, int Ho, int Wo) {
  if (!g || !x || !dw || N <= 0 || C <= 0 || F <= 0 || HH <= 0 || WW <= 0 || Ho <= 0 || Wo <= 0)
    return -1;
  const long ncol = (long)N * Ho * Wo;
  const long kc = (long)C * HH * WW;
  if (!i2c_fits((long)N * C * H * W, ncol) || kc >= 0x7fffffffL) return -1;
  const int HWo = Ho * Wo;
  I2C cv{x, C, H, W, HH, WW, sh, sw, ph, pw, Ho, Wo, (int)kc, db ? 1 : 0};
  Opnd a{g, HWo, (long)F * HWo, HWo}, b{nullptr, 0, 0, 1};
  const bool vec = aligned16(g) && HWo % 4 == 0;
  if (db)
    return run<true, true, false, false, EPI_DW_BIAS, true>(F, (int)kc + 1, (int)ncol, a, b, dw,
                                                            kc, db, 1, vec, cv);
  return run<true, true, false, false, EPI_STORE, true>(F, (int)kc, (int)ncol, a, b, dw, kc,
                                                        nullptr, 1, vec, cv);
}

// dX of a stride-1 convolution as the convolution of the output gradient g
// with the flipped, transposed kernel and padding HH-1-ph / WW-1-pw: the
// reference's dcol = W^T * Gperm followed by col2im (src/autograd.c:515-539,
// 406-434) in one implicit GEMM, M = C, K = F*HH*WW, N = N*H*W.
extern "C" int tt_k_conv2d_dx_implicit(const float *g, const float *w, float *dx, int N, int C,
                                       int H, int W, int F, int HH, int WW, int sh, int sw, int ph,
                                       int pw, int Ho, int Wo) {
  if (!g || !w || !dx || N <= 0 || C <= 0 || F <= 0 || HH <= 0 || WW <= 0) return -1;
  if (sh != 1 || sw != 1 || ph > HH - 1 || pw > WW - 1) return -1;
  if (Ho != H + 2 * ph - HH + 1 || Wo != W + 2 * pw - WW + 1) return -1;
  const long kt = (long)F * HH * WW;
  const long npix = (long)N * H * W;
  if (!i2c_fits((long)N * F * Ho * Wo, npix) || kt > 0x7fffffffL) return -1;
  float *wt = (float *)ttrt_alloc(sizeof(float) * (size_t)kt * C);
  if (!wt) return -2;
  long blocks = (kt * C + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(conv_flip_weights_kernel, dim3((unsigned)blocks), dim3(256), 0, stream(), w,
                     wt, F, C, HH, WW);
  I2C cv{g, F, Ho, Wo, HH, WW, 1, 1, HH - 1 - ph, WW - 1 - pw, H, W, (int)kt, 0};
  Opnd a{wt, kt, 0, 1}, b{nullptr, 0, 0, 1};
  const bool vec = kt % 4 == 0;
  const int rc = run<true, false, true, false, EPI_BIAS_NCHW, true>(
      C, (int)npix, (int)kt, a, b, dx, 0, nullptr, H * W, vec, cv);
  ttrt_free(wt);  // stream-ordered: the GEMM above is queued before any reuse
  return rc;
}
