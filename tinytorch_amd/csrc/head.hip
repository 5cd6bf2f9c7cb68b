// Backward of a classifier layer on gfx950 in one launch: a matmul with few
// output columns (N <= 32) together with the backward of the padones (and
// the reshape or relu before it) that feeds it.
//
// Replaces, for the last layer of the reference's training steps:
//   dW = h_pad^T * dlogits      reference src/autograd.c:87-103 (matmul_tn)
//   dh_pad = dlogits * W^T      reference src/autograd.c:66-84  (matmul_nt)
//   padones backward, reshape backward (a copy) or relu backward
//                               reference src/autograd.c:318-327,348-369
// which the general path runs as three launches (two GEMMs of a few MFLOP
// and the padones backward).  Kernels this small are bound by latency on
// MI355X, so the kernel spreads its work over hundreds of waves with short
// per-lane loops, issues its global loads unconditionally (addresses
// clamped, values selected) and in batches, so a batch costs one memory
// round trip, and stages shared operands in LDS once per workgroup.
//
// Two kinds of workgroups in one grid:
//   dW blocks: 64 rows k of W x 4 columns j (32 x 8 for large M), one
//     output per lane, summed over m ascending from LDS -- the reference
//     matmul_tn order (+0.0, then one multiply and one add per m);
//   dA blocks: 64 columns k x 32 rows m, each lane's 8 outputs summed over j
//     ascending -- the reference matmul_nt order.
// Both are bit-identical to the reference's loops (this file is compiled
// without contraction).  With `gpart` the output gradient is not read: every
// workgroup forms it first, in LDS, from two partial sums of the logits per
// row, the bias and the labels -- the seed of the softmax-CE exactly as
// splitk_reduce_ce_kernel computes it ((0 + p0) + p1 + bias, then ce_row) --
// and workgroup 0 also writes the logits, probabilities, seed and row
// losses that reduction would have written.  dh is written whole (the padones node's gradient)
// and, without its last column, once or twice more: the gradient of the
// padones' input and, when that input is a reshape (a copy) or a relu used
// only here, the gradient of the node before it (for a relu, masked by
// relu output > 0, which equals relu input > 0).

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include "tt_rt.h"
#include "ce_rows.h"
#include "probe.h"
TT_PROBE_DEFINE(head)

namespace {

inline hipStream_t stream() { return (hipStream_t)ttrt_stream(); }
inline int launched() { return hipGetLastError() == hipSuccess ? 0 : -3; }

typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int NT = 256;

// The softmax-CE whose seed the kernel forms itself (kernel argument):
// part = 2 x M x N partial sums of the logits, bias, labels, scale; the
// outputs workgroup 0 writes (each may be NULL).
struct TTHeadCe {
  const float *part, *bias;
  LabU8 lab;
  float scale;
  float *logits, *probs, *seed, *rowloss;
};


// Every padding element of a staged block is loaded from here.
__device__ float g_head_zero[4];

// Stage a rows x COLS block (COLS a power of two <= 64) into LDS:
// dst[r * dstride + c] = src[r * sstride + c] for r < nr and c < nc, else 0,
// for r < rows.  Lane t takes column t % COLS of rows t / COLS + (NT/COLS) u;
// U loads per lane per batch, all issued before the first LDS store.
template <int COLS, int U>
__device__ __forceinline__ void stage_load(float (&v)[U], const float *src,
                                           long sstride, int base, int nr, int nc) {
  constexpr int RPB = NT / COLS;  // rows per pass of the workgroup
  const int c = threadIdx.x % COLS, r0 = threadIdx.x / COLS;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int r = base + r0 + RPB * u;
    const bool ok = r < nr && c < nc;
    v[u] = *(ok ? src + r * sstride + c : g_head_zero);
  }
}

template <int COLS, int U>
__device__ __forceinline__ void stage_store(const float (&v)[U], float *dst, int dstride, int base,
                                            int rows) {
  constexpr int RPB = NT / COLS;
  const int c = threadIdx.x % COLS, r0 = threadIdx.x / COLS;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int r = base + r0 + RPB * u;
    if (r < rows) dst[r * dstride + c] = v[u];
  }
}

// Two blocks of M rows staged together: both blocks' loads of a batch of
// rows are issued before either's LDS stores (one memory round trip per
// batch).  (NT / CA) * UA == (NT / CB) * UB rows per batch.
template <int CA, int UA, int CB, int UB>
__device__ __forceinline__ void stage_pair(float *da, const float *__restrict__ sa, long lda,
                                           int nca, float *db, const float *sb,
                                           long ldb, int ncb, int M) {
  static_assert((NT / CA) * UA == (NT / CB) * UB, "batches of the two blocks differ");
  for (int base = 0; base < M; base += (NT / CA) * UA) {
    float va[UA], vb[UB];
    stage_load<CA, UA>(va, sa, lda, base, M, nca);
    stage_load<CB, UB>(vb, sb, ldb, base, M, ncb);
    stage_store<CA, UA>(va, da, CA, base, M);
    stage_store<CB, UB>(vb, db, CB, base, M);
  }
}

// dW[k][j] for KW rows k and JW = NT / KW columns j of one workgroup: lane t
// takes k = k0 + t % KW, j = j0 + t / KW and sums over m ascending from LDS
// (As: M x KW, Gs: M x JW; the strides are constants, so every LDS read of
// the loop carries its offset in the instruction).
template <int KW, int NC = 16>
__device__ __forceinline__ void head_dw_block(const float *__restrict__ A, int M, int K,
                                              const float *G, int N,
                                              float *__restrict__ dW, int k0, int j0,
                                              float *lds, const TTHeadCe &ce, bool use_ce,
                                              float *gl) {
  constexpr int JW = NT / KW;
  const int tid = threadIdx.x;
  float *As = lds, *Gs = lds + M * KW;
  if (use_ce) {
    // the block of A (M <= 32 * NT / KW rows: one batch) in flight while the
    // seed of every row is formed (its loads issued after the partial sums',
    // which the softmax-CE waits for; workgroup 0 stores the softmax-CE's
    // outputs), then the block's columns of it
    float va[32];
    head_ce_seed<NC, 2>(ce, 0, M, M, N, gl, N, blockIdx.x == 0, gl + M * N,
                        [&]() { stage_load<KW, 32>(va, A + k0, K, 0, M, min(KW, K - k0)); });
    stage_store<KW, 32>(va, As, KW, 0, M);
    __syncthreads();
    for (int i = tid; i < M * JW; i += NT) {
      const int m = i / JW, j = j0 + i % JW;
      Gs[i] = j < N ? gl[m * N + j] : 0.0f;
    }
  } else {
    // batches of 32 * NT / KW rows (128 or 256)
    stage_pair<KW, 32, JW, 32 * JW / KW>(As, A + k0, K, min(KW, K - k0), Gs, G + j0, N,
                                         min(JW, N - j0), M);
  }
  __syncthreads();
  TT_PROBE(0, 1);
  const int kl = tid % KW, jl = tid / KW;
  const int k = k0 + kl, j = j0 + jl;
  if (j >= N || k >= K) return;
  const float *ac = As + kl, *gc = Gs + jl;
  float acc = 0.0f;
  int m = 0;
  for (; m + 16 <= M; m += 16) {
    float a[16], g[16];
#pragma unroll
    for (int u = 0; u < 16; u++) { a[u] = ac[(m + u) * KW]; g[u] = gc[(m + u) * JW]; }
#pragma unroll
    for (int u = 0; u < 16; u++) acc += a[u] * g[u];
  }
  for (; m < M; m++) acc += ac[m * KW] * gc[m * JW];
  dW[(long)k * N + j] = acc;
}


// ---- backward ----
constexpr int DA_M = 32;  // rows m per dA workgroup (8 per lane)
// The output gradient of the classifier for rows [r0, r1) from the partial
// sums of its logits (see above) into gl (row r at gl[(r - r0) * gs]); `out`:
// also store the softmax-CE's outputs of those rows.  The rows' partial sums
// are first loaded whole-workgroup (coalesced) into pp (2 (r1 - r0) N floats
// of LDS) with the rows' labels; GW lanes a row then form its softmax-CE (one
// round for the rows of a block: 2 lanes a row for 128 rows, 8 for 32).
// Every thread calls it (barriers inside).
struct NoLoads {
  __device__ void operator()() const {}
};
// issue(): called once the first partial sums' loads are issued, before the
// wait for them -- loads it issues stay in flight through the softmax-CE
template <int NC, int GW, class Issue = NoLoads>
__device__ __forceinline__ void head_ce_seed(const TTHeadCe &ce, int r0, int r1, int M, int N,
                                             float *gl, int gs, bool out, float *pp,
                                             Issue issue = Issue()) {
  const int n = (r1 - r0) * N;
  const long total = (long)M * N;
  // GW lanes a row (ce_row_group): lane q takes columns [q CPL, q CPL + CPL)
  constexpr int CPL = (NC + GW - 1) / GW;
  const int q = threadIdx.x & (GW - 1);
  float bq[CPL];  // this lane's bias values, loaded with the partial sums
#pragma unroll
  for (int u = 0; u < CPL; u++) bq[u] = ce.bias[min(q * CPL + u, N - 1)];
  // the rows' labels too (read in the loop below, each was a round trip):
  // the first NT loaded into a register here and stored to LDS after the
  // partial sums' loads are issued (stored at once, their round trip would
  // come before those loads)
  int *yl = reinterpret_cast<int *>(pp + 2 * n);
  const int nr = r1 - r0;
  const int y0 = (int)threadIdx.x < nr ? ce.lab[r0 + threadIdx.x] : 0;
  // eight elements a thread in flight before their LDS stores (a loop that
  // stores each load waits a memory round trip per element)
  for (int b = 0; b < n; b += 8 * NT) {
    float v0[8], v1[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = min(b + (int)threadIdx.x + u * NT, n - 1);
      v0[u] = ce.part[(long)r0 * N + i];
      v1[u] = ce.part[total + (long)r0 * N + i];
    }
    if (b == 0) issue();
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int i = b + (int)threadIdx.x + u * NT;
      if (i < n) {
        pp[i] = v0[u];
        pp[n + i] = v1[u];
      }
    }
  }
  if ((int)threadIdx.x < nr) yl[threadIdx.x] = y0;
  for (int i = threadIdx.x + NT; i < nr; i += NT) yl[i] = ce.lab[r0 + i];
  __syncthreads();
  TT_PROBE(0, 6);
  for (int r = r0 + (int)(threadIdx.x / GW); r < r1; r += NT / GW) {
    float lv[CPL], pr[CPL], sr[CPL];
    const float *p0 = pp + (r - r0) * N;
#pragma unroll
    for (int u = 0; u < CPL; u++) {
      const int j = q * CPL + u;
      lv[u] = 0.0f;
      if (j < N) {
        float s = 0.0f;
        s += p0[j];
        s += p0[n + j];
        lv[u] = s + bq[u];
      }
    }
    float lg[CPL];
#pragma unroll
    for (int u = 0; u < CPL; u++) lg[u] = lv[u];
    const float loss = ce_row_group<GW, CPL>(lv, yl[r - r0], N, ce.scale, pr, sr);
#pragma unroll
    for (int u = 0; u < CPL; u++)
      if (q * CPL + u < N) gl[(r - r0) * gs + q * CPL + u] = sr[u];
    if (out) {
#pragma unroll
      for (int u = 0; u < CPL; u++)
        if (q * CPL + u < N) {
          const long o = (long)r * N + q * CPL + u;
          if (ce.logits) ce.logits[o] = lg[u];
          if (ce.probs) ce.probs[o] = pr[u];
          if (ce.seed) ce.seed[o] = sr[u];
        }
      if (ce.rowloss && q == 0) ce.rowloss[r] = loss;
    }
  }
  TT_PROBE(0, 7);
}

template <int NC>
__global__ void __launch_bounds__(NT)
head_bwd_kernel(const float *__restrict__ A, int M, int K, const float *__restrict__ W, int N,
                const float *G, float *__restrict__ dW, float *__restrict__ dA,
                float *__restrict__ d1, float *__restrict__ d2, const float *__restrict__ R,
                int nbw, int KW, int nkw, const unsigned char *__restrict__ codes,
                float *__restrict__ dc, int P2, int Wo2, TTHeadCe ce, int gl_off) {
  TT_PROBE(0, 0);
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nkb = (K + 63) / 64;
  const bool cp = ce.part != nullptr;
  if ((int)blockIdx.x < nbw) {
    // dW blocks: KW rows k x NT / KW columns j
    const int JW = NT / KW;
    const int kb = blockIdx.x % nkw, jb = blockIdx.x / nkw;
    if (KW == 64) head_dw_block<64, NC>(A, M, K, G, N, dW, kb * 64, jb * JW, lds, ce, cp, lds + gl_off);
    else head_dw_block<32, NC>(A, M, K, G, N, dW, kb * 32, jb * JW, lds, ce, cp, lds + gl_off);
    TT_PROBE(0, 2);
    return;
  }
  // dA block: columns [k0, k0 + 64) x rows [m0, m0 + DA_M); Ws, Gs (64 / DA_M x NC)
  const int blk = blockIdx.x - nbw;
  const int k0 = (blk % nkb) * 64, m0 = (blk / nkb) * DA_M;
  float *Ws = lds, *Gs = lds + 64 * NC;
  {  // both blocks' loads in flight before either's LDS stores
    constexpr int UW = 64 / (NT / NC), UG = DA_M / (NT / NC);
    float vw[UW], vg[UG];
    stage_load<NC, UW>(vw, W + (long)k0 * N, N, 0, min(64, K - k0), N);
    if (cp) {
      // the block's rows of the seed, formed here while W is in flight (the
      // first column block stores their softmax-CE outputs when no dW
      // workgroup does)
      head_ce_seed<NC, NT / DA_M>(ce, m0, min(m0 + DA_M, M), M, N, Gs, NC, nbw == 0 && blk % nkb == 0,
                       lds + gl_off);
      stage_store<NC, UW>(vw, Ws, NC, 0, 64);
    } else {
      stage_load<NC, UG>(vg, G + (long)m0 * N, N, 0, min(DA_M, M - m0), N);
      stage_store<NC, UW>(vw, Ws, NC, 0, 64);
      stage_store<NC, UG>(vg, Gs, NC, 0, DA_M);
    }
  }
  const int kl = lane, mg = wave;
  const int k = k0 + kl;
  const int K1 = K - 1;
  constexpr int MI = DA_M / 4;  // rows per lane: m0 + mg + 4 i
  // the relu outputs and pool codes of this lane's outputs, loaded before
  // the barrier, clamped to the matrix (a load issued at its store costs a
  // memory round trip per row)
  float rv[MI];
  unsigned char cv[MI];
  {
    const int kc = k < K1 ? k : K1 - 1;
    if (R && d2) {
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const int m = m0 + mg + 4 * i;
        rv[i] = R[(long)(m < M ? m : M - 1) * K1 + kc];
      }
    }
    if (dc) {
#pragma unroll
      for (int i = 0; i < MI; i++) {
        const int m = m0 + mg + 4 * i;
        cv[i] = codes[(long)(m < M ? m : M - 1) * K1 + kc];
      }
    }
  }
  __syncthreads();
  TT_PROBE(0, 4);
  if (k >= K) return;
  f32x4 w4[NC / 4];
#pragma unroll
  for (int v = 0; v < NC / 4; v++) w4[v] = *(const f32x4 *)(Ws + kl * NC + 4 * v);
  TT_PROBE(0, 8);
  // this lane's window of the pool backward: dc row m starts at 4 m K1 (2Ho2
  // x 2Wo2 per feature map); the divisions once per lane, not per row
  long dco = 0;
  if (dc) {
    const int kq = k < K1 ? k : 0;
    const int fc = kq / P2, rem = kq - fc * P2, h2 = rem / Wo2, w2 = rem - h2 * Wo2;
    dco = ((long)fc * (2 * (P2 / Wo2)) + 2 * h2) * (2 * Wo2) + 2 * w2;
  }
#pragma unroll
  for (int i = 0; i < MI; i++) {
    const int m = m0 + mg + 4 * i;
    if (i == 1) TT_PROBE(0, 9);
    if (m < M) {
      const f32x4 *gr = (const f32x4 *)(Gs + (mg + 4 * i) * NC);
      float s = 0.0f;
#pragma unroll
      for (int v = 0; v < NC / 4; v++) {
        const f32x4 g4 = gr[v];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float t = s + g4[e] * w4[v][e];
          s = 4 * v + e < N ? t : s;
        }
      }
      dA[(long)m * K + k] = s;
      if (k < K1) {
        const long o = (long)m * K1 + k;
        if (d1) d1[o] = s;
        if (d2) d2[o] = R ? (rv[i] > 0.0f ? s : 0.0f) : s;
        if (dc) {
          // d2 is a 2x2 max pool's output gradient (K1 = F x Ho2 x Wo2 per
          // row) whose input was a relu: its pool + relu backward from the
          // window's code (bits 0-1 argmax, 2-5 relu mask), as
          // maxpool2x2_code_bwd_kernel writes it
          const unsigned c = cv[i];
          const float g0 = 0.0f + s;
          auto at = [&](unsigned q) { return ((c & 3) == q && ((c >> (2 + q)) & 1)) ? g0 : 0.0f; };
          float *dr = dc + (long)m * 4 * K1 + dco;
          *reinterpret_cast<float2 *>(dr) = make_float2(at(0), at(1));
          *reinterpret_cast<float2 *>(dr + 2 * Wo2) = make_float2(at(2), at(3));
        }
      }
    }
  }
  TT_PROBE(0, 5);
}

}  // namespace

extern "C" {

static int head_bwd(const float *A, int M, int K, const float *W, int N, const float *G,
                    float *dW, float *dA, float *d1, float *d2, const float *R,
                    const unsigned char *codes, float *dc, int P2, int Wo2,
                    const TTHeadCe *ce = nullptr) {
  if (M <= 0 || K <= 0 || N <= 0 || N > 32 || (!G && !ce) || (!dW && !dA) || (dW && !A) ||
      (dA && !W) || ((d1 || d2) && (!dA || K < 2)))
    return -1;
  if (ce && (!ce->part || !ce->bias || M > TT_CE_ARG_ROWS || N > 16)) return -1;
  const int NC = N <= 16 ? 16 : 32;
  const int KW = (size_t)M * (64 + 4) * sizeof(float) <= 64 * 1024 ? 64 : 32;
  const size_t lds_w = dW ? sizeof(float) * (size_t)M * (KW + NT / KW) : 0;
  const size_t lds_a = dA ? sizeof(float) * (size_t)(64 + DA_M) * NC : 0;
  if (ce && dW && M > 32 * (NT / KW)) return -1;  // one batch of A rows (head_dw_block)
  size_t lds = lds_w > lds_a ? lds_w : lds_a;
  const int gl_off = (int)(lds / sizeof(float));
  if (ce) lds += sizeof(float) * (size_t)(3 * M * N + M);  // output gradient, partials, labels
  if (lds > 64 * 1024) return -1;
  const TTHeadCe none{};
  const TTHeadCe &hc = ce ? *ce : none;
  const long nkb = (K + 63) / 64, nkw = (K + KW - 1) / KW;
  const long nbw = dW ? nkw * ((N + NT / KW - 1) / (NT / KW)) : 0;
  const long nba = dA ? nkb * ((M + DA_M - 1) / DA_M) : 0;
  if (nbw + nba > 0x7fffffffL) return -1;
  const dim3 grid((unsigned)(nbw + nba));
  if (NC == 16)
    hipLaunchKernelGGL(head_bwd_kernel<16>, grid, dim3(NT), lds, stream(), A, M, K, W, N, G, dW,
                       dA, d1, d2, R, (int)nbw, KW, (int)nkw, codes, dc, P2, Wo2, hc, gl_off);
  else
    hipLaunchKernelGGL(head_bwd_kernel<32>, grid, dim3(NT), lds, stream(), A, M, K, W, N, G, dW,
                       dA, d1, d2, R, (int)nbw, KW, (int)nkw, codes, dc, P2, Wo2, hc, gl_off);
  return launched();
}

int tt_k_head_bwd(const float *A, int M, int K, const float *W, int N, const float *G,
                  float *dW, float *dA, float *d1, float *d2, const float *R) {
  return head_bwd(A, M, K, W, N, G, dW, dA, d1, d2, R, nullptr, nullptr, 1, 1);
}

int tt_k_head_bwd_pool(const float *A, int M, int K, const float *W, int N, const float *G,
                       float *dW, float *dA, float *d1, float *d2, const unsigned char *codes,
                       float *dc, int F, int Ho2, int Wo2) {
  if (!codes || !dc || !dA || F <= 0 || Ho2 <= 0 || Wo2 <= 0 ||
      (long)F * Ho2 * Wo2 != (long)K - 1 || ((uintptr_t)dc & 7))
    return -1;
  return head_bwd(A, M, K, W, N, G, dW, dA, d1, d2, nullptr, codes, dc, Ho2 * Wo2, Wo2);
}

}  // extern "C"

int ttk_head_bwd_ce(const float *A, int M, int K, const float *W, int N, const TTHeadCeArgs *a,
                    float *dW, float *dA, float *d1, float *d2, const float *R,
                    const unsigned char *codes, float *dc, int F, int Ho2, int Wo2) {
  if (!a || !a->labels) return -1;
  if (codes && (!dc || !dA || F <= 0 || Ho2 <= 0 || Wo2 <= 0 ||
                (long)F * Ho2 * Wo2 != (long)K - 1 || ((uintptr_t)dc & 7)))
    return -1;
  TTHeadCe ce{};
  ce.part = a->part;
  ce.bias = a->bias;
  ce.scale = a->scale;
  ce.logits = a->logits;
  ce.probs = a->probs;
  ce.seed = a->seed;
  ce.rowloss = a->rowloss;
  if (M > TT_CE_ARG_ROWS) return -1;
  lab_u8_fill(ce.lab, a->labels, M, N);
  return codes ? head_bwd(A, M, K, W, N, nullptr, dW, dA, d1, d2, nullptr, codes, dc, Ho2 * Wo2,
                          Wo2, &ce)
               : head_bwd(A, M, K, W, N, nullptr, dW, dA, d1, d2, R, nullptr, nullptr, 1, 1, &ce);
}
