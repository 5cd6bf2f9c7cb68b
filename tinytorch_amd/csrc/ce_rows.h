// Softmax + mean cross-entropy of a few thousand rows by ONE workgroup of
// 256 threads.  Include it only from files compiled without floating-point
// contraction: with contraction the backend also fuses multiply-adds inside
// the inlined expf / logf, and results move in the last bit.
#pragma once
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include "tt_hip.h"

// Labels handed over inside the kernel arguments (no copy to device memory
// before the launch), one byte each: a label outside [0, cols) is stored as
// 255, which is outside [0, cols) too for cols <= 255 -- the same loss and
// seed as the original label.
struct LabU8 {
  uint8_t v[TT_CE_ARG_ROWS];
  __device__ int operator[](int r) const { return v[r]; }
};

static inline void lab_u8_fill(LabU8 &la, const int32_t *host_labels, long rows, int cols) {
  for (long r = 0; r < rows; r++) {
    const int32_t y = host_labels[r];
    la.v[r] = (uint8_t)(y >= 0 && y < cols ? y : 255);
  }
  for (long r = rows; r < TT_CE_ARG_ROWS; r++) la.v[r] = 255;
}

// Probabilities and seed (p - onehot(y)) * scale of one row of cols logits
// (cols <= MAXC, the row in registers); returns -log max(p_y, 1e-12).
template <int MAXC>
__device__ __forceinline__ float ce_row(const float *__restrict__ xr, int y,
                                        float *__restrict__ pr, float *__restrict__ sr,
                                        int cols, float scale) {
  float v[MAXC];
#pragma unroll
  for (int j = 0; j < MAXC; j++) v[j] = j < cols ? xr[j] : -INFINITY;
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < MAXC; j++) if (j < cols && v[j] > mx) mx = v[j];
  if (mx == -INFINITY) {
#pragma unroll
    for (int j = 0; j < MAXC; j++) v[j] = 1.0f / (float)cols;
  } else {
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < MAXC; j++)
      if (j < cols) { v[j] = expf(v[j] - mx); sum += v[j]; }
#pragma unroll
    for (int j = 0; j < MAXC; j++) v[j] = v[j] / sum;
  }
  float py = 0.0f;
#pragma unroll
  for (int j = 0; j < MAXC; j++)
    if (j < cols) {
      pr[j] = v[j];
      sr[j] = (v[j] - (j == y ? 1.0f : 0.0f)) * scale;
      if (j == y) py = v[j];
    }
  return -logf(fmaxf(py, 1e-12f));
}

// loss_mean[0] = (sum of the 256 per-thread sums acc, added through `part`
// (256 floats of LDS) in a fixed tree) / rows.  Every thread of the
// workgroup calls it; threads 256 and up only take part in the barriers.
__device__ __forceinline__ void ce_mean_tree(float acc, float *part, float *loss_mean,
                                             int rows) {
  const int t = threadIdx.x;
  if (t < 256) part[t] = acc;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (t < o) part[t] += part[t + o];
    __syncthreads();
  }
  if (t == 0) loss_mean[0] = part[0] / (float)rows;
}

// Thread t (of 256) takes rows t, t + 256, ... (ce_row), then the mean of
// the row losses (ce_mean_tree), so the mean is the same run to run.
template <int MAXC, class LAB>
__device__ __forceinline__ void ce_rows_block(const float *__restrict__ x, const LAB &lab,
                                              float *__restrict__ probs,
                                              float *__restrict__ loss_mean,
                                              float *__restrict__ seed, int rows, int cols,
                                              float scale, float *part) {
  float acc = 0.0f;
  for (int r = threadIdx.x; r < rows; r += 256)
    acc += ce_row<MAXC>(x + (long)r * cols, lab[r], probs + (long)r * cols,
                        seed + (long)r * cols, cols, scale);
  ce_mean_tree(acc, part, loss_mean, rows);
}

// ce_row by a group of W lanes (W a power of two, the group's lanes
// consecutive and all active), CPL columns a lane (cols <= W * CPL): lane q =
// threadIdx.x % W holds the logits of columns q * CPL + u in x[u] (ignored
// past cols) and gets those columns' probabilities pj[u] and seeds sj[u];
// every lane of the group returns the row's loss.  The same operations in the
// same order as ce_row, so the same bits: the maximum (order-free; NaN never
// wins, as with the serial strict compare), one expf a column, the sum of the
// exponentials in column order (each lane adds the group's values one by one
// from 0), one division a column.
template <int W, int CPL>
__device__ __forceinline__ float ce_row_group(const float (&x)[CPL], int y, int cols, float scale,
                                              float (&pj)[CPL], float (&sj)[CPL]) {
  const int q = threadIdx.x & (W - 1);
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < CPL; u++)
    if (q * CPL + u < cols && x[u] > mx) mx = x[u];
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) {
    const float t = __shfl_xor(mx, o, W);
    if (t > mx) mx = t;
  }
  float v[CPL];
  if (mx == -INFINITY) {
#pragma unroll
    for (int u = 0; u < CPL; u++) v[u] = 1.0f / (float)cols;
  } else {
    float e[CPL];
#pragma unroll
    for (int u = 0; u < CPL; u++) e[u] = q * CPL + u < cols ? expf(x[u] - mx) : 0.0f;
    float sum = 0.0f;
#pragma unroll
    for (int c = 0; c < W * CPL; c++) {
      const float t = __shfl(e[c % CPL], c / CPL, W);
      if (c < cols) sum += t;
    }
#pragma unroll
    for (int u = 0; u < CPL; u++) v[u] = e[u] / sum;
  }
  float py = 0.0f;
#pragma unroll
  for (int u = 0; u < CPL; u++) {
    const int j = q * CPL + u;
    pj[u] = v[u];
    sj[u] = (v[u] - (j == y ? 1.0f : 0.0f)) * scale;
    if (j == y) py = v[u];
  }
  // the lane that holds column y has its probability, the others 0 (and all
  // 0 for a label out of range): the largest over the group is p_y
#pragma unroll
  for (int o = W / 2; o > 0; o >>= 1) py = fmaxf(py, __shfl_xor(py, o, W));
  // opaque to the optimiser: with a label out of range the argument is the
  // constant 1e-12, and a logf folded at compile time (correctly rounded)
  // can differ in the last bit from the device logf that ce_row runs
  float a = fmaxf(py, 1e-12f);
  asm volatile("" : "+v"(a));
  return -logf(a);
}
