// Phase timestamps for tuning.  Built with -DTT_PHASE_PROBE, a file that
// says TT_PROBE_DEFINE(name) gets its own device array and an exported
// tt_probe_read_<name>(host, n) that copies it back, and TT_PROBE(kid, i)
// records thread 0's s_memrealtime (100 MHz) at point i (< 16) of workgroup
// blockIdx.x (< 1024) of kernel kid (< 4) of that file (TT_PROBE_WAVE: lane
// 0 of each wave).  Without the define
// both expand to nothing.
#pragma once
#include <hip/hip_runtime.h>

#ifdef TT_PHASE_PROBE
#define TT_PROBE_DEFINE(name)                                                           \
  namespace {                                                                           \
  __device__ unsigned long long tt_probe_ts[4 * 1024 * 16];                             \
  }                                                                                     \
  extern "C" int tt_probe_read_##name(unsigned long long *h, int n) {                   \
    return hipMemcpyFromSymbol(h, HIP_SYMBOL(tt_probe_ts),                              \
                               sizeof(unsigned long long) * n) == hipSuccess            \
               ? 0                                                                      \
               : -1;                                                                    \
  }
#define TT_PROBE(kid, i)                                                                \
  do {                                                                                  \
    if (threadIdx.x == 0 && blockIdx.x < 1024)                                          \
      tt_probe_ts[((kid) * 1024 + blockIdx.x) * 16 + (i)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
// the same from lane 0 of every wave (point i chosen per wave by the caller)
#define TT_PROBE_WAVE(kid, i)                                                           \
  do {                                                                                  \
    if ((threadIdx.x & 63) == 0 && blockIdx.x < 1024)                                   \
      tt_probe_ts[((kid) * 1024 + blockIdx.x) * 16 + (i)] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define TT_PROBE_DEFINE(name)
#define TT_PROBE(kid, i) \
  do {                   \
  } while (0)
#define TT_PROBE_WAVE(kid, i) \
  do {                        \
  } while (0)
#endif
