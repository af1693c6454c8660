// Host-side helpers shared by the C-ABI entry points (see include/dryft_decode.h).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/dryft_decode.h"

#define DD_API extern "C" __attribute__((visibility("default")))

namespace dd {

constexpr int DD_ABI_VERSION = 15;

inline bool aligned16(const void* p) { return (((uintptr_t)p) & 15u) == 0; }

// Launch result: the error of the last launch on this thread (0 when it went through).
inline int launch_status() { return (int)hipGetLastError(); }

// GEMV launch helpers (gemv.hip): split-K choice, k per split, workspace size, and the launch
// (h != nullptr selects the residual + RMSNorm epilogue; returns the number of splits).
int pick_splitk(int M, int N, int K);
int kps_for(int K, int sk);
int gemv_nsplit(int K, int sk);
size_t gemv_ws_floats(int M, int N, int K, int sk, bool add_rms);
int launch_gemv(const void* x, const void* W, void* y, void* ws, int* counters, int M, int N,
                int K, int sk, const void* h, const void* lnw, void* hn, float eps,
                hipStream_t stream);

}  // namespace dd

#define DD_REQUIRE(cond)                         \
  do {                                           \
    if (!(cond)) return (int)hipErrorInvalidValue; \
  } while (0)
