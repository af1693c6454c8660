// Greedy token selection over bf16 logits, gfx950.
//
// tok[m] = argmax_v logits[m][v] with torch.argmax's rules: the first index among equal maxima,
// and NaN counts as larger than any number (first NaN wins). Optionally advances the decode
// position(s) afterwards (pos[i] += 1 for i < npos), which ends a decode step
// (engine.py:538-540).
#include "common.h"

namespace dd {

constexpr int AM_THREADS = 1024;

// a beats b?
__device__ __forceinline__ bool am_better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

__global__ void __launch_bounds__(AM_THREADS)
argmax_kernel(const bf16* __restrict__ logits, int V, int64_t* __restrict__ tok,
              int64_t* __restrict__ pos, int npos) {
  __shared__ float sv[AM_THREADS / 64];
  __shared__ int si[AM_THREADS / 64];
  const int m = blockIdx.x;
  const bf16* row = logits + (size_t)m * V;
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const int nvec = ((V & 7) == 0 && (((uintptr_t)row) & 15) == 0) ? V / 8 : 0;
  for (int c = threadIdx.x; c < nvec; c += AM_THREADS) {
    const u32x4 v = ld16_stream(row + (size_t)c * 8);
    const unsigned w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = lo_bf(w[j]), b = hi_bf(w[j]);
      if (am_better(a, c * 8 + 2 * j, bv, bi)) { bv = a; bi = c * 8 + 2 * j; }
      if (am_better(b, c * 8 + 2 * j + 1, bv, bi)) { bv = b; bi = c * 8 + 2 * j + 1; }
    }
  }
  for (int c = nvec * 8 + threadIdx.x; c < V; c += AM_THREADS) {
    const float a = bf2f(row[c]);
    if (am_better(a, c, bv, bi)) { bv = a; bi = c; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) { sv[w] = bv; si[w] = bi; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < AM_THREADS / 64; ++i)
      if (am_better(sv[i], si[i], bv, bi)) { bv = sv[i]; bi = si[i]; }
    tok[m] = bi;
    if (pos != nullptr && m < npos) pos[m] += 1;
  }
}

}  // namespace dd

// ------------------------------------------------------------------------------------------
// C ABI
#include "api.h"

using namespace dd;

DD_API int dd_argmax(const void* logits, int M, int V, int64_t* tok, int64_t* pos, int npos,
                     hipStream_t stream) {
  DD_REQUIRE(logits && tok && M >= 1 && V >= 1 && npos >= 0);
  hipLaunchKernelGGL(argmax_kernel, dim3(M), dim3(AM_THREADS), 0, stream, (const bf16*)logits, V,
                     tok, pos, npos);
  return launch_status();
}
