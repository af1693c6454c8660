// Greedy token selection over bf16 logits, gfx950.
//
// tok[m] = argmax_v logits[m][v] with torch.argmax's rules: the first index among equal maxima,
// and NaN counts as larger than any number (first NaN wins). Optionally advances the decode
// position(s) afterwards (pos[i] += 1 for i < npos), which ends a decode step
// (engine.py:538-540).
#include "common.h"

namespace dd {

constexpr int AM_THREADS = 256;
constexpr int AM_CHUNK = 4096;  // logits per workgroup

// a beats b?
__device__ __forceinline__ bool am_better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

__device__ __forceinline__ void am_wave_reduce(float& bv, int& bi) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
}

// grid (M, P): workgroup (m, p) finds the best of logits[m][p*AM_CHUNK ..) and stores it; the
// last of the P workgroups of row m (per-row counter) reduces the P candidates in chunk order,
// writes tok[m] and advances pos[m] (m < npos). ws: [M][P][2] (value, index).
__global__ void __launch_bounds__(AM_THREADS)
argmax_kernel(const bf16* __restrict__ logits, int V, int64_t* __restrict__ tok,
              int64_t* __restrict__ pos, int npos, float* __restrict__ ws,
              int* __restrict__ counters) {
  __shared__ float sv[AM_THREADS / 64];
  __shared__ int si[AM_THREADS / 64];
  __shared__ int flag;
  const int m = blockIdx.x, p = blockIdx.y, P = gridDim.y;
  const bf16* row = logits + (size_t)m * V;
  const int c0 = p * AM_CHUNK, c1 = min(V, c0 + AM_CHUNK);
  float bv = -INFINITY;
  int bi = 0x7fffffff;
  const bool vec = ((V & 7) == 0) && ((((uintptr_t)row) & 15) == 0);
  if (vec) {
    for (int c = c0 + threadIdx.x * 8; c < c1; c += AM_THREADS * 8) {
      const u32x4 v = ld16_stream(row + c);
      const unsigned w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float a = lo_bf(w[j]), b2 = hi_bf(w[j]);
        if (am_better(a, c + 2 * j, bv, bi)) { bv = a; bi = c + 2 * j; }
        if (am_better(b2, c + 2 * j + 1, bv, bi)) { bv = b2; bi = c + 2 * j + 1; }
      }
    }
  } else {
    for (int c = c0 + threadIdx.x; c < c1; c += AM_THREADS) {
      const float a = bf2f(row[c]);
      if (am_better(a, c, bv, bi)) { bv = a; bi = c; }
    }
  }
  am_wave_reduce(bv, bi);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) { sv[w] = bv; si[w] = bi; }
  __syncthreads();
  const rsrc_t wsr = make_rsrc(ws, (unsigned)((size_t)gridDim.x * P * 8));
  if (threadIdx.x == 0) {
    for (int i = 1; i < AM_THREADS / 64; ++i)
      if (am_better(sv[i], si[i], bv, bi)) { bv = sv[i]; bi = si[i]; }
    stc_f32(wsr, (unsigned)((m * P + p) * 8), bv);
    stc_u32(wsr, (unsigned)((m * P + p) * 8 + 4), (unsigned)bi);
  }
  if (!arrive_last(counters + m, P, &flag)) return;
  if (threadIdx.x < 64) {
    // lane q takes candidates q, q+64, ...; then a wave reduction keeps chunk order on ties
    float best = -INFINITY;
    int besti = 0x7fffffff;
    for (int q = threadIdx.x; q < P; q += 64) {
      const float v = ldc_f32(wsr, (unsigned)((m * P + q) * 8));
      const int i = (int)ldc_u32(wsr, (unsigned)((m * P + q) * 8 + 4));
      if (am_better(v, i, best, besti)) { best = v; besti = i; }
    }
    am_wave_reduce(best, besti);
    if (threadIdx.x == 0) {
      tok[m] = besti;
      if (pos != nullptr && m < npos) pos[m] += 1;
    }
  }
}

}  // namespace dd

// ------------------------------------------------------------------------------------------
// C ABI
#include "api.h"

using namespace dd;

static int am_parts(int V) { return (V + AM_CHUNK - 1) / AM_CHUNK; }

DD_API size_t dd_argmax_ws_bytes(int M, int V) { return (size_t)M * am_parts(V) * 2 * sizeof(float); }

DD_API int dd_argmax(const void* logits, int M, int V, int64_t* tok, int64_t* pos, int npos,
                     void* ws, int* counters, hipStream_t stream) {
  DD_REQUIRE(logits && tok && ws && counters && M >= 1 && V >= 1 && npos >= 0);
  hipLaunchKernelGGL(argmax_kernel, dim3(M, am_parts(V)), dim3(AM_THREADS), 0, stream,
                     (const bf16*)logits, V, tok, pos, npos, (float*)ws, counters);
  return launch_status();
}
