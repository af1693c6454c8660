// Tensorwise fp8 (OCP e4m3, the gfx950 format) quantisation of prefill GEMM activations
// (fused.py:130-149: quant_fp8_tensorwise), two launches:
//   amax_kernel   per-workgroup max |x| over a grid-stride range -> partials[gridDim.x]
//   quant_kernel  every workgroup folds the partials (amax, clamped to >= 1e-6; a NaN in x
//                 makes it NaN, as torch's amax and clamp do), block 0 writes
//                 scale = amax / 448 (the GEMM's dequantisation factor); q = e4m3(x * (448 / amax))
// x is bf16, read as 16-byte vectors (8 elements); the conversion rounds to nearest even and
// turns magnitudes past 464 (half-way to the first value past the largest finite 448, which
// itself rounds to 448) into NaN, as torch's float -> float8_e4m3fn cast does (inputs here are
// scaled to <= 448).
#include "common.h"

namespace dd {
namespace f8 {

constexpr int THREADS = 256;
constexpr int MAXBLK = 1024;

// max that keeps a NaN (torch's amax and clamp propagate it: a NaN anywhere in x makes the scale,
// and so every quantised value, NaN)
__device__ __forceinline__ float nanmax(float a, float b) { return (a != a || a > b) ? a : b; }
__device__ __forceinline__ float wave_nanmax(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = nanmax(v, __shfl_xor(v, o, 64));
  return v;
}

// fp32 -> e4m3fn bits (1 sign, 4 exponent bits with bias 7, 3 mantissa bits; 0x7f/0xff NaN)
__device__ __forceinline__ unsigned e4m3(float x) {
  const unsigned u = __float_as_uint(x);
  const unsigned sign = (u >> 24) & 0x80u;
  const float a = fabsf(x);
  if (!(a <= 464.0f)) return sign | 0x7fu;                 // NaN, inf, out of range (464: 448)
  if (a < 0.015625f) {                                      // below 2^-6: multiples of 2^-9
    const float q = rintf(a * 512.0f);                      // exact scaling, ties to even
    return sign | (unsigned)q;                              // q = 8 is the smallest normal
  }
  const unsigned ua = __float_as_uint(a);
  const unsigned r = (ua + 0x7ffffu + ((ua >> 20) & 1u)) & 0xfff00000u;   // 3 mantissa bits, RNE
  const int e = (int)(r >> 23) - 127;                       // -6 .. 8
  return sign | (unsigned)((e + 7) << 3) | ((r >> 20) & 7u);
}

__global__ void __launch_bounds__(THREADS)
amax_kernel(const u32x4* __restrict__ x, size_t n8, float* __restrict__ partials) {
  __shared__ float red[THREADS / 64];
  float m = 0.f;
  for (size_t i = blockIdx.x * (size_t)THREADS + threadIdx.x; i < n8; i += (size_t)gridDim.x * THREADS) {
    const u32x4 v = x[i];
    const unsigned w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) m = nanmax(m, nanmax(fabsf(lo_bf(w[j])), fabsf(hi_bf(w[j]))));
  }
  m = wave_nanmax(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = red[0];
    for (int k = 1; k < THREADS / 64; ++k) t = nanmax(t, red[k]);
    partials[blockIdx.x] = t;
  }
}

__global__ void __launch_bounds__(THREADS)
quant_kernel(const u32x4* __restrict__ x, size_t n8, const float* __restrict__ partials, int np,
             uint2* __restrict__ out, float* __restrict__ scale) {
  __shared__ float red[THREADS / 64];
  float m = 0.f;
  for (int i = threadIdx.x; i < np; i += THREADS) m = nanmax(m, partials[i]);
  m = wave_nanmax(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  float amax = red[0];
  for (int k = 1; k < THREADS / 64; ++k) amax = nanmax(amax, red[k]);
  amax = nanmax(amax, 1e-6f);
  const float inv = 448.0f / amax;
  if (blockIdx.x == 0 && threadIdx.x == 0) scale[0] = amax / 448.0f;
  for (size_t i = blockIdx.x * (size_t)THREADS + threadIdx.x; i < n8; i += (size_t)gridDim.x * THREADS) {
    const u32x4 v = x[i];
    const unsigned w[4] = {v.x, v.y, v.z, v.w};
    unsigned q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      q[j] = e4m3(lo_bf(w[j]) * inv) | (e4m3(hi_bf(w[j]) * inv) << 8);
    out[i] = make_uint2(q[0] | (q[1] << 16), q[2] | (q[3] << 16));
  }
}

inline int blocks_for(size_t n8) {
  const size_t b = (n8 + THREADS * 8 - 1) / (THREADS * 8);   // about 8 vectors per thread
  return (int)(b < 1 ? 1 : b > MAXBLK ? MAXBLK : b);
}

}  // namespace f8
}  // namespace dd

// ------------------------------------------------------------------------------------------
// C ABI
#include "api.h"

using namespace dd;

DD_API size_t dd_fp8_quant_ws_bytes(size_t n) {
  return (size_t)f8::blocks_for(n / 8) * sizeof(float);
}

DD_API int dd_fp8_quant(const void* x, size_t n, void* out, float* scale, void* ws,
                        hipStream_t stream) {
  DD_REQUIRE(x && out && scale && ws && n >= 8 && n % 8 == 0);
  DD_REQUIRE(aligned16(x) && (((uintptr_t)out) & 7u) == 0);
  const size_t n8 = n / 8;
  const int nb = f8::blocks_for(n8);
  hipLaunchKernelGGL(f8::amax_kernel, dim3(nb), dim3(f8::THREADS), 0, stream, (const u32x4*)x, n8,
                     (float*)ws);
  hipLaunchKernelGGL(f8::quant_kernel, dim3(nb), dim3(f8::THREADS), 0, stream, (const u32x4*)x, n8,
                     (const float*)ws, nb, (uint2*)out, scale);
  return launch_status();
}
