// Row-wise RMSNorm family (one workgroup per activation row), gfx950.
//
// Rounding points follow the reference's RMSNorm (engine.py:107-110): normalise in fp32, round
// to bf16, then multiply by the bf16 weight and round again. Residual adds round to bf16 before
// the norm; a split-K GEMV sum is rounded to bf16 before it is added (engine.py:141).
// Sums of squares are reduced in a fixed order (deterministic).
#include "common.h"

namespace dd {

constexpr int NORM_THREADS = 256;
constexpr int NORM_WAVES = NORM_THREADS / 64;
constexpr int NORM_MAXV = 16;  // values held per thread: N <= 16 * 256 = 4096

// y = bf16(bf16(v * r) * w) for the row held in v[] (element c = tid + j*NORM_THREADS; slots
// past N hold 0); r = 1/sqrt(sum(v^2)/N + eps)
__device__ __forceinline__ void norm_store(const float (&v)[NORM_MAXV], int N,
                                           const bf16* __restrict__ w, bf16* __restrict__ y,
                                           float eps, float* red) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NORM_MAXV; ++j) ss += v[j] * v[j];
  ss = block_sum<NORM_WAVES>(ss, red);
  const float r = rsqrt_ieee(ss / (float)N + eps);
#pragma unroll
  for (int j = 0; j < NORM_MAXV; ++j) {
    const int c = threadIdx.x + j * NORM_THREADS;
    if (c < N) y[c] = f2bf(rbf(v[j] * r) * bf2f(w[c]));
  }
}

// y[m] = rms(x[m]) * w                         grid (M)
__global__ void __launch_bounds__(NORM_THREADS)
rmsnorm_kernel(const bf16* __restrict__ x, const bf16* __restrict__ w, bf16* __restrict__ y, int N,
               float eps) {
  __shared__ float red[NORM_WAVES];
  const size_t row = blockIdx.x;
  float v[NORM_MAXV];
#pragma unroll
  for (int j = 0; j < NORM_MAXV; ++j) {
    const int c = threadIdx.x + j * NORM_THREADS;
    v[j] = c < N ? bf2f(x[row * N + c]) : 0.f;
  }
  norm_store(v, N, w, y + row * N, eps, red);
}

// hn = bf16(x + d); y = rms(hn) * w            grid (M)
__global__ void __launch_bounds__(NORM_THREADS)
add_rmsnorm_kernel(const bf16* __restrict__ x, const bf16* __restrict__ d, const bf16* __restrict__ w,
                   bf16* __restrict__ hn, bf16* __restrict__ y, int N, float eps) {
  __shared__ float red[NORM_WAVES];
  const size_t row = blockIdx.x;
  float v[NORM_MAXV];
#pragma unroll
  for (int j = 0; j < NORM_MAXV; ++j) {
    const int c = threadIdx.x + j * NORM_THREADS;
    v[j] = 0.f;
    if (c < N) {
      const bf16 s = f2bf(bf2f(x[row * N + c]) + bf2f(d[row * N + c]));
      hn[row * N + c] = s;
      v[j] = bf2f(s);
    }
  }
  norm_store(v, N, w, y + row * N, eps, red);
}

// Split-K epilogue: hn = bf16(h + bf16(sum_s ws[s])); y = rms(hn) * w      grid (M)
__global__ void __launch_bounds__(NORM_THREADS)
reduce_add_rmsnorm_kernel(const float* __restrict__ ws, int SK, const bf16* __restrict__ h,
                          const bf16* __restrict__ w, bf16* __restrict__ hn, bf16* __restrict__ y,
                          int M, int N, float eps) {
  __shared__ float red[NORM_WAVES];
  const size_t row = blockIdx.x;
  float v[NORM_MAXV];
#pragma unroll
  for (int j = 0; j < NORM_MAXV; ++j) {
    const int c = threadIdx.x + j * NORM_THREADS;
    v[j] = 0.f;
    if (c < N) {
      float a = 0.f;
      for (int s = 0; s < SK; ++s) a += ws[((size_t)s * M + row) * N + c];
      const bf16 t = f2bf(bf2f(h[row * N + c]) + rbf(a));
      hn[row * N + c] = t;
      v[j] = bf2f(t);
    }
  }
  norm_store(v, N, w, y + row * N, eps, red);
}

// h[m] = embed[tok[m]]; y = rms(h) * w           grid (M)
__global__ void __launch_bounds__(NORM_THREADS)
embed_rmsnorm_kernel(const int64_t* __restrict__ tok, const bf16* __restrict__ embed, int V,
                     const bf16* __restrict__ w, bf16* __restrict__ h, bf16* __restrict__ y, int N,
                     float eps, int* __restrict__ err) {
  __shared__ float red[NORM_WAVES];
  const size_t row = blockIdx.x;
  int64_t t = tok[row];
  if (t < 0 || t >= V) {  // out-of-range id: flag it and read row 0 instead of faulting
    if (threadIdx.x == 0 && err != nullptr) atomicOr(err, 1);
    t = 0;
  }
  float v[NORM_MAXV];
#pragma unroll
  for (int j = 0; j < NORM_MAXV; ++j) {
    const int c = threadIdx.x + j * NORM_THREADS;
    v[j] = 0.f;
    if (c < N) {
      const bf16 s = embed[(size_t)t * N + c];
      h[row * N + c] = s;
      v[j] = bf2f(s);
    }
  }
  norm_store(v, N, w, y + row * N, eps, red);
}

// out[m][n] = bf16(bf16(silu(g)) * u) with [g | u] = gu[m]      grid (ceil(M*I/256))
__global__ void silu_mul_kernel(const bf16* __restrict__ gu, bf16* __restrict__ out, int M, int I) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (size_t)M * I) return;
  const size_t row = i / I, col = i % I;
  const float g = bf2f(gu[row * 2 * I + col]);
  const float u = bf2f(gu[row * 2 * I + I + col]);
  const float s = rbf(g / (1.0f + expf(-g)));
  out[i] = f2bf(s * u);
}

}  // namespace dd

// ------------------------------------------------------------------------------------------
// C ABI
#include "api.h"

using namespace dd;

DD_API int dd_rmsnorm(const void* x, const void* w, void* y, int M, int N, float eps,
                      hipStream_t stream) {
  DD_REQUIRE(x && w && y && M >= 1 && N >= 1 && N <= NORM_MAXV * NORM_THREADS);
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(M), dim3(NORM_THREADS), 0, stream, (const bf16*)x,
                     (const bf16*)w, (bf16*)y, N, eps);
  return launch_status();
}

DD_API int dd_add_rmsnorm(const void* x, const void* d, const void* w, void* hn, void* y, int M,
                          int N, float eps, hipStream_t stream) {
  DD_REQUIRE(x && d && w && hn && y && M >= 1 && N >= 1 && N <= NORM_MAXV * NORM_THREADS);
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3(M), dim3(NORM_THREADS), 0, stream, (const bf16*)x,
                     (const bf16*)d, (const bf16*)w, (bf16*)hn, (bf16*)y, N, eps);
  return launch_status();
}

DD_API int dd_gemv_add_rmsnorm(const void* x, const void* W, const void* h, const void* lnw,
                               void* hn, void* y, int M, int N, int K, float eps, int splitk,
                               void* ws, hipStream_t stream) {
  DD_REQUIRE(x && W && h && lnw && hn && y && ws);
  DD_REQUIRE(M >= 1 && M <= 16 && N >= 1 && N <= NORM_MAXV * NORM_THREADS && K >= 8 && K % 8 == 0);
  DD_REQUIRE(aligned16(x) && aligned16(W));
  if (splitk <= 0) splitk = pick_splitk(M, N, K);
  const int got = launch_gemv(x, W, nullptr, ws, M, N, K, splitk, /*partials=*/true, stream);
  hipLaunchKernelGGL(reduce_add_rmsnorm_kernel, dim3(M), dim3(NORM_THREADS), 0, stream,
                     (const float*)ws, got, (const bf16*)h, (const bf16*)lnw, (bf16*)hn, (bf16*)y,
                     M, N, eps);
  return launch_status();
}

DD_API int dd_embed_rmsnorm(const int64_t* tok, const void* embed, int V, const void* w, void* h,
                            void* y, int M, int N, float eps, int* err, hipStream_t stream) {
  DD_REQUIRE(tok && embed && w && h && y && M >= 1 && V >= 1 && N >= 1 &&
             N <= NORM_MAXV * NORM_THREADS);
  hipLaunchKernelGGL(embed_rmsnorm_kernel, dim3(M), dim3(NORM_THREADS), 0, stream, tok,
                     (const bf16*)embed, V, (const bf16*)w, (bf16*)h, (bf16*)y, N, eps, err);
  return launch_status();
}

DD_API int dd_silu_mul(const void* gu, void* out, int M, int I, hipStream_t stream) {
  DD_REQUIRE(gu && out && M >= 1 && I >= 1);
  const size_t n = (size_t)M * I;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     (const bf16*)gu, (bf16*)out, M, I);
  return launch_status();
}
