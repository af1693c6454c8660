// Skinny GEMV family for decode (M <= 16 activation rows), gfx950.
//
//   out[m][n] = sum_k x[m][k] * W[n][k]          (F.linear semantics, W row-major [N, K])
//
// Design
//  * A workgroup of 4 waves owns one 16-row tile of W (NR tiles for the fused gate/up variant)
//    over a K range. The 4 waves interleave over 32-wide k-steps, so at any moment the
//    workgroup streams 256 contiguous bytes of every W row it owns.
//  * Each k-step is one v_mfma_f32_16x16x32_bf16: A = 16 W rows x 32 k (each lane loads 16
//    contiguous bytes straight from HBM into the A operand), B = x^T (32 k x 16 activation rows;
//    rows >= M are clamped reads whose output columns are discarded). MFMA makes the
//    contraction free at every M <= 16; the kernel is bound by the weight stream alone.
//  * fp32 accumulation. Cross-wave reduction through LDS in fixed wave order, split-K partials
//    summed in fixed split order: results are deterministic run to run.
//  * U k-steps of loads are issued before the matching MFMAs so that each wave keeps
//    U x (NR + 1) 16-byte loads per lane in flight.
#include "common.h"

namespace dd {

constexpr int GEMV_WAVES = 4;
constexpr int GEMV_THREADS = GEMV_WAVES * 64;

// Accumulate NR 16-row tiles over k in [k0, k1). W tile t starts at row rows[t].
// Requires K % 8 == 0 (16-byte aligned rows); k0 is a multiple of 32.
template <int NR, int U>
__device__ __forceinline__ void gemv_accumulate(const bf16* __restrict__ x, int M, int K,
                                                const bf16* __restrict__ W, const int* rows,
                                                int nrows_total, int k0, int k1, f32x4 acc[NR]) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int m = r < M ? r : M - 1;
  const bf16* xp = x + (size_t)m * K + g * 8;
  const bf16* wp[NR];
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    int row = rows[t] + r;
    row = row < nrows_total ? row : nrows_total - 1;
    wp[t] = W + (size_t)row * K + g * 8;
  }
  const int nfull = (k1 - k0) >> 5;  // complete 32-wide k-steps
  int ks = wave;
  // main loop: U k-steps per wave per iteration
  for (; ks + (U - 1) * GEMV_WAVES < nfull; ks += U * GEMV_WAVES) {
    u32x4 wv[U][NR], xv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = k0 + (ks + u * GEMV_WAVES) * 32;
#pragma unroll
      for (int t = 0; t < NR; ++t) wv[u][t] = ld16_stream(wp[t] + k);
      xv[u] = ld16(xp + k);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int t = 0; t < NR; ++t) acc[t] = mfma16x16x32(wv[u][t], xv[u], acc[t]);
  }
  for (; ks < nfull; ks += GEMV_WAVES) {
    const int k = k0 + ks * 32;
    u32x4 xv = ld16(xp + k);
#pragma unroll
    for (int t = 0; t < NR; ++t) acc[t] = mfma16x16x32(ld16_stream(wp[t] + k), xv, acc[t]);
  }
  // ragged tail (K range not a multiple of 32): one partial k-step, owned by wave (nfull % 4)
  const int ktail = k0 + nfull * 32;
  if (ktail < k1 && wave == (nfull & (GEMV_WAVES - 1))) {
    const bool ok = ktail + g * 8 < k1;  // 8-element chunks are whole because K % 8 == 0
    u32x4 zero = {0u, 0u, 0u, 0u};
    u32x4 xv = ok ? ld16(xp + ktail) : zero;
#pragma unroll
    for (int t = 0; t < NR; ++t) acc[t] = mfma16x16x32(ok ? ld16_stream(wp[t] + ktail) : zero, xv, acc[t]);
  }
}

// Sum the 4 waves' accumulators in wave order; result valid in wave 0 (returned there).
template <int NR>
__device__ __forceinline__ void gemv_wave_reduce(f32x4 acc[NR], float* red /* [3][NR][64][4] */) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < NR; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(((wave - 1) * NR + t) * 64 + lane) * 4 + i] = acc[t][i];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 1; w < GEMV_WAVES; ++w)
#pragma unroll
      for (int t = 0; t < NR; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] += red[(((w - 1) * NR + t) * 64 + lane) * 4 + i];
  }
}

// grid (ceil(N/16), SK). partials == 0 (only with SK == 1): y[m*ldy + n] = bf16(sum);
// otherwise fp32 ws[(s*M + m)*N + n] = sum over split s.
template <int U>
__global__ void __launch_bounds__(GEMV_THREADS)
gemv_kernel(const bf16* __restrict__ x, const bf16* __restrict__ W, bf16* __restrict__ y,
            float* __restrict__ ws, int M, int N, int K, int kps, int ldy, int partials) {
  __shared__ float red[(GEMV_WAVES - 1) * 64 * 4];
  const int n0 = blockIdx.x * 16;
  const int s = blockIdx.y;
  const int k0 = s * kps;
  const int k1 = min(K, k0 + kps);
  f32x4 acc[1] = {{0.f, 0.f, 0.f, 0.f}};
  int rows[1] = {n0};
  gemv_accumulate<1, U>(x, M, K, W, rows, N, k0, k1, acc);
  gemv_wave_reduce<1>(acc, red);
  if ((threadIdx.x >> 6) != 0) return;
  const int lane = threadIdx.x & 63;
  const int m = lane & 15;
  if (m >= M) return;
  const int nb = n0 + (lane >> 4) * 4;
  if (!partials) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (nb + i < N) y[(size_t)m * ldy + nb + i] = f2bf(acc[0][i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (nb + i < N) ws[((size_t)s * M + m) * N + nb + i] = acc[0][i];
  }
}

// Fused gate/up GEMV + SiLU epilogue. Wgu = [gate (I rows); up (I rows)], K columns.
// out[m][n] = bf16( bf16(silu(bf16 g)) * bf16 u )  -- the rounding points of
// silu_mul(linear(x, wgu)) in the reference (engine.py:144-146, fused.py:677-682).
template <int U>
__global__ void __launch_bounds__(GEMV_THREADS)
gemv_silu_kernel(const bf16* __restrict__ x, const bf16* __restrict__ Wgu, bf16* __restrict__ out,
                 int M, int I, int K) {
  __shared__ float red[(GEMV_WAVES - 1) * 2 * 64 * 4];
  const int n0 = blockIdx.x * 16;
  f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
  // Rows past the end of a partial last tile read neighbouring valid rows; their outputs are
  // never stored (nb + i < I below).
  int rows[2] = {n0, I + n0};
  gemv_accumulate<2, U>(x, M, K, Wgu, rows, 2 * I, 0, K, acc);
  gemv_wave_reduce<2>(acc, red);
  if ((threadIdx.x >> 6) != 0) return;
  const int lane = threadIdx.x & 63;
  const int m = lane & 15;
  if (m >= M) return;
  const int nb = n0 + (lane >> 4) * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (nb + i < I) {
      const float gg = rbf(acc[0][i]);
      const float uu = rbf(acc[1][i]);
      const float sg = rbf(gg / (1.0f + expf(-gg)));
      out[(size_t)m * I + nb + i] = f2bf(sg * uu);
    }
  }
}

// Sum SK fp32 partials (fixed order) -> bf16.  grid ceil(M*N/256)
__global__ void splitk_reduce_kernel(const float* __restrict__ ws, bf16* __restrict__ y, int SK,
                                     int MN) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= MN) return;
  float a = 0.f;
  for (int s = 0; s < SK; ++s) a += ws[(size_t)s * MN + i];
  y[i] = f2bf(a);
}

}  // namespace dd

// ------------------------------------------------------------------------------------------
// C ABI
#include "api.h"

namespace dd {

// Split-K heuristic for the MI355X (256 CUs): keep one 16-row tile per workgroup and split K
// until the grid has at least ~2 workgroups per CU, keeping >= 512 k per split.
int pick_splitk(int M, int N, int K) {
  (void)M;
  const int tiles = (N + 15) / 16;
  int sk = 1;
  while (tiles * sk < 512 && K / (sk * 2) >= 512 && sk < 8) sk *= 2;
  return sk;
}

int kps_for(int K, int sk) { return ((K + sk - 1) / sk + 31) / 32 * 32; }

int launch_gemv(const void* x, const void* W, void* y, void* ws, int M, int N, int K, int sk,
                bool partials, hipStream_t stream) {
  const int kps = kps_for(K, sk);
  const int nsplit = (K + kps - 1) / kps;
  dim3 grid((N + 15) / 16, nsplit);
  hipLaunchKernelGGL(gemv_kernel<8>, grid, dim3(GEMV_THREADS), 0, stream, (const bf16*)x,
                     (const bf16*)W, (bf16*)y, (float*)ws, M, N, K, kps, N,
                     (int)(partials || nsplit > 1));
  return nsplit;
}

}  // namespace dd

using namespace dd;

DD_API int dd_abi_version(void) { return DD_ABI_VERSION; }

DD_API int dd_gemv_splitk(int M, int N, int K) { return pick_splitk(M, N, K); }

// Bytes of fp32 partials for a split (at least one split's worth, which the fused
// add+norm path always uses).
DD_API size_t dd_gemv_ws_bytes(int M, int N, int K, int splitk) {
  if (splitk <= 0) splitk = pick_splitk(M, N, K);
  const int kps = kps_for(K, splitk);
  const int nsplit = (K + kps - 1) / kps;
  return (size_t)(nsplit < 1 ? 1 : nsplit) * M * N * sizeof(float);
}

DD_API int dd_gemv(const void* x, const void* W, void* y, int M, int N, int K, int splitk, void* ws,
                   hipStream_t stream) {
  DD_REQUIRE(x && W && y && M >= 1 && M <= 16 && N >= 1 && K >= 8 && K % 8 == 0);
  DD_REQUIRE(aligned16(x) && aligned16(W));
  if (splitk <= 0) splitk = pick_splitk(M, N, K);
  const int nsplit = (K + kps_for(K, splitk) - 1) / kps_for(K, splitk);
  DD_REQUIRE(nsplit == 1 || ws != nullptr);
  launch_gemv(x, W, y, ws, M, N, K, splitk, /*partials=*/false, stream);
  if (nsplit > 1) {
    const int MN = M * N;
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((MN + 255) / 256), dim3(256), 0, stream,
                       (const float*)ws, (bf16*)y, nsplit, MN);
  }
  return launch_status();
}

DD_API int dd_gate_up_silu(const void* x, const void* Wgu, void* out, int M, int I, int K,
                           hipStream_t stream) {
  DD_REQUIRE(x && Wgu && out && M >= 1 && M <= 16 && I >= 1 && K >= 8 && K % 8 == 0);
  DD_REQUIRE(aligned16(x) && aligned16(Wgu));
  hipLaunchKernelGGL(gemv_silu_kernel<8>, dim3((I + 15) / 16), dim3(GEMV_THREADS), 0, stream,
                     (const bf16*)x, (const bf16*)Wgu, (bf16*)out, M, I, K);
  return launch_status();
}
