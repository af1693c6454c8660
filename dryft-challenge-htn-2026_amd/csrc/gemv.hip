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

// Epilogue modes of gemv_kernel.
//   GEMV_OUT      y = bf16(x.W^T)
//   GEMV_ADD_RMS  hn = bf16(h + bf16(x.W^T)); y = bf16(bf16(hn * r) * lnw),
//                 r = 1/sqrt(mean(hn^2) + eps) over each full row (engine.py:140-142)
// grid (ceil(N/16), nsplit). With nsplit > 1 every split stores its fp32 partial tile and the
// last split to arrive for a tile (per-tile counter) sums the partials in split order. In
// GEMV_ADD_RMS the tile finisher also adds the residual and stores the tile's per-row sum of
// squares; the last tile to finish (global counter) normalises every row.
// Workspace (floats): partials [nsplit][M][N] | hn32 [M][N] | ss [ntiles][M].
// Counters: [ntiles] per tile, then 1 global; zero before the launch, zero after it.
enum { GEMV_OUT = 0, GEMV_ADD_RMS = 1 };

template <int U, int MODE>
__global__ void __launch_bounds__(GEMV_THREADS)
gemv_kernel(const bf16* __restrict__ x, const bf16* __restrict__ W, bf16* __restrict__ y,
            float* __restrict__ ws, int* __restrict__ counters, int M, int N, int K, int kps,
            const bf16* __restrict__ h, const bf16* __restrict__ lnw, bf16* __restrict__ hn,
            float eps) {
  __shared__ float red[(GEMV_WAVES - 1) * 64 * 4];
  __shared__ float tile[16][17];
  __shared__ float rrow[16];
  __shared__ int flag;
  const int n0 = blockIdx.x * 16;
  const int s = blockIdx.y;
  const int nsplit = gridDim.y;
  const int ntiles = gridDim.x;
  const int k0 = s * kps;
  const int k1 = min(K, k0 + kps);
  f32x4 acc[1] = {{0.f, 0.f, 0.f, 0.f}};
  int rows[1] = {n0};
  gemv_accumulate<1, U>(x, M, K, W, rows, N, k0, k1, acc);
  gemv_wave_reduce<1>(acc, red);
  const int lane = threadIdx.x & 63;
  if (threadIdx.x < 64) {
#pragma unroll
    for (int i = 0; i < 4; ++i) tile[lane & 15][(lane >> 4) * 4 + i] = acc[0][i];
  }
  __syncthreads();
  // one tile element per thread: row m, column n0 + c
  const int m = threadIdx.x >> 4, c = threadIdx.x & 15, n = n0 + c;
  const bool mine = m < M && n < N;
  float v = mine ? tile[m][c] : 0.f;
  const unsigned MN = (unsigned)(M * N);
  const rsrc_t wsr = make_rsrc(ws, (unsigned)(((MODE == GEMV_ADD_RMS) ? (size_t)nsplit * MN + MN / 2 + 1 + (size_t)ntiles * M
                                                                       : (size_t)nsplit * MN) * 4));
  if (nsplit > 1) {
    if (mine) stc_f32(wsr, (unsigned)(((size_t)s * M + m) * N + n) * 4, v);
    if (!arrive_last(counters + blockIdx.x, nsplit, &flag)) return;
    float part[16];
#pragma unroll
    for (int sp = 0; sp < 16; ++sp)
      part[sp] = (mine && sp < nsplit) ? ldc_f32(wsr, (unsigned)(((size_t)sp * M + m) * N + n) * 4) : 0.f;
    v = 0.f;
#pragma unroll
    for (int sp = 0; sp < 16; ++sp) v += part[sp];  // split order
  }
  if (MODE == GEMV_OUT) {
    if (mine) y[(size_t)m * N + n] = f2bf(v);
    return;
  }
  // GEMV_ADD_RMS: residual, tile sum of squares, then the last tile normalises every row.
  // hn goes out twice: plainly (the returned tensor) and through sc1 as bf16 into the
  // workspace (read back by the finishing workgroup).
  const unsigned hn_off = (unsigned)((size_t)nsplit * MN * 4);          // bf16 [M][N]
  const unsigned ss_off = hn_off + ((MN * 2 + 3) & ~3u);                 // f32 [ntiles][M]
  float hv = 0.f;
  if (mine) {
    const bf16 hb = f2bf(bf2f(h[(size_t)m * N + n]) + rbf(v));
    hv = bf2f(hb);
    hn[(size_t)m * N + n] = hb;
    stc_b16(wsr, hn_off + (unsigned)((size_t)m * N + n) * 2, hb);
  }
  float q = hv * hv;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);  // sum over the 16 columns, fixed order
  if (c == 0 && m < M) stc_f32(wsr, ss_off + (unsigned)((size_t)blockIdx.x * M + m) * 4, q);
  if (!arrive_last(counters + ntiles, ntiles, &flag)) return;
  if (threadIdx.x < 16 * 16) {
    // rows split over 16 lanes each: lane j of row m sums tiles j, j+16, ... then a 16-lane sum
    const int mm = threadIdx.x >> 4, j = threadIdx.x & 15;
    float t = 0.f;
    if (mm < M)
      for (int tl = j; tl < ntiles; tl += 16) t += ldc_f32(wsr, ss_off + (unsigned)(tl * M + mm) * 4);
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) t += __shfl_xor(t, o, 64);
    if (j == 0 && mm < M) rrow[mm] = rsqrt_ieee(t / (float)N + eps);
  }
  __syncthreads();
  // y = bf16(bf16(hn * r) * lnw), 8 elements per 16-byte load (N % 8 == 0 here: K-side checks
  // guarantee 16-byte rows; the scalar tail handles any remainder)
  const bool al = ((((uintptr_t)y) | ((uintptr_t)lnw)) & 15) == 0;
  const int nvec = (N % 8 == 0 && al) ? (int)(MN / 8) : 0;
  for (int e = threadIdx.x; e < nvec; e += GEMV_THREADS) {
    const u32x4 hv8 = ldc_b128(wsr, hn_off + (unsigned)e * 16);
    const int mm = (e * 8) / N, nn = (e * 8) % N;
    const u32x4 w8 = ld16(lnw + nn);
    const float r = rrow[mm];
    const unsigned hw[4] = {hv8.x, hv8.y, hv8.z, hv8.w}, ww[4] = {w8.x, w8.y, w8.z, w8.w};
    unsigned o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned lo = f2bf(rbf(lo_bf(hw[j]) * r) * lo_bf(ww[j]));
      const unsigned hi = f2bf(rbf(hi_bf(hw[j]) * r) * hi_bf(ww[j]));
      o[j] = lo | (hi << 16);
    }
    *(u32x4*)(y + (size_t)e * 8) = u32x4{o[0], o[1], o[2], o[3]};
  }
  for (int e = nvec * 8 + threadIdx.x; e < (int)MN; e += GEMV_THREADS) {
    const int mm = e / N, nn = e % N;
    const unsigned pair = ldc_u32(wsr, hn_off + ((unsigned)e * 2 & ~3u));
    const float hx = (e & 1) ? hi_bf(pair) : lo_bf(pair);
    y[e] = f2bf(rbf(hx * rrow[mm]) * bf2f(lnw[nn]));
  }
}

// GEMV_OUT without a K split, NR 16-row tiles of W per workgroup: each lane's x load feeds NR
// MFMAs instead of one (at M = 16 the x operand is as many bytes per k-step as one W tile).
// Every tile's k order and wave-reduction order are those of gemv_kernel, so the outputs are
// the same bits. Rows past N are clamped reads whose outputs are not stored.
template <int U, int NR>
__global__ void __launch_bounds__(GEMV_THREADS)
gemv_multi_kernel(const bf16* __restrict__ x, const bf16* __restrict__ W, bf16* __restrict__ y,
                  int M, int N, int K) {
  __shared__ float red[(GEMV_WAVES - 1) * NR * 64 * 4];
  const int n0 = blockIdx.x * 16 * NR;
  f32x4 acc[NR];
  int rows[NR];
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    rows[t] = n0 + 16 * t;
  }
  gemv_accumulate<NR, U>(x, M, K, W, rows, N, 0, K, acc);
  gemv_wave_reduce<NR>(acc, red);
  if ((threadIdx.x >> 6) != 0) return;
  const int lane = threadIdx.x & 63;
  const int m = lane & 15;
  if (m >= M) return;
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    const int nb = n0 + 16 * t + (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (nb + i < N) y[(size_t)m * N + nb + i] = f2bf(acc[t][i]);
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

}  // namespace dd

// ------------------------------------------------------------------------------------------
// C ABI
#include "api.h"

namespace dd {

// Split-K heuristic for the MI355X (256 CUs): keep one 16-row tile per workgroup and split K
// until the grid has at least ~2 workgroups per CU, keeping >= 512 k per split; grids still
// under 1024 workgroups split further while >= 1024 k per split remain (down, 2560 x 9728: 8
// splits instead of 4, 15.8 -> 15.3 us at M = 1, 21.8 -> 20.3 at M = 16, graph-timed).
int pick_splitk(int M, int N, int K) {
  (void)M;
  const int tiles = (N + 15) / 16;
  int sk = 1;
  while (sk < 8 && ((tiles * sk < 512 && K / (sk * 2) >= 512) ||
                    (tiles * sk < 1024 && K / (sk * 2) >= 1024)))
    sk *= 2;
  return sk;
}

// 16-row tiles per workgroup of an unsplit GEMV_OUT launch: at M >= 8 the most (4, 2, 1) that
// still leave 1024 workgroups. Graph-timed on MI355X, lm_head (151936 x 2560): M = 16 269 -> 223
// us with four tiles; M = 1 177 -> 200 us (one tile kept there: x is one row, its loads hit the
// same lines, and four times the workgroups keep more loads in flight).
int gemv_tiles_per_wg(int M, int N) {
  const int tiles = (N + 15) / 16;
  if (M < 8) return 1;
  return tiles / 4 >= 1024 ? 4 : tiles / 2 >= 1024 ? 2 : 1;
}

int kps_for(int K, int sk) { return ((K + sk - 1) / sk + 31) / 32 * 32; }

int gemv_nsplit(int K, int sk) {
  const int kps = kps_for(K, sk);
  return (K + kps - 1) / kps;
}

size_t gemv_ws_floats(int M, int N, int K, int sk, bool add_rms) {
  const int nsplit = gemv_nsplit(K, sk);
  size_t f = nsplit > 1 ? (size_t)nsplit * M * N : 0;
  // add_rms: partials | hn as bf16 (rounded up to whole floats) | per-tile sums of squares
  if (add_rms) f = (size_t)nsplit * M * N + ((size_t)M * N + 1) / 2 + (size_t)((N + 15) / 16) * M;
  return f;
}

int launch_gemv(const void* x, const void* W, void* y, void* ws, int* counters, int M, int N,
                int K, int sk, const void* h, const void* lnw, void* hn, float eps,
                hipStream_t stream) {
  const int kps = kps_for(K, sk);
  const int nsplit = (K + kps - 1) / kps;
  dim3 grid((N + 15) / 16, nsplit);
  const int nr = h == nullptr && nsplit == 1 ? gemv_tiles_per_wg(M, N) : 1;
  if (nr == 4)
    hipLaunchKernelGGL((gemv_multi_kernel<4, 4>), dim3((N + 63) / 64), dim3(GEMV_THREADS), 0,
                       stream, (const bf16*)x, (const bf16*)W, (bf16*)y, M, N, K);
  else if (nr == 2)
    hipLaunchKernelGGL((gemv_multi_kernel<8, 2>), dim3((N + 31) / 32), dim3(GEMV_THREADS), 0, stream,
                       (const bf16*)x, (const bf16*)W, (bf16*)y, M, N, K);
  else if (h == nullptr)
    hipLaunchKernelGGL((gemv_kernel<8, GEMV_OUT>), grid, dim3(GEMV_THREADS), 0, stream,
                       (const bf16*)x, (const bf16*)W, (bf16*)y, (float*)ws, counters, M, N, K,
                       kps, nullptr, nullptr, nullptr, 0.f);
  else
    hipLaunchKernelGGL((gemv_kernel<8, GEMV_ADD_RMS>), grid, dim3(GEMV_THREADS), 0, stream,
                       (const bf16*)x, (const bf16*)W, (bf16*)y, (float*)ws, counters, M, N, K,
                       kps, (const bf16*)h, (const bf16*)lnw, (bf16*)hn, eps);
  return nsplit;
}

}  // namespace dd

using namespace dd;

DD_API int dd_abi_version(void) { return DD_ABI_VERSION; }

DD_API int dd_gemv_splitk(int M, int N, int K) { return pick_splitk(M, N, K); }

// Bytes of fp32 partials for a split (at least one split's worth, which the fused
// add+norm path always uses).
// Bytes of fp32 workspace dd_gemv needs (0 without split-K).
DD_API size_t dd_gemv_ws_bytes(int M, int N, int K, int splitk) {
  if (splitk <= 0) splitk = pick_splitk(M, N, K);
  return gemv_ws_floats(M, N, K, splitk, false) * sizeof(float);
}

// Ints of zeroed counters dd_gemv / dd_gemv_add_rmsnorm need: one per 16-column tile + 1.
DD_API int dd_gemv_counters(int N) { return (N + 15) / 16 + 1; }

DD_API int dd_gemv(const void* x, const void* W, void* y, int M, int N, int K, int splitk, void* ws,
                   int* counters, hipStream_t stream) {
  DD_REQUIRE(x && W && y && M >= 1 && M <= 16 && N >= 1 && K >= 8 && K % 8 == 0);
  DD_REQUIRE(aligned16(x) && aligned16(W));
  if (splitk <= 0) splitk = pick_splitk(M, N, K);
  DD_REQUIRE(gemv_nsplit(K, splitk) <= 16);
  DD_REQUIRE(gemv_nsplit(K, splitk) == 1 || (ws != nullptr && counters != nullptr));
  launch_gemv(x, W, y, ws, counters, M, N, K, splitk, nullptr, nullptr, nullptr, 0.f, stream);
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
