// Decode qkv_post: per-head RMSNorm of q and k, RoPE at each row's own position, k/v written
// into the static cache, q written in the attention layout -- one pass, gfx950.
//
// Input  qkv [B*S, (NH + 2*NKV) * HD]  (the fused QKV GEMV output, q | k | v columns)
// Output q   [B, NKV, S, G, HD]        (rows (s, g) contiguous per kv head, G = NH / NKV)
//        kc, vc [B, NKV, cap, HD]       row (b, h, pos[b*pos_stride] + s) overwritten
//
// Rounding points follow the reference (engine.py:107-115, 166-187; fused.py:191-200, 442-475):
//   n = bf16(bf16(x * r) * w), r = 1/sqrt(mean(x^2) + eps)     (x = the bf16 head vector)
//   out[d]    = bf16(bf16(n[d] * cos[d]) + bf16(-n[d+64] * sin[d]))      d < 64
//   out[d+64] = bf16(bf16(n[d+64] * cos[d+64]) + bf16(n[d] * sin[d+64]))
// v is copied bit for bit.
//
// grid (tokens, ceil(heads / 4)): each of the 4 waves of a workgroup handles one head; lane l
// holds dims l and l+64, i.e. exactly one rotate-half pair, so RoPE needs no data exchange.
#include "common.h"

namespace dd {

constexpr int QKV_THREADS = 256;

__global__ void __launch_bounds__(QKV_THREADS)
qkv_post_decode_kernel(const bf16* __restrict__ qkv, const bf16* __restrict__ qn,
                       const bf16* __restrict__ kn, const bf16* __restrict__ cos_t,
                       const bf16* __restrict__ sin_t, const int64_t* __restrict__ pos,
                       int pos_stride, bf16* __restrict__ q, bf16* __restrict__ kc,
                       bf16* __restrict__ vc, int S, int NH, int NKV, int cap, int rope_rows,
                       float eps, int* __restrict__ err) {
  constexpr int HD = 128, HALF = 64;
  const int t = blockIdx.x;
  const int b = t / S, s = t % S;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int G = NH / NKV;
  const int total = (NH + 2 * NKV) * HD;
  const int64_t position = pos[(size_t)b * pos_stride] + s;
  const bool pos_ok = position >= 0 && position < cap && position < rope_rows;
  if (!pos_ok) {  // never write outside the cache; report instead
    if (threadIdx.x == 0 && err != nullptr) atomicOr(err, 2);
    return;
  }
  const bf16* row = qkv + (size_t)t * total;
  const size_t cb = (size_t)position * HD;
  const float c1 = bf2f(cos_t[cb + lane]), c2 = bf2f(cos_t[cb + HALF + lane]);
  const float s1 = bf2f(sin_t[cb + lane]), s2 = bf2f(sin_t[cb + HALF + lane]);
  const int h = blockIdx.y * (QKV_THREADS / 64) + wave;
  if (h < NH + 2 * NKV) {
    const bf16* base = row + h * HD;
    const bf16 x1b = base[lane], x2b = base[HALF + lane];
    if (h >= NH + NKV) {  // v: straight copy into the cache
      bf16* vo = vc + (((size_t)b * NKV + (h - NH - NKV)) * cap + position) * HD;
      vo[lane] = x1b;
      vo[HALF + lane] = x2b;
      return;
    }
    const float f1 = bf2f(x1b), f2 = bf2f(x2b);
    const float ss = wave_sum(f1 * f1 + f2 * f2);
    const float r = rsqrt_ieee(ss / (float)HD + eps);
    const bf16* wn = h < NH ? qn : kn;
    const float n1 = rbf(rbf(f1 * r) * bf2f(wn[lane]));
    const float n2 = rbf(rbf(f2 * r) * bf2f(wn[HALF + lane]));
    const bf16 o1 = f2bf(rbf(n1 * c1) + rbf(-n2 * s1));
    const bf16 o2 = f2bf(rbf(n2 * c2) + rbf(n1 * s2));
    bf16* dst;
    if (h < NH) {
      dst = q + ((((size_t)b * NKV + h / G) * S + s) * G + h % G) * HD;
    } else {
      dst = kc + (((size_t)b * NKV + (h - NH)) * cap + position) * HD;
    }
    dst[lane] = o1;
    dst[HALF + lane] = o2;
  }
}

}  // namespace dd

// ------------------------------------------------------------------------------------------
// C ABI
#include "api.h"

using namespace dd;

DD_API int dd_qkv_post_decode(const void* qkv, const void* qn, const void* kn, const void* cos_t,
                              const void* sin_t, int rope_rows, const int64_t* pos, int pos_stride,
                              void* q, void* kc, void* vc, int B, int S, int NH, int NKV, int HD,
                              int cap, float eps, int* err, hipStream_t stream) {
  DD_REQUIRE(qkv && qn && kn && cos_t && sin_t && pos && q && kc && vc);
  DD_REQUIRE(HD == 128 && B >= 1 && S >= 1 && NKV >= 1 && NH >= NKV && NH % NKV == 0);
  DD_REQUIRE(cap >= 1 && rope_rows >= 1 && (pos_stride == 0 || pos_stride == 1));
  const int heads = NH + 2 * NKV;
  hipLaunchKernelGGL(qkv_post_decode_kernel, dim3(B * S, (heads + 3) / 4), dim3(QKV_THREADS), 0, stream,
                     (const bf16*)qkv, (const bf16*)qn, (const bf16*)kn, (const bf16*)cos_t,
                     (const bf16*)sin_t, pos, pos_stride, (bf16*)q, (bf16*)kc, (bf16*)vc, S, NH,
                     NKV, cap, rope_rows, eps, err);
  return launch_status();
}
