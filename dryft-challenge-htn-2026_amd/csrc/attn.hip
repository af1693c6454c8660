// Split-KV GQA decode attention with an in-kernel log-sum-exp combine, gfx950.
//
//   out[b*W + s][(kvh*G + g)*HD + d] = softmax_j(q . k_j * HD^-0.5) . v_j
//   over keys j = 0 .. pos[b] + s  of kv head kvh (query row r = s*G + g of that head)
//
// Inputs  q  [B, NKV, W, G, HD] bf16      kc, vc [B, NKV, cap, HD] bf16 (zero-initialised cache)
//         pos int64, row b at pos[b * pos_stride]
// Output  out [B*W, NH*HD] bf16
//
// Work split: one workgroup per (b*NKV + kvh, split) over a fixed key chunk of C keys, so ragged
// lengths balance across the grid (a split past the row's length exits at once). Inside, the 4
// waves take 32-key blocks round-robin and keep their own online-softmax state:
//   S^T = K . Q^T   on MFMA 16x16x32 (A = 16 keys x 32 dims loaded straight from HBM,
//                   B = Q^T held in registers), fp32 scores in the log2 domain;
//   O^T += V^T . P^T  on MFMA (A = V^T read transposed from an LDS copy of the V block,
//                   B = P^T, which is exactly the lanes' own S^T accumulators rounded to bf16 --
//                   the key order inside the contraction is permuted to make that local).
// P is rounded to bf16 before PV and the running sum l uses the fp32 P (the reference's fused
// kernel does the same, fused.py:511-525). The waves merge through LDS; a single-split row
// writes bf16 directly, otherwise fp32 partials (acc, m, l) go to ws and the last split to
// arrive (per (b, kvh) counter) combines them in split order and resets the counter.
#include "common.h"

namespace dd {

constexpr int ATT_THREADS = 256;
constexpr int ATT_WAVES = 4;
constexpr int HD = 128;
constexpr int VROW = HD + 8;  // padded LDS row (elements) for the V block: 272 bytes

struct AttnShared {
  union {
    bf16 v[ATT_WAVES][32][VROW];                // per-wave V block
    float mrg[ATT_WAVES][16][HD];               // wave partial O (one 16-row block at a time)
  } u;
  float ms[ATT_WAVES][16];
  float ls[ATT_WAVES][16];
  int last;
};

template <int RB>
__global__ void __launch_bounds__(ATT_THREADS)
attn_decode_kernel(const bf16* __restrict__ q, const bf16* __restrict__ kc,
                   const bf16* __restrict__ vc, const int64_t* __restrict__ pos, int pos_stride,
                   bf16* __restrict__ out, float* __restrict__ ws, int* __restrict__ counters,
                   int W, int G, int NKV, int cap, int chunk, int nsplit_max, float scale_log2) {
  __shared__ AttnShared sh;
  const int bk = blockIdx.x;
  const int split = blockIdx.y;
  const int b = bk / NKV, kvh = bk % NKV;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int R = W * G;
  const int64_t p0 = pos[(size_t)b * pos_stride];
  const int L = (int)min<int64_t>(p0 + W, (int64_t)cap);  // keys 0 .. L-1 exist
  const int nsplit = (L + chunk - 1) / chunk;
  if (split >= nsplit) return;
  const int start = split * chunk;
  const int end = min(start + chunk, L);

  const bf16* qb = q + (size_t)bk * R * HD;
  const bf16* kb_ = kc + (size_t)bk * cap * HD;
  const bf16* vb_ = vc + (size_t)bk * cap * HD;

  // Q^T operand (B of the S^T MFMA): lane holds q[row rb*16 + l16][kb*32 + g4*8 .. +8]
  u32x4 qreg[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = rb * 16 + l16;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      if (row < R) qreg[rb][kb] = ld16(qb + (size_t)row * HD + kb * 32 + g4 * 8);
      else qreg[rb][kb] = u32x4{0u, 0u, 0u, 0u};
    }
  }
  // causal limit of this lane's query row (as a key index, inclusive)
  int lim[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int row = rb * 16 + l16;
    lim[rb] = (int)p0 + (row < R ? row : R - 1) / G;
  }

  f32x4 acc[RB][8];
  float m_run[RB], l_run[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m_run[rb] = -INFINITY;
    l_run[rb] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[rb][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  bf16(*vs)[VROW] = sh.u.v[wave];
  const int nblk = (end - start + 31) >> 5;
  for (int bi = wave; bi < nblk; bi += ATT_WAVES) {
    const int j0 = start + bi * 32;
    // K operand loads: 2 tiles of 16 keys x 4 dim blocks
    u32x4 kreg[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      int key = j0 + t * 16 + l16;
      key = key < cap ? key : cap - 1;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) kreg[t][kb] = ld16(kb_ + (size_t)key * HD + kb * 32 + g4 * 8);
    }
    // V block -> registers -> LDS (natural [key][dim] layout)
    u32x4 vreg[8];
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int c = it * 64 + lane;
      int key = j0 + (c >> 4);
      key = key < cap ? key : cap - 1;
      vreg[it] = ld16(vb_ + (size_t)key * HD + (c & 15) * 8);
    }
    // S^T tiles
    f32x4 sc[2][RB];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) d = mfma16x16x32(kreg[t][kb], qreg[rb][kb], d);
        sc[t][rb] = d;
      }
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int c = it * 64 + lane;
      *(u32x4*)&vs[c >> 4][(c & 15) * 8] = vreg[it];
    }
    // online softmax per 16-row block; P^T operand packed as bf16 pairs
    u32x4 pB[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      float sv[8];
      float mloc = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = j0 + t * 16 + g4 * 4 + i;
          const bool ok = key < end && key <= lim[rb];
          const float v = ok ? sc[t][rb][i] * scale_log2 : -INFINITY;
          sv[t * 4 + i] = v;
          mloc = fmaxf(mloc, v);
        }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
      const float m_new = fmaxf(m_run[rb], mloc);
      const float msafe = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2_hw(m_run[rb] - msafe);
      float psum = 0.f;
      unsigned pk[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float pa = exp2_hw(sv[2 * j] - msafe);
        const float pb = exp2_hw(sv[2 * j + 1] - msafe);
        psum += pa + pb;
        pk[j] = (unsigned)f2bf(pa) | ((unsigned)f2bf(pb) << 16);
      }
      psum += __shfl_xor(psum, 16, 64);
      psum += __shfl_xor(psum, 32, 64);
      l_run[rb] = l_run[rb] * alpha + psum;
      m_run[rb] = m_new;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[rb][dt] *= alpha;
      pB[rb] = u32x4{pk[0], pk[1], pk[2], pk[3]};
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // O^T += V^T . P^T ; V^T operand: dim dt*16 + l16, keys {g4*4 + i} then {16 + g4*4 + i}
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int d = dt * 16 + l16;
      unsigned a[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ka = (j < 2) ? (g4 * 4 + 2 * j) : (16 + g4 * 4 + 2 * (j - 2));
        a[j] = (unsigned)vs[ka][d] | ((unsigned)vs[ka + 1][d] << 16);
      }
      const u32x4 va = {a[0], a[1], a[2], a[3]};
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][dt] = mfma16x16x32(va, pB[rb], acc[rb][dt]);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- merge the 4 waves, one 16-row block at a time ----
  const size_t wsrow = HD + 2;
  const rsrc_t wsr = make_rsrc(ws, (unsigned)((size_t)gridDim.x * nsplit_max * R * wsrow * 4));
  for (int rb = 0; rb < RB; ++rb) {
    __syncthreads();  // V staging area is reused for the merge
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) sh.u.mrg[wave][l16][dt * 16 + g4 * 4 + i] = acc[rb][dt][i];
    if (g4 == 0) {
      sh.ms[wave][l16] = m_run[rb];
      sh.ls[wave][l16] = l_run[rb];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 16 * HD; e += ATT_THREADS) {
      const int rr = e / HD, d = e % HD;
      const int row = rb * 16 + rr;
      if (row >= R) continue;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < ATT_WAVES; ++w) M = fmaxf(M, sh.ms[w][rr]);
      const float Ms = M == -INFINITY ? 0.f : M;
      float o = 0.f, l = 0.f;
#pragma unroll
      for (int w = 0; w < ATT_WAVES; ++w) {
        const float f = exp2_hw(sh.ms[w][rr] - Ms);
        o += sh.u.mrg[w][rr][d] * f;
        l += sh.ls[w][rr] * f;
      }
      if (nsplit == 1) {
        const int sq = row / G, gq = row % G;
        out[((size_t)b * W + sq) * (NKV * G * HD) + ((size_t)kvh * G + gq) * HD + d] = f2bf(o / l);
      } else {
        const unsigned p = (unsigned)((((size_t)bk * nsplit_max + split) * R + row) * wsrow) * 4;
        stc_f32(wsr, p + d * 4, o);
        if (d == 0) {
          stc_f32(wsr, p + HD * 4, M);
          stc_f32(wsr, p + (HD + 1) * 4, l);
        }
      }
    }
  }
  if (nsplit == 1) return;

  // ---- last split to arrive combines (split order); partials travel through sc1 ----
  if (!arrive_last(counters + bk, nsplit, &sh.last)) return;
  for (int e = threadIdx.x; e < R * HD; e += ATT_THREADS) {
    const int row = e / HD, d = e % HD;
    const unsigned p = (unsigned)(((size_t)bk * nsplit_max * R + row) * wsrow) * 4;
    const unsigned sstride = (unsigned)(R * wsrow) * 4;
    float M = -INFINITY;
    for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, ldc_f32(wsr, p + sp * sstride + HD * 4));
    float o = 0.f, l = 0.f;
    for (int sp = 0; sp < nsplit; ++sp) {
      const unsigned ps = p + sp * sstride;
      const float f = exp2_hw(ldc_f32(wsr, ps + HD * 4) - M);
      o += ldc_f32(wsr, ps + d * 4) * f;
      l += ldc_f32(wsr, ps + (HD + 1) * 4) * f;
    }
    const int sq = row / G, gq = row % G;
    out[((size_t)b * W + sq) * (NKV * G * HD) + ((size_t)kvh * G + gq) * HD + d] = f2bf(o / l);
  }
}

template __global__ void attn_decode_kernel<1>(const bf16*, const bf16*, const bf16*, const int64_t*, int,
                                               bf16*, float*, int*, int, int, int, int, int, int, float);
template __global__ void attn_decode_kernel<2>(const bf16*, const bf16*, const bf16*, const int64_t*, int,
                                               bf16*, float*, int*, int, int, int, int, int, int, float);

}  // namespace dd

// ------------------------------------------------------------------------------------------
// C ABI
#include "api.h"

using namespace dd;

// Keys per split: aim for ~1024 workgroups over a full cache (256 CUs x 4), in multiples of
// 128 keys (one 32-key block per wave), never below 128.
DD_API int dd_attn_chunk(int B, int NKV, int cap) {
  if (B < 1 || NKV < 1 || cap < 1) return 128;
  const long long keys = (long long)B * NKV * cap;
  long long c = (keys + 1023) / 1024;
  c = (c + 127) / 128 * 128;
  return (int)(c < 128 ? 128 : c);
}

DD_API size_t dd_attn_ws_bytes(int B, int W, int NH, int NKV, int HD, int cap, int chunk) {
  if (chunk <= 0) chunk = dd_attn_chunk(B, NKV, cap);
  if (B < 1 || NKV < 1 || NH < NKV || W < 1 || HD < 1 || cap < 1) return 0;
  const size_t nsplit = (size_t)(cap + chunk - 1) / chunk;
  const size_t R = (size_t)W * (NH / NKV);
  return (size_t)B * NKV * nsplit * R * (HD + 2) * sizeof(float);
}

DD_API int dd_attn_decode(const void* q, const void* kc, const void* vc, const int64_t* pos,
                          int pos_stride, void* out, void* ws, int* counters, int B, int W, int NH,
                          int NKV, int HD, int cap, int chunk, hipStream_t stream) {
  DD_REQUIRE(q && kc && vc && pos && out && ws && counters);
  DD_REQUIRE(HD == 128 && B >= 1 && W >= 1 && NKV >= 1 && NH >= NKV && NH % NKV == 0 && cap >= 1);
  DD_REQUIRE(pos_stride == 0 || pos_stride == 1);
  const int G = NH / NKV;
  DD_REQUIRE(W * G <= 32);
  DD_REQUIRE(aligned16(q) && aligned16(kc) && aligned16(vc));
  if (chunk <= 0) chunk = dd_attn_chunk(B, NKV, cap);
  DD_REQUIRE(chunk % 32 == 0);
  const int nsplit_max = (cap + chunk - 1) / chunk;
  const float scale_log2 = (1.0f / sqrtf((float)HD)) * 1.4426950408889634f;
  dim3 grid(B * NKV, nsplit_max);
  if (W * G <= 16)
    hipLaunchKernelGGL(attn_decode_kernel<1>, grid, dim3(ATT_THREADS), 0, stream, (const bf16*)q,
                       (const bf16*)kc, (const bf16*)vc, pos, pos_stride, (bf16*)out, (float*)ws,
                       counters, W, G, NKV, cap, chunk, nsplit_max, scale_log2);
  else
    hipLaunchKernelGGL(attn_decode_kernel<2>, grid, dim3(ATT_THREADS), 0, stream, (const bf16*)q,
                       (const bf16*)kc, (const bf16*)vc, pos, pos_stride, (bf16*)out, (float*)ws,
                       counters, W, G, NKV, cap, chunk, nsplit_max, scale_log2);
  return launch_status();
}

// ---------------------------------------------------------------------------------------------
// No-allocation variant: the split partials and the per-(row, kv head) counters live in a
// file-scope device array instead of caller workspaces. Each device holds its own copy of the
// array (for the life of the process); host code reaches it only through the address
// hipGetSymbolAddress returns for the current device, looked up once per device.
namespace dd {
constexpr size_t NOALLOC_WS_BYTES = size_t(24) << 20;   // split partials (dd_attn_ws_bytes)
constexpr int NOALLOC_COUNTERS = 4096;                  // B * NKV combine counters
static __device__ __align__(256) unsigned char scratch[NOALLOC_WS_BYTES + NOALLOC_COUNTERS * 4];

__global__ void zero_ints_kernel(int* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

}  // namespace dd

#include <mutex>

namespace {
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[NOALLOC_MAX_DEVICES];   // device address of `scratch`, per device

// Address of this device's scratch array. The first call on a device looks it up and clears the
// counters synchronously (so no later call, on any stream, can overlap the clear); a first call
// made while `stream` is being captured into a graph returns hipErrorStreamCaptureUnsupported
// instead, since the clear could only be recorded, not done.
int noalloc_scratch(hipStream_t stream, unsigned char** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES)
    return (int)hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (g_noalloc_ptr[dev] == nullptr) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) return (int)hipErrorInvalidValue;
    if (cap != hipStreamCaptureStatusNone) return (int)hipErrorStreamCaptureUnsupported;
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(dd::scratch));
    if (e != hipSuccess) return (int)e;
    if (ptr == nullptr) return (int)hipErrorInvalidSymbol;
    int* counters = (int*)((unsigned char*)ptr + dd::NOALLOC_WS_BYTES);
    hipLaunchKernelGGL(dd::zero_ints_kernel, dim3((dd::NOALLOC_COUNTERS + 255) / 256), dim3(256),
                       0, stream, counters, dd::NOALLOC_COUNTERS);
    const int st = dd::launch_status();
    if (st != 0) return st;
    e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return (int)e;
    g_noalloc_ptr[dev] = ptr;
  }
  *out = (unsigned char*)g_noalloc_ptr[dev];
  return 0;
}
}  // namespace

DD_API int dd_attn_decode_noalloc(const void* q, const void* kc, const void* vc,
                                  const int64_t* pos, int pos_stride, void* out, int B, int W,
                                  int NH, int NKV, int HD, int cap, hipStream_t stream) {
  DD_REQUIRE(q && kc && vc && pos && out);
  DD_REQUIRE(HD == 128 && B >= 1 && W >= 1 && NKV >= 1 && NH >= NKV && NH % NKV == 0 && cap >= 1);
  DD_REQUIRE(pos_stride == 0 || pos_stride == 1);
  DD_REQUIRE(W * (NH / NKV) <= 32);
  DD_REQUIRE(aligned16(q) && aligned16(kc) && aligned16(vc));
  const int chunk = dd_attn_chunk(B, NKV, cap);
  // the static array bounds the shapes this entry point takes
  if (dd_attn_ws_bytes(B, W, NH, NKV, HD, cap, chunk) > dd::NOALLOC_WS_BYTES ||
      (long long)B * NKV > dd::NOALLOC_COUNTERS)
    return (int)hipErrorOutOfMemory;
  unsigned char* base = nullptr;
  const int e = noalloc_scratch(stream, &base);
  if (e != 0) return e;
  return dd_attn_decode(q, kc, vc, pos, pos_stride, out, base, (int*)(base + dd::NOALLOC_WS_BYTES),
                        B, W, NH, NKV, HD, cap, chunk, stream);
}

