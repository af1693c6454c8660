// Prefill (the prompt pass, engine.py:459-515 with pos = None), gfx950: token-major q/k
// RMSNorm + RoPE + K/V cache write, and causal GQA flash attention over the cache. Both take a
// packed ("varlen") batch: the B prompts' tokens laid end to end, T tokens in all, prompt b
// holding tokens seq_start[b] .. seq_start[b+1] - 1 at positions 0 .. len_b - 1, so a ragged
// batch prefills in one launch per kernel instead of one pass per prompt length.
//
// qkv_prefill_kernel: one workgroup of 4 waves per token, a wave per head in turn (the raw heads
// of a batch of 8 requested together); lane l holds dims 2l and 2l + 1 (4-byte accesses), its
// rotate-half partners in lane l ^ 32. Rounding points as the reference's
// (engine.py:107-115, 166-187; fused.py:191-200, 221-257):
//   n = bf16(bf16(x * r) * w), r = 1/sqrt(mean(x^2) + eps)
//   out[d]    = bf16(bf16(n[d] * cos[d]) + bf16(-n[d+64] * sin[d]))        d < 64
//   out[d+64] = bf16(bf16(n[d+64] * cos[d+64]) + bf16(n[d] * sin[d+64]))
// q goes to q_out [T, NH, HD] (token-major), k (normalised, rotated) and v (bit copy) to the
// cache [B, NKV, cap, HD] at (b, kv head, position).
//
// flash_prefill_kernel: one workgroup of 4 waves per (tile of 16 NTT tokens of one prompt, kv
// head). Wave w takes token tile w / (G / HPW) and HPW of the kv head's G query heads, so each K
// and V^T fragment a wave reads from LDS feeds HPW query tiles; the 4 waves stage every 32-key
// block (K row-major, V transposed) into LDS once for the whole tile, the next block's global
// loads in flight during the current block. Per block: S^T = K.Q^T on MFMA 16x16x32 (A = 16 keys
// x 32 dims from LDS, B = Q^T held in registers), causal mask key <= token position, online
// softmax in the log2 domain (scale HD^-0.5 log2 e), P rounded to bf16 (fused.py:335),
// O^T += V^T.P^T; the key order inside each P.V contraction is the one each lane's S^T
// accumulators hold, so P never leaves the lane. A wave skips the blocks past its last token.
// Tiles holding a prompt's last tokens (the longest causal prefixes) are scheduled first.
#include "common.h"

namespace dd {
namespace pf {

constexpr int HD = 128;
constexpr int HALF = 64;
constexpr int NWAVE_F = 4;             // waves per flash workgroup
constexpr int KB = 32;                 // keys per block
constexpr int MAXG = 8;                // query heads per kv head
constexpr int KROW = HD + 8;           // LDS K row (elements): 272 bytes
constexpr int VROW = KB + 4;           // LDS V^T row (elements): 72 bytes (18 words: the 4
                                       // dim rows one staging store spans fall in 4 disjoint
                                       // 16-bank ranges)

// The value of lane l ^ 16 (l ^ 32) through gfx950's v_permlane16_swap (v_permlane32_swap), a
// VALU operation, instead of the LDS round trip (ds_bpermute) __shfl_xor compiles to: swapping a
// register with itself leaves each lane the pair (value of the lower row, value of the upper row).
__device__ __forceinline__ float lane_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32) ? r[0] : r[1]);
}

// prompt and position of packed token t (seq_start: B + 1 ascending offsets)
__device__ __forceinline__ void locate(const int* __restrict__ seq_start, int B, int t, int& b, int& p) {
  int lo = 0, hi = B - 1;
  while (lo < hi) {                    // last b with seq_start[b] <= t
    const int mid = (lo + hi + 1) >> 1;
    if (seq_start[mid] <= t) lo = mid;
    else hi = mid - 1;
  }
  b = lo;
  p = t - seq_start[lo];
}

// heads of one wave whose loads are in flight together (a wave takes heads wave, wave + 4, ..)
constexpr int QKV_HPB = 8;

__global__ void __launch_bounds__(256)
qkv_prefill_kernel(const bf16* __restrict__ qkv, const bf16* __restrict__ qn,
                   const bf16* __restrict__ kn, const bf16* __restrict__ cos_t,
                   const bf16* __restrict__ sin_t, const int* __restrict__ seq_start, int B,
                   int last_only, bf16* __restrict__ q_out, bf16* __restrict__ kc,
                   bf16* __restrict__ vc, int NH, int NKV, int cap, int rope_rows, float eps,
                   int* __restrict__ err) {
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int b, p;
  locate(seq_start, B, t, b, p);
  const int len = seq_start[b + 1] - seq_start[b];
  if (p < 0 || p >= len || p >= cap || p >= rope_rows) {   // never write outside the cache
    if (threadIdx.x == 0 && err != nullptr) atomicOr(err, 2);
    return;
  }
  // last_only: q of each prompt's last token only, at row b (the last layer's queries)
  const int h_first = last_only && p != len - 1 ? NH : 0;
  const int nheads = NH + 2 * NKV;
  // lane l holds dims 2l and 2l + 1 (4-byte accesses); its rotate-half partner is lane l ^ 32.
  // The token's cos/sin row and both norm weights are loaded once; then per batch of QKV_HPB
  // heads every raw head is requested before the first is used (one memory latency per batch).
  const int d = 2 * lane;
  const size_t cb = (size_t)p * HD + d;
  const unsigned cw = *(const unsigned*)(cos_t + cb), sw = *(const unsigned*)(sin_t + cb);
  const unsigned wq = *(const unsigned*)(qn + d), wk = *(const unsigned*)(kn + d);
  const bf16* row = qkv + (size_t)t * nheads * HD + d;
  for (int h0 = h_first + wave; h0 < nheads; h0 += 4 * QKV_HPB) {
    unsigned xw[QKV_HPB];
#pragma unroll
    for (int i = 0; i < QKV_HPB; ++i) {
      const int h = h0 + 4 * i;
      xw[i] = h < nheads ? *(const unsigned*)(row + (size_t)h * HD) : 0u;
    }
#pragma unroll
    for (int i = 0; i < QKV_HPB; ++i) {
      const int h = h0 + 4 * i;
      if (h >= nheads) break;
      if (h >= NH + NKV) {             // v: a straight copy into the cache
        *(unsigned*)(vc + (((size_t)b * NKV + (h - NH - NKV)) * cap + p) * HD + d) = xw[i];
        continue;
      }
      const unsigned ww = h < NH ? wq : wk;
      const float x0 = lo_bf(xw[i]), x1 = hi_bf(xw[i]);
      const float ss = wave_sum(x0 * x0 + x1 * x1);
      const float r = rsqrt_ieee(ss / (float)HD + eps);
      const float n0 = rbf(rbf(x0 * r) * lo_bf(ww));
      const float n1 = rbf(rbf(x1 * r) * hi_bf(ww));
      const float pn0 = __shfl_xor(n0, 32, 64), pn1 = __shfl_xor(n1, 32, 64);
      // first half: n cos - n[d + 64] sin; second half: n cos + n[d - 64] sin
      const float sg = lane < 32 ? -1.0f : 1.0f;
      const float o0 = rbf(n0 * lo_bf(cw)) + rbf(sg * pn0 * lo_bf(sw));
      const float o1 = rbf(n1 * hi_bf(cw)) + rbf(sg * pn1 * hi_bf(sw));
      bf16* dst = h < NH ? q_out + ((size_t)(last_only ? b : t) * NH + h) * HD
                         : kc + (((size_t)b * NKV + (h - NH)) * cap + p) * HD;
      *(unsigned*)(dst + d) = pk_bf16(o0, o1);
    }
  }
}

struct FlashShared {
  bf16 k[KB][KROW];                    // the block's keys, row-major
  bf16 vt[HD][VROW];                   // the block's values, transposed: [dim][key]
};

// Tile index -> (prompt, first token position) for tiles of TQ tokens. ntile[b] = ceil(len_b /
// TQ); tiles are numbered prompt by prompt, and workgroup x takes tile (total - 1 - x), so the
// last tiles of the prompts (their longest causal prefixes) go first. last_only: one tile per
// prompt, the one holding its last token.
__device__ __forceinline__ bool tile_of(const int* __restrict__ seq_start, int B, int x, bool last_only,
                                        int TQ, int& b, int& p0) {
  if (last_only) {
    if (x >= B) return false;
    b = x;
    const int len = seq_start[b + 1] - seq_start[b];
    if (len <= 0) return false;
    p0 = ((len - 1) / TQ) * TQ;
    return true;
  }
  int total = 0;
  for (int i = 0; i < B; ++i) total += (seq_start[i + 1] - seq_start[i] + TQ - 1) / TQ;
  const int idx = total - 1 - x;
  if (idx < 0) return false;
  int acc = 0;
  for (int i = 0; i < B; ++i) {
    const int n = (seq_start[i + 1] - seq_start[i] + TQ - 1) / TQ;
    if (idx < acc + n) {
      b = i;
      p0 = (idx - acc) * TQ;
      return true;
    }
    acc += n;
  }
  return false;
}

// q [T, NH, HD] token-major; out [T, NH * HD] (last_only: [B, NH, HD] / [B, NH * HD], row b =
// prompt b's last token). HPW query heads per wave, NTT 16-token tiles per workgroup, with
// NTT * (NH / NKV) / HPW = 4 waves.
#ifndef DD_PF_MINB
#define DD_PF_MINB 2
#endif
template <int HPW, int NTT>
__global__ void __launch_bounds__(64 * NWAVE_F, DD_PF_MINB)
flash_prefill_kernel(const bf16* __restrict__ q, const bf16* __restrict__ kc, const bf16* __restrict__ vc,
                     const int* __restrict__ seq_start, int B, int T, bf16* __restrict__ out,
                     int NH, int NKV, int cap, int last_only, float scale_log2) {
  __shared__ FlashShared sh;
  constexpr int TQ = 16 * NTT;
  int b = 0, p0 = 0;
  if (!tile_of(seq_start, B, blockIdx.x, last_only != 0, TQ, b, p0)) return;
  const int G = NH / NKV, kvh = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int wpt = G / HPW;                                    // waves per token tile
  const int tt = wave / wpt;                                  // this wave's token tile
  const int head0 = kvh * G + (wave - tt * wpt) * HPW;        // its first query head
  const int s0 = seq_start[b], len = seq_start[b + 1] - s0;
  if (s0 < 0 || len <= 0 || s0 + len > T || len > cap) return;   // inconsistent offsets: no access
  const int pq = p0 + tt * 16 + l16;                          // this lane's query token position
  const bool qok = last_only ? pq == len - 1 : pq < len;
  // the wave's token tile: its last valid position (blocks past it are skipped), and whether
  // any of its lanes holds a query at all
  const int tfirst = p0 + tt * 16;
  const bool wact = last_only ? (len - 1 >= tfirst && len - 1 < tfirst + 16) : tfirst < len;
  const int wlast = min(tfirst + 15, len - 1);
  const int plast = min(p0 + TQ, len) - 1;                    // last query position of the tile
  const int nblk = plast / KB + 1;
  // Q^T operands: lane = token l16, dims kb * 32 + g4 * 8 ..
  u32x4 qreg[HPW][4];
#pragma unroll
  for (int h = 0; h < HPW; ++h)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      qreg[h][kb] = qok ? *(const u32x4*)(q + ((size_t)(last_only ? b : s0 + pq) * NH + head0 + h) * HD +
                                          kb * 32 + g4 * 8)
                        : u32x4{0u, 0u, 0u, 0u};
  f32x4 acc[HPW][8];
  float m_run[HPW], l_run[HPW];
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) acc[h][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const size_t kvbase = ((size_t)b * NKV + kvh) * cap * HD;
  // staging per block: K as 512 16-byte chunks (2 a thread: key c / 16, dims (c % 16) 8 ..);
  // V as 256 pairs of 16-byte chunks (one a thread: keys 2 kp and 2 kp + 1 at dims dg 8 ..,
  // kp = t % 16, dg = t / 16), stored transposed as 4-byte words holding both keys of one dim
  constexpr int CPT = KB * HD / 8 / (64 * NWAVE_F);
  static_assert(KB * HD / 16 == 64 * NWAVE_F, "one V chunk pair per thread");
  u32x4 kst[CPT], vst[2];
  const int vkp = (int)threadIdx.x & 15, vdg = (int)threadIdx.x >> 4;
  auto fetch = [&](int key0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = (int)threadIdx.x + i * 64 * NWAVE_F;
      const int key = min(key0 + (c >> 4), cap - 1);
      kst[i] = *(const u32x4*)(kc + kvbase + (size_t)key * HD + (c & 15) * 8);
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const int key = min(key0 + 2 * vkp + r, cap - 1);
      vst[r] = *(const u32x4*)(vc + kvbase + (size_t)key * HD + vdg * 8);
    }
  };
  fetch(0);
  for (int blk = 0; blk < nblk; ++blk) {
    const int key0 = blk * KB;
    __syncthreads();                                          // the previous block is consumed
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = (int)threadIdx.x + i * 64 * NWAVE_F;
      *(u32x4*)&sh.k[c >> 4][(c & 15) * 8] = kst[i];
    }
    {
      const unsigned w0[4] = {vst[0].x, vst[0].y, vst[0].z, vst[0].w};   // key 2 kp
      const unsigned w1[4] = {vst[1].x, vst[1].y, vst[1].z, vst[1].w};   // key 2 kp + 1
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        *(unsigned*)&sh.vt[vdg * 8 + 2 * j][2 * vkp] = (w0[j] & 0xffffu) | (w1[j] << 16);
        *(unsigned*)&sh.vt[vdg * 8 + 2 * j + 1][2 * vkp] = (w0[j] >> 16) | (w1[j] & 0xffff0000u);
      }
    }
    __syncthreads();
    if (blk + 1 < nblk) fetch(key0 + KB);                     // in flight during this block
    if (!wact || key0 > wlast) continue;                      // wave-uniform: nothing to add
    // S^T = K.Q^T: two 16-key halves; D layout: key = t * 16 + g4 * 4 + i, query column l16
    u32x4 ka[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) ka[t][kb] = *(const u32x4*)&sh.k[t * 16 + l16][kb * 32 + g4 * 8];
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      f32x4 sc[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) d = mfma16x16x32(ka[t][kb], qreg[h][kb], d);
        sc[t] = d;
      }
      float sv[8];
      float mloc = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = key0 + t * 16 + g4 * 4 + i;
          const float v = qok && key <= pq ? sc[t][i] * scale_log2 : -INFINITY;
          sv[t * 4 + i] = v;
          mloc = fmaxf(mloc, v);
        }
      mloc = fmaxf(mloc, lane_xor16(mloc));
      mloc = fmaxf(mloc, lane_xor32(mloc));
      const float m_new = fmaxf(m_run[h], mloc);
      const float msafe = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = exp2_hw(m_run[h] - msafe);
      float psum = 0.f;
      unsigned pk[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float pa = exp2_hw(sv[2 * jj] - msafe);
        const float pb = exp2_hw(sv[2 * jj + 1] - msafe);
        psum += pa + pb;
        pk[jj] = pk_bf16(pa, pb);
      }
      psum += lane_xor16(psum);
      psum += lane_xor32(psum);
      l_run[h] = l_run[h] * alpha + psum;
      m_run[h] = m_new;
      const u32x4 pB = {pk[0], pk[1], pk[2], pk[3]};
      // O^T += V^T.P^T; V^T operand: dims dt * 16 + l16, keys g4 * 4 .. + 3 and
      // 16 + g4 * 4 .. + 3 (the keys the lane's P values belong to)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const int d = dt * 16 + l16;
        const u32x2 lo = *(const u32x2*)&sh.vt[d][g4 * 4];
        const u32x2 hi = *(const u32x2*)&sh.vt[d][16 + g4 * 4];
        acc[h][dt] *= alpha;
        acc[h][dt] = mfma16x16x32(u32x4{lo.x, lo.y, hi.x, hi.y}, pB, acc[h][dt]);
      }
    }
  }
  // out: O^T D layout: dim dt * 16 + g4 * 4 + i, token column l16
  if (!qok) return;
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    bf16* orow = last_only ? out + ((size_t)b * NH + head0 + h) * HD
                           : out + ((size_t)(s0 + pq) * NH + head0 + h) * HD;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) orow[dt * 16 + g4 * 4 + i] = f2bf(acc[h][dt][i] / l_run[h]);
  }
}

}  // namespace pf
}  // namespace dd

// ------------------------------------------------------------------------------------------
// C ABI
#include "api.h"

using namespace dd;

DD_API int dd_qkv_post_prefill(const void* qkv, const void* qn, const void* kn, const void* cos_t,
                               const void* sin_t, int rope_rows, const int* seq_start, int B, int T,
                               int last_only, void* q_out, void* kc, void* vc, int NH, int NKV,
                               int HD, int cap, float eps, int* err, hipStream_t stream) {
  DD_REQUIRE(qkv && qn && kn && cos_t && sin_t && seq_start && q_out && kc && vc);
  DD_REQUIRE(HD == 128 && B >= 1 && T >= 1 && NKV >= 1 && NH >= NKV && NH % NKV == 0);
  DD_REQUIRE(cap >= 1 && rope_rows >= 1);
  DD_REQUIRE((long long)T * (NH + 2 * NKV) * HD < (1ll << 40));
  hipLaunchKernelGGL(pf::qkv_prefill_kernel, dim3(T), dim3(256), 0, stream,
                     (const bf16*)qkv, (const bf16*)qn, (const bf16*)kn, (const bf16*)cos_t,
                     (const bf16*)sin_t, seq_start, B, last_only, (bf16*)q_out, (bf16*)kc,
                     (bf16*)vc, NH, NKV, cap, rope_rows, eps, err);
  return launch_status();
}

DD_API int dd_attn_prefill(const void* q, const void* kc, const void* vc, const int* seq_start,
                           int B, int T, int last_only, void* out, int NH, int NKV, int HD, int cap,
                           hipStream_t stream) {
  DD_REQUIRE(q && kc && vc && seq_start && out);
  DD_REQUIRE(HD == 128 && B >= 1 && T >= 1 && NKV >= 1 && NH >= NKV && NH % NKV == 0);
  const int G = NH / NKV;
  DD_REQUIRE((G == 1 || G == 2 || G == 4 || G == 8) && cap >= 1);
  DD_REQUIRE(aligned16(q) && aligned16(kc) && aligned16(vc));
  // HD^-0.5 log2(e), formed in double and rounded once (the reference passes the product of two
  // Python floats to a float32 kernel argument)
  const float scale_log2 = (float)(1.0 / sqrt((double)HD) * 1.4426950408889634);
  // 4 waves: HPW heads x (16 NTT tokens) per wave group; tiles per launch at most T / TQ + B
  auto launch = [&](auto kern, int TQ) {
    const int ntiles = last_only ? B : T / TQ + B;
    hipLaunchKernelGGL(kern, dim3(ntiles, NKV), dim3(64 * pf::NWAVE_F), 0, stream, (const bf16*)q,
                       (const bf16*)kc, (const bf16*)vc, seq_start, B, T, (bf16*)out, NH, NKV, cap,
                       last_only, scale_log2);
  };
  switch (G) {
    case 1: launch(pf::flash_prefill_kernel<1, 4>, 64); break;
    case 2: launch(pf::flash_prefill_kernel<2, 4>, 64); break;
#ifndef DD_PF_G4
#define DD_PF_G4 2
#endif
    case 4:
      if (DD_PF_G4 == 4) launch(pf::flash_prefill_kernel<4, 4>, 64);   // 4 heads x 16 tokens a wave
      else launch(pf::flash_prefill_kernel<2, 2>, 32);                  // 2 heads x 16 tokens a wave
      break;
    default: launch(pf::flash_prefill_kernel<2, 1>, 16); break;   // G = 8: 4 waves per token tile
  }
  return launch_status();
}
