// Prefill (the prompt pass, engine.py:459-515 with pos = None), gfx950: token-major q/k
// RMSNorm + RoPE + K/V cache write, and causal GQA flash attention over the cache. Both take a
// packed ("varlen") batch: the B prompts' tokens laid end to end, T tokens in all, prompt b
// holding tokens seq_start[b] .. seq_start[b+1] - 1 at positions 0 .. len_b - 1, so a ragged
// batch prefills in one launch per kernel instead of one pass per prompt length.
//
// qkv_prefill_kernel: one workgroup per 16 tokens, a 16-lane group per token taking its heads in
// turn (the raw heads of a batch of 8 requested together); lane j holds dims 4j .. 4j + 3 and
// their rotate-half partners 64 + 4j .. (two 8-byte accesses). Rounding points as the reference's
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
// block (K and V row-major, V^T read by transposing LDS loads) into LDS once for the whole tile,
// the next block's global loads in flight during the current block. Per block: S^T = K.Q^T on
// MFMA 16x16x32 (A = 16 keys x 32 dims from LDS, B = Q^T held in registers), causal mask key <=
// token position (only on the blocks that reach into the tile), online
// softmax in the log2 domain (scale HD^-0.5 log2 e), P rounded to bf16 (fused.py:335),
// O^T += V^T.P^T; the key order inside each P.V contraction is the one each lane's S^T
// accumulators hold, so P never leaves the lane. A wave skips the blocks past its last token.
// Tiles holding a prompt's last tokens (the longest causal prefixes) are scheduled first.
// flash_prefill_dma_kernel: the same arithmetic for G = 4 with one query head per wave, its
// 32-key blocks staged by LDS-DMA loads into two swizzled LDS buffers (the G = 4 default).
#include <type_traits>

#include "common.h"

namespace dd {
namespace pf {

constexpr int HD = 128;
constexpr int HALF = 64;
constexpr int KB = 32;                 // keys per block
constexpr int MAXG = 8;                // query heads per kv head
constexpr int KROW = HD + 8;           // LDS K / V row (elements): 272 bytes

// Max and sum over the lane pairs l, l ^ 16 (rows16) and l, l ^ 32 (rows32) through gfx950's
// v_permlane16_swap / v_permlane32_swap, VALU operations, instead of the LDS round trip
// (ds_bpermute) __shfl_xor compiles to. Swapping a register with itself leaves the pair (value of
// the lower row, value of the upper row) in every lane, so the pair's max or sum needs no
// lane-dependent select; the sum adds the lower row's value first in every lane, the same bits as
// either order.
__device__ __forceinline__ float max_rows16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_rows32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_rows16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_rows32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
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

// One workgroup per 16 tokens: each 16-lane group takes one token's heads in turn, QKV_HPB heads'
// loads in flight together. Lane j of a group holds dims 4j .. 4j + 3 and 64 + 4j .. 64 + 4j + 3
// (two 8-byte accesses), so both rotate-half partners of every dim are in the lane; the head's
// sum of squares is the lane's 8 squares added in order, then reduced over the 16 lanes.
constexpr int QKV_TPW = 16;            // tokens per workgroup (4 waves x 4 groups)
#ifndef DD_QKV_HPB
#define DD_QKV_HPB 8
#endif
constexpr int QKV_HPB = DD_QKV_HPB;

__device__ __forceinline__ float group16_sum(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__global__ void __launch_bounds__(256)
qkv_prefill_kernel(const bf16* __restrict__ qkv, const bf16* __restrict__ qn,
                   const bf16* __restrict__ kn, const bf16* __restrict__ cos_t,
                   const bf16* __restrict__ sin_t, const int* __restrict__ seq_start, int B, int T,
                   int last_only, bf16* __restrict__ q_out, bf16* __restrict__ kc,
                   bf16* __restrict__ vc, int NH, int NKV, int cap, int rope_rows, float eps,
                   int* __restrict__ err) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 15;
  const int t = blockIdx.x * QKV_TPW + wave * 4 + (lane >> 4);   // this group's token
  if (t >= T) return;                                             // whole group
  int b, p;
  locate(seq_start, B, t, b, p);
  const int len = seq_start[b + 1] - seq_start[b];
  if (p < 0 || p >= len || p >= cap || p >= rope_rows) {   // never write outside the cache
    if (j == 0 && err != nullptr) atomicOr(err, 2);
    return;
  }
  // last_only: q of each prompt's last token only, at row b (the last layer's queries)
  const int h_first = last_only && p != len - 1 ? NH : 0;
  const int nheads = NH + 2 * NKV;
  const int d0 = 4 * j, d1 = 64 + 4 * j;
  const size_t cb = (size_t)p * HD;
  const u32x2 c0 = *(const u32x2*)(cos_t + cb + d0), c1 = *(const u32x2*)(cos_t + cb + d1);
  const u32x2 s0 = *(const u32x2*)(sin_t + cb + d0), s1 = *(const u32x2*)(sin_t + cb + d1);
  const u32x2 q0 = *(const u32x2*)(qn + d0), q1 = *(const u32x2*)(qn + d1);
  const u32x2 k0 = *(const u32x2*)(kn + d0), k1 = *(const u32x2*)(kn + d1);
  const float cw[8] = {lo_bf(c0.x), hi_bf(c0.x), lo_bf(c0.y), hi_bf(c0.y),
                       lo_bf(c1.x), hi_bf(c1.x), lo_bf(c1.y), hi_bf(c1.y)};
  const float sw[8] = {lo_bf(s0.x), hi_bf(s0.x), lo_bf(s0.y), hi_bf(s0.y),
                       lo_bf(s1.x), hi_bf(s1.x), lo_bf(s1.y), hi_bf(s1.y)};
  const bf16* row = qkv + (size_t)t * nheads * HD;
  for (int h0 = h_first; h0 < nheads; h0 += QKV_HPB) {
    u32x2 xa[QKV_HPB], xb[QKV_HPB];
#pragma unroll
    for (int i = 0; i < QKV_HPB; ++i) {
      const int h = h0 + i;
      xa[i] = h < nheads ? *(const u32x2*)(row + (size_t)h * HD + d0) : u32x2{0u, 0u};
      xb[i] = h < nheads ? *(const u32x2*)(row + (size_t)h * HD + d1) : u32x2{0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < QKV_HPB; ++i) {
      const int h = h0 + i;
      if (h >= nheads) break;
      if (h >= NH + NKV) {             // v: a straight copy into the cache
        bf16* dst = vc + (((size_t)b * NKV + (h - NH - NKV)) * cap + p) * HD;
        *(u32x2*)(dst + d0) = xa[i];
        *(u32x2*)(dst + d1) = xb[i];
        continue;
      }
      const u32x2 wa = h < NH ? q0 : k0, wb = h < NH ? q1 : k1;
      const float w[8] = {lo_bf(wa.x), hi_bf(wa.x), lo_bf(wa.y), hi_bf(wa.y),
                          lo_bf(wb.x), hi_bf(wb.x), lo_bf(wb.y), hi_bf(wb.y)};
      const float x[8] = {lo_bf(xa[i].x), hi_bf(xa[i].x), lo_bf(xa[i].y), hi_bf(xa[i].y),
                          lo_bf(xb[i].x), hi_bf(xb[i].x), lo_bf(xb[i].y), hi_bf(xb[i].y)};
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) ss += x[k] * x[k];
      ss = group16_sum(ss);
      const float r = rsqrt_ieee(ss / (float)HD + eps);
      float n[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) n[k] = rbf(rbf(x[k] * r) * w[k]);
      // first half: n cos - n[d + 64] sin; second half: n cos + n[d - 64] sin
      float o[8];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        o[k] = rbf(n[k] * cw[k]) + rbf(-n[k + 4] * sw[k]);
        o[k + 4] = rbf(n[k + 4] * cw[k + 4]) + rbf(n[k] * sw[k + 4]);
      }
      bf16* dst = h < NH ? q_out + ((size_t)(last_only ? b : t) * NH + h) * HD
                         : kc + (((size_t)b * NKV + (h - NH)) * cap + p) * HD;
      *(u32x2*)(dst + d0) = u32x2{pk_bf16(o[0], o[1]), pk_bf16(o[2], o[3])};
      *(u32x2*)(dst + d1) = u32x2{pk_bf16(o[4], o[5]), pk_bf16(o[6], o[7])};
    }
  }
}

struct FlashShared {
  bf16 k[KB][KROW];                    // the block's keys, row-major
  bf16 v[KB][KROW];                    // the block's values, row-major (read transposed)
};

// ds_read_b64_tr_b16 (gfx950), a transposing LDS read: when lane (l16, g4) of a wave addresses
// row g4 * 4 + l16 / 4, columns c0 + 4 (l16 % 4) .. + 3 of a row-major bf16 array, it receives
// column c0 + l16 of rows g4 * 4 .. g4 * 4 + 3 (the MFMA operand of the transposed block).
typedef short i16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_read_tr16(const bf16* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(const_cast<bf16*>(p)));
  return __builtin_bit_cast(u32x2, v);
}

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
// NTT * (NH / NKV) / HPW = NWAVE_F waves; MINB workgroups per CU (the register budget).
#ifndef DD_PF_MINB1
#define DD_PF_MINB1 4
#endif
#ifndef DD_PF_MINB
#define DD_PF_MINB 2
#endif
template <int HPW, int NTT, int NWAVE_F, int MINB>
__global__ void __launch_bounds__(64 * NWAVE_F, MINB)
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
  // staging per block: K and V as 512 16-byte chunks each, 2 of each a thread (chunk c: key
  // c / 16, dims (c % 16) 8 ..), both stored row-major. Buffer loads over this (sequence, kv
  // head)'s cache rows: the per-lane offsets are fixed and the block's key0 goes in the scalar
  // offset; keys past the cache read zeros (they are masked).
  constexpr int CPT = KB * HD / 8 / (64 * NWAVE_F);
  static_assert(CPT * 64 * NWAVE_F * 8 == KB * HD, "whole chunks per thread");
  const rsrc_t kr = make_rsrc(kc + kvbase, (unsigned)((size_t)cap * HD * 2));
  const rsrc_t vr = make_rsrc(vc + kvbase, (unsigned)((size_t)cap * HD * 2));
  unsigned coff[CPT];
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = (int)threadIdx.x + i * 64 * NWAVE_F;
    coff[i] = (unsigned)((c >> 4) * HD * 2 + (c & 15) * 16);
  }
  u32x4 kst[CPT], vst[CPT];
  auto fetch = [&](int key0) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      kst[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, coff[i], (unsigned)key0 * HD * 2, 0);
      vst[i] = __builtin_amdgcn_raw_buffer_load_b128(vr, coff[i], (unsigned)key0 * HD * 2, 0);
    }
  };
  // V^T operand addressing (see lds_read_tr16)
  const int trow = g4 * 4 + (l16 >> 2), tcol = 4 * (l16 & 3);
  // One block: stage it, request the next, then (the wave's keys permitting) add it. MASKED: the
  // causal mask key <= query position; blocks wholly before the tile's first query need none.
  auto block = [&](int blk, auto masked) {
    constexpr bool MASKED = decltype(masked)::value;
    const int key0 = blk * KB;
    __syncthreads();                                          // the previous block is consumed
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = (int)threadIdx.x + i * 64 * NWAVE_F;
      *(u32x4*)&sh.k[c >> 4][(c & 15) * 8] = kst[i];
      *(u32x4*)&sh.v[c >> 4][(c & 15) * 8] = vst[i];
    }
    __syncthreads();
    if (blk + 1 < nblk) fetch(key0 + KB);                     // in flight during this block
    if (!wact || key0 > wlast) return;                        // wave-uniform: nothing to add
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
          const float v = !MASKED || (qok && key <= pq) ? sc[t][i] * scale_log2 : -INFINITY;
          sv[t * 4 + i] = v;
          mloc = fmaxf(mloc, v);
        }
      mloc = max_rows32(max_rows16(mloc));
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
      psum = sum_rows32(sum_rows16(psum));
      l_run[h] = l_run[h] * alpha + psum;
      m_run[h] = m_new;
      const u32x4 pB = {pk[0], pk[1], pk[2], pk[3]};
      // O^T += V^T.P^T; V^T operand: dims dt * 16 + l16, keys g4 * 4 .. + 3 and
      // 16 + g4 * 4 .. + 3 (the keys the lane's P values belong to)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const u32x2 lo = lds_read_tr16(&sh.v[trow][dt * 16 + tcol]);
        const u32x2 hi = lds_read_tr16(&sh.v[16 + trow][dt * 16 + tcol]);
        acc[h][dt] *= alpha;
        acc[h][dt] = mfma16x16x32(u32x4{lo.x, lo.y, hi.x, hi.y}, pB, acc[h][dt]);
      }
    }
  };
  // blocks whose last key is at or before the workgroup's first query position: no mask; then the
  // blocks that reach into the tile
  const int nfull = min(nblk, (p0 + 1) / KB);
  fetch(0);
  for (int blk = 0; blk < nfull; ++blk) block(blk, std::integral_constant<bool, false>{});
  for (int blk = nfull; blk < nblk; ++blk) block(blk, std::integral_constant<bool, true>{});
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

// The same attention (one query head per wave, 16 tokens, G = 4 waves per workgroup) with the
// 32-key blocks staged by LDS-DMA loads (buffer_load_dwordx4 ... lds: lane i's 16 bytes land at
// the wave's LDS base + 16 i) into two buffers: block j + 1 streams into one while block j is
// read from the other, with one barrier per block and no staging registers. Rows are 256 bytes,
// unpadded; 16-byte chunks are XOR-swizzled so that the MFMA operand reads meet distinct banks:
// K chunk c of key r at position c ^ (r % 16) (a K read: 16 consecutive keys, one chunk), V chunk
// c of key r at c ^ 2 (r % 8) (a transposing V read: 4 consecutive keys, a pair of chunks).
// The DMA writer picks, per lane, the source chunk whose swizzled position is its own. The loop is
// unrolled by two so each buffer is a separate LDS object at every access.
struct FlashDmaBuf {
  bf16 k[KB * HD];
  bf16 v[KB * HD];
};

template <int MINB>
__global__ void __launch_bounds__(256, MINB)
flash_prefill_dma_kernel(const bf16* __restrict__ q, const bf16* __restrict__ kc, const bf16* __restrict__ vc,
                         const int* __restrict__ seq_start, int B, int T, bf16* __restrict__ out,
                         int NH, int NKV, int cap, int last_only, float scale_log2) {
  __shared__ __attribute__((aligned(16))) FlashDmaBuf sb0;
  __shared__ __attribute__((aligned(16))) FlashDmaBuf sb1;
  constexpr int TQ = 16;
  int b = 0, p0 = 0;
  if (!tile_of(seq_start, B, blockIdx.x, last_only != 0, TQ, b, p0)) return;
  const int G = NH / NKV, kvh = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int head = kvh * G + wave;                              // this wave's query head
  const int s0 = seq_start[b], len = seq_start[b + 1] - s0;
  if (s0 < 0 || len <= 0 || s0 + len > T || len > cap) return;   // inconsistent offsets: no access
  const int pq = p0 + l16;                                      // this lane's query token position
  const bool qok = last_only ? pq == len - 1 : pq < len;
  const bool wact = last_only ? (len - 1 >= p0 && len - 1 < p0 + 16) : p0 < len;
  const int wlast = min(p0 + 15, len - 1);
  const int nblk = wlast / KB + 1;
  u32x4 qreg[4];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb)
    qreg[kb] = qok ? *(const u32x4*)(q + ((size_t)(last_only ? b : s0 + pq) * NH + head) * HD + kb * 32 + g4 * 8)
                   : u32x4{0u, 0u, 0u, 0u};
  f32x4 acc[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const size_t kvbase = ((size_t)b * NKV + kvh) * cap * HD;
  const rsrc_t kr = make_rsrc(kc + kvbase, (unsigned)((size_t)cap * HD * 2));
  const rsrc_t vr = make_rsrc(vc + kvbase, (unsigned)((size_t)cap * HD * 2));
  // DMA: wave w writes LDS positions (2 w + j) 64 + lane (16-byte chunks) of each matrix
  unsigned koff[2], voff[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int p = (2 * wave + j) * 64 + lane, r = p >> 4, c = p & 15;
    koff[j] = (unsigned)(r * HD * 2 + ((c ^ (r & 15)) * 16));
    voff[j] = (unsigned)(r * HD * 2 + ((c ^ (2 * (r & 7))) * 16));
  }
  typedef __attribute__((address_space(3))) void* lds_t;
  auto issue = [&](FlashDmaBuf& s, int key0) {
    const unsigned so = (unsigned)key0 * HD * 2;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(kr, (lds_t)&s.k[(2 * wave + j) * 512], 16, koff[j], so, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(vr, (lds_t)&s.v[(2 * wave + j) * 512], 16, voff[j], so, 0, 0);
    }
  };
  // MFMA operand addresses (elements) inside a buffer
  int ka_off[2][4];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int r = t * 16 + l16, c = kb * 4 + g4;
      ka_off[t][kb] = r * HD + ((c ^ (r & 15)) << 3);
    }
  const int trow = g4 * 4 + (l16 >> 2), tcol = 4 * (l16 & 3);
  int vt_off[2][8];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const int r = hh * 16 + trow, col = dt * 16 + tcol;
      vt_off[hh][dt] = r * HD + ((((col >> 3) ^ (2 * (r & 7)))) << 3) + (col & 7);
    }
  const int nfull = min(nblk, (p0 + 1) / KB);                  // blocks that need no causal mask
  // one block: wait for its DMA (this wave's, then every wave's through the barrier), start the
  // next block's DMA into the other buffer (free: every wave is past its previous block), then
  // (the wave's keys permitting) add it
  auto block = [&](const FlashDmaBuf& cur, FlashDmaBuf& nxt, int blk) {
    const int key0 = blk * KB;
    __builtin_amdgcn_s_waitcnt(0x0f70);                        // vmcnt(0)
    __syncthreads();
    if (blk + 1 < nblk) issue(nxt, key0 + KB);
    if (!wact || key0 > wlast) return;                          // wave-uniform: nothing to add
    const bool masked = blk >= nfull;
    f32x4 sc[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) d = mfma16x16x32(*(const u32x4*)&cur.k[ka_off[t][kb]], qreg[kb], d);
      sc[t] = d;
    }
    float sv[8];
    float mloc = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = key0 + t * 16 + g4 * 4 + i;
        const float v = !masked || (qok && key <= pq) ? sc[t][i] * scale_log2 : -INFINITY;
        sv[t * 4 + i] = v;
        mloc = fmaxf(mloc, v);
      }
    mloc = max_rows32(max_rows16(mloc));
    const float m_new = fmaxf(m_run, mloc);
    const float msafe = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2_hw(m_run - msafe);
    float psum = 0.f;
    unsigned pk[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float pa = exp2_hw(sv[2 * jj] - msafe);
      const float pb = exp2_hw(sv[2 * jj + 1] - msafe);
      psum += pa + pb;
      pk[jj] = pk_bf16(pa, pb);
    }
    psum = sum_rows32(sum_rows16(psum));
    l_run = l_run * alpha + psum;
    m_run = m_new;
    const u32x4 pB = {pk[0], pk[1], pk[2], pk[3]};
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const u32x2 lo = lds_read_tr16(&cur.v[vt_off[0][dt]]);
      const u32x2 hi = lds_read_tr16(&cur.v[vt_off[1][dt]]);
      acc[dt] *= alpha;
      acc[dt] = mfma16x16x32(u32x4{lo.x, lo.y, hi.x, hi.y}, pB, acc[dt]);
    }
  };
  issue(sb0, 0);
  for (int blk = 0; blk < nblk; blk += 2) {
    block(sb0, sb1, blk);
    if (blk + 1 < nblk) block(sb1, sb0, blk + 1);
  }
  if (!qok) return;
  bf16* orow = last_only ? out + ((size_t)b * NH + head) * HD : out + ((size_t)(s0 + pq) * NH + head) * HD;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) orow[dt * 16 + g4 * 4 + i] = f2bf(acc[dt][i] / l_run);
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
  hipLaunchKernelGGL(pf::qkv_prefill_kernel, dim3((T + pf::QKV_TPW - 1) / pf::QKV_TPW), dim3(256), 0,
                     stream, (const bf16*)qkv, (const bf16*)qn, (const bf16*)kn, (const bf16*)cos_t,
                     (const bf16*)sin_t, seq_start, B, T, last_only, (bf16*)q_out, (bf16*)kc,
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
  auto launch = [&](auto kern, int TQ, int nw) {
    const int ntiles = last_only ? B : T / TQ + B;
    hipLaunchKernelGGL(kern, dim3(ntiles, NKV), dim3(64 * nw), 0, stream, (const bf16*)q,
                       (const bf16*)kc, (const bf16*)vc, seq_start, B, T, (bf16*)out, NH, NKV, cap,
                       last_only, scale_log2);
  };
  switch (G) {
    case 1: launch(pf::flash_prefill_kernel<1, 4, 4, DD_PF_MINB>, 64, 4); break;
    case 2: launch(pf::flash_prefill_kernel<2, 4, 4, DD_PF_MINB>, 64, 4); break;
// G = 4 (Qwen3): one query head per wave, 16 tokens per workgroup, four workgroups per CU (four
// waves per SIMD). configs[4]'s packed prompts, one process alternating builds, us per layer, the
// same bits throughout: two heads per wave (211 VGPRs, two workgroups per CU) 368; one head per
// wave with register staging (108 VGPRs) 338; with the LDS-DMA double buffer (116 VGPRs, 32 KB
// of LDS) 314-322 against 347-354 on the same boxes. Eight waves per workgroup (32 tokens, half
// the barriers and DMA issues per token) 370, with the DMA double buffer 353 against 320; five or
// six workgroups per CU spill (349 with DMA; 676 / 805 without). The DMA kernel's last
// block may reach past a prompt's keys but not past the cache: it needs cap % 32 == 0 (the
// engine's capacities are multiples of 128), else the register-staged kernel runs.
#ifndef DD_PF_G4
#define DD_PF_G4 5
#endif
    case 4:
      if (DD_PF_G4 == 5 && cap % pf::KB == 0) launch(pf::flash_prefill_dma_kernel<DD_PF_MINB1>, 16, 4);
      else if (DD_PF_G4 == 2) launch(pf::flash_prefill_kernel<2, 2, 4, DD_PF_MINB>, 32, 4);
      else launch(pf::flash_prefill_kernel<1, 1, 4, DD_PF_MINB1>, 16, 4);
      break;
    default: launch(pf::flash_prefill_kernel<2, 1, 4, DD_PF_MINB>, 16, 4); break;   // G = 8
  }
  return launch_status();
}
