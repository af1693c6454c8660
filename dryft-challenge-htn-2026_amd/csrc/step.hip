// Persistent decode step for MI355X (gfx950): one launch runs a whole Qwen3-shape decode step.
//
// Grid: one 512-thread workgroup per CU, all co-resident. The step is a fixed list of phases:
//   0            embedding gather  h = embed[tok], per-64-column sums of squares
//   per layer    QKV GEMV (+ per-head q/k RMSNorm, RoPE, K/V cache write)
//                split-KV attention (+ log-sum-exp combine)
//                O GEMV (+ residual, sums of squares)
//                gate/up GEMV (+ SiLU x up)
//                down GEMV (+ residual, sums of squares)
//   last         lm_head GEMV (+ logits, argmax, pos += 1)
// with a grid barrier between phases.
//
// GEMV phases stream weights that were re-laid out once into "MFMA tile order" (dd_tile_weight):
// the A operand of one v_mfma_f32_16x16x32_bf16 (16 rows x 32 k) is one contiguous 1 KB block
// in lane order, so every weight load instruction of a wave reads 1 KB contiguous (a 16-row x
// 64-byte pattern only reaches ~70% of the HBM bandwidth on MI355X). NR tiles that share a group
// of rows sit next to each other per 32-k step ("step" = NR blocks). Each workgroup owns a
// contiguous range of steps (stream-K): equal bytes per CU; a row group cut between workgroups
// is finished by the last of its contributors to arrive (partials in split order: deterministic).
// The activation operand x of a phase is staged once into LDS per workgroup (only the k window
// that workgroup needs), with the RMSNorm of the residual stream applied on the way in.
//
// Barriers are split: a workgroup arrives (after its stores completed), then issues the weight
// loads of the next phase, then waits -- the HBM stream keeps going through the barrier.
//
// Cross-workgroup data inside the launch moves with sc1 stores/loads (served at the device
// coherence point, see common.h); every spin has a wall-clock timeout that raises a flag
// instead of hanging.
#include "common.h"

namespace dd {
namespace st {

constexpr int NWAVE = 8;
constexpr int NTHR = NWAVE * 64;
constexpr int HD = 128;
constexpr int SSG = 64;      // residual columns per sum-of-squares group (O/down row group)
constexpr int MAXM = 16;
constexpr int BATCH = 8;     // weight blocks (1 KB each) per prefetch batch per wave

enum : int { F_WQKV = 0, F_WO, F_WGU, F_WD, F_LN1, F_LN2, F_QN, F_KN, F_KC, F_VC, NFIELD = 16 };

// counters (ints)
constexpr int C_BAR = 0;          // [64 * (1 + xcd)]: arrivals of the XCD's workgroups
constexpr int C_EXIT = 640;
constexpr int C_GROUP = 1024;     // per row-group fixup counters
constexpr int C_ATT = C_GROUP + 8192;
constexpr int C_AM = C_ATT + 512;
constexpr int C_TOTAL = C_AM + 64;

// error flags
constexpr int E_TOKEN = 1, E_POS = 2, E_TIMEOUT = 4, E_GEOM = 8;

// tiles per row group of each GEMV phase (log2)
constexpr int LNR_QKV = 1, LNR_O = 2, LNR_GU = 1, LNR_D = 2, LNR_LM = 1;

// Thread index read through an opaque move: values derived from it cannot be hoisted out of
// the phase that computes them, so they do not stay live (in registers or spilled) across the
// whole step.
__device__ __forceinline__ int tid() {
  int t = (int)threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// Wave index within the workgroup, as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(tid() >> 6); }

// A pointer read from LDS (the layer table) lands in vector registers; buffer descriptors built
// from it would then be looped over per distinct value. It is the same in every lane: move it
// to scalar registers.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(long long v) {
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)((unsigned long long)v >> 32));
  return (T*)(((unsigned long long)hi << 32) | lo);
}

// Optional timing trace (compiled in only with -DDD_STEP_TRACE, for profiling builds): wall
// clock (100 MHz) per workgroup at phase milestones, read back with dd_step_trace.
constexpr int TR_PHASES = 192, TR_EVENTS = 12;
#ifdef DD_STEP_TRACE
__device__ unsigned long long g_trace[1024 * TR_PHASES * TR_EVENTS];
#define STEP_TRACE(p, ev)                                                                    \
  do {                                                                                      \
    if (tid() == 0 && (p) < TR_PHASES)                                                      \
      g_trace[((size_t)blockIdx.x * TR_PHASES + (p)) * TR_EVENTS + (ev)] = wall_clock64();   \
  } while (0)
#else
#define STEP_TRACE(p, ev) \
  do {                    \
  } while (0)
#endif

struct Args {
  const int64_t* layers;             // [L][NFIELD] device pointers
  const bf16* embed;                 // [V][H] natural layout (gather)
  const bf16* lm_t;                  // lm_head, tiled with NR = 2
  const bf16* fnorm;                 // final RMSNorm weight [H]
  const bf16* cos_t;
  const bf16* sin_t;
  int64_t* tok;                      // [M] in: this step's tokens, out: next tokens
  int64_t* pos;                      // [M] per-row positions, += 1 at the end
  bf16* h;                           // [2L+1][M][H] residual stream, one slot per producer
  bf16* qkv;                         // [L][M][(NH + 2 NKV) * HD] raw q|k|v
  bf16* attn;                        // [L][M][NH*HD]
  bf16* mbuf;                        // [L][M][I]
  bf16* logits;                      // [M][V]
  float* ws;
  int* ctr;
  int* err;
  int L, M, H, NH, NKV, I, V, cap, rope_rows;
  float eps;
  int phase_begin, phase_end;
  unsigned off_ss, off_part, off_att, off_am;   // workspace offsets (floats); ss: [2L+1][64][16]
  unsigned ws_floats;
};

// The steps of a phase are split into equal contiguous workgroup ranges in units of `unit`
// steps: 1 (stream-K: equal bytes per workgroup; a row group cut between workgroups is finished
// by its last contributor) or nk (whole row groups per workgroup: no cross-workgroup partials,
// balanced when there are many groups per workgroup or the epilogue needs the whole group).
struct Geo {                         // one GEMV phase for this workgroup
  const bf16* W;
  rsrc_t wr;                         // this workgroup's steps s0 .. s1 of W (range-checked)
  int lnr, nk, ngroups, S, unit, nu, s0, s1;
};

__device__ __forceinline__ Geo make_geo(const bf16* W, int rows, int K, int lnr, bool whole) {
  Geo g;
  g.W = W;
  g.lnr = lnr;
  g.nk = K >> 5;
  g.ngroups = rows >> (4 + lnr);
  g.S = g.ngroups * g.nk;
  g.unit = whole ? g.nk : 1;
  g.nu = whole ? g.ngroups : g.S;
  g.s0 = (int)((unsigned)g.nu * blockIdx.x / gridDim.x) * g.unit;
  g.s1 = (int)((unsigned)g.nu * (blockIdx.x + 1) / gridDim.x) * g.unit;
  g.wr = make_rsrc(W + ((size_t)g.s0 << (9 + lnr)), (unsigned)((g.s1 - g.s0) << (10 + lnr)));
  return g;
}

// workgroup owning global step s
__device__ __forceinline__ int wg_of_step(const Geo& g, int s) {
  return (int)(((unsigned)(s / g.unit + 1) * gridDim.x - 1) / (unsigned)g.nu);
}

// Activation buffers are write-once within a launch: the residual stream h has one slot per
// phase that produces it (embedding -> 0, O of layer l -> 2l+1, down of layer l -> 2l+2), raw
// q|k|v, attention output and SiLU output one slot per layer. A slot is only read after the phase that
// writes it (through to the device coherence point, sc1) and every cache is clean at launch
// start, so no cache can hold a stale copy: readers use plain cached loads, and each XCD's L2
// fetches a line once for all its workgroups.
constexpr int SS_SLOT = 64 * MAXM;   // floats per sums-of-squares slot ([H/64 <= 64][16])
__device__ __forceinline__ bf16* h_slot(const Args& a, int k) {
  return a.h + (size_t)k * a.M * a.H;
}
__device__ __forceinline__ float* ss_slot(const Args& a, int k) {
  return a.ws + a.off_ss + (size_t)k * SS_SLOT;
}
__device__ __forceinline__ bf16* qkv_slot(const Args& a, int l) {
  return a.qkv + (size_t)l * a.M * (a.NH + 2 * a.NKV) * HD;
}
__device__ __forceinline__ bf16* attn_slot(const Args& a, int l) {
  return a.attn + (size_t)l * a.M * a.NH * HD;
}
__device__ __forceinline__ bf16* m_slot(const Args& a, int l) {
  return a.mbuf + (size_t)l * a.M * a.I;
}
// split-attention partials of a layer ([G][2][heads per kv head][ATT_REC] fp32): write-once
__device__ __forceinline__ float* att_part(const Args& a, int l) {
  return a.ws + a.off_att + (size_t)l * gridDim.x * 2 * (a.NH / a.NKV) * (HD + 4);
}
// plain (cached) 16-byte buffer load; out-of-range offsets read zeros
__device__ __forceinline__ u32x4 ldb128(rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// first step of workgroup c's range (ranges of workgroups between two owners may be empty)
__device__ __forceinline__ int step0_of(const Geo& g, int c) {
  return (int)((unsigned)g.nu * c / gridDim.x) * g.unit;
}

// Issue the wave's weight loads for wave-step index j0 .. (a batch of BATCH blocks). The loads
// are unconditional buffer loads through the workgroup's range descriptor: a step past the
// range reads zeros without touching memory, and with no branches around the loads the compiler
// waits for each buffer register on its own (vmcnt(n)) instead of draining the queue. The whole
// offset is in the VGPR operand: the SGPR offset is not range-checked.
constexpr int CP_NT = 2;   // buffer cache-policy bit nt (streaming)

template <int NR>
__device__ __forceinline__ void issue_batch(const Geo& g, int j0, u32x4 (&buf)[BATCH]) {
  const int lane = tid() & 63, wave = wave_id();
#pragma unroll
  for (int b = 0; b < BATCH; ++b) {
    const int u = b / NR, t = b % NR;
    const int sl = wave + NWAVE * (j0 + u);          // step relative to s0
    buf[b] = __builtin_amdgcn_raw_buffer_load_b128(g.wr, lane * 16 + ((sl * NR + t) << 10), 0,
                                                   CP_NT);
  }
}

// GEMV phases carve their LDS out of one region: per-wave partial tiles (NR x 8 KB), the
// reduced group tile, then the staged activation window.
constexpr int GBUF = 112 * 1024;
constexpr int RES_BYTES = 8 * 16 * (MAXM + 1) * 4;
__host__ __device__ constexpr int x_capacity(int NR) { return GBUF - NR * NWAVE * 256 * 4 - RES_BYTES; }

constexpr int LNW_KS = 128;                   // k-steps of the norm weight staged in LDS
constexpr int MAXG = 512;                     // workgroups (CUs) the step kernel supports
constexpr int MAXG_HEADS = 8;                 // query heads per kv head
constexpr int MAXL = 64;                      // layers
constexpr int LFIELDS = 10;                   // layer-table fields the phases read

struct Shared {
  union {
    unsigned char g[GBUF];                    // GEMV phases (see GemvLds)
    struct {                                  // attention
      bf16 v[NWAVE][32][HD + 8];
      float mrg[NWAVE][MAXG_HEADS][HD];
      bf16 qn[32][HD];                        // normalised, rotated query heads of the segments
    } a;
  } u;
  float rs[MAXM];                             // per-row 1/rms of the staged x
  float rsp[NTHR / MAXM][MAXM];               // partial sums of squares behind rs
  float ms[NWAVE][16];
  float ls[NWAVE][16];
  float bestv[MAXM];
  int besti[MAXM];
  int flag;
  int bail;                                   // a barrier wait timed out: stop waiting
  int xrs;                                    // staged x row stride (bytes)
  int xksf, xnw;                              // staged window: first k-step, width
  int units[MAXM + 1];                        // attention unit prefix sums
  int seg[32][4];                             // attention segments: b, kvh, first block, blocks
  int nseg, segnext;
  long long posv[MAXM];                       // this step's positions (read once at launch)
  int afirst[MAXG + 1];                       // attention: first unit of each workgroup
  int aG;                                     // attention: workgroups holding units
  long long ltab[MAXL][LFIELDS];              // the layer table, copied once per launch
  int pinfo[MAXM * 32][8];                    // O staging: per (row, kv head) fw, lw, record
                                              // offsets of its first 3 contributors (-1: none), S
  bf16 lnw[LNW_KS * 32];                      // staged norm weight window (<= LNW_KS k-steps)
};

static_assert(sizeof(Shared) <= 160 * 1024, "LDS budget of one CU");

// ---------------------------------------------------------------------------------------------
template <int NR>
struct GemvLds {
  float (*red)[NR][256];                      // [NWAVE][NR][256]
  float (*res)[MAXM + 1];                     // [NR*16][MAXM+1]
  unsigned char* x;
  __device__ explicit GemvLds(Shared& sh)
      : red((float(*)[NR][256])sh.u.g),
        res((float(*)[MAXM + 1])(sh.u.g + NR * NWAVE * 256 * 4)),
        x(sh.u.g + NR * NWAVE * 256 * 4 + RES_BYTES) {}
};

// barrier (split)
__device__ __forceinline__ void bar_arrive(const Args& a, unsigned epoch) {
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();
  if (tid() == 0)                            // no return value: nothing to wait for
    __hip_atomic_fetch_add((unsigned*)a.ctr + C_BAR + 64 * (1 + (blockIdx.x & 7)), 1u,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Released when every XCD's counter has all its workgroups' arrivals: lanes 0..7 of wave 0 read
// the 8 counters in one load, so the release is one memory latency after the last arrival.
__device__ __forceinline__ void bar_wait(const Args& a, Shared& sh, unsigned epoch) {
  if (wave_id() == 0 && !sh.bail) {
    const int lane = tid() & 63;
    const unsigned target = epoch * (unsigned)(gridDim.x >> 3);
    const rsrc_t cr = make_rsrc(a.ctr + C_BAR, 9 * 64 * 4);
    const unsigned off = lane < 8 ? (unsigned)(64 * (1 + lane) * 4) : 0xfffffff0u;
    const unsigned long long t0 = wall_clock64();
    for (;;) {
      const unsigned v = ldc_u32(cr, off);
      if (__all(lane >= 8 || v >= target)) break;
      __builtin_amdgcn_s_sleep(2);
      if (wall_clock64() - t0 > 20000000ull) {  // 200 ms: report, stop waiting from now on
        if (lane == 0) {
          atomicOr(a.err, E_TIMEOUT);
          sh.bail = 1;
        }
        break;
      }
    }
  }
  __builtin_amdgcn_s_barrier();
}

// ---------------------------------------------------------------------------------------------
// activation staging: x window [ksf, ksf + nw) (cyclic over nk k-steps) of an [M][K] source into
// LDS rows of stride xrs bytes. NORM: x = bf16(bf16(h * r[m]) * lnw[k]) with r from the ss groups.
// Every load of a batch is issued before the first is used (one memory latency per batch of
// SBATCH items per thread), and the first batch is in flight while r is reduced. The norm
// weight window (the same for every row) is staged once into LDS.
constexpr int SBATCH = 12;

__device__ __forceinline__ unsigned stage_off(int it, int nw, int ksf, int nk, int K, int* lds) {
  const int m = it / (nw * 4);
  const int rem = it - m * nw * 4;
  const int w = rem >> 2, e = rem & 3;
  int ks = ksf + w;
  if (ks >= nk) ks -= nk;
  *lds = w * 64 + e * 16;
  return (unsigned)((size_t)m * K + ks * 32 + e * 8);
}

// The norm weight of the window does not depend on the previous phase: its load is issued before
// the barrier wait (thread t < 4 * window holds 16 bytes of k-step t / 4).
__device__ __forceinline__ u32x4 lnw_prefetch(const Geo& g, const bf16* lnw, int K) {
  const int t = tid();
  const int ksf = g.s1 > g.s0 ? g.s0 % g.nk : 0;
  const int nw = g.s1 > g.s0 ? min(g.s1 - g.s0, g.nk) : 0;
  int ks = ksf + (t >> 2);
  if (ks >= g.nk) ks -= g.nk;
  const rsrc_t r = make_rsrc(lnw, (unsigned)(K * 2));
  return ldb128(r, t < nw * 4 ? (unsigned)((ks * 32 + (t & 3) * 8) * 2) : 0xfffffff0u);
}

__device__ __forceinline__ void stage_x(const Args& a, Shared& sh, unsigned char* xb, const Geo& g,
                                        int K, const bf16* src, const bf16* lnw, u32x4 lwv,
                                        const float* ss, int p) {
  const int M = a.M;
  const int t = tid();
  int ksf = 0, nw = 0;
  if (g.s1 > g.s0) {
    ksf = g.s0 % g.nk;
    nw = min(g.s1 - g.s0, g.nk);
  }
  const int xrs = nw * 64 + 16;
  const int W = nw * 4;                       // 16-byte items per row
  const int items = M * W;
  const rsrc_t sr = make_rsrc(src, (unsigned)((size_t)M * K * 2));
  // thread t takes items t, t + NTHR, ... (item = m * W + r); (m, r) advance without dividing
  const int Wd = W > 0 ? W : 1;
  const int dq = NTHR / Wd, dr = NTHR - dq * Wd;
  int cm = t / Wd, cr = t - (t / Wd) * Wd;    // the thread's next item
  u32x4 v[SBATCH];
  int lo_[SBATCH], m_[SBATCH];                // LDS byte offset within the row, row (-1: none)
  auto issue = [&]() {
#pragma unroll
    for (int b = 0; b < SBATCH; ++b) {
      const bool ok = cm < M;
      const int w = cr >> 2, e = cr & 3;
      int ks = ksf + w;
      if (ks >= g.nk) ks -= g.nk;
      lo_[b] = w * 64 + e * 16;
      m_[b] = ok ? cm : -1;
      v[b] = ldb128(sr, ok ? (unsigned)((cm * K + ks * 32 + e * 8) * 2) : 0xfffffff0u);
      cr += dr;
      cm += dq;
      if (cr >= Wd) {
        cr -= Wd;
        ++cm;
      }
    }
  };
  // the sums of squares behind r are loaded first (one latency with the window): thread (q, m)
  // takes groups q and q + 32 of row m (H / SSG <= 64), unconditionally (range-checked)
  const int rm = t & (MAXM - 1), rq = t / MAXM;
  float ss0 = 0.f, ss1 = 0.f;
  if (lnw != nullptr) {
    const rsrc_t ssr = make_rsrc(ss, (unsigned)(SS_SLOT * 4));
    const int nq = a.H / SSG;
    ss0 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        ssr, rm < M && rq < nq ? (unsigned)((rq * MAXM + rm) * 4) : 0xfffffff0u, 0, 0));
    ss1 = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
        ssr, rm < M && rq + NTHR / MAXM < nq ? (unsigned)(((rq + NTHR / MAXM) * MAXM + rm) * 4)
                                             : 0xfffffff0u, 0, 0));
  }
  issue();
  // norm phases have K = H <= 64 * SSG (checked on the host): the window fits LNW_KS k-steps
  if (lnw != nullptr) {
    if (t < nw * 4) *(u32x4*)&sh.lnw[t * 8] = lwv;
    // r[m] = 1/sqrt(sum_q ss[q][m] / H + eps): row m adds the 32 partials in order
    sh.rsp[rq][rm] = ss0 + ss1;
    __syncthreads();
    if (t < M) {
      float r = 0.f;
#pragma unroll 8
      for (int q = 0; q < NTHR / MAXM; ++q) r += sh.rsp[q][t];
      sh.rs[t] = rsqrt_ieee(r / (float)a.H + a.eps);
    }
  }
  STEP_TRACE(p, 8);
  if (t == 0) {
    sh.xrs = xrs;
    sh.xksf = ksf;
    sh.xnw = nw;
  }
  __syncthreads();
  for (int base = 0; base < items; base += SBATCH * NTHR) {
    if (base > 0) issue();
#pragma unroll
    for (int b = 0; b < SBATCH; ++b) {
      const int m = m_[b];
      if (m < 0) break;
      u32x4 x = v[b];
      if (lnw != nullptr) {
        const float r = sh.rs[m];
        const u32x4 wv = *(const u32x4*)&sh.lnw[(lo_[b] >> 4) * 8];
        const unsigned hw[4] = {x.x, x.y, x.z, x.w}, ww[4] = {wv.x, wv.y, wv.z, wv.w};
        unsigned o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          o[j] = pk_bf16(rbf(lo_bf(hw[j]) * r) * lo_bf(ww[j]), rbf(hi_bf(hw[j]) * r) * hi_bf(ww[j]));
        x = u32x4{o[0], o[1], o[2], o[3]};
      }
      *(u32x4*)(xb + m * xrs + lo_[b]) = x;
    }
  }
  STEP_TRACE(p, 9);
  __syncthreads();
}

// ---------------------------------------------------------------------------------------------
// GEMV epilogues. `res[row][m]` holds the fp32 sums of the group's NR*16 weight rows.
enum { EPI_QKV = 0, EPI_RES = 1, EPI_SILU = 2, EPI_LOGITS = 3 };

__device__ __forceinline__ void epi_qkv(const Args& a, float (*res)[MAXM + 1], int layer, int grp) {
  // raw q|k|v rows grp*32 .. +32 for every token (q/k RMSNorm, RoPE and the K/V cache write
  // happen in the attention phase, which holds whole heads)
  constexpr int ROWS = 16 << LNR_QKV;
  const int M = a.M;
  const int t = tid();
  const int r = t % ROWS, m = t / ROWS;
  const int nqkv = (a.NH + 2 * a.NKV) * HD;
  if (m < M) {
    const rsrc_t qr = make_rsrc(qkv_slot(a, layer), (unsigned)((size_t)M * nqkv * 2));
    stc_b16(qr, (unsigned)((size_t)m * nqkv + grp * ROWS + r) * 2, f2bf(res[r][m]));
  }
}

// The residual input of the thread's two columns (thread t: row t / 32, columns 2 (t % 32) ..),
// loaded when the group's flush starts so that its latency is off the finisher's chain.
__device__ __forceinline__ unsigned epi_res_input(const Args& a, int grp, int hk) {
  const int t = tid();
  const int m = t >> 5, c2 = (t & 31) * 2;
  const rsrc_t hin = make_rsrc(h_slot(a, hk - 1), (unsigned)((size_t)a.M * a.H * 2));
  return __builtin_amdgcn_raw_buffer_load_b32(
      hin, m < a.M ? (unsigned)((size_t)m * a.H + grp * SSG + c2) * 2 : 0xfffffff0u, 0, 0);
}

__device__ __forceinline__ void epi_res(const Args& a, float (*res)[MAXM + 1], int grp, int hk,
                                        unsigned hv2) {
  // 64 residual columns grp*64 .. : h[hk] = bf16(h[hk-1] + bf16(sum)); ss[hk][grp][m] = sum h^2
  const int M = a.M;
  const int t = tid();
  const int m = t >> 5, c2 = (t & 31) * 2;   // two columns per thread
  const unsigned bytes = (unsigned)((size_t)M * a.H * 2);
  const rsrc_t hout = make_rsrc(h_slot(a, hk), bytes);
  float q = 0.f;
  if (m < M) {
    const unsigned off = (unsigned)((size_t)m * a.H + grp * SSG + c2) * 2;
    const float h0 = rbf(lo_bf(hv2) + rbf(res[c2][m]));
    const float h1 = rbf(hi_bf(hv2) + rbf(res[c2 + 1][m]));
    stc_u32(hout, off, (unsigned)f2bf(h0) | ((unsigned)f2bf(h1) << 16));
    q = h0 * h0 + h1 * h1;
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
  if (m < M && (t & 31) == 0) {
    const rsrc_t ssr = make_rsrc(ss_slot(a, hk), (unsigned)(SS_SLOT * 4));
    stc_f32(ssr, (unsigned)(grp * MAXM + m) * 4, q);
  }
}

__device__ __forceinline__ void epi_silu(const Args& a, float (*res)[MAXM + 1], int grp, int layer) {
  // rows 0..15: gate features grp*16.., rows 16..31: the matching up rows
  const int M = a.M;
  const int t = tid();
  if (t >= 16 * MAXM) return;
  const int m = t >> 4, f = t & 15;
  if (m >= M) return;
  const float g = rbf(res[f][m]);
  const float u = rbf(res[16 + f][m]);
  const float s = rbf(g / (1.0f + expf(-g)));
  const rsrc_t mr = make_rsrc(m_slot(a, layer), (unsigned)((size_t)M * a.I * 2));
  stc_b16(mr, (unsigned)((size_t)m * a.I + grp * 16 + f) * 2, f2bf(s * u));
}

__device__ __forceinline__ bool am_better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

__device__ __forceinline__ void epi_logits(const Args& a, Shared& sh, float (*res)[MAXM + 1], int grp) {
  // 32 vocab rows grp*32 ..; logits out + the workgroup's running argmax per token
  const int M = a.M;
  const int t = tid();
  const int m = t >> 5, v = t & 31;
  float val = -INFINITY;
  int idx = 0x7fffffff;
  if (m < M) {
    const bf16 b = f2bf(res[v][m]);
    const int col = grp * 32 + v;
    a.logits[(size_t)m * a.V + col] = b;
    val = bf2f(b);
    idx = col;
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) {
    const float ov = __shfl_xor(val, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (am_better(ov, oi, val, idx)) { val = ov; idx = oi; }
  }
  if (m < M && v == 0 && am_better(val, idx, sh.bestv[m], sh.besti[m])) {
    sh.bestv[m] = val;
    sh.besti[m] = idx;
  }
}

// Run the epilogue of a row group whose fp32 sums are in res.
template <int EPI>
__device__ __forceinline__ void run_epilogue(const Args& a, Shared& sh, float (*res)[MAXM + 1],
                                             int grp, int layer, unsigned hres) {
  if (EPI == EPI_QKV) epi_qkv(a, res, layer, grp);
  else if (EPI == EPI_RES) epi_res(a, res, grp, layer, hres);   // layer: output h slot
  else if (EPI == EPI_SILU) epi_silu(a, res, grp, layer);
  else epi_logits(a, sh, res, grp);
}

// Reduce the waves' tiles of one row group and finish it: directly when this workgroup owns the
// whole group, else through partials, finished by the last contributor to arrive (partials
// summed in workgroup order, CB contributors' loads in flight at once; an empty contributor
// adds +0).
template <int NR, int EPI>
__device__ __forceinline__ void flush_group(const Args& a, Shared& sh, const Geo& g, int grp, int layer,
                            f32x4 (&acc)[NR], int p = -1) {
  const int lane = tid() & 63, wave = wave_id();
  const int M = a.M;
  GemvLds<NR> L(sh);
  const unsigned hres = EPI == EPI_RES ? epi_res_input(a, grp, layer) : 0u;
#pragma unroll
  for (int t = 0; t < NR; ++t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) L.red[wave][t][lane * 4 + i] = acc[t][i];
    acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): LDS writes done (vmcnt untouched)
  __builtin_amdgcn_s_barrier();
  // res[row][m], row = t*16 + (lane/16)*4 + i of the D layout, m = lane % 16
  for (int e = tid(); e < NR * 256; e += NTHR) {
    const int t = e >> 8, ln = (e >> 2) & 63, i = e & 3;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) s += L.red[w][t][ln * 4 + i];
    L.res[t * 16 + (ln >> 4) * 4 + i][ln & 15] = s;
  }
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_s_barrier();
  const int first = wg_of_step(g, grp * g.nk);
  const int last = wg_of_step(g, (grp + 1) * g.nk - 1);
  bool finish = true;
  if (first != last) {
    // partial: slot 0 = the group holding this workgroup's first step, slot 1 = its last
    const int rows = NR * 16;
    const unsigned slot_floats = (unsigned)(rows * MAXM);
    const rsrc_t pr = make_rsrc(a.ws + a.off_part, (unsigned)(gridDim.x * 2 * slot_floats * 4));
    const int myslot = (grp == g.s0 / g.nk) ? 0 : 1;
    // whole [rows][MAXM] tiles (columns >= M carry finite values nobody reads): no division
    constexpr int PE = NR * 16 * MAXM;       // floats per partial
    const unsigned mybase = (blockIdx.x * 2 + myslot) * slot_floats * 4;
    for (int e = tid(); e < PE; e += NTHR) stc_f32(pr, mybase + e * 4, L.res[e >> 4][e & 15]);
    // contributors: the workgroups first..last whose step range is not empty
    int ncontrib = 0;
    for (int c = first; c <= last; ++c) ncontrib += step0_of(g, c + 1) > step0_of(g, c);
    STEP_TRACE(p, 4);
    finish = arrive_last(a.ctr + C_GROUP + grp, ncontrib, &sh.flag);
    STEP_TRACE(p, 5);
    if (finish) {
      constexpr int EPT = (PE + NTHR - 1) / NTHR;
      constexpr int CB = 8;
      constexpr unsigned NONE = 0x80000000u;  // past the descriptor's range: reads 0
      float acc[EPT];
#pragma unroll
      for (int i = 0; i < EPT; ++i) acc[i] = 0.f;
      for (int c0 = first; c0 <= last; c0 += CB) {
        // contributor record bases (workgroup-uniform), then every load unconditional
        unsigned cb[CB];
        int cs = step0_of(g, c0);
#pragma unroll
        for (int j = 0; j < CB; ++j) {
          const int c = c0 + j;
          const int cn = step0_of(g, c + 1);
          const bool ok = c <= last && cn > cs;
          cb[j] = ok ? (unsigned)((c * 2 + (cs >= grp * g.nk ? 0 : 1)) * slot_floats * 4) : NONE;
          cs = cn;
        }
        float pv[EPT][CB];
#pragma unroll
        for (int i = 0; i < EPT; ++i) {
          const int e = tid() + i * NTHR;
#pragma unroll
          for (int j = 0; j < CB; ++j) pv[i][j] = ldc_f32(pr, (e < PE ? cb[j] : NONE) + e * 4);
        }
#pragma unroll
        for (int i = 0; i < EPT; ++i)
#pragma unroll
          for (int j = 0; j < CB; ++j) acc[i] += pv[i][j];
      }
#pragma unroll
      for (int i = 0; i < EPT; ++i) {
        const int e = tid() + i * NTHR;
        if (e < PE) L.res[e >> 4][e & 15] = acc[i];
      }
      __syncthreads();
      STEP_TRACE(p, 6);
    }
  }
  if (finish) run_epilogue<EPI>(a, sh, L.res, grp, layer, hres);
  if (finish && first != last) STEP_TRACE(p, 7);
  __builtin_amdgcn_s_waitcnt(0xc07f);
  __builtin_amdgcn_s_barrier();
}

// Consume U wave-steps j0 .. j0+U-1 from a prefetch buffer (static register indices: data still
// in flight is never copied, so each MFMA waits only for its own loads). A wave's steps inside
// one batch span at most two row groups (nk >= NWAVE * U): `cur` accumulates the oldest unflushed
// group, `nxt` the one after it.
template <int NR>
__device__ __forceinline__ void gemv_consume(const Geo& g, const u32x4 (&buf)[BATCH], int j0,
                                             int nmine, int gcur, const unsigned char* xrow_p,
                                             int ksf, f32x4 (&cur)[NR], f32x4 (&nxt)[NR]) {
  constexpr int U = BATCH / NR;
  const int wave = wave_id();
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = j0 + u;
    if (j < nmine) {
      const int s = g.s0 + wave + NWAVE * j;
      const int grp = s / g.nk;
      int w = s - grp * g.nk - ksf;
      if (w < 0) w += g.nk;
      const u32x4 xv = *(const u32x4*)(xrow_p + w * 64);
      if (grp == gcur) {
#pragma unroll
        for (int t = 0; t < NR; ++t) cur[t] = mfma16x16x32(buf[u * NR + t], xv, cur[t]);
      } else {
#pragma unroll
        for (int t = 0; t < NR; ++t) nxt[t] = mfma16x16x32(buf[u * NR + t], xv, nxt[t]);
      }
    }
  }
}

// Flush the row groups this wave has moved past (all remaining ones when done): every wave of
// the workgroup flushes every group of the range in order (flush_group synchronises them).
template <int NR, int EPI>
__device__ __forceinline__ void gemv_flush_to(const Args& a, Shared& sh, const Geo& g, int layer,
                                              int target, int seg0, int& flushed,
                                              f32x4 (&cur)[NR], f32x4 (&nxt)[NR], int p) {
  while (flushed < target) {
    flush_group<NR, EPI>(a, sh, g, seg0 + flushed, layer, cur, p);   // leaves cur zeroed
#pragma unroll
    for (int t = 0; t < NR; ++t) {
      cur[t] = nxt[t];
      nxt[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    ++flushed;
  }
}

// Consume this workgroup's steps of a GEMV phase. On entry A/B hold (in flight) the wave's
// batches 0 and 1; batches alternate between them. Returns with nothing in flight.
template <int NR, int EPI>
__device__ __forceinline__ void gemv_phase(const Args& a, Shared& sh, const Geo& g, int layer,
                                           u32x4 (&A)[BATCH], u32x4 (&B)[BATCH], int p) {
  constexpr int U = BATCH / NR;   // steps per batch
  const int lane = tid() & 63, wave = wave_id();
  const int M = a.M;
  const int nmine = g.s1 - g.s0 > wave ? (g.s1 - g.s0 - wave + NWAVE - 1) / NWAVE : 0;
  const int seg0 = g.s1 > g.s0 ? g.s0 / g.nk : 0;
  const int nseg = g.s1 > g.s0 ? (g.s1 - 1) / g.nk - seg0 + 1 : 0;
  const unsigned char* xrow_p =
      GemvLds<NR>(sh).x + min(lane & 15, M - 1) * sh.xrs + (lane >> 4) * 16;
  const int ksf = sh.xksf;
  f32x4 cur[NR], nxt[NR];
#pragma unroll
  for (int t = 0; t < NR; ++t) {
    cur[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    nxt[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  int flushed = 0;
  // group of the wave's step j
  auto grp_of = [&](int j) { return (g.s0 + wave + NWAVE * j) / g.nk - seg0; };
  for (int j0 = 0;; j0 += 2 * U) {
    if (j0 < nmine) {
      gemv_consume<NR>(g, A, j0, nmine, seg0 + flushed, xrow_p, ksf, cur, nxt);
      issue_batch<NR>(g, j0 + 2 * U, A);
      __builtin_amdgcn_sched_barrier(0);    // keep the refill ahead of the next batch's MFMAs
      gemv_flush_to<NR, EPI>(a, sh, g, layer, grp_of(min(j0 + U, nmine) - 1), seg0, flushed,
                             cur, nxt, p);
    }
    if (j0 + U < nmine) {
      gemv_consume<NR>(g, B, j0 + U, nmine, seg0 + flushed, xrow_p, ksf, cur, nxt);
      issue_batch<NR>(g, j0 + 3 * U, B);
      __builtin_amdgcn_sched_barrier(0);
    }
    const bool done = j0 + 2 * U >= nmine;
    gemv_flush_to<NR, EPI>(a, sh, g, layer,
                           done ? nseg : grp_of(min(j0 + 2 * U, nmine) - 1), seg0, flushed,
                           cur, nxt, p);
    if (done) break;
  }
}

// ---------------------------------------------------------------------------------------------
// attention. The 32-key blocks of every (row, kv head) are laid end to end (row-major, then kv
// head) and split into equal contiguous workgroup ranges, so every workgroup streams the same
// number of K/V bytes whatever the per-row context lengths. A workgroup takes its range as
// segments, one per (row, kv head) it touches; its 8 waves share a segment's blocks.
// Per segment: the G query heads are RMS-normalised and rotated from the raw q|k|v (engine.py
// qkv_post), the segment holding the newest block also normalises/rotates k and writes K/V at
// pos; then S^T = K.Q^T and O^T += V^T.P^T on MFMA (P rounded to bf16), the waves merge through
// LDS, and a (row, kv head) split over workgroups is combined (log-sum-exp, in workgroup order)
// by the last contributor to arrive.

// q/k head RMSNorm and RoPE for one head held by a wave: lane l holds dims l and l + 64, with
// the norm weight (w0, w1) and the position's cos/sin values (c0, c1, s0, s1) of those dims.
__device__ __forceinline__ void head_norm_rope(const Args& a, float& x0, float& x1, float w0,
                                               float w1, float c0, float c1, float s0, float s1,
                                               bool rope) {
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float r = rsqrt_ieee(ss / (float)HD + a.eps);
  const float n0 = rbf(rbf(x0 * r) * w0);
  const float n1 = rbf(rbf(x1 * r) * w1);
  if (rope) {
    x0 = rbf(rbf(n0 * c0) + rbf(-n1 * s0));
    x1 = rbf(rbf(n1 * c1) + rbf(n0 * s1));
  } else {
    x0 = n0;
    x1 = n1;
  }
}

// The units are split over the first Ga workgroups, Ga = min(grid, T / ATT_MINU): a small
// workload (short contexts, B = 1) stays on fewer workgroups, so a (row, kv head) is split over
// few contributors. Partition arithmetic stays in 32 bits (units x workgroups < 2^31, checked
// on the host).
constexpr int ATT_MINU = 16;
__device__ __forceinline__ int attn_owner(int T, int Ga, int i) {  // workgroup of global unit i
  return (int)(((unsigned)(i + 1) * Ga - 1) / (unsigned)T);
}
__device__ __forceinline__ int attn_first(int T, int Ga, int c) {  // first unit of workgroup c
  return c >= Ga ? T : (int)((unsigned)T * c / Ga);
}

// Partition units of one (row, kv head): ATT_OVH units for its fixed per-segment latency
// (prologue, wave merge, output) followed by one unit per 32-key block, so a workgroup holding
// many short segments gets fewer blocks.
constexpr int ATT_OVH = 12;
constexpr int ATT_REC = HD + 4;      // split partial record: o[128], m, l, 2 pad (16-byte rows)
constexpr int ATT_QN = 32;           // query heads of all segments of one prologue round
constexpr int SA_PQ = 3;             // contributors per (row, kv head) whose records the O
                                     // staging loads in its first pass

// units[b]: first partition unit of row b (rows with no keys have none); units[M] = total
__device__ __forceinline__ void attn_partition(const Args& a, Shared& sh, bool flag_errors) {
  if (tid() < 64) {                          // wave 0: lane b = row b, prefix sum by shuffles
    const int b = tid();
    int cnt = 0;
    if (b < a.M) {
      const int64_t p = sh.posv[b];
      if (flag_errors && (p < 0 || p >= a.cap || p >= a.rope_rows) && blockIdx.x == 0)
        atomicOr(a.err, E_POS);
      const int Lb = (int)min<int64_t>(max<int64_t>(p + 1, 0), (int64_t)a.cap);
      const int nblk = (Lb + 31) >> 5;
      cnt = nblk > 0 ? a.NKV * (ATT_OVH + nblk) : 0;
    }
    int inc = cnt;
#pragma unroll
    for (int o = 1; o <= MAXM; o <<= 1) {      // lanes 0..MAXM: lane M sums all M rows
      const int v = __shfl_up(inc, o, 64);
      if (b >= o) inc += v;
    }
    if (b <= a.M) sh.units[b] = inc - cnt;   // lane M: cnt = 0, inc = total
  }
  __syncthreads();
  const int T = sh.units[a.M];
  const int Ga = max(1, min((int)gridDim.x, T / ATT_MINU));
  for (int c = tid(); c <= (int)gridDim.x; c += NTHR) sh.afirst[c] = attn_first(T, Ga, c);
  if (tid() == 0) sh.aG = Ga;
  __syncthreads();
}

// The attention partition depends only on this step's positions: computed once per launch,
// with the O staging's per-(row, kv head) contributor table (fw, lw, record offsets of the
// first contributors, S).
__device__ __forceinline__ void attn_setup(const Args& a, Shared& sh, bool flag_errors) {
  const int M = a.M, NKV = a.NKV, G = a.NH / a.NKV;
  attn_partition(a, sh, flag_errors);
  const int T = sh.units[M];
  for (int pi = tid(); pi < M * NKV; pi += NTHR) {
    const int m = pi / NKV, kvh = pi - m * NKV;
    const int64_t pp = sh.posv[m];
    const int Lb = (int)min<int64_t>(max<int64_t>(pp + 1, 0), (int64_t)a.cap);
    const int nblk = (Lb + 31) >> 5;
    int* pin = sh.pinfo[pi];
    if (nblk == 0) {
      pin[0] = 0;
      pin[1] = -1;                                                  // no keys: zeros
      for (int q = 0; q < SA_PQ; ++q) pin[2 + q] = -1;
      continue;
    }
    const int S = sh.units[m] + kvh * (ATT_OVH + nblk);
    const int fw = attn_owner(T, sh.aG, S + ATT_OVH), lw = attn_owner(T, sh.aG, S + ATT_OVH + nblk - 1);
    pin[0] = fw;
    pin[1] = lw;
#pragma unroll
    for (int q = 0; q < SA_PQ; ++q) {
      const int c = fw + q;
      const bool ok = lw > fw && c <= lw && sh.afirst[c + 1] > sh.afirst[c];
      pin[2 + q] = ok ? (int)(((c * 2 + (sh.afirst[c] >= S ? 0 : 1)) * G) * ATT_REC * 4) : -1;
    }
    pin[6] = S;
  }
  __syncthreads();
}

__device__ __forceinline__ void attention_phase(const Args& a, Shared& sh, int layer, int p) {
  const int M = a.M, NKV = a.NKV, NH = a.NH, G = NH / NKV;
  const int lane = tid() & 63, wave = wave_id();
  const int l16 = lane & 15, g4 = lane >> 4;
  const long long* lp = sh.ltab[layer];
  bf16* kc = uniform_ptr<bf16>(lp[F_KC]);
  bf16* vc = uniform_ptr<bf16>(lp[F_VC]);
  const bf16* qnw = uniform_ptr<const bf16>(lp[F_QN]);
  const bf16* knw = uniform_ptr<const bf16>(lp[F_KN]);
  const int nqkv = (NH + 2 * NKV) * HD;
  const float scale_log2 = (1.0f / sqrtf((float)HD)) * 1.4426950408889634f;
  STEP_TRACE(p, 4);
  const int i0 = sh.afirst[blockIdx.x], i1 = sh.afirst[blockIdx.x + 1];
  const unsigned kvbytes = (unsigned)((size_t)M * NKV * a.cap * HD * 2);
  const rsrc_t kwr = make_rsrc(kc, kvbytes), vwr = make_rsrc(vc, kvbytes);
  const rsrc_t rawr = make_rsrc(qkv_slot(a, layer), (unsigned)((size_t)M * nqkv * 2));
  const rsrc_t qwr = make_rsrc(qnw, HD * 2), kwr_n = make_rsrc(knw, HD * 2);
  const rsrc_t cosr = make_rsrc(a.cos_t, (unsigned)((size_t)a.rope_rows * HD * 2));
  const rsrc_t sinr = make_rsrc(a.sin_t, (unsigned)((size_t)a.rope_rows * HD * 2));
  const rsrc_t orr = make_rsrc(attn_slot(a, layer), (unsigned)((size_t)M * NH * HD * 2));
  const unsigned rec = ATT_REC;
  const rsrc_t pr = make_rsrc(att_part(a, layer), (unsigned)((size_t)gridDim.x * 2 * G * rec * 4));
  const int maxseg = ATT_QN / G;
  bool first_seg = true;
  for (int i = i0; i < i1;) {
    // ---- this round's segments: (row, kv head) pairs whose blocks meet [i, i1)
    if (tid() == 0) {
      int n = 0, u = i;
      while (u < i1 && n < maxseg) {
        int b = 0;
        while (b + 1 < M && sh.units[b + 1] <= u) ++b;
        const int Lb = (int)min<int64_t>(max<int64_t>(sh.posv[b] + 1, 0), (int64_t)a.cap);
        const int nblk = (Lb + 31) >> 5;
        const int per = ATT_OVH + nblk;
        const int kvh = (u - sh.units[b]) / per;
        const int S = sh.units[b] + kvh * per;                      // pair start (overhead units)
        const int lo = max(u, S + ATT_OVH), hi = min(i1, S + per);
        if (hi > lo) {
          sh.seg[n][0] = b;
          sh.seg[n][1] = kvh;
          sh.seg[n][2] = lo - S - ATT_OVH;
          sh.seg[n][3] = hi - lo;
          ++n;
        }
        u = S + per;
      }
      sh.nseg = n;
      sh.segnext = u;                                               // where the next round starts
    }
    __syncthreads();
    const int nsg = sh.nseg;
    const int inext = sh.segnext;
    // one 32-key block of K (S^T operand: lane = key l16 of half t, dims kb*32 + g4*8) and V
    // (rows of 16 keys x 8 dims, transposed through LDS below)
    u32x4 kreg[2][4], vreg[8];
    auto load_block = [&](size_t kvbase, int key0) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        int key = key0 + t * 16 + l16;
        key = key < a.cap ? key : a.cap - 1;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) kreg[t][kb] = ld16(kc + kvbase + (size_t)key * HD + kb * 32 + g4 * 8);
      }
#pragma unroll
      for (int it = 0; it < 8; ++it) {
        const int cc = it * 64 + lane;
        int key = key0 + (cc >> 4);
        key = key < a.cap ? key : a.cap - 1;
        vreg[it] = ld16(vc + kvbase + (size_t)key * HD + (cc & 15) * 8);
      }
    };
    // the wave's first block of the round's first segment is loaded before the prologue, so its
    // latency overlaps the prologue, unless it is the pair's newest block (whose key at pos the
    // prologue writes)
    bool pre = false;                        // kreg/vreg hold the wave's next block
    if (nsg > 0) {
      const int b = sh.seg[0][0], kvh = sh.seg[0][1], j0 = sh.seg[0][2], ns = sh.seg[0][3];
      const int Lb = (int)min<int64_t>(max<int64_t>(sh.posv[b] + 1, 0), (int64_t)a.cap);
      pre = wave < ns && j0 + wave != ((Lb + 31) >> 5) - 1;
      if (pre) load_block((size_t)(b * NKV + kvh) * a.cap * HD, (j0 + wave) * 32);
    }
    // ---- prologue for every segment of the round: q heads normalised + rotated into LDS; the
    // segment holding the newest block also writes K/V of position pos
    for (int task = wave; task < nsg * (G + 2); task += NWAVE) {
      const int sg = task / (G + 2), tk = task - sg * (G + 2);
      const int b = sh.seg[sg][0], kvh = sh.seg[sg][1];
      const int64_t p0 = sh.posv[b];
      const int Lb = (int)min<int64_t>(max<int64_t>(p0 + 1, 0), (int64_t)a.cap);
      const bool newest = sh.seg[sg][2] + sh.seg[sg][3] == ((Lb + 31) >> 5);
      const bool pok = p0 >= 0 && p0 < a.cap && p0 < a.rope_rows;
      if (tk >= G && !(newest && pok)) continue;
      const int col = tk < G ? (kvh * G + tk) * HD : tk == G ? (NH + kvh) * HD : (NH + NKV + kvh) * HD;
      const unsigned ro = (unsigned)((size_t)b * nqkv + col) * 2;
      // every load of the task is issued before the first use (one memory latency): raw head,
      // norm weight, cos/sin row (row 0 stands in for an invalid position)
      const rsrc_t wr = tk < G ? qwr : kwr_n;
      const unsigned cb = (unsigned)((pok ? p0 : 0) * HD) * 2;
      float x0 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rawr, ro + lane * 2, 0, 0));
      float x1 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rawr, ro + (lane + 64) * 2, 0, 0));
      const float w0 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(wr, lane * 2, 0, 0));
      const float w1 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(wr, (lane + 64) * 2, 0, 0));
      const float c0 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(cosr, cb + lane * 2, 0, 0));
      const float c1 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(cosr, cb + (lane + 64) * 2, 0, 0));
      const float s0 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(sinr, cb + lane * 2, 0, 0));
      const float s1 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(sinr, cb + (lane + 64) * 2, 0, 0));
      if (tk <= G) head_norm_rope(a, x0, x1, w0, w1, c0, c1, s0, s1, pok);
      if (tk < G) {
        sh.u.a.qn[sg * G + tk][lane] = f2bf(x0);
        sh.u.a.qn[sg * G + tk][lane + 64] = f2bf(x1);
      } else {
        const rsrc_t cr = tk == G ? kwr : vwr;
        const unsigned co = (unsigned)(((size_t)(b * NKV + kvh) * a.cap + p0) * HD * 2);
        stc_b16(cr, co + lane * 2, f2bf(x0));
        stc_b16(cr, co + (lane + 64) * 2, f2bf(x1));
      }
    }
    __builtin_amdgcn_s_waitcnt(0);          // K/V at pos written through before anyone reads it
    __syncthreads();
    if (first_seg) STEP_TRACE(p, 5);
    for (int sg = 0; sg < nsg; ++sg) {
      const int b = sh.seg[sg][0], kvh = sh.seg[sg][1], j0 = sh.seg[sg][2], nseg = sh.seg[sg][3];
      const int64_t p0 = sh.posv[b];
      const int Lb = (int)min<int64_t>(max<int64_t>(p0 + 1, 0), (int64_t)a.cap);
      const int nblk = (Lb + 31) >> 5;
      const int bk = b * NKV + kvh;
      const size_t kvbase = (size_t)bk * a.cap * HD;
      const int S = sh.units[b] + kvh * (ATT_OVH + nblk);
      // Q^T operand (rows = the G query heads of this kv head; rows >= G zero)
      u32x4 qreg[4];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        qreg[kb] = l16 < G ? *(const u32x4*)&sh.u.a.qn[sg * G + l16][kb * 32 + g4 * 8]
                           : u32x4{0u, 0u, 0u, 0u};
      f32x4 acc[8];
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) acc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
      float m_run = -INFINITY, l_run = 0.f;
      bf16(*vs)[HD + 8] = sh.u.a.v[wave];
      for (int k = wave; k < nseg; k += NWAVE) {
        const int key0 = (j0 + k) * 32;
        if (!pre) load_block(kvbase, key0);
        f32x4 sc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) d = mfma16x16x32(kreg[t][kb], qreg[kb], d);
          sc[t] = d;
        }
#pragma unroll
        for (int it = 0; it < 8; ++it) {
          const int cc = it * 64 + lane;
          *(u32x4*)&vs[cc >> 4][(cc & 15) * 8] = vreg[it];
        }
        // K and V of this block are consumed: the wave's next block (in this segment, else its
        // first block of the next one) streams in during the softmax, P.V and merge
        pre = false;
        if (k + NWAVE < nseg) {
          load_block(kvbase, key0 + NWAVE * 32);
          pre = true;
        } else if (sg + 1 < nsg && wave < sh.seg[sg + 1][3]) {
          load_block((size_t)(sh.seg[sg + 1][0] * NKV + sh.seg[sg + 1][1]) * a.cap * HD,
                     (sh.seg[sg + 1][2] + wave) * 32);
          pre = true;
        }
        float sv[8];
        float mloc = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int key = key0 + t * 16 + g4 * 4 + q;
            const float v = key < Lb ? sc[t][q] * scale_log2 : -INFINITY;
            sv[t * 4 + q] = v;
            mloc = fmaxf(mloc, v);
          }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
        const float m_new = fmaxf(m_run, mloc);
        const float msafe = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(m_run - msafe);
        float psum = 0.f;
        unsigned pk[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float pa = exp2f(sv[2 * jj] - msafe);
          const float pb = exp2f(sv[2 * jj + 1] - msafe);
          psum += pa + pb;
          pk[jj] = pk_bf16(pa, pb);
        }
        psum += __shfl_xor(psum, 16, 64);
        psum += __shfl_xor(psum, 32, 64);
        l_run = l_run * alpha + psum;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[dt] *= alpha;
        const u32x4 pB = {pk[0], pk[1], pk[2], pk[3]};
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const int d = dt * 16 + l16;
          unsigned av[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int ka = (jj < 2) ? (g4 * 4 + 2 * jj) : (16 + g4 * 4 + 2 * (jj - 2));
            av[jj] = (unsigned)vs[ka][d] | ((unsigned)vs[ka + 1][d] << 16);
          }
          acc[dt] = mfma16x16x32(u32x4{av[0], av[1], av[2], av[3]}, pB, acc[dt]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      // merge the waves (rows < G)
      __syncthreads();
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (l16 < G) sh.u.a.mrg[wave][l16][dt * 16 + g4 * 4 + q] = acc[dt][q];
      if (g4 == 0) {
        sh.ms[wave][l16] = m_run;
        sh.ls[wave][l16] = l_run;
      }
      __syncthreads();
      // a (row, kv head) whose blocks all lie in this workgroup is finished here; one split over
      // workgroups leaves (o, m, l) partials, combined by the O projection's staging
      const bool whole = j0 == 0 && nseg == nblk;
      const int myslot = first_seg ? 0 : 1;
      first_seg = false;
      for (int e = tid(); e < G * HD; e += NTHR) {
        const int row = e / HD, d = e % HD;
        float Mx = -INFINITY;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) Mx = fmaxf(Mx, sh.ms[w][row]);
        const float Ms = Mx == -INFINITY ? 0.f : Mx;
        float o = 0.f, l = 0.f;
#pragma unroll
        for (int w = 0; w < NWAVE; ++w) {
          const float f = exp2f(sh.ms[w][row] - Ms);
          o += sh.u.a.mrg[w][row][d] * f;
          l += sh.ls[w][row] * f;
        }
        if (whole) {
          stc_b16(orr, (unsigned)(((size_t)b * NH + kvh * G + row) * HD + d) * 2, f2bf(o / l));
        } else {
          const unsigned pb = (unsigned)(((blockIdx.x * 2 + myslot) * G + row) * rec) * 4;
          stc_f32(pr, pb + d * 4, o);
          if (d == 0) {
            stc_f32(pr, pb + HD * 4, Mx);
            stc_f32(pr, pb + (HD + 1) * 4, l);
          }
        }
      }
      __syncthreads();
    }
    i = inext;
  }
  STEP_TRACE(p, 6);
}

// ---------------------------------------------------------------------------------------------
// embedding gather: workgroup q < H/64 copies columns q*64.. of every row, stores ss[q][m]
__device__ __forceinline__ void embed_phase(const Args& a, Shared& sh) {
  const int M = a.M;
  const int q = blockIdx.x;
  if (q >= a.H / SSG) return;
  const int t = tid();
  const int m = t >> 5, c2 = (t & 31) * 2;
  float s = 0.f;
  if (m < M) {
    int64_t tk = a.tok[m];
    if (tk < 0 || tk >= a.V) {
      if (c2 == 0) atomicOr(a.err, E_TOKEN);
      tk = 0;
    }
    const unsigned v2 = *(const unsigned*)(a.embed + (size_t)tk * a.H + q * SSG + c2);
    const rsrc_t hr = make_rsrc(h_slot(a, 0), (unsigned)((size_t)M * a.H * 2));
    stc_u32(hr, (unsigned)((size_t)m * a.H + q * SSG + c2) * 2, v2);
    s = lo_bf(v2) * lo_bf(v2) + hi_bf(v2) * hi_bf(v2);
  }
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  if (m < M && (t & 31) == 0) {
    const rsrc_t ssr = make_rsrc(ss_slot(a, 0), (unsigned)(SS_SLOT * 4));
    stc_f32(ssr, (unsigned)(q * MAXM + m) * 4, s);
  }
}

// ---------------------------------------------------------------------------------------------
// phase table
enum { P_EMB = 0, P_QKV = 1, P_ATT = 2, P_O = 3, P_GU = 4, P_D = 5, P_LM = 6 };

__device__ __forceinline__ int phase_kind(const Args& a, int p, int* layer) {
  if (p == 0) { *layer = -1; return P_EMB; }
  if (p == 1 + 5 * a.L) { *layer = -1; return P_LM; }
  *layer = (p - 1) / 5;
  return P_QKV + (p - 1) % 5;
}

__device__ __forceinline__ bool phase_geo(const Args& a, const Shared& sh, int p, Geo* g) {
  int layer;
  const int kind = phase_kind(a, p, &layer);
  const long long* lp = layer >= 0 ? sh.ltab[layer] : nullptr;
  switch (kind) {
    case P_QKV: *g = make_geo(uniform_ptr<const bf16>(lp[F_WQKV]), (a.NH + 2 * a.NKV) * HD, a.H, LNR_QKV, true); return true;
    case P_O:   *g = make_geo(uniform_ptr<const bf16>(lp[F_WO]), a.H, a.NH * HD, LNR_O, false); return true;
    case P_GU:  *g = make_geo(uniform_ptr<const bf16>(lp[F_WGU]), 2 * a.I, a.H, LNR_GU, false); return true;
    case P_D:   *g = make_geo(uniform_ptr<const bf16>(lp[F_WD]), a.H, a.I, LNR_D, false); return true;
    case P_LM:  *g = make_geo(a.lm_t, a.V, a.H, LNR_LM, true); return true;
    default: return false;
  }
}

// Staging of the O projection's input x = the attention output of `layer`. A (row, kv head)
// split over attention workgroups is combined here from its (o, m, l) partials (log-sum-exp,
// online in workgroup order) on the way into LDS, and also written to the attention slot.
// The partials are write-once per layer (plain cached loads); every load of a thread's items
// is issued before the first combine.
constexpr int SA_IPT = 3;            // items per thread per batch

__device__ __forceinline__ void stage_attn(const Args& a, Shared& sh, unsigned char* xb, const Geo& g,
                                           int layer, int p) {
  const int M = a.M, NKV = a.NKV, NH = a.NH, G = NH / NKV;
  const int K = NH * HD;
  const int t = tid();
  int ksf = 0, nw = 0;
  if (g.s1 > g.s0) {
    ksf = g.s0 % g.nk;
    nw = min(g.s1 - g.s0, g.nk);
  }
  const int xrs = nw * 64 + 16;
  const int items = M * nw * 4;
  STEP_TRACE(p, 8);
  const rsrc_t orr = make_rsrc(attn_slot(a, layer), (unsigned)((size_t)M * K * 2));
  const rsrc_t pr = make_rsrc(att_part(a, layer), (unsigned)((size_t)gridDim.x * 2 * G * ATT_REC * 4));
  if (t == 0) {
    sh.xrs = xrs;
    sh.xksf = ksf;
    sh.xnw = nw;
  }
  const int gsh = __builtin_ctz(G);
  for (int base = 0; base < items; base += SA_IPT * NTHR) {
    int lds[SA_IPT], m_[SA_IPT], pi_[SA_IPT], hh_[SA_IPT], d0_[SA_IPT];
    unsigned eo_[SA_IPT];
    u32x4 xd[SA_IPT];
    float mv[SA_IPT][SA_PQ], lv[SA_IPT][SA_PQ];
    u32x4 oa[SA_IPT][SA_PQ], ob[SA_IPT][SA_PQ];
    // pass 1: every load
#pragma unroll
    for (int b = 0; b < SA_IPT; ++b) {
      const int it = base + t + b * NTHR;
      const bool valid = it < items;
      const unsigned eo = stage_off(valid ? it : 0, nw > 0 ? nw : 1, ksf, g.nk > 0 ? g.nk : 1, K, &lds[b]);
      const int m = valid ? it / (nw * 4) : 0;
      const int col = (int)(eo - (unsigned)m * K);
      const int h = col >> 7, kvh = h >> gsh;
      hh_[b] = h & (G - 1);
      d0_[b] = col & (HD - 1);
      m_[b] = valid ? m : -1;
      eo_[b] = eo;
      const int pi = m * NKV + kvh;
      pi_[b] = pi;
      const int fw = sh.pinfo[pi][0], lw = sh.pinfo[pi][1];
      xd[b] = ldb128(orr, valid && fw == lw ? eo * 2 : 0xfffffff0u);
      const unsigned hoff = (unsigned)(hh_[b] * ATT_REC * 4);
#pragma unroll
      for (int q = 0; q < SA_PQ; ++q) {
        const int r = sh.pinfo[pi][2 + q];
        const bool ok = valid && r >= 0;
        const unsigned ro = (unsigned)r + hoff;
        mv[b][q] = ok ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, ro + HD * 4, 0, 0)) : -INFINITY;
        lv[b][q] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, ok ? ro + (HD + 1) * 4 : 0xfffffff0u, 0, 0));
        oa[b][q] = ldb128(pr, ok ? ro + d0_[b] * 4 : 0xfffffff0u);
        ob[b][q] = ldb128(pr, ok ? ro + (d0_[b] + 4) * 4 : 0xfffffff0u);
      }
    }
    // pass 2: combine (contributors beyond the first SA_PQ are loaded here, rarely)
#pragma unroll
    for (int b = 0; b < SA_IPT; ++b) {
      if (m_[b] < 0) continue;
      const int pi = pi_[b];
      const int fw = sh.pinfo[pi][0], lw = sh.pinfo[pi][1];
      u32x4 x = xd[b];
      if (lw > fw) {
        float Mx = -INFINITY, l = 0.f, o[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = 0.f;
        auto add = [&](float mq, float lq, u32x4 qa, u32x4 qb) {
          if (mq == -INFINITY) return;
          const float Mn = fmaxf(Mx, mq);
          const float fo = exp2f(Mx - Mn), fn = exp2f(mq - Mn);
          const float ov[8] = {__uint_as_float(qa.x), __uint_as_float(qa.y), __uint_as_float(qa.z),
                               __uint_as_float(qa.w), __uint_as_float(qb.x), __uint_as_float(qb.y),
                               __uint_as_float(qb.z), __uint_as_float(qb.w)};
#pragma unroll
          for (int j = 0; j < 8; ++j) o[j] = o[j] * fo + ov[j] * fn;
          l = l * fo + lq * fn;
          Mx = Mn;
        };
#pragma unroll
        for (int q = 0; q < SA_PQ; ++q) add(mv[b][q], lv[b][q], oa[b][q], ob[b][q]);
        const int S = sh.pinfo[pi][6];
        for (int c = fw + SA_PQ; c <= lw; ++c) {
          if (sh.afirst[c + 1] <= sh.afirst[c]) continue;
          const unsigned ro = (unsigned)(((c * 2 + (sh.afirst[c] >= S ? 0 : 1)) * G + hh_[b]) * ATT_REC) * 4;
          add(__uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, ro + HD * 4, 0, 0)),
              __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(pr, ro + (HD + 1) * 4, 0, 0)),
              ldb128(pr, ro + d0_[b] * 4), ldb128(pr, ro + (d0_[b] + 4) * 4));
        }
        const float il = 1.0f / l;
        x = u32x4{pk_bf16(o[0] * il, o[1] * il), pk_bf16(o[2] * il, o[3] * il),
                  pk_bf16(o[4] * il, o[5] * il), pk_bf16(o[6] * il, o[7] * il)};
        // the attention slot copy is written by one workgroup only: the one whose range holds
        // this k-step of row group 0
        if (g.s0 + (lds[b] >> 6) < g.nk) stc_b128(orr, eo_[b] * 2, x);
      }
      *(u32x4*)(xb + m_[b] * xrs + lds[b]) = x;
    }
  }
  STEP_TRACE(p, 9);
  __syncthreads();
}

// One GEMV phase: arrive at the barrier (sync), start this phase's weight stream, wait, stage
// the activation window, consume. The prefetch registers live only inside this call.
template <int LNR, int EPI, bool ATTN_X = false>
__device__ __forceinline__ void run_gemv(const Args& a, Shared& sh, const Geo& g, int p, int layer,
                                         bool sync, unsigned epoch, int K, const bf16* src,
                                         const bf16* lnw, const float* ss) {
  constexpr int NR = 1 << LNR;
  u32x4 A[BATCH], B[BATCH];
  STEP_TRACE(p, 0);
  if (sync) bar_arrive(a, epoch);
  issue_batch<NR>(g, 0, A);
  issue_batch<NR>(g, BATCH / NR, B);
  const u32x4 lwv = (!ATTN_X && lnw != nullptr) ? lnw_prefetch(g, lnw, K) : u32x4{0u, 0u, 0u, 0u};
  if (sync) bar_wait(a, sh, epoch);
  STEP_TRACE(p, 1);
  if (ATTN_X) stage_attn(a, sh, GemvLds<NR>(sh).x, g, layer >> 1, p);   // layer: output h slot 2l+1
  else stage_x(a, sh, GemvLds<NR>(sh).x, g, K, src, lnw, lwv, ss, p);
  STEP_TRACE(p, 2);
  gemv_phase<NR, EPI>(a, sh, g, layer, A, B, p);
  STEP_TRACE(p, 3);
}

__global__ void __launch_bounds__(NTHR, 1) decode_step_kernel(Args a) {
  extern __shared__ unsigned char smem_raw[];
  Shared& sh = *(Shared*)smem_raw;
  unsigned epoch = 0;
  if (tid() < MAXM) {
    sh.bestv[tid()] = -INFINITY;
    sh.besti[tid()] = 0x7fffffff;
  }
  if (tid() == 0) sh.bail = 0;
  if (tid() < a.M) sh.posv[tid()] = a.pos[tid()];
  for (int e = tid(); e < a.L * LFIELDS; e += NTHR)
    sh.ltab[e / LFIELDS][e % LFIELDS] = a.layers[(size_t)(e / LFIELDS) * NFIELD + e % LFIELDS];
  __syncthreads();
  {
    // attention phases are p = 2 + 5l: position errors are flagged when one of them runs
    const int l0 = a.phase_begin <= 2 ? 0 : (a.phase_begin - 2 + 4) / 5;
    attn_setup(a, sh, l0 < a.L && 2 + 5 * l0 < a.phase_end);
  }
  for (int p = a.phase_begin; p < a.phase_end; ++p) {
    int layer;
    const int kind = phase_kind(a, p, &layer);
    const long long* lp = layer >= 0 ? sh.ltab[layer] : nullptr;
    const bool sync = p > a.phase_begin;
    if (sync) ++epoch;
    Geo g;
    phase_geo(a, sh, p, &g);
    switch (kind) {
      case P_QKV:
        run_gemv<LNR_QKV, EPI_QKV>(a, sh, g, p, layer, sync, epoch, a.H, h_slot(a, 2 * layer),
                                   uniform_ptr<const bf16>(lp[F_LN1]), ss_slot(a, 2 * layer));
        break;
      case P_O:
        run_gemv<LNR_O, EPI_RES, true>(a, sh, g, p, 2 * layer + 1, sync, epoch, a.NH * HD,
                                 attn_slot(a, layer), nullptr, nullptr);
        break;
      case P_GU:
        run_gemv<LNR_GU, EPI_SILU>(a, sh, g, p, layer, sync, epoch, a.H, h_slot(a, 2 * layer + 1),
                                   uniform_ptr<const bf16>(lp[F_LN2]), ss_slot(a, 2 * layer + 1));
        break;
      case P_D:
        run_gemv<LNR_D, EPI_RES>(a, sh, g, p, 2 * layer + 2, sync, epoch, a.I, m_slot(a, layer),
                                 nullptr, nullptr);
        break;
      case P_LM:
        run_gemv<LNR_LM, EPI_LOGITS>(a, sh, g, p, 0, sync, epoch, a.H, h_slot(a, 2 * a.L), a.fnorm,
                                     ss_slot(a, 2 * a.L));
        break;
      default:
        STEP_TRACE(p, 0);
        if (sync) {
          bar_arrive(a, epoch);
          bar_wait(a, sh, epoch);
        }
        STEP_TRACE(p, 1);
        if (kind == P_EMB) embed_phase(a, sh);
        else attention_phase(a, sh, layer, p);
        STEP_TRACE(p, 3);
        break;
    }
    if (kind == P_LM) {
      // argmax over the workgroups' candidates; the last workgroup writes tok, advances pos
      const rsrc_t cr = make_rsrc(a.ws + a.off_am, (unsigned)(gridDim.x * MAXM * 2 * 4));
      if (tid() < (unsigned)a.M) {
        stc_f32(cr, (unsigned)((blockIdx.x * MAXM + tid()) * 2) * 4, sh.bestv[tid()]);
        stc_u32(cr, (unsigned)((blockIdx.x * MAXM + tid()) * 2 + 1) * 4, (unsigned)sh.besti[tid()]);
      }
      if (arrive_last(a.ctr + C_AM, gridDim.x, &sh.flag)) {
        // one wave per row: lanes scan the workgroups' candidates, then a wave reduction
        const int lane = tid() & 63;
        for (int m = wave_id(); m < a.M; m += NWAVE) {
          float bv = -INFINITY;
          int bi = 0x7fffffff;
          for (int w = lane; w < (int)gridDim.x; w += 64) {
            const float v = ldc_f32(cr, (unsigned)((w * MAXM + m) * 2) * 4);
            const int i = (int)ldc_u32(cr, (unsigned)((w * MAXM + m) * 2 + 1) * 4);
            if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
          }
#pragma unroll
          for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, 64);
            const int oi = __shfl_xor(bi, o, 64);
            if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
          }
          if (lane == 0) {
            a.tok[m] = bi;
            a.pos[m] = sh.posv[m] + 1;
          }
        }
      }
    }
  }
  // exit: the last workgroup out resets the barrier counters for the next launch
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid() == 0) {
    const int old = __hip_atomic_fetch_add(a.ctr + C_EXIT, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == (int)gridDim.x - 1) {
      __hip_atomic_store(a.ctr + C_BAR, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      for (int x = 0; x < 8; ++x)
        __hip_atomic_store(a.ctr + C_BAR + 64 * (1 + x), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(a.ctr + C_EXIT, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------------------------
// weight re-layout into MFMA tile order. Block (group gi, k-step ks, tile t) holds rows
// src_row(gi, t, r), r = 0..15, columns ks*32 .. +32, lane l's 16 bytes = row l%16, k (l/16)*8.
// gate/up (gu_I > 0, NR = 2): tile 0 = gate rows gi*16.., tile 1 = up rows gu_I + gi*16...
__global__ void tile_weight_kernel(const bf16* __restrict__ src, bf16* __restrict__ dst, int N, int K,
                                   int lnr, int gu_I) {
  const size_t nblocks = (size_t)(N >> 4) * (K >> 5);
  const size_t blk = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= nblocks) return;
  const int lane = threadIdx.x & 63;
  const int nk = K >> 5;
  const int NR = 1 << lnr;
  const size_t step = blk >> lnr;
  const int t = (int)(blk & (NR - 1));
  const int gi = (int)(step / nk), ks = (int)(step % nk);
  const int r = lane & 15;
  int row;
  if (gu_I > 0) row = (t == 0 ? 0 : gu_I) + gi * 16 + r;
  else row = ((gi << lnr) + t) * 16 + r;
  const u32x4 v = *(const u32x4*)(src + (size_t)row * K + ks * 32 + (lane >> 4) * 8);
  *(u32x4*)(dst + (blk << 9) + lane * 8) = v;
}

}  // namespace st
}  // namespace dd

// ------------------------------------------------------------------------------------------
// C ABI
#include "api.h"

using namespace dd;
using namespace dd::st;

static int step_grid(int* G_out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return (int)hipErrorInvalidDevice;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return (int)hipErrorInvalidDevice;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute((const void*)decode_step_kernel,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(Shared)) !=
        hipSuccess)
      return (int)hipErrorInvalidConfiguration;
    attr_set = true;
  }
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, decode_step_kernel, NTHR, sizeof(Shared)) !=
      hipSuccess || occ < 1)
    return (int)hipErrorInvalidConfiguration;
  *G_out = cus & ~7;   // barrier groups workgroups by XCD (8 per device)
  if (*G_out < 8 || *G_out > MAXG) return (int)hipErrorInvalidConfiguration;
  return 0;
}

struct WsLayout { size_t ss, part, att, am, total; };

static WsLayout ws_layout(int L, int G, int G_heads) {
  WsLayout w;
  w.ss = 0;
  w.part = (size_t)(2 * L + 1) * SS_SLOT;                   // ss: [2L+1][H/64 <= 64][16]
  w.att = w.part + (size_t)G * 2 * 128 * MAXM;              // GEMV: 2 slots of <= 128 rows x 16
  w.am = w.att + (size_t)L * G * 2 * G_heads * ATT_REC;    // attention: per layer, 2 slots
  w.total = w.am + (size_t)G * MAXM * 2;
  return w;
}

DD_API int dd_step_grid(void) {
  int G = 0;
  return step_grid(&G) == 0 ? G : -1;
}

DD_API int dd_step_counters(void) { return C_TOTAL; }

DD_API int dd_step_nr(int matrix) {
  const int lnr[5] = {LNR_QKV, LNR_O, LNR_GU, LNR_D, LNR_LM};
  return matrix >= 0 && matrix < 5 ? 1 << lnr[matrix] : 0;
}

DD_API size_t dd_step_ws_bytes(int L, int NH, int NKV) {
  int G = 0;
  if (L < 1 || NKV < 1 || NH < NKV || step_grid(&G) != 0) return 0;
  return ws_layout(L, G, NH / NKV).total * sizeof(float);
}

DD_API size_t dd_tiled_bytes(int N, int K) { return (size_t)N * K * 2; }

DD_API int dd_tile_weight(const void* src, void* dst, int N, int K, int nr, int gate_up_I,
                          hipStream_t stream) {
  DD_REQUIRE(src && dst && K % 32 == 0 && (nr == 1 || nr == 2 || nr == 4 || nr == 8));
  const int lnr = nr == 1 ? 0 : nr == 2 ? 1 : nr == 4 ? 2 : 3;
  DD_REQUIRE(N % (16 * nr) == 0);
  DD_REQUIRE(gate_up_I == 0 || (nr == 2 && N == 2 * gate_up_I));
  DD_REQUIRE(aligned16(src) && aligned16(dst));
  const size_t nblocks = (size_t)(N / 16) * (K / 32);
  hipLaunchKernelGGL(tile_weight_kernel, dim3((unsigned)((nblocks + 3) / 4)), dim3(256), 0, stream,
                     (const bf16*)src, (bf16*)dst, N, K, lnr, gate_up_I);
  return launch_status();
}

// Model geometry the phases take (Qwen3 family, head_dim 128); G > 0 also checks that every
// GEMV phase's staged activation window fits the LDS x buffer with that many workgroups.
static bool geometry_ok(int L, int H, int NH, int NKV, int I, int V, int M, int G) {
  if (!(M >= 1 && M <= MAXM && L >= 1 && NKV >= 1 && NH >= NKV && NH % NKV == 0 &&
        NH / NKV <= MAXG_HEADS && ((NH / NKV) & (NH / NKV - 1)) == 0 && L <= MAXL))
    return false;
  if (MAXM * NKV > C_AM - C_ATT) return false;            // one combine counter per (row, kv head)
  if (!(H % SSG == 0 && H / SSG <= 64 && I % 16 == 0 && V % 32 == 0)) return false;
  const int K_of[5] = {H, NH * HD, H, I, H};
  const int rows_of[5] = {(NH + 2 * NKV) * HD, H, 2 * I, H, V};
  const int lnr_of[5] = {LNR_QKV, LNR_O, LNR_GU, LNR_D, LNR_LM};
  const bool whole_of[5] = {true, false, false, false, true};   // as in phase_geo
  for (int q = 0; q < 5; ++q) {
    const int K = K_of[q], rows = rows_of[q], lnr = lnr_of[q];
    if (K % 32 != 0 || rows % (16 << lnr) != 0) return false;
    const int nk = K / 32;
    if (nk < NWAVE * (BATCH >> lnr)) return false;       // a batch spans at most two row groups
    if ((rows >> (4 + lnr)) > C_ATT - C_GROUP) return false;
    if (G > 0) {
      const long long S = (long long)(rows >> (4 + lnr)) * nk;
      const long long per = (S + G - 1) / G;
      const long long nw = whole_of[q] || per > nk ? nk : per;
      if ((nw * 64 + 16) * M > (long long)x_capacity(1 << lnr)) return false;
      if (S * (G + 1) >= (1ll << 31)) return false;           // 32-bit partition arithmetic
    }
  }
  return true;
}

DD_API int dd_step_supported(int L, int H, int NH, int NKV, int I, int V, int M) {
  int G = 0;
  if (step_grid(&G) != 0) return 0;
  return geometry_ok(L, H, NH, NKV, I, V, M, G) ? 1 : 0;
}

DD_API int dd_decode_step(const int64_t* layer_table, int L, const void* embed, const void* lm_tiled,
                          const void* final_norm, const void* cos_t, const void* sin_t,
                          int rope_rows, int64_t* tok, int64_t* pos, void* h, void* qkv,
                          void* attn, void* mbuf, void* logits, void* ws, int* counters, int* err,
                          int M, int H, int NH, int NKV, int I, int V, int cap, float eps,
                          int phase_begin, int phase_end, hipStream_t stream) {
  DD_REQUIRE(layer_table && embed && lm_tiled && final_norm && cos_t && sin_t && tok && pos);
  DD_REQUIRE(h && qkv && attn && mbuf && logits && ws && counters && err);
  DD_REQUIRE(geometry_ok(L, H, NH, NKV, I, V, M, 0));
  DD_REQUIRE(cap >= 1 && rope_rows >= 1 && rope_rows <= (1 << 23));   // cos/sin byte ranges < 2^31
  DD_REQUIRE(phase_begin >= 0 && phase_begin < phase_end && phase_end <= 2 + 5 * L);
  int G = 0;
  const int e = step_grid(&G);
  if (e != 0) return e;
  DD_REQUIRE(geometry_ok(L, H, NH, NKV, I, V, M, G));
  // attention partition units (32-bit arithmetic in the kernel)
  DD_REQUIRE((long long)MAXM * NKV * (ATT_OVH + cap / 32 + 1) * (G + 1) < (1ll << 31));
  const WsLayout w = ws_layout(L, G, NH / NKV);
  Args a;
  a.layers = layer_table;
  a.embed = (const bf16*)embed;
  a.lm_t = (const bf16*)lm_tiled;
  a.fnorm = (const bf16*)final_norm;
  a.cos_t = (const bf16*)cos_t;
  a.sin_t = (const bf16*)sin_t;
  a.tok = tok;
  a.pos = pos;
  a.h = (bf16*)h;
  a.qkv = (bf16*)qkv;
  a.attn = (bf16*)attn;
  a.mbuf = (bf16*)mbuf;
  a.logits = (bf16*)logits;
  a.ws = (float*)ws;
  a.ctr = counters;
  a.err = err;
  a.L = L; a.M = M; a.H = H; a.NH = NH; a.NKV = NKV; a.I = I; a.V = V;
  a.cap = cap; a.rope_rows = rope_rows; a.eps = eps;
  a.phase_begin = phase_begin;
  a.phase_end = phase_end;
  a.off_ss = (unsigned)w.ss;
  a.off_part = (unsigned)w.part;
  a.off_att = (unsigned)w.att;
  a.off_am = (unsigned)w.am;
  a.ws_floats = (unsigned)w.total;
  hipLaunchKernelGGL(decode_step_kernel, dim3(G), dim3(NTHR), sizeof(Shared), stream, a);
  return launch_status();
}

#ifdef DD_STEP_TRACE
// Profiling builds only: copy the timing trace ([1024][192][12] u64) to host memory.
DD_API int dd_step_trace(void* host, size_t bytes) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace), bytes, 0, hipMemcpyDeviceToHost);
}
#endif
