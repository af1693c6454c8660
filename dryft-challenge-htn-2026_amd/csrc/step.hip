// Persistent decode step for MI355X (gfx950): one launch runs a whole Qwen3-shape decode step.
//
// Grid: one 512-thread workgroup per CU, all co-resident. The step is a fixed list of phases:
//   0            embedding gather  h = embed[tok], per-workgroup sums of squares
//   per layer    QKV GEMV (raw q|k|v)
//                attention (q/k RMSNorm + RoPE + K/V cache write, split-KV, log-sum-exp combine)
//                O GEMV (+ residual, sums of squares)
//                gate/up GEMV (+ SiLU x up)
//                down GEMV (+ residual, sums of squares)
//   last         lm_head GEMV (+ logits, argmax, pos += 1)
// with a grid barrier between phases.
//
// The same launch also runs the verify-shaped step (engine.py:542-547): B sequences of W tokens,
// M = B W rows, token s of sequence b at position pos[b] + s attending keys 0 .. pos[b] + s. The
// kernel is instantiated for NM 16-row activation tiles: NM = 1 for decode (M <= 16, W = 1) and
// NM = 5 for verify (M <= 80): every weight tile then feeds NM MFMAs, and each (sequence, kv
// head) reads its K/V once for all its W G query rows.
//
// GEMV phases: every workgroup owns whole output rows over the whole K (rows split evenly over
// the workgroups: 10 rows of O/down, 24 of QKV, 38 gate+up feature pairs, ~594 vocabulary rows
// at Qwen3-4B widths on 256 CUs), so no output is ever split between workgroups: no partial
// sums, no finishing hand-offs, each workgroup runs its own epilogue. A workgroup's rows are
// processed in chunks of up to T 16-row MFMA tiles; its 8 waves split the 32-column k-steps
// (wave w takes k-steps w, w + 8, ...) and meet once per chunk in LDS. Weights are streamed from
// a copy re-laid out once (dd_tile_weight): per workgroup and chunk, k-step-major, so one wave
// load of a tile reads rows x 64 contiguous bytes. The activation operand (16 rows x K) is loaded
// by each wave straight into MFMA B-operand registers from the L2 (each XCD's L2 fetches it
// once), RMS-normalised in registers where the phase takes a normalised input.
//
// Barriers are split: a workgroup arrives (after its stores completed), then issues the weight
// loads of the next phase, then waits -- the HBM stream keeps going through the barrier.
//
// Cross-workgroup data inside the launch moves with sc1 stores (written through to the device
// coherence point, see common.h); every spin has a wall-clock timeout that raises a flag instead
// of hanging.
#include "common.h"

namespace dd {
namespace st {

constexpr int NWAVE = 8;
constexpr int NTHR = NWAVE * 64;
constexpr int HD = 128;
constexpr int MAXB = 16;                 // sequences of one launch
constexpr int MAXW = 5;                  // tokens per sequence (verify width)
constexpr int MAXROWS = 80;              // activation rows M = B W
constexpr unsigned OOB = 0x80000000u;   // buffer offset past every range: the load reads 0
#ifndef DD_BAR_SLEEP
#define DD_BAR_SLEEP 2       // s_sleep between barrier polls (units of 64 cycles)
#endif

enum : int { F_WQKV = 0, F_WO, F_WGU, F_WD, F_LN1, F_LN2, F_QN, F_KN, F_KC, F_VC, NFIELD = 16 };

// counters (ints)
constexpr int C_BAR = 0;          // [64 * (1 + xcd)]: arrivals of the XCD's workgroups
constexpr int C_EXIT = 640;
constexpr int C_ATT = 1024;       // per (row, kv head) attention combine counters
constexpr int C_AM = C_ATT + 512;
constexpr int C_SPL = C_AM + 64;   // per workgroup pair: split O / down arrivals
constexpr int C_TOTAL = C_SPL + 256;

// error flags
constexpr int E_TOKEN = 1, E_POS = 2, E_TIMEOUT = 4, E_GEOM = 8;

// The GEMV matrices and their per-workgroup layout: T tiles (16 rows each) per chunk, KB k-steps
// per prefetch batch, NBUF batches in the wave's ring (all but the one being consumed are in
// flight), UPR weight rows per unit of the partition (gate/up: one unit = one feature = its gate
// row and its up row, kept in the same chunk for the SiLU epilogue).
enum : int { M_QKV = 0, M_O = 1, M_GU = 2, M_D = 3, M_LM = 4, NMAT = 5 };
#ifndef DD_KB_OD
#define DD_KB_OD 8
#endif
// ring depths (measured per step at B = 16 / B = 1 against 2 slots everywhere: 3 slots for O,
// gate/up, down and lm_head -4.1% / -3.6%; 4 for gate/up or O, or 3-4 for QKV, are slower)
#ifndef DD_NBUF_QKV
#define DD_NBUF_QKV 2
#endif
#ifndef DD_NBUF_O
#define DD_NBUF_O 3
#endif
#ifndef DD_NBUF_GU
#define DD_NBUF_GU 3
#endif
#ifndef DD_NBUF_D
#define DD_NBUF_D 3
#endif
#ifndef DD_NBUF_LM
#define DD_NBUF_LM 3
#endif
#ifndef DD_NPRE
#define DD_NPRE 2
#endif
__host__ __device__ constexpr int mat_T(int k) { return k == M_QKV ? 2 : k == M_GU ? 5 : k == M_LM ? 8 : 1; }
__host__ __device__ constexpr int mat_KB1(int k) { return k == M_QKV ? 2 : k == M_GU ? 1 : k == M_LM ? 1 : DD_KB_OD; }
__host__ __device__ constexpr int mat_NBUF1(int k) {
  return k == M_LM ? DD_NBUF_LM : k == M_QKV ? DD_NBUF_QKV : k == M_GU ? DD_NBUF_GU : k == M_D ? DD_NBUF_D : DD_NBUF_O;
}
// Ring slots whose weight loads are issued before the barrier wait; the rest go out right after
// it, so the stream continues while the activation and 1/rms loads are in flight. More slots
// before the wait only delay the release (measured: gate/up with all of 3-4 slots before the
// wait is slower than 2 before it).
#ifndef DD_NPRE_D
#define DD_NPRE_D DD_NPRE
#endif
#ifndef DD_NPRE_GU
#define DD_NPRE_GU DD_NPRE
#endif
__host__ __device__ constexpr int mat_npre_max(int k) { return k == M_D ? DD_NPRE_D : k == M_GU ? DD_NPRE_GU : DD_NPRE; }
// weight rows per partition unit: gate/up 2 (a feature's gate and up rows), else 1
__host__ __device__ constexpr int mat_UPR(int k) { return k == M_GU ? 2 : 1; }
// units per chunk: this (with the partition) fixes the tiled weight layout, for every NM
__host__ __device__ constexpr int mat_CAPU(int k) { return mat_T(k) * 16 / mat_UPR(k); }
constexpr int TMAX = 8;
// 80-row (verify) instantiation: k-steps per prefetch batch (O/down, other phases) and ring depth
// (measured at B = 16, W = 5 with 2-tile passes: 4 slots 6.37 against 6.15 ms; 4 slots of one
// k-step for O/down 6.28). Gate/up (6 tiles per pass) and lm_head (4) keep 2 slots: their tile
// partials take the registers (B = 16, W = 5: 5.13 ms; 3 slots with 4-tile passes 5.58, 2 slots
// 5.48, and 2-tile passes with 3 slots 5.69)
#ifndef DD_V_KB
#define DD_V_KB 1
#endif
#ifndef DD_V_KBOD
#define DD_V_KBOD 2
#endif
#ifndef DD_V_NBUF
#define DD_V_NBUF 3
#endif
#ifndef DD_V_NBUF_GU
#define DD_V_NBUF_GU 2
#endif
#ifndef DD_V_NBUF_LM
#define DD_V_NBUF_LM 2
#endif

// With NM > 1 a chunk is streamed in sub-passes of TS of its tiles (the tile partials of all NM
// activation tiles must fit the registers): QKV (2 tiles), O and down (1), gate/up (6: up to 48
// features, three gate tiles and their matching up tiles; a chunk holds 40) one pass, lm_head 2
// passes of 64 rows; every pass reads the whole 80-row activation, so fewer passes read less.
// The cross-wave reduction of a pass takes RED_TILES tile partials per round. The tiled layout
// is the decode step's: a pass reads its tiles' rows at every k-step of the chunk.
#ifndef DD_V_TS_GU
#define DD_V_TS_GU 6                          // 80-row gate/up: tiles per pass (paired layout)
#endif
// 80-row gate/up in the decode step's chunk layout (1): one pass over the chunk's 5 row tiles
// (its nf gate rows, then its nf up rows), reduced in rounds into one buffer of all 80 rows, the
// SiLU epilogue once after the last round. (0: passes of DD_V_TS_GU tiles pairing 16-feature
// gate and up tiles, so every reduction round ends with its own SiLU epilogue; 6 tiles = 48
// feature slots for the chunk's 40, a sixth of the MFMAs and tile partials on empty rows.)
#ifndef DD_V_GU_FLAT
#define DD_V_GU_FLAT 1
#endif
#ifndef DD_V_TS_LM
#define DD_V_TS_LM 4                          // 80-row lm_head: tiles per pass
#endif
template <int NM> struct MatCfg {
  static constexpr int TS(int k) {
    return NM == 1 ? mat_T(k)
         : k == M_GU ? (DD_V_GU_FLAT ? mat_T(M_GU) : DD_V_TS_GU)
         : k == M_LM ? DD_V_TS_LM : (mat_T(k) < 2 ? mat_T(k) : 2);
  }
  static constexpr int NSUB(int k) {
    return NM == 1 ? 1
         : k == M_GU && !DD_V_GU_FLAT ? (mat_CAPU(M_GU) + 8 * TS(k) - 1) / (8 * TS(k))
         : mat_T(k) / TS(k);
  }
  static constexpr int KB(int k) { return NM == 1 ? mat_KB1(k) : (k == M_O || k == M_D) ? DD_V_KBOD : DD_V_KB; }
  static constexpr int NBUF(int k) {
    return NM == 1 ? mat_NBUF1(k) : k == M_GU ? DD_V_NBUF_GU : k == M_LM ? DD_V_NBUF_LM : DD_V_NBUF;
  }
  static constexpr int NPRE(int k) { return NBUF(k) < mat_npre_max(k) ? NBUF(k) : mat_npre_max(k); }
};

// first unit of workgroup c when n units are split evenly over G workgroups (n * G < 2^32)
__host__ __device__ inline int part_lo(int n, int G, int c) {
  return (int)(((unsigned)n * (unsigned)c) / (unsigned)G);
}

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
constexpr int TR_PHASES = 192, TR_EVENTS = 20;
#ifdef DD_STEP_TRACE
__device__ unsigned long long g_trace[1024 * TR_PHASES * TR_EVENTS];
#define STEP_TRACE(p, ev)                                                                    \
  do {                                                                                      \
    if (tid() == 0 && (p) < TR_PHASES)                                                      \
      g_trace[((size_t)blockIdx.x * TR_PHASES + (p)) * TR_EVENTS + (ev)] = wall_clock64();   \
  } while (0)
// per wave: event ev + wave, recorded by the wave's lane 0
#define STEP_TRACE_WAVE(p, ev)                                                               \
  do {                                                                                      \
    if ((tid() & 63) == 0 && (p) < TR_PHASES)                                               \
      g_trace[((size_t)blockIdx.x * TR_PHASES + (p)) * TR_EVENTS + (ev) + (tid() >> 6)] =   \
          wall_clock64();                                                                   \
  } while (0)
#else
#define STEP_TRACE(p, ev) \
  do {                    \
  } while (0)
#define STEP_TRACE_WAVE(p, ev) \
  do {                         \
  } while (0)
#endif

struct Args {
  const int64_t* layers;             // [L][NFIELD] device pointers
  const bf16* embed;                 // [V][H] natural layout (gather)
  const bf16* lm_t;                  // lm_head, tiled (M_LM)
  const bf16* fnorm;                 // final RMSNorm weight [H]
  const bf16* cos_t;
  const bf16* sin_t;
  const int64_t* tok;                // [M] this step's tokens (row m = b W + s)
  int64_t* otok;                     // [M] argmax of each row's logits (may alias tok)
  int64_t* pos;                      // [B] per-sequence positions; += 1 at the end when W == 1
  bf16* h;                           // [2L+1][M][H] residual stream, one slot per producer
  bf16* qkv;                         // [L][M][(NH + 2 NKV) * HD] raw q|k|v
  bf16* attn;                        // [L][M][NH*HD]
  bf16* mbuf;                        // [L][M][I]
  bf16* logits;                      // [M][V]
  float* ws;
  int* ctr;
  int* err;
  int L, M, B, W, H, NH, NKV, I, V, cap, rope_rows;
  float eps;
  int phase_begin, phase_end;
  int phase_cur;                     // trace builds: the phase being run
  unsigned off_ss, off_att, off_am;  // workspace offsets (floats); ss: [2L+1][G][16 NM]
  unsigned off_spl;                  // split O / down partials: [2L][G][2][16][16 NM]
};

// Activation slots that feed a GEMV (h, attention output, SiLU output; K columns, M rows) are
// stored k-step-major: element (m, k) at ((k / 32) * M + m) * 32 + k % 32, so the B operand of one
// 32-column k-step (all M rows) is M * 64 contiguous bytes: one wave load per 16 rows.
__device__ __forceinline__ unsigned xoff(int m, int k, int M) {
  return (unsigned)((((k >> 5) * M + m) << 5) + (k & 31));
}

// Activation buffers are write-once within a launch: the residual stream h has one slot per
// phase that produces it (embedding -> 0, O of layer l -> 2l+1, down of layer l -> 2l+2), raw
// q|k|v, attention output and SiLU output one slot per layer. A slot is only read after the phase
// that writes it (through to the device coherence point, sc1) and every cache is clean at launch
// start, so no cache can hold a stale copy: readers use plain cached loads, and each XCD's L2
// fetches a line once for all its workgroups. The sums of squares behind the RMSNorms follow the
// same rule: slot k holds one [16 NM] partial per workgroup (its columns of h slot k).
__device__ __forceinline__ bf16* h_slot(const Args& a, int k) {
  return a.h + (size_t)k * a.M * a.H;
}
template <int NM>
__device__ __forceinline__ float* ss_slot(const Args& a, int k) {
  return a.ws + a.off_ss + (size_t)k * gridDim.x * 16 * NM;
}
// The raw q|k|v slot is head-grouped: row m holds, per kv head h, its G = NH / NKV q heads, then
// k head h, then v head h (128 columns each), so one kv head's projection is a contiguous range
// of QKV rows (dd_tile_weight lays the QKV weight out in the same row order).
__device__ __forceinline__ bf16* qkv_slot(const Args& a, int l) {
  return a.qkv + (size_t)l * a.M * (a.NH + 2 * a.NKV) * HD;
}

// XCD-local QKV -> attention hand-off. With a multiple of 8 kv heads (and of 8 workgroups), XCD x
// (workgroups c with c % 8 == x) computes the QKV rows of kv heads [x NKV / 8, (x + 1) NKV / 8)
// and runs the attention of exactly those heads, so the attention phase waits for its own XCD's
// arrivals only: 8 attention groups (measured at B = 16: 1.0% per step). With fewer than
// DD_ATT_XCD_MINM sequences an XCD's attention is one or two (sequence, head) pairs on a few
// workgroups and the local wait measured no gain (B = 1: 0.5% slower), so those steps, and
// geometries without a multiple of 8 kv heads, use one group (every workgroup, every head) and
// the full barrier. The choice depends only on the launch's arguments, so the QKV and attention
// phases agree on it.
#ifndef DD_ATT_XCD
#define DD_ATT_XCD 1
#endif
#ifndef DD_ATT_XCD_MINM
#define DD_ATT_XCD_MINM 3
#endif
__device__ __forceinline__ int att_groups(const Args& a) {
  return DD_ATT_XCD && a.B >= DD_ATT_XCD_MINM && (a.NKV & 7) == 0 && (gridDim.x & 7) == 0 ? 8 : 1;
}
__device__ __forceinline__ bf16* attn_slot(const Args& a, int l) {
  return a.attn + (size_t)l * a.M * a.NH * HD;
}
__device__ __forceinline__ bf16* m_slot(const Args& a, int l) {
  return a.mbuf + (size_t)l * a.M * a.I;
}
// split-attention partials of a layer ([G][2][query rows per pair][ATT_REC] fp32): write-once.
// A (sequence, kv head) pair has R = W G query rows: its W tokens times the G query heads of the
// kv head, row r = s G + g.
constexpr int ATT_REC = HD + 4;      // o[128], m, l, 2 pad (16-byte rows)
__device__ __forceinline__ int att_rows(const Args& a) { return a.W * (a.NH / a.NKV); }
__device__ __forceinline__ float* att_part(const Args& a, int l) {
  return a.ws + a.off_att + (size_t)l * gridDim.x * 2 * att_rows(a) * ATT_REC;
}
// plain (cached) 16-byte buffer load; out-of-range offsets read zeros
__device__ __forceinline__ u32x4 ldb128(rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
constexpr int CP_NT = 2;   // buffer cache-policy bit nt (streaming)

constexpr int MAXG = 512;                     // workgroups (CUs) the step kernel supports
constexpr int MAXG_HEADS = 8;                 // query heads per kv head
constexpr int MAXR = 32;                      // query rows per (sequence, kv head): W G
constexpr int MAXL = 64;                      // layers
constexpr int LFIELDS = 10;                   // layer-table fields the phases read
constexpr int MAXH = 4096;                    // hidden size (norm weight staged in LDS)
constexpr int ATT_MAXSEG = 8;                 // attention segments of one round
constexpr int ATT_QN = 64;                    // query rows (all segments) of one round
constexpr int ATT_KVN = 32;                   // new K/V rows (all segments) of one round
constexpr int ATT_PAIRS = 64;                 // pairs of one attention group (pair-aligned)
constexpr int LGS_ROWS = 1024;                // GEMV output units per workgroup staged in LDS
constexpr int RED_TILES = 10;                 // per-wave partial tiles of one chunk pass
// row stride (floats) of the attention merge buffer: 576 bytes, so the 16-byte writes of a
// wave's 4 x 4 (row, dim-group) lanes fall on 16 distinct 16-byte bank groups
constexpr int MRG_STRIDE = HD + 16;
constexpr int RES_FLOATS = 2592;              // reduced rows of one pass: 128 x 17, 32 x 81

struct Shared {
  union {
    struct {                                  // GEMV phases
      float red[NWAVE][RED_TILES][256];       // per-wave partial tiles of a chunk pass
      float res[RES_FLOATS];                  // the pass's reduced rows: [rows][16 NM + 1]
      bf16 lgs[16][LGS_ROWS];                 // outputs of the chunks before the last (NM = 1)
    } g;
    struct {                                  // attention
      union {
        bf16 v[NWAVE][32][HD + 8];            // per-wave V block (inside the block loop)
        float mrg[NWAVE][16][MRG_STRIDE];     // per-wave O of one 16-row query tile (after it)
      } vm;
      bf16 qn[ATT_QN][HD];                    // normalised, rotated query rows of the segments
      bf16 kvn[ATT_KVN][HD];                  // per segment and new token: k (normalised,
                                              // rotated), v
    } a;
  } u;
  float lnw[MAXH];                            // norm weight of a normalised-input GEMV phase (fp32)
  float rs[MAXROWS];                          // per-row 1/rms of the phase's input
  float rsp[NWAVE][MAXROWS];                  // per-wave partial sums of squares behind rs
  float ms[NWAVE][MAXR];
  float ls[NWAVE][MAXR];
  float bestv[MAXROWS];
  int besti[MAXROWS];
  int flag;
  int bail;                                   // a barrier wait timed out: stop waiting
  int units[MAXB + 1];                        // attention unit prefix sums (per sequence)
  int aovh;                                   // attention: overhead units per pair
  int apm;                                    // attention: pair-aligned partition
  int pf[ATT_PAIRS + 1];                      // pair-aligned: first workgroup of each pair
  int seg[32][4];                             // attention segments: b, kvh, first block, blocks
  int nseg, segnext;
  long long pseq[MAXB];                       // this step's sequence positions (read at launch)
  int afirst[MAXG + 1];                       // attention: first unit of each workgroup
  int aG;                                     // attention: workgroups holding units
  long long ltab[MAXL][LFIELDS];              // the layer table, copied once per launch
};

static_assert(sizeof(Shared) <= 160 * 1024, "LDS budget of one CU");

// LDS-only wait + workgroup barrier (outstanding global loads are not waited for)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
}

// The value of lane l ^ 16 (l ^ 32) through gfx950's v_permlane16_swap (v_permlane32_swap)
// instead of an LDS round trip (ds_bpermute, which __shfl_xor compiles to): swapping a register
// with itself leaves each lane the pair (value of the lower row, value of the upper row).
__device__ __forceinline__ float lane_xor16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((tid() & 16) ? r[0] : r[1]);
}
__device__ __forceinline__ float lane_xor32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((tid() & 32) ? r[0] : r[1]);
}

// 0 + x[0] + x[1] + .. + x[7] (in that order) for x[w] = p[w * stride] in LDS, the eight loads
// issued together: left to itself the register-bound scheduler waits for each load (or pair)
// before issuing the next, one LDS round trip per wave's partial.
__device__ __forceinline__ float lds_sum8(const float* p, int stride) {
  float x[NWAVE];
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) x[w] = p[w * stride];
  __builtin_amdgcn_sched_barrier(0);
  float v = 0.f;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) v += x[w];
  return v;
}

// Transposing LDS read of four 16-bit elements (gfx950 ds_read_b64_tr_b16), per 16-lane group:
// output lane j receives element j % 4 of the 8-byte rows that source lanes j / 4, j / 4 + 4,
// j / 4 + 8, j / 4 + 12 address (in that order, low half first). `p` is 8-byte aligned LDS.
typedef short i16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ u32x2 lds_read_tr16(const bf16* p) {
  const i16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(const_cast<bf16*>(p)));
  return __builtin_bit_cast(u32x2, v);
}

// ---------------------------------------------------------------------------------------------
// barrier (split)
__device__ __forceinline__ void bar_arrive(const Args& a, unsigned epoch) {
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_s_barrier();
  if (tid() == 0)                            // no return value: nothing to wait for
    __hip_atomic_fetch_add((unsigned*)a.ctr + C_BAR + 64 * (1 + (blockIdx.x & 7)), 1u,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Released when every XCD's counter has all its workgroups' arrivals: wave 0 reads the 8
// counters with 8 scalar loads in flight together (DD_BAR_SPOLL; else lanes 0..7 in one vector
// load), so the release is one memory latency after the last arrival. xcd_local: only this
// workgroup's XCD's arrivals are waited for.
#ifndef DD_BAR_SPOLL
#define DD_BAR_SPOLL 1
#endif
// One scalar (SMEM) load of a counter, past the scalar cache (glc): counted by lgkmcnt, so a
// poll does not wait for the wave's own vector loads in flight.
__device__ __forceinline__ unsigned spoll_u32(const int* p) {
  unsigned v;
  asm volatile("s_load_dword %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}
// the smallest of the 8 XCD barrier counters (256 bytes apart from C_BAR + 64), all 8 loads in
// flight together
__device__ __forceinline__ unsigned spoll_min8(const int* bar) {
  unsigned v0, v1, v2, v3, v4, v5, v6, v7;
  asm volatile(
      "s_load_dword %0, %8, 0x100 glc\n\t"
      "s_load_dword %1, %8, 0x200 glc\n\t"
      "s_load_dword %2, %8, 0x300 glc\n\t"
      "s_load_dword %3, %8, 0x400 glc\n\t"
      "s_load_dword %4, %8, 0x500 glc\n\t"
      "s_load_dword %5, %8, 0x600 glc\n\t"
      "s_load_dword %6, %8, 0x700 glc\n\t"
      "s_load_dword %7, %8, 0x800 glc\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(v0), "=&s"(v1), "=&s"(v2), "=&s"(v3), "=&s"(v4), "=&s"(v5), "=&s"(v6), "=&s"(v7)
      : "s"(bar)
      : "memory");
  return min(min(min(v0, v1), min(v2, v3)), min(min(v4, v5), min(v6, v7)));
}

__device__ __forceinline__ void bar_wait(const Args& a, Shared& sh, unsigned epoch,
                                         bool xcd_local = false) {
  if (DD_BAR_SPOLL && wave_id() == 0 && !sh.bail) {
    const unsigned target = epoch * (unsigned)(gridDim.x >> 3);
    const unsigned long long t0 = wall_clock64();
    const int* mine = a.ctr + C_BAR + 64 * (1 + (int)(blockIdx.x & 7));
    for (;;) {
      const unsigned v = xcd_local ? spoll_u32(mine) : spoll_min8(a.ctr + C_BAR);
      if (v >= target) break;
      __builtin_amdgcn_s_sleep(DD_BAR_SLEEP);
      if (wall_clock64() - t0 > 20000000ull) {  // 200 ms: report, stop waiting from now on
        if ((tid() & 63) == 0) {
          atomicOr(a.err, E_TIMEOUT);
          sh.bail = 1;
        }
        break;
      }
    }
    STEP_TRACE(a.phase_cur, 11);             // the poller saw the release
  } else if (wave_id() == 0 && !sh.bail) {
    const int lane = tid() & 63;
    const unsigned target = epoch * (unsigned)(gridDim.x >> 3);
    const rsrc_t cr = make_rsrc(a.ctr + C_BAR, 9 * 64 * 4);
    const bool mine = lane < 8 && (!xcd_local || lane == (int)(blockIdx.x & 7));
    const unsigned off = mine ? (unsigned)(64 * (1 + lane) * 4) : 0xfffffff0u;
    const unsigned long long t0 = wall_clock64();
    for (;;) {
      const unsigned v = ldc_u32(cr, off);
      if (__all(!mine || v >= target)) break;
      __builtin_amdgcn_s_sleep(DD_BAR_SLEEP);
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
// GEMV phases

// This workgroup's share of one GEMV phase: units u0 .. u0 + nu of the matrix, nch chunks of up
// to CAPU units, each streamed in nsub passes (NM > 1: a pass takes TS of the chunk's tiles), a
// pass in nbpc prefetch batches (every wave has J = nk / 8 k-steps, wave w's i-th being k-step
// w + 8 i; batch bb holds its k-steps bb KB .. bb KB + KB - 1); nb batches in all.
struct Geo {
  rsrc_t wr;                         // the workgroup's weight region (all its chunks)
  int K, nk, J, u0, nu, nch, nsub, nbpc, nb;
};

template <int KIND, int NM>
__device__ __forceinline__ Geo make_geo(const bf16* W, int nunits, int K, int c) {
  constexpr int UPR = mat_UPR(KIND), CAPU = mat_CAPU(KIND), KB = MatCfg<NM>::KB(KIND);
  Geo g;
  g.K = K;
  g.nk = K >> 5;
  g.J = g.nk >> 3;
  const int u0 = part_lo(nunits, gridDim.x, c);
  const int u1 = part_lo(nunits, gridDim.x, c + 1);
  g.u0 = u0;
  g.nu = u1 - u0;
  g.nch = (g.nu + CAPU - 1) / CAPU;
  g.nsub = MatCfg<NM>::NSUB(KIND);
  g.nbpc = (g.J + KB - 1) / KB;
  g.nb = g.nch * g.nsub * g.nbpc;
  g.wr = make_rsrc(W + (size_t)u0 * UPR * K, (unsigned)((size_t)g.nu * UPR * K * 2));
  return g;
}

// weight rows of chunk ch
template <int KIND>
__device__ __forceinline__ int chunk_rows(const Geo& g, int ch) {
  return min(mat_CAPU(KIND), g.nu - ch * mat_CAPU(KIND)) * mat_UPR(KIND);
}

// A batch position (chunk, pass within it, batch within the pass), advanced one batch at a
// time: the stream's hot loop does no divisions.
struct Cur {
  int ch, sp, bb;
};
__device__ __forceinline__ void advance(const Geo& g, Cur& c) {
  if (++c.bb == g.nbpc) {
    c.bb = 0;
    if (++c.sp == g.nsub) {
      c.sp = 0;
      ++c.ch;
    }
  }
}

// One prefetch batch of a wave: KB k-steps, each TS weight tiles (MFMA A operands) and NM
// activation blocks (B operands: lane l = row 16 n + l % 16, columns (l / 16) * 8 .. +8 of the
// k-step).
template <int KIND, int NM>
struct Buf {
  u32x4 w[MatCfg<NM>::KB(KIND)][MatCfg<NM>::TS(KIND)];
  u32x4 x[MatCfg<NM>::KB(KIND)][NM];
};

// Per-lane byte offsets of batch 0 of a pass's weight tiles and of the activation blocks; batch
// bb adds bb * step, passed as the loads' scalar offset. A lane whose row is past the chunk (or
// past the M activation rows) holds an offset past every range: its loads read zeros without
// memory traffic, unconditionally, so the compiler waits for each register on its own.
template <int KIND, int NM>
struct WOff {
  unsigned o[MatCfg<NM>::KB(KIND)][MatCfg<NM>::TS(KIND)];
  unsigned step;
};
template <int KIND, int NM>
struct XOff {
  unsigned o[MatCfg<NM>::KB(KIND)][NM];
  unsigned step;
};

// Chunk row of tile t's lane row l16 in pass sp, or -1 past the chunk. NM = 1: one pass over
// the chunk's T tiles. NM > 1: TS tiles per pass; gate/up passes take the gate rows of up to
// 8 TS features (tiles 0 .. TS/2 - 1) and the matching up rows (tiles TS/2 ..; the chunk holds
// its nf gate rows, then its nf up rows).
template <int KIND, int NM>
__device__ __forceinline__ int pass_row(int rows, int sp, int t, int l16) {
  constexpr int TS = MatCfg<NM>::TS(KIND);
  if (NM > 1 && KIND == M_GU && !DD_V_GU_FLAT) {   // tiles 0 .. TS/2 - 1 gate rows, then their up rows
    constexpr int th = TS / 2;
    const int nf = rows >> 1, f = 16 * (th * sp + (t < th ? t : t - th)) + l16;
    return f < nf ? (t < th ? f : nf + f) : -1;
  }
  const int j = 16 * (TS * sp + t) + l16;
  return j < rows ? j : -1;
}

template <int KIND, int NM>
__device__ __forceinline__ void set_chunk(const Geo& g, int ch, int sp, WOff<KIND, NM>& w) {
  constexpr int TS = MatCfg<NM>::TS(KIND), KB = MatCfg<NM>::KB(KIND), CAPU = mat_CAPU(KIND),
                UPR = mat_UPR(KIND);
  const int lane = tid() & 63, wave = wave_id();
  const int rows = ch < g.nch ? chunk_rows<KIND>(g, ch) : 0;
  const unsigned cbase = (unsigned)(ch * CAPU * UPR) * (unsigned)g.K * 2u;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int t = 0; t < TS; ++t) {
      const int j = pass_row<KIND, NM>(rows, sp, t, lane & 15);
      w.o[kb][t] = j >= 0 ? cbase + (unsigned)((wave + NWAVE * kb) * rows + j) * 64u +
                                (unsigned)(lane >> 4) * 16u
                          : OOB;
    }
  w.step = (unsigned)(NWAVE * KB * rows) * 64u;
}

template <int KIND, int NM>
__device__ __forceinline__ XOff<KIND, NM> make_xoff(int M) {
  constexpr int KB = MatCfg<NM>::KB(KIND);
  const int lane = tid() & 63, wave = wave_id();
  XOff<KIND, NM> x;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb)
#pragma unroll
    for (int n = 0; n < NM; ++n) {
      const int m = 16 * n + (lane & 15);
      x.o[kb][n] = m < M ? (unsigned)(((wave + NWAVE * kb) * M + m) * 64 + (lane >> 4) * 16) : OOB;
    }
  x.step = (unsigned)(NWAVE * KB * M) * 64u;
  return x;
}

// Loads of batch bb of the pass `w` describes; a k-step past K (in a pass's last batch) reads
// zeros (out-of-range offset).
template <int KIND, int NM>
__device__ __forceinline__ void issue_w(const Geo& g, const WOff<KIND, NM>& w, int bb, Buf<KIND, NM>& b) {
  constexpr int TS = MatCfg<NM>::TS(KIND), KB = MatCfg<NM>::KB(KIND);
  const unsigned so = (unsigned)bb * w.step;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const bool ok = bb * KB + kb < g.J;
#pragma unroll
    for (int t = 0; t < TS; ++t)
      b.w[kb][t] = __builtin_amdgcn_raw_buffer_load_b128(g.wr, ok ? w.o[kb][t] : OOB, ok ? so : 0u, CP_NT);
  }
}

template <int KIND, int NM>
__device__ __forceinline__ void issue_x(const Geo& g, rsrc_t xr, const XOff<KIND, NM>& x, int bb, Buf<KIND, NM>& b) {
  constexpr int KB = MatCfg<NM>::KB(KIND);
  const unsigned so = (unsigned)bb * x.step;
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    const bool ok = bb * KB + kb < g.J;
#pragma unroll
    for (int n = 0; n < NM; ++n)
      b.x[kb][n] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? x.o[kb][n] : OOB, ok ? so : 0u, 0);
  }
}

// Two fp32 values rounded to bf16 (nearest even) by one packed conversion, the same instruction
// the compiler emits for a single conversion. Written as inline asm so that the pair is not split
// back into two single-value conversions (each with its own shift back to fp32) when only the
// rounded values are used.
__device__ __forceinline__ unsigned cvt_pk_bf16(float lo, float hi) {
  unsigned y;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(y) : "v"(lo), "v"(hi));
  return y;
}

// x = bf16(bf16(h * r) * w) for the 8 values of one B-operand register; w (8 values) in fp32.
// Per pair of values: 2 unpacks, 2 multiplies, one packed rounding, 2 unpacks, 2 multiplies, one
// packed rounding (10 VALU instructions; 13 with per-value rounding and bf16 weights).
__device__ __forceinline__ u32x4 norm8(u32x4 x, float r, f32x4 wa, f32x4 wb) {
  const unsigned hw[4] = {x.x, x.y, x.z, x.w};
  const float w[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
  unsigned o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const unsigned y = cvt_pk_bf16(lo_bf(hw[j]) * r, hi_bf(hw[j]) * r);
    o[j] = pk_bf16(lo_bf(y) * w[2 * j], hi_bf(y) * w[2 * j + 1]);
  }
  return u32x4{o[0], o[1], o[2], o[3]};
}

template <int KIND, int NM, bool NORM>
__device__ __forceinline__ void consume(const Geo& g, const Shared& sh, const Buf<KIND, NM>& b, int bb,
                                        const float (&r)[NM],
                                        f32x4 (&acc)[MatCfg<NM>::TS(KIND)][NM]) {
  constexpr int TS = MatCfg<NM>::TS(KIND), KB = MatCfg<NM>::KB(KIND);
  const int lane = tid() & 63, wave = wave_id();
#pragma unroll
  for (int kb = 0; kb < KB; ++kb) {
    u32x4 xv[NM];
    f32x4 wa = {0.f, 0.f, 0.f, 0.f}, wb = {0.f, 0.f, 0.f, 0.f};
    if (NORM) {
      const int ks = wave + NWAVE * min(bb * KB + kb, g.J - 1);
      const float* wp = &sh.lnw[ks * 32 + (lane >> 4) * 8];
      wa = *(const f32x4*)wp;
      wb = *(const f32x4*)(wp + 4);
    }
#pragma unroll
    for (int n = 0; n < NM; ++n) xv[n] = NORM ? norm8(b.x[kb][n], r[n], wa, wb) : b.x[kb][n];
    // tiles past the pass's rows hold zeros (their loads were out of range): no guard, so the
    // tiles' MFMAs issue back to back
#pragma unroll
    for (int t = 0; t < TS; ++t)
#pragma unroll
      for (int n = 0; n < NM; ++n) acc[t][n] = mfma16x16x32(b.w[kb][t], xv[n], acc[t][n]);
  }
}

// epilogues: `res` holds the fp32 sums of the pass's weight rows for every activation row
enum { EPI_QKV = 0, EPI_RES = 1, EPI_SILU = 2, EPI_LOGITS = 3 };

__device__ __forceinline__ bool am_better(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

// am_better without short-circuit evaluation: the same result, as lane-mask arithmetic and one
// select (the branching form compiles to divergent branches per value, which the 80-row lm_head,
// with 100 candidates per lane, cannot afford)
__device__ __forceinline__ bool am_better_nb(float av, int ai, float bv, int bi) {
  const bool an = av != av, bn = bv != bv, lt = ai < bi;
  const bool r_nan = an & (!bn | lt);
  const bool r_num = (av > bv) | ((av == bv) & lt);
  return (an | bn) ? r_nan : r_num;
}

template <int KIND, int NM, int EPI, bool STAGE>
__device__ __forceinline__ void chunk_epilogue(const Args& a, Shared& sh, const Geo& g, int ch, int sp,
                                               int r, int rows, int ua, int oslot,
                                               const unsigned (&hin)[NM]);

// Reduce the waves' tiles of pass (ch, sp) and run its epilogue. oslot: QKV/SILU the layer, RES
// the h slot written (its input is slot oslot - 1, preloaded per thread in hin).
template <int KIND, int NM, int EPI, bool STAGE>
__device__ __forceinline__ void chunk_end(const Args& a, Shared& sh, const Geo& g, int ch, int sp,
                                          f32x4 (&acc)[MatCfg<NM>::TS(KIND)][NM], int oslot,
                                          const unsigned (&hin)[NM]) {
  constexpr int TS = MatCfg<NM>::TS(KIND), CAPU = mat_CAPU(KIND), MS = 16 * NM, RW = MS + 1;
  // RT tiles per reduction round (all NM activation tiles of each), NR rounds. Paired gate/up
  // rounds (NM > 1, DD_V_GU_FLAT 0) pair gate tile r with its up tile r + TS / 2 and run the
  // epilogue per round; flat gate/up (FLAT) reduces every round into one buffer of all the
  // chunk's rows (the LDS staging area, unused by 80-row steps) and runs the epilogue once.
  constexpr bool FLAT = NM > 1 && KIND == M_GU && DD_V_GU_FLAT;
  constexpr int RT = TS * NM <= RED_TILES ? TS : RED_TILES / NM;
  constexpr int NR = FLAT ? (TS + RT - 1) / RT : TS / RT;
  static_assert((FLAT || TS % RT == 0) && RT * NM <= RED_TILES && RT * 16 * RW <= RES_FLOATS, "reduction rounds");
  static_assert(!FLAT || TS * 16 * RW * 4 <= (int)sizeof(sh.u.g.lgs), "flat gate/up rows fit the staging area");
  static_assert(NR == 1 || NM > 1, "several reduction rounds only in the 80-row instantiation");
  static_assert(NR == 1 || EPI == EPI_SILU || EPI == EPI_LOGITS, "several rounds: gate/up, lm_head");
  const int lane = tid() & 63, wave = wave_id();
  const int M = a.M;
  const int rows = chunk_rows<KIND>(g, ch);
  const int ua = g.u0 + ch * CAPU;            // first unit of the chunk
  float* resb = FLAT ? (float*)&sh.u.g.lgs[0][0] : sh.u.g.res;
  STEP_TRACE(a.phase_cur, 7);
  STEP_TRACE_WAVE(a.phase_cur, 12);          // this wave's last batch of the chunk consumed
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    constexpr int RT0 = RT;
    const int ntr = FLAT ? min(RT0, TS - r * RT0) : RT0;   // tiles of this round (compile-time)
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const int tt = EPI == EPI_SILU && NR > 1 && !FLAT ? (i == 0 ? r : r + TS / 2) : r * RT + i;
      if (tt < TS) {
#pragma unroll
        for (int n = 0; n < NM; ++n) {
          *(f32x4*)&sh.u.g.red[wave][i * NM + n][lane * 4] = acc[tt][n];
          acc[tt][n] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
      }
    }
    lds_barrier();
    // res[row j][m]: j = i * 16 + (lane / 16) * 4 + q of the D layout (FLAT: the chunk row, the
    // round's first tile r RT), m = 16 n + lane % 16
    const int jb = FLAT ? 16 * r * RT : 0;
    for (int e = tid(); e < ntr * NM * 256; e += NTHR) {
      const int tn = e >> 8, ln = (e >> 2) & 63, q = e & 3;
      const int i = tn / NM, n = tn - i * NM;
      const float s = lds_sum8(&sh.u.g.red[0][tn][e & 255], RED_TILES * 256);
      resb[(jb + i * 16 + (ln >> 4) * 4 + q) * RW + 16 * n + (ln & 15)] = s;
    }
    lds_barrier();
    if (!FLAT || r == NR - 1) chunk_epilogue<KIND, NM, EPI, STAGE>(a, sh, g, ch, sp, r, rows, ua, oslot, hin);
  }
  STEP_TRACE(a.phase_cur, 8);
}

// The epilogue of reduction round r of pass (ch, sp): `res` holds the fp32 sums of the round's
// RT tiles of rows for every activation row.
template <int KIND, int NM, int EPI, bool STAGE>
__device__ __forceinline__ void chunk_epilogue(const Args& a, Shared& sh, const Geo& g, int ch, int sp,
                                               int r, int rows, int ua, int oslot,
                                               const unsigned (&hin)[NM]) {
  constexpr int TS = MatCfg<NM>::TS(KIND), CAPU = mat_CAPU(KIND), MS = 16 * NM, RW = MS + 1;
  constexpr int RT = TS * NM <= RED_TILES ? TS : RED_TILES / NM;
  const int M = a.M;
  const int t = tid();
  if (EPI == EPI_QKV) {
    // raw q|k|v columns of the pass's rows for every token (q/k RMSNorm, RoPE and the K/V cache
    // write happen in the attention phase, which holds whole heads)
    const int nqkv = (a.NH + 2 * a.NKV) * HD;
    const int j0 = 16 * TS * sp, nj = min(16 * TS, rows - j0);
    const rsrc_t qr = make_rsrc(qkv_slot(a, oslot), (unsigned)((size_t)M * nqkv * 2));
    for (int e = t; e < nj * M; e += NTHR) {
      const int m = e / nj, j = e - m * nj;
      const bf16 v = f2bf(sh.u.g.res[j * RW + m]);
      if (STAGE) sh.u.g.lgs[m][ch * CAPU + j0 + j] = v;
      else stc_b16(qr, (unsigned)((size_t)m * nqkv + ua + j0 + j) * 2, v);
    }
  } else if (EPI == EPI_RES) {
    // residual columns ua .. ua + rows (<= 16, one pass): h[oslot] = bf16(h[oslot-1] + bf16(sum));
    // ss[oslot][wg][m] = sum over the columns of h^2 (thread t: row 16 n + t / 16, column t % 16)
    const rsrc_t hout = make_rsrc(h_slot(a, oslot), (unsigned)((size_t)M * a.H * 2));
    const rsrc_t ssr = make_rsrc(ss_slot<NM>(a, oslot), (unsigned)(gridDim.x * MS * 4));
#pragma unroll
    for (int n = 0; n < NM; ++n) {
      if (t < 256) {
        const int m = 16 * n + (t >> 4), j = t & 15;
        float q = 0.f;
        if (m < M && j < rows) {
          const float hv = rbf(bf2f((bf16)hin[n]) + rbf(sh.u.g.res[j * RW + m]));
          stc_b16(hout, xoff(m, ua + j, M) * 2, f2bf(hv));
          q = hv * hv;
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
        if (j == 0) stc_f32(ssr, (unsigned)(blockIdx.x * MS + m) * 4, q);
      }
    }
  } else if (EPI == EPI_SILU) {
    // NM = 1 and flat 80-row gate/up: chunk rows 0 .. nf: gate features ua.., rows nf .. 2 nf:
    // the matching up rows. Paired 80-row passes: round rows 0 .. 16: gate features ua + f0..,
    // rows 16 .. 32: their up rows.
    constexpr bool FLAT = NM > 1 && DD_V_GU_FLAT;
    const float* resb = FLAT ? (const float*)&sh.u.g.lgs[0][0] : sh.u.g.res;
    const int nfc = rows >> 1;
    const int f0 = NM == 1 || FLAT ? 0 : 16 * (TS / 2 * sp + r);
    const int nf = NM == 1 || FLAT ? nfc : min(16, nfc - f0);
    const int up = NM == 1 || FLAT ? nfc : 16;
    const rsrc_t mr = make_rsrc(m_slot(a, oslot), (unsigned)((size_t)M * a.I * 2));
    for (int e = t; e < nf * M; e += NTHR) {
      const int m = e / nf, f = e - m * nf;
      const float gv = rbf(resb[f * RW + m]);
      const float uv = rbf(resb[(up + f) * RW + m]);
      const float sl = rbf(gv / (1.0f + expf(-gv)));
      if (STAGE) sh.u.g.lgs[m][ch * CAPU + f0 + f] = f2bf(sl * uv);
      else stc_b16(mr, xoff(m, ua + f0 + f, M) * 2, f2bf(sl * uv));
    }
  } else {
    // vocabulary rows of the round: logits out + the workgroup's running argmax per token
    const int j0 = 16 * (TS * sp + RT * r), nj = min(16 * RT, rows - j0);
    const int r0 = ua + j0;
#pragma unroll
    for (int n = 0; n < NM; ++n) {
      const int m = 16 * n + (t >> 5), v = t & 31;
      float val = -INFINITY;
      int idx = 0x7fffffff;
      if (m < M) {
        for (int j = v; j < nj; j += 32) {
          const bf16 bv = f2bf(sh.u.g.res[j * RW + m]);
          const int col = r0 + j;
          if (STAGE) sh.u.g.lgs[m][ch * CAPU + j0 + j] = bv;   // written out after the stream
          else a.logits[(size_t)m * a.V + col] = bv;
          const float fv = bf2f(bv);
          if (am_better(fv, col, val, idx)) {
            val = fv;
            idx = col;
          }
        }
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
  }
  lds_barrier();
}

// The refill side of a phase's weight stream: the next batch to request (rc) and the load
// offsets of rc's pass. Past the workgroup's share rc's chunk has no rows, so every load of a
// request reads zeros without memory traffic: requests are unconditional.
template <int KIND, int NM>
struct Refill {
  Cur rc;
  int wch, wsp;                              // pass `wo` describes
  WOff<KIND, NM> wo;
};

// Request the next batch into ring slot b (weights, and the activation when `x`).
template <int KIND, int NM>
__device__ __forceinline__ void refill(const Geo& g, rsrc_t xr, const XOff<KIND, NM>& xo,
                                       Refill<KIND, NM>& f, Buf<KIND, NM>& b, bool x) {
  if (f.rc.ch != f.wch || f.rc.sp != f.wsp) {   // the next pass (or none: past the share)
    set_chunk<KIND, NM>(g, f.rc.ch, f.rc.sp, f.wo);
    f.wch = f.rc.ch;
    f.wsp = f.rc.sp;
  }
  issue_w<KIND, NM>(g, f.wo, f.rc.bb, b);
  if (x) issue_x<KIND, NM>(g, xr, xo, f.rc.bb, b);
  advance(g, f.rc);
}

// O and down (EPI_RES): the second wave of each SIMD (waves 4 .. 7) runs the phase's loads at
// issue priority 1. Under equal priority the older wave of a SIMD has its loads served first and
// the other finishes its last batch 1.4 (O) / 3.9 (down) us later; with the order reversed the
// step measured 0.2% (B = 16) / 0.8% (B = 1) faster. (For QKV and gate/up, reversing the order
// moves the same lag to waves 0 .. 3 and is slower.)
#ifndef DD_RES_PRIO
#define DD_RES_PRIO 1
#endif

// The batch loop of a GEMV phase: consume each batch from its ring slot and refill the slot with
// the next batch to request. With NM = 1 the loop holds no global store when the workgroup has
// one chunk (MODE 0: its epilogue follows the loop) or stages its earlier chunks' outputs in LDS
// (MODE 1), so the compiler waits for each ring register on its own (a global store in the loop
// would make it wait for every load in flight instead). With NM > 1 (MODE 2) every pass but the
// last writes its outputs from the loop.
template <int KIND, int NM, bool NORM, int EPI, int MODE>
__device__ __forceinline__ void stream_loop(const Args& a, Shared& sh, const Geo& g, rsrc_t xr,
                                            const XOff<KIND, NM>& xo, Refill<KIND, NM>& f,
                                            Buf<KIND, NM> (&ring)[MatCfg<NM>::NBUF(KIND)],
                                            const float (&r)[NM],
                                            f32x4 (&acc)[MatCfg<NM>::TS(KIND)][NM], int oslot,
                                            const unsigned (&hin)[NM]) {
  constexpr int NBUF = MatCfg<NM>::NBUF(KIND);
  Cur cc = {0, 0, 0};
  auto step = [&](Buf<KIND, NM>& b) {
    consume<KIND, NM, NORM>(g, sh, b, cc.bb, r, acc);
    refill<KIND, NM>(g, xr, xo, f, b, true);
    __builtin_amdgcn_sched_barrier(0);        // keep the refill ahead of the next batch's MFMAs
    if (MODE != 0 && cc.bb == g.nbpc - 1 && !(cc.ch + 1 == g.nch && cc.sp + 1 == g.nsub))
      chunk_end<KIND, NM, EPI, MODE == 1>(a, sh, g, cc.ch, cc.sp, acc, oslot, hin);
    advance(g, cc);
  };
  // the first round of the ring on its own (its activation loads went out after the other
  // slots' weights), then whole rounds (every slot consumed: the loop's entry and back edge
  // carry the same loads in flight, so each batch waits for its own registers only), then the
  // remaining batches
  int bi = 0;
  if (g.nb >= NBUF) {
#pragma unroll
    for (int s = 0; s < NBUF; ++s) step(ring[s]);
    for (bi = NBUF; bi + NBUF <= g.nb; bi += NBUF) {
#pragma unroll
      for (int s = 0; s < NBUF; ++s) step(ring[s]);
    }
  }
#pragma unroll
  for (int s = 0; s < NBUF - 1; ++s)
    if (bi + s < g.nb) step(ring[s]);
  if (DD_RES_PRIO && EPI == EPI_RES) __builtin_amdgcn_s_setprio(0);
}

// Partition index of this workgroup in GEMV phase KIND: the QKV phase of 8 attention groups
// gives XCD x the indices x G / 8 .. (x + 1) G / 8 - 1, whose units are its kv heads' rows
// (head-grouped, so part_lo(n, G, x G / 8) = x n / 8 is a head boundary).
template <int KIND>
__device__ __forceinline__ int gemv_part(const Args& a) {
  return KIND == M_QKV && att_groups(a) == 8
             ? (int)((blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3))
             : (int)blockIdx.x;
}

// 1/rms of every activation row of an 80-row step into sh.rs (MS = 16 NM rows): the rows'
// sums of squares are [G][MS] per-workgroup partials. Thread t (t < SUBS * NRG) takes the 4
// rows of row group t % NRG of the partials t / NRG + SUBS i, all requested before the first is
// added; the SUBS subset sums then meet in LDS and are added in subset order.
template <int NM>
__device__ __forceinline__ void wide_rows_rsqrt(const Args& a, Shared& sh, const float* ss) {
  constexpr int MS = 16 * NM;
  constexpr int NRG = MS / 4, SUBS = NTHR / NRG, NIT = (MAXG + SUBS - 1) / SUBS, HALF = (NIT + 1) / 2;
  const int rg = tid() % NRG, k = tid() / NRG;
  const rsrc_t ssr = make_rsrc(ss, (unsigned)(gridDim.x * MS * 4));
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int hb = 0; hb < 2; ++hb) {
    u32x4 v[HALF];
#pragma unroll
    for (int i = 0; i < HALF; ++i) {
      const int cw = k + SUBS * (hb * HALF + i);
      v[i] = ldb128(ssr, k < SUBS && cw < (int)gridDim.x ? (unsigned)((cw * MS + 4 * rg) * 4) : OOB);
    }
#pragma unroll
    for (int i = 0; i < HALF; ++i)
      s += f32x4{__uint_as_float(v[i].x), __uint_as_float(v[i].y), __uint_as_float(v[i].z),
                 __uint_as_float(v[i].w)};
  }
  float* part = &sh.u.g.red[0][0][0];      // [SUBS][MS] (the reduction buffer is free here)
  if (k < SUBS) *(f32x4*)&part[k * MS + 4 * rg] = s;
  lds_barrier();
  if (tid() < MS) {
    float v = 0.f;
    for (int kk = 0; kk < SUBS; ++kk) v += part[kk * MS + tid()];
    sh.rs[tid()] = rsqrt_ieee(v / (float)a.H + a.eps);
  }
  lds_barrier();
}

// One GEMV phase: arrive at the barrier (sync), start this phase's weight stream, wait, then
// stream the activation with the remaining weights, one pass epilogue at a time.
//   NORM: the input is rmsnorm(x) * lnw, 1/rms from the per-workgroup sums of squares `ss`
//   EPI_RES: the residual input is h slot oslot - 1, loaded before the wait (it was written two
//            or more barriers earlier)
template <int KIND, int NM, bool NORM, int EPI>
__device__ __forceinline__ void run_gemv(const Args& a, Shared& sh, int p, bool sync, unsigned epoch,
                                         const bf16* W, int nunits, int K, const bf16* x,
                                         const bf16* lnw, const float* ss, int oslot) {
  constexpr int TS = MatCfg<NM>::TS(KIND), NBUF = MatCfg<NM>::NBUF(KIND), MS = 16 * NM;
  const Geo g = make_geo<KIND, NM>(W, nunits, K, gemv_part<KIND>(a));
  const int M = a.M;
  Buf<KIND, NM> ring[NBUF];
  STEP_TRACE(p, 0);
  if (sync) bar_arrive(a, epoch);
  STEP_TRACE(p, 9);
  // loads independent of the previous phase, issued first (so they are the first to complete)
  u32x4 lw = {0u, 0u, 0u, 0u};
  if (NORM) lw = ldb128(make_rsrc(lnw, (unsigned)(K * 2)), tid() * 8 < K ? (unsigned)(tid() * 16) : OOB);
  unsigned hin[NM];
#pragma unroll
  for (int n = 0; n < NM; ++n) {
    hin[n] = 0;
    if (EPI == EPI_RES) {
      const int m = 16 * n + (tid() >> 4), j = tid() & 15;
      const rsrc_t hr = make_rsrc(h_slot(a, oslot - 1), (unsigned)((size_t)M * a.H * 2));
      constexpr int UPR = mat_UPR(KIND);
      hin[n] = __builtin_amdgcn_raw_buffer_load_b16(
          hr, tid() < 256 && m < M && j < g.nu * UPR ? xoff(m, g.u0 * UPR + j, M) * 2 : OOB, 0, 0);
    }
  }
  constexpr int NPRE = MatCfg<NM>::NPRE(KIND);
  Refill<KIND, NM> f;
  f.rc = Cur{0, 0, 0};
  f.wch = 0;
  f.wsp = 0;
  set_chunk<KIND, NM>(g, 0, 0, f.wo);
  const XOff<KIND, NM> xo = make_xoff<KIND, NM>(M);
  if (DD_RES_PRIO && EPI == EPI_RES && wave_id() >= NWAVE / 2) __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int s = 0; s < NPRE; ++s) refill<KIND, NM>(g, g.wr, xo, f, ring[s], false);   // weights only
  if (NORM && tid() * 8 < K) {
    *(f32x4*)&sh.lnw[tid() * 8] = f32x4{lo_bf(lw.x), hi_bf(lw.x), lo_bf(lw.y), hi_bf(lw.y)};
    *(f32x4*)&sh.lnw[tid() * 8 + 4] = f32x4{lo_bf(lw.z), hi_bf(lw.z), lo_bf(lw.w), hi_bf(lw.w)};
  }
  if (sync) bar_wait(a, sh, epoch);
  STEP_TRACE(p, 1);
  const rsrc_t xr = make_rsrc(x, (unsigned)((size_t)M * K * 2));
  constexpr int NSV = NM == 1 ? MAXG * 4 / NTHR : 1;   // 16-byte sums-of-squares items per thread
  u32x4 sv[NSV];
  if (NORM && NM == 1) {
    // the sums of squares behind 1/rms: [G][16] partials, thread t adds items t, t + NTHR, ..
    // (16 bytes = 4 rows of one partial; every item of thread t holds rows 4 (t % 4) ..)
    const rsrc_t ssr = make_rsrc(ss, (unsigned)(gridDim.x * 16 * 4));
#pragma unroll
    for (int i = 0; i < NSV; ++i) {
      const int q = tid() + i * NTHR;
      sv[i] = ldb128(ssr, q < (int)gridDim.x * 4 ? (unsigned)(q * 16) : OOB);
    }
  }
  {
    Cur xc = {0, 0, 0};                      // the activation of the batches requested before the wait
#pragma unroll
    for (int s = 0; s < NPRE; ++s) {
      issue_x<KIND, NM>(g, xr, xo, xc.bb, ring[s]);
      advance(g, xc);
    }
  }
#pragma unroll
  for (int s = NPRE; s < NBUF; ++s) refill<KIND, NM>(g, xr, xo, f, ring[s], true);
  float r[NM];
#pragma unroll
  for (int n = 0; n < NM; ++n) r[n] = 0.f;
  if (NORM && NM == 1) {
    const int lane = tid() & 63, wave = wave_id();
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NSV; ++i)
      s += f32x4{__uint_as_float(sv[i].x), __uint_as_float(sv[i].y), __uint_as_float(sv[i].z),
                 __uint_as_float(sv[i].w)};
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] += __shfl_xor(s[i], o, 64);
    }
    if (lane < 4) {
#pragma unroll
      for (int i = 0; i < 4; ++i) sh.rsp[wave][lane * 4 + i] = s[i];
    }
    lds_barrier();
    if (tid() < 16) {
      const float v = lds_sum8(&sh.rsp[0][tid()], MAXROWS);
      sh.rs[tid()] = rsqrt_ieee(v / (float)a.H + a.eps);
    }
    lds_barrier();
    r[0] = sh.rs[tid() & 15];
  } else if (NORM) {
    wide_rows_rsqrt<NM>(a, sh, ss);
#pragma unroll
    for (int n = 0; n < NM; ++n) r[n] = sh.rs[16 * n + (tid() & 15)];
  }
  STEP_TRACE(p, 2);
  f32x4 acc[TS][NM];
#pragma unroll
  for (int t = 0; t < TS; ++t)
#pragma unroll
    for (int n = 0; n < NM; ++n) acc[t][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (EPI == EPI_RES) {                      // O / down: one chunk of one pass (H <= 16 G, checked)
    stream_loop<KIND, NM, NORM, EPI, 0>(a, sh, g, xr, xo, f, ring, r, acc, oslot, hin);
    if (g.nch == 1) chunk_end<KIND, NM, EPI, false>(a, sh, g, 0, 0, acc, oslot, hin);
  } else if (g.nch > 0 && NM > 1) {
    // several passes: each but the last writes its outputs from the stream loop
    stream_loop<KIND, NM, NORM, EPI, 2>(a, sh, g, xr, xo, f, ring, r, acc, oslot, hin);
    chunk_end<KIND, NM, EPI, false>(a, sh, g, g.nch - 1, g.nsub - 1, acc, oslot, hin);
  } else if (g.nch > 0) {
    // several chunks (O / down have one: H <= 16 G): the earlier chunks' outputs are staged in
    // LDS (at most LGS_ROWS units, checked on the host) and written out after the stream
    stream_loop<KIND, NM, NORM, EPI, 1>(a, sh, g, xr, xo, f, ring, r, acc, oslot, hin);
    chunk_end<KIND, NM, EPI, false>(a, sh, g, g.nch - 1, 0, acc, oslot, hin);
    const int R = (g.nch - 1) * mat_CAPU(KIND);           // staged units
    for (int e = tid(); e < R * M; e += NTHR) {
      const int m = e / R, j = e - m * R;
      const bf16 v = sh.u.g.lgs[m][j];
      if (EPI == EPI_LOGITS) {
        a.logits[(size_t)m * a.V + g.u0 + j] = v;
      } else if (EPI == EPI_QKV) {
        const int nqkv = (a.NH + 2 * a.NKV) * HD;
        stc_b16(make_rsrc(qkv_slot(a, oslot), (unsigned)((size_t)M * nqkv * 2)),
                (unsigned)((size_t)m * nqkv + g.u0 + j) * 2, v);
      } else {
        stc_b16(make_rsrc(m_slot(a, oslot), (unsigned)((size_t)M * a.I * 2)), xoff(m, g.u0 + j, M) * 2, v);
      }
    }
  }
  if (EPI == EPI_RES && g.nch == 0 && tid() < MS) {   // no columns here: a zero partial
    const rsrc_t ssr = make_rsrc(ss_slot<NM>(a, oslot), (unsigned)(gridDim.x * MS * 4));
    stc_f32(ssr, (unsigned)(blockIdx.x * MS + tid()) * 4, 0.f);
  }
  STEP_TRACE(p, 3);
}

// ---------------------------------------------------------------------------------------------
// lm_head of an 80-row step (NM > 1). The row-owned GEMV above splits a pass's k-steps over the
// waves and reduces the waves' tile partials in LDS; with ~594 vocabulary rows per workgroup
// (37 tiles) and 5 activation tiles per k-step its registers hold 4 weight tiles per pass, so
// the lm_head took 10 passes, each re-reading and re-normalising the whole 80-row activation
// (410 KB per CU per pass) and reducing 20 tile partials. Here the waves split the vocabulary
// rows instead: wave w owns tiles w, w + 8, .. (LMW of them per round) over the whole K, so its
// accumulators hold complete sums (no cross-wave reduction), and the normalised activation is
// staged in LDS one stage of LMKC k-steps at a time, loaded and normalised once per workgroup
// and round (one round when the tiles fit 8 LMW) and read by every wave from LDS. Each wave keeps
// a ring of LMKC k-steps of its weight tiles in flight; the next stage's activation is loaded at
// the start of a stage and normalised into the other LDS buffer at its end.
#ifndef DD_V_LMW
#define DD_V_LMW 5                            // vocabulary tiles per wave and round
#endif
#ifndef DD_V_LMKC
#define DD_V_LMKC 3                           // k-steps per activation stage (= weight ring depth)
#endif
#ifndef DD_V_LM_WIDE
#define DD_V_LM_WIDE 1
#endif
template <int NM>
__device__ __forceinline__ void run_lm_wide(const Args& a, Shared& sh, int p, bool sync, unsigned epoch) {
  constexpr int MS = 16 * NM, TW = DD_V_LMW, KC = DD_V_LMKC, CAPU = mat_CAPU(M_LM);
  constexpr int NXI = (KC * MS * 4 + NTHR - 1) / NTHR;       // 16-byte staging items per thread
  static_assert(2 * KC * MS * 64 + NWAVE * MS * 8 <= (int)sizeof(float) * NWAVE * RED_TILES * 256,
                "staging buffers and argmax candidates fit the reduction buffer");
  static_assert(MS * CAPU * 2 <= 2 * KC * MS * 64, "a chunk's logits fit the staging buffers");
  const int K = a.H, M = a.M;
  const Geo g = make_geo<M_LM, NM>(a.lm_t, a.V, K, (int)blockIdx.x);
  const int lane = tid() & 63, wave = wave_id(), l16 = lane & 15, g4 = lane >> 4;
  const int nk = g.nk, nst = (nk + KC - 1) / KC;
  const int nt = g.nch > 0 ? (g.nch - 1) * (CAPU / 16) + (chunk_rows<M_LM>(g, g.nch - 1) + 15) / 16 : 0;
  const int nround = (nt + NWAVE * TW - 1) / (NWAVE * TW);
  const bf16* x = h_slot(a, 2 * a.L);
  const rsrc_t xr = make_rsrc(x, (unsigned)((size_t)M * K * 2));
  unsigned char* stg = (unsigned char*)&sh.u.g.red[0][0][0];   // [2][KC][MS][64 bytes]
  float* candv = (float*)(stg + 2 * KC * MS * 64);             // [NWAVE][MS]
  int* candi = (int*)(candv + NWAVE * MS);

  // tile slot i of round rd: the lane's byte offset at k-step 0 and the per-k-step stride
  unsigned wo[TW], wst[TW];
  auto set_round = [&](int rd) {
#pragma unroll
    for (int i = 0; i < TW; ++i) {
      const int t = rd * NWAVE * TW + wave + NWAVE * i;
      const int ch = t >> 3, tt = t & 7;
      const int rows = t < nt ? chunk_rows<M_LM>(g, ch) : 0;
      const int j = tt * 16 + l16;
      wst[i] = (unsigned)rows * 64u;
      wo[i] = j < rows ? (unsigned)(ch * CAPU) * (unsigned)K * 2u + (unsigned)j * 64u + (unsigned)g4 * 16u : OOB;
    }
  };
  auto issue_w = [&](int ks, u32x4 (&w)[TW]) {
#pragma unroll
    for (int i = 0; i < TW; ++i)
      w[i] = __builtin_amdgcn_raw_buffer_load_b128(g.wr, ks < nk && wo[i] != OOB ? wo[i] + (unsigned)ks * wst[i] : OOB,
                                                    0u, CP_NT);
  };
  // activation stage s: item e = (k-step ks of the stage, row m, 16-byte quarter q)
  auto stage_load = [&](int s, u32x4 (&v)[NXI]) {
#pragma unroll
    for (int i = 0; i < NXI; ++i) {
      const int e = tid() + i * NTHR;
      const int ksl = e / (MS * 4), rem = e - ksl * MS * 4, m = rem >> 2, q = rem & 3;
      const int ks = s * KC + ksl;
      v[i] = ldb128(xr, e < KC * MS * 4 && ks < nk && m < M ? (unsigned)((ks * M + m) * 64 + q * 16) : OOB);
    }
  };
  auto stage_store = [&](int s, const u32x4 (&v)[NXI]) {
    unsigned char* dst = stg + (s & 1) * KC * MS * 64;
#pragma unroll
    for (int i = 0; i < NXI; ++i) {
      const int e = tid() + i * NTHR;
      if (e < KC * MS * 4) {
        const int ksl = e / (MS * 4), rem = e - ksl * MS * 4, m = rem >> 2, q = rem & 3;
        const int ks = s * KC + ksl;
        u32x4 y = {0u, 0u, 0u, 0u};
        if (ks < nk) {
          const float* wp = &sh.lnw[ks * 32 + q * 8];
          y = norm8(v[i], sh.rs[m], *(const f32x4*)wp, *(const f32x4*)(wp + 4));
        }
        *(u32x4*)(dst + (ksl * MS + m) * 64 + q * 16) = y;
      }
    }
  };

  STEP_TRACE(p, 0);
  if (sync) bar_arrive(a, epoch);
  STEP_TRACE(p, 9);
  const u32x4 lw = ldb128(make_rsrc(a.fnorm, (unsigned)(K * 2)), tid() * 8 < K ? (unsigned)(tid() * 16) : OOB);
  u32x4 ring[KC][TW];
  set_round(0);
#pragma unroll
  for (int j = 0; j < KC; ++j) issue_w(j, ring[j]);          // independent of the last phase
  if (tid() * 8 < K) {
    *(f32x4*)&sh.lnw[tid() * 8] = f32x4{lo_bf(lw.x), hi_bf(lw.x), lo_bf(lw.y), hi_bf(lw.y)};
    *(f32x4*)&sh.lnw[tid() * 8 + 4] = f32x4{lo_bf(lw.z), hi_bf(lw.z), lo_bf(lw.w), hi_bf(lw.w)};
  }
  if (sync) bar_wait(a, sh, epoch);
  STEP_TRACE(p, 1);
  wide_rows_rsqrt<NM>(a, sh, ss_slot<NM>(a, 2 * a.L));        // sh.rs; ends with a barrier
  STEP_TRACE(p, 2);
  float bv[NM];
  int bi[NM];
#pragma unroll
  for (int n = 0; n < NM; ++n) {
    bv[n] = -INFINITY;
    bi[n] = 0x7fffffff;
  }
  for (int rd = 0; rd < nround; ++rd) {
    if (rd > 0) {
      set_round(rd);
#pragma unroll
      for (int j = 0; j < KC; ++j) issue_w(j, ring[j]);
    }
    {
      u32x4 v[NXI];
      stage_load(0, v);
      stage_store(0, v);
    }
    __syncthreads();
    f32x4 acc[TW][NM];
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
      for (int n = 0; n < NM; ++n) acc[i][n] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s < nst; ++s) {
      u32x4 v[NXI];
      if (s + 1 < nst) stage_load(s + 1, v);
      const unsigned char* src = stg + (s & 1) * KC * MS * 64;
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        u32x4 xv[NM];
#pragma unroll
        for (int n = 0; n < NM; ++n) xv[n] = *(const u32x4*)(src + (j * MS + 16 * n + l16) * 64 + g4 * 16);
#pragma unroll
        for (int i = 0; i < TW; ++i)
#pragma unroll
          for (int n = 0; n < NM; ++n) acc[i][n] = mfma16x16x32(ring[j][i], xv[n], acc[i][n]);
        issue_w((s + 1) * KC + j, ring[j]);                    // past nk: reads zeros
        __builtin_amdgcn_sched_barrier(0);
      }
      if (s + 1 < nst) stage_store(s + 1, v);
      __syncthreads();
    }
    STEP_TRACE(p, 7);
    // Logits of the round, one tile slot at a time: the 8 waves' tiles of slot i are chunk
    // rd TW + i (tile t = chunk 8 t + wave), so they meet in LDS as [row][128 columns] (the
    // staging buffers are free now) and go out as row-contiguous runs (lane-consecutive
    // columns); each lane also keeps a running argmax per activation row of its own values.
    bf16* lgb = (bf16*)stg;                                     // [MS][CAPU]
#pragma unroll
    for (int i = 0; i < TW; ++i) {
      const int ch = rd * TW + i;
      const int rows = ch < g.nch ? chunk_rows<M_LM>(g, ch) : 0;
#pragma unroll
      for (int n = 0; n < NM; ++n) {
        const int m = 16 * n + l16;
        unsigned pk[2];
#pragma unroll
        for (int q = 0; q < 4; q += 2) {
          const bf16 b0 = f2bf(acc[i][n][q]), b1 = f2bf(acc[i][n][q + 1]);
          pk[q >> 1] = (unsigned)b0 | ((unsigned)b1 << 16);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int j = wave * 16 + g4 * 4 + q + h;
            const int col = g.u0 + ch * CAPU + j;
            const float fv = bf2f(h ? b1 : b0);
            const bool up = (m < M) & (j < rows) & am_better_nb(fv, col, bv[n], bi[n]);
            bv[n] = up ? fv : bv[n];
            bi[n] = up ? col : bi[n];
          }
        }
        *(u32x2*)&lgb[m * CAPU + wave * 16 + g4 * 4] = u32x2{pk[0], pk[1]};
      }
      lds_barrier();
      const int nr = rows > 0 ? M * rows : 0;
      bf16* out = a.logits + g.u0 + ch * CAPU;
      for (int e = tid(); e < nr; e += NTHR) {
        const int m = e / rows, j = e - m * rows;
        out[(size_t)m * a.V + j] = lgb[m * CAPU + j];
      }
      lds_barrier();
    }
  }
  // the lanes of a row (l16 + 16 g4) meet by shuffles, the waves in LDS
#pragma unroll
  for (int n = 0; n < NM; ++n) {
#pragma unroll
    for (int o = 16; o < 64; o <<= 1) {
      const float ov = __shfl_xor(bv[n], o, 64);
      const int oi = __shfl_xor(bi[n], o, 64);
      const bool up = am_better_nb(ov, oi, bv[n], bi[n]);
      bv[n] = up ? ov : bv[n];
      bi[n] = up ? oi : bi[n];
    }
    if (g4 == 0) {
      candv[wave * MS + 16 * n + l16] = bv[n];
      candi[wave * MS + 16 * n + l16] = bi[n];
    }
  }
  lds_barrier();
  if (tid() < M) {
    float v = sh.bestv[tid()];
    int ix = sh.besti[tid()];
    for (int w = 0; w < NWAVE; ++w)
      if (am_better_nb(candv[w * MS + tid()], candi[w * MS + tid()], v, ix)) {
        v = candv[w * MS + tid()];
        ix = candi[w * MS + tid()];
      }
    sh.bestv[tid()] = v;
    sh.besti[tid()] = ix;
  }
  lds_barrier();
  STEP_TRACE(p, 3);
}

// ---------------------------------------------------------------------------------------------
// Down (and optionally O) with the reduction dimension split over workgroup pairs, for 80-row
// steps (NM = 5) and for decode steps of at least DD_SPL_MINM rows. Row-owned, a workgroup of
// these phases holds ~10 output rows (one 16-row tile) and reads the whole activation for them:
// at 80 rows 655 KB (O) / 1.56 MB (down) per CU through its vector memory pipeline, which set the
// phases' time (measured: without those loads the verify step took 4.0 instead of 6.0 ms, O +
// down 48 -> 23 us per layer); at 16 rows down still reads 311 KB of activation per CU against
// 195 KB of weights. Here workgroups c and c ^ 8 (one XCD) share the decode partition's chunks of
// c & ~8 and (c & ~8) + 8 as two tiles, each takes half of the k-steps of both, so a CU reads
// half the activation for the same weight bytes. Each writes its fp32 partial (write-once slot
// per layer and phase); the second to arrive adds the other's (one commutative add: the same bits
// whichever arrives last) and runs the residual epilogue for both chunks, writing the pair's
// sums-of-squares partial into the first member's slot and a zero into the other's. The exchange
// adds ~3 us to the phase's tail: it pays for down (33.8 -> 26.9 us per layer at B = 16, W = 5;
// decode step 2.739 -> 2.679 ms at B = 16, but not at B = 1, whose activation is 16x smaller),
// not for O (16.4 -> 16.9 at W = 5, verify step 5.70 ms with down only, 5.79 with both; decode
// 2.70 -> 2.78 ms). Exchanging through the XCD's L2 (plain stores and loads, pair counters in
// cached memory) measured slower (5.76).
#ifndef DD_V_SPLIT
#define DD_V_SPLIT 1
#endif
#ifndef DD_SPL_O
#define DD_SPL_O 0                            // split O as well (80-row steps)
#endif
// decode steps split down from this many rows (measured, ms per step, unsplit -> split: B = 16
// 2.739 -> 2.679, B = 8 2.324 -> 2.301, B = 4 2.167 -> 2.150, B = 1 1.977 -> 1.980); 16-row verify
// steps take the choice of the decode step of their B sequences, so that the reduction order of
// their row 0 is the decode step's
#ifndef DD_SPL_MINM
#define DD_SPL_MINM 4
#endif
// ring batches (one k-step each) and how many are requested before the barrier wait: 16 rows
// stream 3 KB per k-step and wave, 80 rows 7 KB (measured at 16 rows, B = 16: 8 / 6 batches
// 2.707 ms, 10 / 8 2.700, 12 / 10 2.705, 12 / 8 2.724, 14 / 12 2.748)
template <int NM> constexpr int spl_nb() { return NM == 1 ? 10 : 3; }
template <int NM> constexpr int spl_npre() { return NM == 1 ? 8 : 2; }
// one workgroup's partial: [2 tiles][16 rows][16 NM]
__host__ __device__ constexpr int spl_floats(int NM) { return 2 * 16 * 16 * NM; }

__device__ __forceinline__ bool res_split_ok(int K) {
  return DD_V_SPLIT && (gridDim.x & 15) == 0 && ((K >> 5) & 15) == 0;
}

template <int KIND, int NM>
__device__ __forceinline__ void run_res_split(const Args& a, Shared& sh, int p, bool sync, unsigned epoch,
                                              const bf16* W, int N, int K, const bf16* x, int oslot) {
  constexpr int MS = 16 * NM, RW = MS + 1, NB = spl_nb<NM>(), NPRE = spl_npre<NM>();
  constexpr int SPLF = spl_floats(NM);
  const int G = gridDim.x, c = blockIdx.x, c0 = c & ~8, mem = (c >> 3) & 1;
  const int M = a.M;
  const int lane = tid() & 63, wave = wave_id(), l16 = lane & 15, g4 = lane >> 4;
  STEP_TRACE(p, 0);
  if (sync) bar_arrive(a, epoch);
  STEP_TRACE(p, 9);
  // the pair's chunks (rows u0[t] .. u0[t] + nr[t], nr <= 16: H <= 16 G is checked on the host)
  int u0[2], nr[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    u0[t] = part_lo(N, G, c0 + 8 * t);
    nr[t] = part_lo(N, G, c0 + 8 * t + 1) - u0[t];
  }
  // the residual input of both chunks' columns (thread t < 256: row 16 n + t / 16, column t % 16)
  const rsrc_t hr = make_rsrc(h_slot(a, oslot - 1), (unsigned)((size_t)M * a.H * 2));
  unsigned hin[2][NM];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int n = 0; n < NM; ++n) {
      const int m = 16 * n + (tid() >> 4), j = tid() & 15;
      hin[t][n] = __builtin_amdgcn_raw_buffer_load_b16(
          hr, tid() < 256 && m < M && j < nr[t] ? xoff(m, u0[t] + j, M) * 2 : OOB, 0, 0);
    }
  // weights: tile t is chunk t, laid out k-step-major ([k-step][nr[t] rows][32]); this member
  // takes k-steps mem * half .. + half, wave w the k-steps mem * half + w + 8 i (i < J)
  const rsrc_t wr = make_rsrc(W + (size_t)u0[0] * K, (unsigned)((size_t)(u0[1] + nr[1] - u0[0]) * K * 2));
  const int half = K >> 6, J = half >> 3, ks = mem * half + wave;
  unsigned wo[2], wst[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    wo[t] = l16 < nr[t] ? (unsigned)((u0[t] - u0[0]) * K * 2) + (unsigned)((ks * nr[t] + l16) * 64 + g4 * 16)
                        : OOB;
    wst[t] = (unsigned)(NWAVE * nr[t] * 64);
  }
  unsigned xo[NM];
#pragma unroll
  for (int n = 0; n < NM; ++n) {
    const int m = 16 * n + l16;
    xo[n] = m < M ? (unsigned)((ks * M + m) * 64 + g4 * 16) : OOB;
  }
  const unsigned xst = (unsigned)(NWAVE * M * 64);
  const rsrc_t xr = make_rsrc(x, (unsigned)((size_t)M * K * 2));
  struct SB {
    u32x4 w[2];
    u32x4 x[NM];
  };
  SB ring[NB];
  // batch bb of this wave (k-steps past J read zeros without memory traffic)
  auto issue_wt = [&](int bb, SB& b) {
    const bool ok = bb < J;
#pragma unroll
    for (int t = 0; t < 2; ++t)
      b.w[t] = __builtin_amdgcn_raw_buffer_load_b128(wr, ok ? wo[t] : OOB, ok ? (unsigned)bb * wst[t] : 0u, CP_NT);
  };
  auto issue_xt = [&](int bb, SB& b) {
    const bool ok = bb < J;
#pragma unroll
    for (int n = 0; n < NM; ++n)
      b.x[n] = __builtin_amdgcn_raw_buffer_load_b128(xr, ok ? xo[n] : OOB, ok ? (unsigned)bb * xst : 0u, 0);
  };
  if (DD_RES_PRIO && wave >= NWAVE / 2) __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int b = 0; b < NPRE; ++b) issue_wt(b, ring[b]);
  if (sync) bar_wait(a, sh, epoch);
  STEP_TRACE(p, 1);
#pragma unroll
  for (int b = 0; b < NPRE; ++b) issue_xt(b, ring[b]);
#pragma unroll
  for (int b = NPRE; b < NB; ++b) {
    issue_wt(b, ring[b]);
    issue_xt(b, ring[b]);
  }
  STEP_TRACE(p, 2);
  f32x4 acc[2][NM];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int n = 0; n < NM; ++n) acc[t][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto step = [&](SB& b, int bi) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int n = 0; n < NM; ++n) acc[t][n] = mfma16x16x32(b.w[t], b.x[n], acc[t][n]);
    issue_wt(bi + NB, b);
    issue_xt(bi + NB, b);
    __builtin_amdgcn_sched_barrier(0);
  };
  // whole rounds of the ring (batch bi in slot bi % NB), then the remaining batches
  int bi = 0;
  for (; bi + NB <= J; bi += NB) {
#pragma unroll
    for (int b = 0; b < NB; ++b) step(ring[b], bi + b);
  }
#pragma unroll
  for (int b = 0; b < NB - 1; ++b)
    if (bi + b < J) step(ring[b], bi + b);
  if (DD_RES_PRIO) __builtin_amdgcn_s_setprio(0);
  STEP_TRACE(p, 7);
  STEP_TRACE_WAVE(p, 12);
  // cross-wave reduction: res[(16 t + row) RW + m] (rows of the D layout, as in chunk_end)
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int n = 0; n < NM; ++n) *(f32x4*)&sh.u.g.red[wave][t * NM + n][lane * 4] = acc[t][n];
  lds_barrier();
  for (int e = tid(); e < 2 * NM * 256; e += NTHR) {
    const int tn = e >> 8, ln = (e >> 2) & 63, i = e & 3;
    const int t = tn / NM, n = tn - t * NM;
    const float v = lds_sum8(&sh.u.g.red[0][tn][e & 255], RED_TILES * 256);
    sh.u.g.res[(t * 16 + (ln >> 4) * 4 + i) * RW + 16 * n + (ln & 15)] = v;
  }
  lds_barrier();
  // this member's partial out, then the pair's arrival
  const unsigned pbytes = (unsigned)((size_t)G * SPLF * 4);
  const rsrc_t pr = make_rsrc(a.ws + a.off_spl + (size_t)(oslot - 1) * G * SPLF, pbytes);
  for (int e = tid(); e < 2 * 16 * MS; e += NTHR) {
    const int t = e / (16 * MS), j = (e / MS) & 15, m = e % MS;
    if (j < nr[t] && m < M)
      stc_f32(pr, (unsigned)(c * SPLF + e) * 4, sh.u.g.res[(t * 16 + j) * RW + m]);
  }
  const rsrc_t ssr = make_rsrc(ss_slot<NM>(a, oslot), (unsigned)(G * MS * 4));
  if (arrive_last(a.ctr + C_SPL + (c & 7) * (MAXG / 16) + (c >> 4), 2, &sh.flag)) {
    const int co = c ^ 8;
    for (int e = tid(); e < 2 * 16 * MS; e += NTHR) {
      const int t = e / (16 * MS), j = (e / MS) & 15, m = e % MS;
      if (j < nr[t] && m < M)
        sh.u.g.res[(t * 16 + j) * RW + m] += ldc_f32(pr, (unsigned)(co * SPLF + e) * 4);
    }
    lds_barrier();
    // h[oslot] = bf16(h[oslot - 1] + bf16(sum)) for both chunks' columns; ss[oslot][c][m] = the
    // sum of h^2 over them
    const rsrc_t hout = make_rsrc(h_slot(a, oslot), (unsigned)((size_t)M * a.H * 2));
#pragma unroll
    for (int n = 0; n < NM; ++n) {
      if (tid() < 256) {
        const int m = 16 * n + (tid() >> 4), j = tid() & 15;
        float q = 0.f;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (m < M && j < nr[t]) {
            const float hv = rbf(bf2f((bf16)hin[t][n]) + rbf(sh.u.g.res[(t * 16 + j) * RW + m]));
            stc_b16(hout, xoff(m, u0[t] + j, M) * 2, f2bf(hv));
            q += hv * hv;
          }
        }
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
        // the pair's sum in the slot of its first member, a zero in the other's, whichever
        // member arrives last: the consumers add the G slots in a fixed order, so a sum placed
        // by arrival order would change the bits of 1/rms from run to run
        if (j == 0) {
          stc_f32(ssr, (unsigned)(c0 * MS + m) * 4, q);
          stc_f32(ssr, (unsigned)((c0 + 8) * MS + m) * 4, 0.f);
        }
      }
    }
  }
  lds_barrier();
  STEP_TRACE(p, 3);
}

// ---------------------------------------------------------------------------------------------
// attention. The 32-key blocks of every (sequence, kv head) are laid end to end (sequence-major,
// then kv head) and split into equal contiguous workgroup ranges, so every workgroup streams the
// same number of K/V bytes whatever the per-sequence context lengths. A workgroup takes its range
// as segments, one per (sequence, kv head) it touches; its 8 waves share a segment's blocks.
// A pair (sequence b, kv head) has R = W G query rows, row r = s G + g: token s (activation row
// b W + s, position pos[b] + s) and query head g of the kv head; row r attends keys 0 .. pos[b] + s.
// Per segment: its query rows are RMS-normalised and rotated from the raw q|k|v (engine.py
// qkv_post); a segment whose blocks hold new keys (positions pos[b] .. pos[b] + W - 1) also
// normalises/rotates those tokens' k and writes K/V there (its blocks take the new keys from
// those values, so nothing waits for the cache write); then S^T = K.Q^T and O^T += V^T.P^T on
// MFMA (P rounded to bf16; NQT 16-column query tiles), the waves merge through LDS, and a pair
// split over workgroups is combined (log-sum-exp, in workgroup order) by the last contributor.

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
// workload (short contexts, B = 1) stays on fewer workgroups, at least ATT_MINU units each
// (measured at B = 1: 8 is 2.3% faster per step than 16; with the split overhead units 6 is 0.6%
// faster than 8 and 12 is 2% slower; later 4 is 0.7% faster than 6, 3 and 5 in between; B = 16
// and the verify step are the same for 4-12). Partition arithmetic stays in 32 bits (units x
// workgroups < 2^31, checked on the host).
#ifndef DD_ATT_MINU
#define DD_ATT_MINU 4
#endif
constexpr int ATT_MINU = DD_ATT_MINU;
__device__ __forceinline__ int attn_owner(int T, int Ga, int i) {  // workgroup of global unit i
  return (int)(((unsigned)(i + 1) * Ga - 1) / (unsigned)T);
}
__device__ __forceinline__ int attn_first(int T, int Ga, int c) {  // first unit of workgroup c
  return c >= Ga ? T : (int)((unsigned)T * c / Ga);
}

// Partition units of one (sequence, kv head): att_ovh(B, W) units for its fixed per-segment latency
// (prologue, wave merge, output) followed by one unit per 32-key block, so a workgroup holding
// many short segments gets fewer blocks. With one or two sequences the few pairs are spread over
// more workgroups by a larger weight (B = 16 best at 12; at B = 1 any weight from 8 to 48
// measured the same with ATT_MINU 8; with ATT_MINU 4, 48 is 0.1% faster than 24 and 12 0.2%
// slower). A verify-shaped segment (W G query rows: prologue and
// merge of two query tiles) weighs more: 36 (B = 16, W = 5: 6.48 -> 6.19 ms per step; 48 and
// 64 measured 6.27 and 6.35).
#ifndef DD_ATT_OVH_SMALL
#define DD_ATT_OVH_SMALL 48
#endif
#ifndef DD_ATT_OVH
#define DD_ATT_OVH 12
#endif
#ifndef DD_ATT_OVH_W
#define DD_ATT_OVH_W 36                  // verify-shaped steps (W > 1)
#endif
constexpr int cmax(int x, int y) { return x > y ? x : y; }
constexpr int ATT_OVH_MAX = cmax(DD_ATT_OVH_SMALL, cmax(DD_ATT_OVH, DD_ATT_OVH_W));
// Of a pair's overhead units, att_ovh_head(ovh) sit before its blocks and the rest after them:
// a workgroup whose range holds the end of one pair and the start of the next pays both parts,
// one whose range starts or ends at a pair boundary only one.
#ifndef DD_ATT_OVH_HEAD2
#define DD_ATT_OVH_HEAD2 1                // halves of the overhead before the blocks (0, 1 or 2)
#endif
__host__ __device__ constexpr int att_ovh_head(int ovh) { return ovh * DD_ATT_OVH_HEAD2 / 2; }
__host__ __device__ constexpr int att_ovh(int B, int W) {
  return B <= 2 ? DD_ATT_OVH_SMALL : W > 1 ? DD_ATT_OVH_W : DD_ATT_OVH;
}
#ifndef DD_ATT_NOPRE
#define DD_ATT_NOPRE 1               // waves 0 .. n-1 request no K/V block before the barrier wait
#endif
#ifndef DD_ATT_KPRE
#define DD_ATT_KPRE 1                // K half of the first block before the wait (see below)
#endif
constexpr int ATT_CB = 4;            // contributors whose partials one combine pass loads

// Keys the attention of sequence b covers this step: its cache below pos plus its W new tokens,
// counted as at least ATT_WPAD new tokens (a key past pos + W - 1 is masked for every row, and its
// cache slot exists: the count stops at cap). The count sets the partition of the key blocks, so a
// decode step (W = 1) and a verify step of up to ATT_WPAD tokens at the same positions split and
// combine every (sequence, kv head) pair at the same blocks: row 0 of such a verify step then
// gives the decode step's bits (speculation stays token-identical to plain decoding).
#ifndef DD_ATT_WPAD
#define DD_ATT_WPAD 4
#endif
__device__ __forceinline__ int seq_keys(const Args& a, const Shared& sh, int b) {
  return (int)min<int64_t>(max<int64_t>(sh.pseq[b] + max(a.W, DD_ATT_WPAD), 0), (int64_t)a.cap);
}
// every new token of sequence b has a valid cache slot and rope row
__device__ __forceinline__ bool seq_pos_ok(const Args& a, const Shared& sh, int b) {
  const int64_t p = sh.pseq[b];
  return p >= 0 && p + a.W <= a.cap && p + a.W <= a.rope_rows;
}

// units[b]: first partition unit of sequence b (sequences with no keys have none);
// units[B] = total. The partition depends only on this step's positions: computed once per launch.
//
// Verify-shaped steps of the 80-row instantiation (W > 1) use a pair-aligned partition instead: a
// segment there costs as much as ~21 blocks (prologue of W G query rows and 2 W new K/V rows,
// merge of two query tiles, partials), so the unit partition's per-pair overhead units, which a
// workgroup pays whether or not it holds the pair's blocks, left workgroups with 6 to 43 blocks
// (ends 14-37 us after the release at B = 16). Here every workgroup holds one segment: pair q
// gets n_q = ceil(nb_q / X)
// workgroups and an even split of its nb_q blocks, X the smallest share (>= DD_ATT_PAIR_MIN)
// whose workgroups fit the group.
#ifndef DD_ATT_PAIR
#define DD_ATT_PAIR 1
#endif
#ifndef DD_ATT_PAIR_MIN
#define DD_ATT_PAIR_MIN 8                   // blocks: one per wave
#endif
__device__ __forceinline__ int wave_sum_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}
template <int NM>
__device__ __forceinline__ void attn_partition(const Args& a, Shared& sh, bool flag_errors) {
  const int P = att_groups(a), hpg = a.NKV / P, Gl = (int)gridDim.x / P;
  // The 16-row instantiation partitions verify steps (W > 1) exactly as decode steps (unit
  // partition, the decode weight), so that their row 0 reproduces the decode step.
  const bool pm = DD_ATT_PAIR && NM > 1 && a.W > 1 && a.B * hpg <= min(ATT_PAIRS, Gl);
  const int ovh = pm ? 0 : att_ovh(a.B, NM == 1 ? 1 : a.W);
  if (tid() < 64) {                          // wave 0: lane b = sequence b, prefix sum by shuffles
    const int b = tid();
    int cnt = 0;
    if (b < a.B) {
      if (flag_errors && !seq_pos_ok(a, sh, b) && blockIdx.x == 0) atomicOr(a.err, E_POS);
      const int nblk = (seq_keys(a, sh, b) + 31) >> 5;
      cnt = nblk > 0 ? hpg * (ovh + nblk) : 0;
    }
    int inc = cnt;
#pragma unroll
    for (int o = 1; o <= MAXB; o <<= 1) {      // lanes 0..MAXB: lane B sums all B sequences
      const int v = __shfl_up(inc, o, 64);
      if (b >= o) inc += v;
    }
    if (b <= a.B) sh.units[b] = inc - cnt;   // lane B: cnt = 0, inc = total
  }
  __syncthreads();
  const int T = sh.units[a.B];
  if (pm) {
    if (tid() < 64) {
      // lane q: pair q = (sequence q / hpg, the group's kv head h0 + q % hpg), nb blocks from unit S
      const int q = tid(), np = a.B * hpg;
      const int bq = q < np ? q / hpg : 0;
      const int nb = q < np ? (sh.units[bq + 1] - sh.units[bq]) / hpg : 0;
      const int S = q < np ? sh.units[bq] + (q - bq * hpg) * nb : T;
      int lo = DD_ATT_PAIR_MIN, hi = max(lo, wave_max_i(nb));
      while (lo < hi) {                        // uniform across the wave
        const int mid = (lo + hi) >> 1;
        if (wave_sum_i((nb + mid - 1) / mid) <= Gl) hi = mid;
        else lo = mid + 1;
      }
      const int n = (nb + lo - 1) / lo;
      int inc = n;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int v = __shfl_up(inc, o, 64);
        if (q >= o) inc += v;
      }
      const int f = inc - n, Ga = __shfl(inc, 63, 64);
      if (q <= np) sh.pf[q] = f;             // lane np: f = Ga
      for (int j = 0; j < n; ++j) sh.afirst[f + j] = S + (int)((unsigned)nb * j / n);
      for (int c = Ga + q; c <= Gl; c += 64) sh.afirst[c] = T;
      if (q == 0) sh.aG = max(1, Ga);
    }
  } else {
    const int Ga = max(1, min(Gl, T / ATT_MINU));
    for (int c = tid(); c <= Gl; c += NTHR) sh.afirst[c] = attn_first(T, Ga, c);
    if (tid() == 0) sh.aG = Ga;
  }
  if (tid() == 0) {
    sh.aovh = ovh;
    sh.apm = pm;
  }
  __syncthreads();
}

// Combine the (o, m, l) partials of a (sequence, kv head) split over attention workgroups
// fw .. lw (in workgroup order) into the bf16 attention output; run by the last contributor to
// arrive. Pair start S: a contributor's record is its slot 0 when the pair is its first segment.
// The combine with two query tiles (R = W G rows, 20 at W = 5). Merging element by element
// (a thread's 5 elements, each with its own round of loads) kept the combining workgroup 3.2-3.8
// us past its arrival. Here thread t takes 8 consecutive dims of one row (R x 16 threads): per
// contributor two 16-byte loads of o and one of (m, l), all ATT_CB contributors' loads in flight
// together, the merge in registers in contributor order (the same operations on the same values
// as the per-element merge), and one 16-byte store of the 8 outputs.
#ifndef DD_ATT_CMB_1R
#define DD_ATT_CMB_1R 1
#endif
__device__ __forceinline__ void attn_combine_1r(const Args& a, const Shared& sh, int layer, int b,
                                                int kvh, int S, int fw, int lw, int P, int gx) {
  constexpr int DPT = 8, TPR = HD / DPT;                  // dims per thread, threads per row
  const int NH = a.NH, G = a.NH / a.NKV, R = att_rows(a);
  const int t = tid();
  if (t >= R * TPR) return;
  const int row = t / TPR, d0 = (t - row * TPR) * DPT;
  const int ovt = sh.aovh - att_ovh_head(sh.aovh);
  const rsrc_t pr = make_rsrc(att_part(a, layer), (unsigned)((size_t)gridDim.x * 2 * R * ATT_REC * 4));
  const rsrc_t orr = make_rsrc(attn_slot(a, layer), (unsigned)((size_t)a.M * NH * HD * 2));
  float Mx = -INFINITY, l = 0.f, o[DPT];
#pragma unroll
  for (int i = 0; i < DPT; ++i) o[i] = 0.f;
  for (int c0 = fw; c0 <= lw; c0 += ATT_CB) {
    u32x4 oa[ATT_CB], ob[ATT_CB], ml[ATT_CB];
#pragma unroll
    for (int j = 0; j < ATT_CB; ++j) {
      const int c = c0 + j;
      const bool ok = c <= lw && sh.afirst[c + 1] > sh.afirst[c];
      const unsigned ro =
          (unsigned)((((c * P + gx) * 2 + (sh.afirst[c] >= S - ovt ? 0 : 1)) * R + row) * ATT_REC) * 4;
      oa[j] = ldc_b128(pr, ok ? ro + d0 * 4 : OOB);
      ob[j] = ldc_b128(pr, ok ? ro + (d0 + 4) * 4 : OOB);
      ml[j] = ok ? ldc_b128(pr, ro + HD * 4) : u32x4{0xff800000u, 0u, 0u, 0u};   // m = -inf: skipped
    }
#pragma unroll
    for (int j = 0; j < ATT_CB; ++j) {
      const float mv = __uint_as_float(ml[j].x), lv = __uint_as_float(ml[j].y);
      if (mv == -INFINITY) continue;
      const float Mn = fmaxf(Mx, mv);
      const float fo = exp2_hw(Mx - Mn), fn = exp2_hw(mv - Mn);
      const float ov[DPT] = {__uint_as_float(oa[j].x), __uint_as_float(oa[j].y), __uint_as_float(oa[j].z),
                             __uint_as_float(oa[j].w), __uint_as_float(ob[j].x), __uint_as_float(ob[j].y),
                             __uint_as_float(ob[j].z), __uint_as_float(ob[j].w)};
#pragma unroll
      for (int i = 0; i < DPT; ++i) o[i] = o[i] * fo + ov[i] * fn;
      l = l * fo + lv * fn;
      Mx = Mn;
    }
  }
  const float inv = 1.0f / l;
  const int s = row / G, g = row - s * G;
  stc_b128(orr, xoff(b * a.W + s, (kvh * G + g) * HD + d0, a.M) * 2,
           u32x4{pk_bf16(o[0] * inv, o[1] * inv), pk_bf16(o[2] * inv, o[3] * inv),
                 pk_bf16(o[4] * inv, o[5] * inv), pk_bf16(o[6] * inv, o[7] * inv)});
}

__device__ __forceinline__ void attn_combine(const Args& a, const Shared& sh, int layer, int b,
                                             int kvh, int S, int fw, int lw, int P, int gx) {
  const int NH = a.NH, G = a.NH / a.NKV, R = att_rows(a);
  // overhead units after the previous pair's blocks: a contributor whose range starts at or past
  // them has this pair as its first segment (record slot 0)
  const int ovt = sh.aovh - att_ovh_head(sh.aovh);
  const rsrc_t pr = make_rsrc(att_part(a, layer), (unsigned)((size_t)gridDim.x * 2 * R * ATT_REC * 4));
  const rsrc_t orr = make_rsrc(attn_slot(a, layer), (unsigned)((size_t)a.M * NH * HD * 2));
  for (int e = tid(); e < R * HD; e += NTHR) {
    const int row = e / HD, d = e - row * HD;
    float Mx = -INFINITY, l = 0.f, o = 0.f;
    for (int c0 = fw; c0 <= lw; c0 += ATT_CB) {
      float mv[ATT_CB], lv[ATT_CB], ov[ATT_CB];
#pragma unroll
      for (int j = 0; j < ATT_CB; ++j) {
        const int c = c0 + j;
        const bool ok = c <= lw && sh.afirst[c + 1] > sh.afirst[c];
        const unsigned ro =
            ok ? (unsigned)((((c * P + gx) * 2 + (sh.afirst[c] >= S - ovt ? 0 : 1)) * R + row) * ATT_REC) * 4
               : OOB;
        mv[j] = ok ? ldc_f32(pr, ro + HD * 4) : -INFINITY;
        lv[j] = ldc_f32(pr, ok ? ro + (HD + 1) * 4 : OOB);
        ov[j] = ldc_f32(pr, ok ? ro + d * 4 : OOB);
      }
#pragma unroll
      for (int j = 0; j < ATT_CB; ++j) {
        if (mv[j] == -INFINITY) continue;
        const float Mn = fmaxf(Mx, mv[j]);
        const float fo = exp2_hw(Mx - Mn), fn = exp2_hw(mv[j] - Mn);
        o = o * fo + ov[j] * fn;
        l = l * fo + lv[j] * fn;
        Mx = Mn;
      }
    }
    const int s = row / G, g = row - s * G;
    stc_b16(orr, xoff(b * a.W + s, (kvh * G + g) * HD + d, a.M) * 2, f2bf(o * (1.0f / l)));
  }
}

// A split segment's arrival and the next segment's first K/V block: 0 = the block requested during
// the segment's last block (its arrival then also waits for it), 1 = after the arrival's stores
// with one query tile (decode), 2 = after them in both instantiations.
#ifndef DD_ATT_DEFER
#define DD_ATT_DEFER 1
#endif
template <int NQT> __device__ constexpr bool att_defer() {
  return DD_ATT_DEFER == 2 || (DD_ATT_DEFER == 1 && NQT == 1);
}

// The attention prologue's head tasks packed four to a wave instruction (16 lanes each) or one
// per wave: 0 = never, 1 = with two query tiles (verify), 2 = when a round has more tasks than
// waves, 3 = always.
#ifndef DD_ATT_PACK
#define DD_ATT_PACK 1
#endif
template <int NQT> __device__ __forceinline__ bool att_pack(int ntasks) {
  return DD_ATT_PACK == 3 || (DD_ATT_PACK == 1 && NQT > 1) || (DD_ATT_PACK == 2 && ntasks > NWAVE);
}

// The attention phase. The K/V cache below each sequence's position does not depend on this
// step, so the first round's segments are laid out and every wave's first K/V block is requested
// before the barrier wait (sync: the phase waits for the QKV phase here).
template <int NQT>
__device__ __forceinline__ void attention_phase(const Args& a, Shared& sh, int layer, int p, bool sync,
                                                unsigned epoch) {
  const int M = a.M, W = a.W, NKV = a.NKV, NH = a.NH, G = NH / NKV, R = W * G;
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
  // attention group gx of P (XCD gx when P = 8) takes kv heads h0 .. h0 + NKV / P - 1; the
  // partition (sh.units, sh.afirst) is over its heads and its workgroups li = 0 .. G / P - 1
  const int P = att_groups(a), gx = (int)blockIdx.x % P, li = (int)blockIdx.x / P;
  const int h0 = gx * (NKV / P);
  const int i0 = sh.afirst[li], i1 = sh.afirst[li + 1];
  const int Tu = sh.units[a.B], Ga = sh.aG;
  const int ovh = sh.aovh, ova = att_ovh_head(ovh);
  const unsigned kvbytes = (unsigned)((size_t)a.B * NKV * a.cap * HD * 2);
  const rsrc_t kwr = make_rsrc(kc, kvbytes), vwr = make_rsrc(vc, kvbytes);
  const rsrc_t rawr = make_rsrc(qkv_slot(a, layer), (unsigned)((size_t)M * nqkv * 2));
  const rsrc_t qwr = make_rsrc(qnw, HD * 2), kwr_n = make_rsrc(knw, HD * 2);
  const rsrc_t cosr = make_rsrc(a.cos_t, (unsigned)((size_t)a.rope_rows * HD * 2));
  const rsrc_t sinr = make_rsrc(a.sin_t, (unsigned)((size_t)a.rope_rows * HD * 2));
  const rsrc_t orr = make_rsrc(attn_slot(a, layer), (unsigned)((size_t)M * NH * HD * 2));
  const unsigned rec = ATT_REC;
  const rsrc_t pr = make_rsrc(att_part(a, layer), (unsigned)((size_t)gridDim.x * 2 * R * rec * 4));
  const int maxseg = min(min(ATT_QN / R, ATT_MAXSEG), ATT_KVN / (2 * W));
  bool first_seg = true;
  // one 32-key block of K (S^T operand: lane = key l16 of half t, dims kb*32 + g4*8) and V
  // (rows of 16 keys x 8 dims, transposed through LDS below)
  u32x4 kreg[2][4], vreg[8];
  auto load_k = [&](size_t kvbase, int key0) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      int key = key0 + t * 16 + l16;
      key = key < a.cap ? key : a.cap - 1;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) kreg[t][kb] = ld16(kc + kvbase + (size_t)key * HD + kb * 32 + g4 * 8);
    }
  };
  auto load_v = [&](size_t kvbase, int key0) {
#pragma unroll
    for (int it = 0; it < 8; ++it) {
      const int cc = it * 64 + lane;
      int key = key0 + (cc >> 4);
      key = key < a.cap ? key : a.cap - 1;
      vreg[it] = ld16(vc + kvbase + (size_t)key * HD + (cc & 15) * 8);
    }
  };
  auto load_block = [&](size_t kvbase, int key0) {
    load_k(kvbase, key0);
    load_v(kvbase, key0);
  };
  // One query tile and the XCD-local wait (B >= 3): before the barrier wait the waves request
  // only the K half of their first block, its V half after the prologue. The full blocks (112 KB
  // per CU) take ~4 us to issue when every CU requests at once; the last wave to finish issuing
  // set the release (s_barrier) at 6.5 us after the XCD's last QKV arrival, the poller having
  // seen it at 2.0 us (trace build: release 6.3 -> 3.8 us, attention span 27.7 -> 26.7 us per
  // layer; step B = 16 2.589 -> 2.579 ms. B = 1, whose few attention workgroups are not issue
  // bound, measured 1.928 -> 1.950 with the split and keeps whole blocks; so does the two-tile
  // instantiation: 4.788 -> 4.927 ms per verify step with the split.)
  const bool KPRE = DD_ATT_KPRE && NQT == 1 && P == 8;
  bool vpend = false;
  // ---- a round's segments: (sequence, kv head) pairs whose blocks meet [i, i1), then the wave's
  // first block of the round's first segment (its latency overlaps the prologue; before the
  // barrier wait wave 0, the poller, requests nothing so its poll is not queued behind a block)
  auto start_round = [&](int i, bool before_wait) {
    if (tid() == 0) {
      int n = 0, u = i;
      while (u < i1 && n < maxseg) {
        int b = 0;
        while (b + 1 < a.B && sh.units[b + 1] <= u) ++b;
        const int nblk = (seq_keys(a, sh, b) + 31) >> 5;
        const int per = ovh + nblk;
        const int kvh = h0 + (u - sh.units[b]) / per;
        const int S = sh.units[b] + (kvh - h0) * per;               // pair start (overhead units)
        const int lo = max(u, S + ova), hi = min(i1, S + ova + nblk);
        if (hi > lo) {
          sh.seg[n][0] = b;
          sh.seg[n][1] = kvh;
          sh.seg[n][2] = lo - S - ova;
          sh.seg[n][3] = hi - lo;
          ++n;
        }
        u = S + per;
      }
      sh.nseg = n;
      sh.segnext = u;                                               // where the next round starts
    }
    __syncthreads();
    bool pre = false;
    if (sh.nseg > 0) {
      const int b = sh.seg[0][0], kvh = sh.seg[0][1], j0 = sh.seg[0][2], ns = sh.seg[0][3];
      pre = wave < ns && !(before_wait && wave < DD_ATT_NOPRE);   // wave 0 polls the barrier
      if (pre) {
        if (KPRE && before_wait) {
          load_k((size_t)(b * NKV + kvh) * a.cap * HD, (j0 + wave) * 32);
          vpend = true;
        } else {
          load_block((size_t)(b * NKV + kvh) * a.cap * HD, (j0 + wave) * 32);
        }
      }
    }
    if (before_wait) STEP_TRACE_WAVE(p, 12);   // the wave's pre-wait requests issued
    return pre;
  };
  bool pre = start_round(i0, sync);                // kreg/vreg hold the wave's next block
  if (sync) bar_wait(a, sh, epoch, P == 8);
  STEP_TRACE(p, 1);
  for (int i = i0; i < i1;) {
    if (i != i0) pre = start_round(i, false);
    const int nsg = sh.nseg;
    const int inext = sh.segnext;
    // ---- prologue for every segment of the round: its query rows normalised + rotated into
    // LDS; a segment whose blocks hold new keys also normalises/rotates those tokens' k, and
    // copies their v (task t of a segment: t < R query row t, then W k rows, then W v rows).
    // Packed (att_pack): four tasks per wave instruction, 16 lanes per task, lane l of a task
    // holding dims 4l .. 4l + 3 and their rotate-half partners 64 + 4l .. (8-byte accesses), so a
    // round of 32 tasks (a verify segment's 30) costs one memory latency. Every load of a task is
    // issued before the first use; descriptors stay wave-uniform (the q and k norm weights are
    // two loads, the one a task does not use out of range).
    const int TK = R + 2 * W, NT = nsg * TK;
    if (att_pack<NQT>(NT)) {
      const int grp = lane >> 4, gl = lane & 15;
      constexpr int HALF = HD / 2;
      for (int t0 = wave * 4; t0 < NT; t0 += NWAVE * 4) {
        const int task = min(t0 + grp, NT - 1);
        const int sg = task / TK, tk = task - sg * TK;
        const int b = sh.seg[sg][0], kvh = sh.seg[sg][1];
        const int64_t p0 = sh.pseq[b];
        const int key_lo = sh.seg[sg][2] * 32, key_hi = (sh.seg[sg][2] + sh.seg[sg][3]) * 32;
        const bool hasnew = key_lo < p0 + W && key_hi > p0;
        const bool pok = seq_pos_ok(a, sh, b);
        const bool act = t0 + grp < NT && (tk < R || (hasnew && pok));
        const int s = tk < R ? tk / G : tk < R + W ? tk - R : tk - R - W;
        const int hcol = tk < R ? tk - s * G : tk < R + W ? G : G + 1;   // head-grouped: q heads, k, v
        const int col = (kvh * (G + 2) + hcol) * HD;
        const unsigned ro = (unsigned)((size_t)(b * W + s) * nqkv + col) * 2 + gl * 8;
        const unsigned cb = (unsigned)((pok ? p0 + s : 0) * HD) * 2 + gl * 8;
        const unsigned wo = (unsigned)gl * 8;
        const u32x2 xl = __builtin_amdgcn_raw_buffer_load_b64(rawr, act ? ro : OOB, 0, 0);
        const u32x2 xh = __builtin_amdgcn_raw_buffer_load_b64(rawr, act ? ro + HALF * 2 : OOB, 0, 0);
        const bool isq = tk < R, isk = tk >= R && tk < R + W;
        const u32x2 ql = __builtin_amdgcn_raw_buffer_load_b64(qwr, act && isq ? wo : OOB, 0, 0);
        const u32x2 qh = __builtin_amdgcn_raw_buffer_load_b64(qwr, act && isq ? wo + HALF * 2 : OOB, 0, 0);
        const u32x2 kl = __builtin_amdgcn_raw_buffer_load_b64(kwr_n, act && isk ? wo : OOB, 0, 0);
        const u32x2 kh = __builtin_amdgcn_raw_buffer_load_b64(kwr_n, act && isk ? wo + HALF * 2 : OOB, 0, 0);
        const u32x2 cl = __builtin_amdgcn_raw_buffer_load_b64(cosr, act ? cb : OOB, 0, 0);
        const u32x2 ch = __builtin_amdgcn_raw_buffer_load_b64(cosr, act ? cb + HALF * 2 : OOB, 0, 0);
        const u32x2 sl = __builtin_amdgcn_raw_buffer_load_b64(sinr, act ? cb : OOB, 0, 0);
        const u32x2 sh2 = __builtin_amdgcn_raw_buffer_load_b64(sinr, act ? cb + HALF * 2 : OOB, 0, 0);
        // x[i], i < 4: dim 4 gl + i; x[4 + i]: dim 64 + 4 gl + i (the partner of x[i])
        float x[8], w[8], c[8], sn[8];
        const u32x2 wl = {ql.x | kl.x, ql.y | kl.y}, wh = {qh.x | kh.x, qh.y | kh.y};
        const unsigned xw[4] = {xl.x, xl.y, xh.x, xh.y}, ww[4] = {wl.x, wl.y, wh.x, wh.y};
        const unsigned cw[4] = {cl.x, cl.y, ch.x, ch.y}, sw[4] = {sl.x, sl.y, sh2.x, sh2.y};
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          x[2 * j] = lo_bf(xw[j]);
          x[2 * j + 1] = hi_bf(xw[j]);
          w[2 * j] = lo_bf(ww[j]);
          w[2 * j + 1] = hi_bf(ww[j]);
          c[2 * j] = lo_bf(cw[j]);
          c[2 * j + 1] = hi_bf(cw[j]);
          sn[2 * j] = lo_bf(sw[j]);
          sn[2 * j + 1] = hi_bf(sw[j]);
        }
        // 1/rms of the head: its 16 lanes' sums of squares (outside any branch: every lane
        // of the group takes part)
        float ss = 0.f;
  #pragma unroll
        for (int i = 0; i < 8; ++i) ss += x[i] * x[i];
  #pragma unroll
        for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o, 64);
        const float r = rsqrt_ieee(ss / (float)HD + a.eps);
        unsigned out[4] = {xw[0], xw[1], xw[2], xw[3]};     // v rows: a bit copy
        if (tk < R + W) {
          float n[8], y[8];
  #pragma unroll
          for (int i = 0; i < 8; ++i) n[i] = rbf(rbf(x[i] * r) * w[i]);
  #pragma unroll
          for (int i = 0; i < 4; ++i) {
            y[i] = pok ? rbf(rbf(n[i] * c[i]) + rbf(-n[i + 4] * sn[i])) : n[i];
            y[i + 4] = pok ? rbf(rbf(n[i + 4] * c[i + 4]) + rbf(n[i] * sn[i + 4])) : n[i + 4];
          }
  #pragma unroll
          for (int j = 0; j < 4; ++j) out[j] = pk_bf16(y[2 * j], y[2 * j + 1]);
        }
        if (act) {
          bf16* dst = tk < R ? sh.u.a.qn[sg * R + tk] : sh.u.a.kvn[2 * (sg * W + s) + (tk < R + W ? 0 : 1)];
          *(u32x2*)&dst[4 * gl] = u32x2{out[0], out[1]};
          *(u32x2*)&dst[HALF + 4 * gl] = u32x2{out[2], out[3]};
        }
      }
    } else {
      // one task per wave: lane l holds dims l and l + 64
      for (int task = wave; task < nsg * TK; task += NWAVE) {
        const int sg = task / TK, tk = task - sg * TK;
        const int b = sh.seg[sg][0], kvh = sh.seg[sg][1];
        const int64_t p0 = sh.pseq[b];
        const int key_lo = sh.seg[sg][2] * 32, key_hi = (sh.seg[sg][2] + sh.seg[sg][3]) * 32;
        const bool hasnew = key_lo < p0 + W && key_hi > p0;
        const bool pok = seq_pos_ok(a, sh, b);
        if (tk >= R && !(hasnew && pok)) continue;
        const int s = tk < R ? tk / G : tk < R + W ? tk - R : tk - R - W;
        const int hcol = tk < R ? tk - s * G : tk < R + W ? G : G + 1;   // head-grouped: q heads, k, v
        const int col = (kvh * (G + 2) + hcol) * HD;
        const unsigned ro = (unsigned)((size_t)(b * W + s) * nqkv + col) * 2;
        // every load of the task is issued before the first use (one memory latency): raw head,
        // norm weight, cos/sin row (row 0 stands in for an invalid position)
        const rsrc_t wr = tk < R ? qwr : kwr_n;
        const unsigned cb = (unsigned)((pok ? p0 + s : 0) * HD) * 2;
        float x0 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rawr, ro + lane * 2, 0, 0));
        float x1 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rawr, ro + (lane + 64) * 2, 0, 0));
        const float w0 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(wr, lane * 2, 0, 0));
        const float w1 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(wr, (lane + 64) * 2, 0, 0));
        const float c0 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(cosr, cb + lane * 2, 0, 0));
        const float c1 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(cosr, cb + (lane + 64) * 2, 0, 0));
        const float s0 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(sinr, cb + lane * 2, 0, 0));
        const float s1 = bf2f((unsigned short)__builtin_amdgcn_raw_buffer_load_b16(sinr, cb + (lane + 64) * 2, 0, 0));
        if (tk < R + W) head_norm_rope(a, x0, x1, w0, w1, c0, c1, s0, s1, pok);
        bf16* dst = tk < R ? sh.u.a.qn[sg * R + tk] : sh.u.a.kvn[2 * (sg * W + s) + (tk < R + W ? 0 : 1)];
        dst[lane] = f2bf(x0);
        dst[lane + 64] = f2bf(x1);
      }
    }
    if (vpend) {                                // the first block's V half (see KPRE above)
      load_v((size_t)(sh.seg[0][0] * NKV + sh.seg[0][1]) * a.cap * HD, (sh.seg[0][2] + wave) * 32);
      vpend = false;
    }
    lds_barrier();
    if (first_seg) STEP_TRACE(p, 5);
    for (int sg = 0; sg < nsg; ++sg) {
      const int b = sh.seg[sg][0], kvh = sh.seg[sg][1], j0 = sh.seg[sg][2], nseg = sh.seg[sg][3];
      const int64_t p0 = sh.pseq[b];
      const int Lb = seq_keys(a, sh, b);
      const int nblk = (Lb + 31) >> 5;
      const int bk = b * NKV + kvh;
      const size_t kvbase = (size_t)bk * a.cap * HD;
      const int S = sh.units[b] + (kvh - h0) * (ovh + nblk);
      // the new keys p0 .. p0 + W - 1 take their K/V from the prologue (when positions are valid)
      const bool pok = seq_pos_ok(a, sh, b);
      // Q^T operands (rows = the pair's R query rows, 16 per tile; rows >= R zero)
      u32x4 qreg[NQT][4];
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
          qreg[qt][kb] = 16 * qt + l16 < R ? *(const u32x4*)&sh.u.a.qn[sg * R + 16 * qt + l16][kb * 32 + g4 * 8]
                                           : u32x4{0u, 0u, 0u, 0u};
      // causal limit of this lane's query column in each tile: keys <= p0 + s of its row
      int lim[NQT];
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt) {
        const int r = min(16 * qt + l16, R - 1);
        lim[qt] = (int)min<int64_t>(p0 + r / G, (int64_t)Lb - 1);
      }
      // a pair whose blocks all lie in this workgroup is finished here; one split over
      // workgroups leaves (o, m, l) partials, combined by its last contributor to arrive
      const bool whole = j0 == 0 && nseg == nblk;
      const bool defer = att_defer<NQT>() && !whole;   // next segment's block after the arrival
      f32x4 acc[NQT][8];
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) acc[qt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
      float m_run[NQT], l_run[NQT];
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt) {
        m_run[qt] = -INFINITY;
        l_run[qt] = 0.f;
      }
      bf16(*vs)[HD + 8] = sh.u.a.vm.v[wave];
      for (int k = wave; k < nseg; k += NWAVE) {
        const int key0 = (j0 + k) * 32;
        if (!pre) load_block(kvbase, key0);
        if (pok && key0 < p0 + W && key0 + 32 > p0) {
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            const int dk = key0 + t * 16 + l16 - (int)p0;
#pragma unroll
            for (int kb = 0; kb < 4; ++kb)
              if (dk >= 0 && dk < W) kreg[t][kb] = *(const u32x4*)&sh.u.a.kvn[2 * (sg * W + dk)][kb * 32 + g4 * 8];
          }
#pragma unroll
          for (int it = 0; it < 8; ++it) {
            const int cc = it * 64 + lane;
            const int dk = key0 + (cc >> 4) - (int)p0;
            if (dk >= 0 && dk < W) vreg[it] = *(const u32x4*)&sh.u.a.kvn[2 * (sg * W + dk) + 1][(cc & 15) * 8];
          }
        }
        f32x4 sc[2][NQT];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int qt = 0; qt < NQT; ++qt) {
            f32x4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) d = mfma16x16x32(kreg[t][kb], qreg[qt][kb], d);
            sc[t][qt] = d;
          }
#pragma unroll
        for (int it = 0; it < 8; ++it) {
          const int cc = it * 64 + lane;
          *(u32x4*)&vs[cc >> 4][(cc & 15) * 8] = vreg[it];
        }
        // K and V of this block are consumed: the wave's next block (in this segment, else its
        // first block of the next one) streams in during the softmax, P.V and merge. After a
        // split segment the next segment's block is requested at the arrival instead (below).
        pre = false;
        if (k + NWAVE < nseg) {
          load_block(kvbase, key0 + NWAVE * 32);
          pre = true;
        } else if (!defer && sg + 1 < nsg && wave < sh.seg[sg + 1][3]) {
          load_block((size_t)(sh.seg[sg + 1][0] * NKV + sh.seg[sg + 1][1]) * a.cap * HD,
                     (sh.seg[sg + 1][2] + wave) * 32);
          pre = true;
        }
        u32x4 pB[NQT];
        float alpha[NQT];
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) {
          float sv[8];
          float mloc = -INFINITY;
#pragma unroll
          for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int key = key0 + t * 16 + g4 * 4 + q;
              const float v = key <= lim[qt] ? sc[t][qt][q] * scale_log2 : -INFINITY;
              sv[t * 4 + q] = v;
              mloc = fmaxf(mloc, v);
            }
          // (the two-tile instantiation keeps the LDS shuffles: its register allocation spills more
          // with the swaps)
          mloc = fmaxf(mloc, NQT == 1 ? lane_xor16(mloc) : __shfl_xor(mloc, 16, 64));
          mloc = fmaxf(mloc, NQT == 1 ? lane_xor32(mloc) : __shfl_xor(mloc, 32, 64));
          const float m_new = fmaxf(m_run[qt], mloc);
          const float msafe = m_new == -INFINITY ? 0.f : m_new;
          alpha[qt] = exp2_hw(m_run[qt] - msafe);
          float psum = 0.f;
          unsigned pk[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const float pa = exp2_hw(sv[2 * jj] - msafe);
            const float pb = exp2_hw(sv[2 * jj + 1] - msafe);
            psum += pa + pb;
            pk[jj] = pk_bf16(pa, pb);
          }
          psum += NQT == 1 ? lane_xor16(psum) : __shfl_xor(psum, 16, 64);
          psum += NQT == 1 ? lane_xor32(psum) : __shfl_xor(psum, 32, 64);
          l_run[qt] = l_run[qt] * alpha[qt] + psum;
          m_run[qt] = m_new;
          pB[qt] = u32x4{pk[0], pk[1], pk[2], pk[3]};
        }
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt)
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) acc[qt][dt] *= alpha[qt];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // V^T operand of dim tile dt: lane (l16, g4) needs V[key][dt 16 + l16] for keys g4 4 + q
        // and 16 + g4 4 + q (q = 0..3, the lane-local P key order): two transposing LDS loads
        // (ds_read_b64_tr_b16: output lane j of a 16-lane group gets element j % 4 of the 8-byte
        // rows that source lanes j / 4 + 4 q address), each source lane addressing 4 dims of one
        // key. 16 loads per block instead of 64 two-byte loads, which the register-bound compiler
        // issued two at a time, each pair waited for (decode B = 16 2.661 -> 2.617 ms, B = 1
        // 1.975 -> 1.954; verify 4.794 -> 4.781).
        const int trow = g4 * 4 + (l16 >> 2), tcol = 4 * (l16 & 3);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const u32x2 lo = lds_read_tr16(&vs[trow][dt * 16 + tcol]);
          const u32x2 hi = lds_read_tr16(&vs[16 + trow][dt * 16 + tcol]);
#pragma unroll
          for (int qt = 0; qt < NQT; ++qt)
            acc[qt][dt] = mfma16x16x32(u32x4{lo.x, lo.y, hi.x, hi.y}, pB[qt], acc[qt][dt]);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
      // the waves' running max and sum of every query row
      if (g4 == 0) {
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt)
          if (16 * qt + l16 < R) {
            sh.ms[wave][16 * qt + l16] = m_run[qt];
            sh.ls[wave][16 * qt + l16] = l_run[qt];
          }
      }
      // the cache's K/V of the new keys in this segment's blocks (read by later steps only;
      // complete before the phase's barrier). Each lane stores one 16-byte chunk of K and the
      // same chunk of V through the two uniform descriptors: a descriptor chosen per lane would
      // be compiled as a loop over the distinct descriptors, and under register pressure the
      // verify instantiation's allocation of such a loop reloaded a spilled half-descriptor into
      // the registers its next iteration reads (a store through a wrong base address).
      if (pok && tid() < 16 * W) {
        const int sn = tid() >> 4, ch = tid() & 15;
        const int key = (int)p0 + sn;
        if (key >= j0 * 32 && key < (j0 + nseg) * 32) {
          const unsigned co = (unsigned)(((size_t)bk * a.cap + key) * HD * 2) + ch * 16;
          stc_b128(kwr, co, *(const u32x4*)&sh.u.a.kvn[2 * (sg * W + sn)][ch * 8]);
          stc_b128(vwr, co, *(const u32x4*)&sh.u.a.kvn[2 * (sg * W + sn) + 1][ch * 8]);
        }
      }
      const int myslot = first_seg ? 0 : 1;
      first_seg = false;
      // merge the waves one 16-row query tile at a time (the V buffers hold the tile)
#pragma unroll
      for (int qt = 0; qt < NQT; ++qt) {
        __syncthreads();
        if (16 * qt + l16 < R) {
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) *(f32x4*)&sh.u.a.vm.mrg[wave][l16][dt * 16 + g4 * 4] = acc[qt][dt];
        }
        __syncthreads();
        const int nr = min(16, R - 16 * qt);
        for (int e = tid(); e < nr * HD; e += NTHR) {
          const int rl = e / HD, d = e - rl * HD, row = 16 * qt + rl;
          // every wave's max, sum and output of this element read at once (one LDS latency)
          float mv[NWAVE], lv[NWAVE], ov[NWAVE];
#pragma unroll
          for (int w = 0; w < NWAVE; ++w) {
            mv[w] = sh.ms[w][row];
            lv[w] = sh.ls[w][row];
            ov[w] = sh.u.a.vm.mrg[w][rl][d];
          }
          float Mx = -INFINITY;
#pragma unroll
          for (int w = 0; w < NWAVE; ++w) Mx = fmaxf(Mx, mv[w]);
          const float Ms = Mx == -INFINITY ? 0.f : Mx;
          float o = 0.f, l = 0.f;
#pragma unroll
          for (int w = 0; w < NWAVE; ++w) {
            const float f = exp2_hw(mv[w] - Ms);
            o += ov[w] * f;
            l += lv[w] * f;
          }
          if (whole) {
            const int s = row / G, g = row - s * G;
            stc_b16(orr, xoff(b * W + s, (kvh * G + g) * HD + d, M) * 2, f2bf(o / l));
          } else {
            const unsigned pb = (unsigned)(((blockIdx.x * 2 + myslot) * R + row) * rec) * 4;
            stc_f32(pr, pb + d * 4, o);
            if (d == 0) {
              stc_f32(pr, pb + HD * 4, Mx);
              stc_f32(pr, pb + (HD + 1) * 4, l);
            }
          }
        }
      }
      if (sg == 0) STEP_TRACE(p, 7);            // merged, outputs / partials stored
      if (!whole) {
        int fw, lw, nc = 0;
        if (sh.apm) {                          // the pair's workgroups, each holding blocks
          const int q = b * (NKV / P) + (kvh - h0);
          fw = sh.pf[q];
          lw = sh.pf[q + 1] - 1;
          nc = lw - fw + 1;
        } else {
          fw = attn_owner(Tu, Ga, S + ova);
          lw = attn_owner(Tu, Ga, S + ova + nblk - 1);
          for (int c = fw; c <= lw; ++c) nc += sh.afirst[c + 1] > sh.afirst[c];
        }
        // The arrival (as arrive_last): every thread's partial stores complete, then one
        // counter increment. Vector memory operations complete in issue order, so with `defer`
        // the next segment's first block is requested only now: requested before the stores,
        // the store wait would also wait for it. The waves request it right behind the
        // increment, and only wave 0 waits for the increment's return.
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        int* cnt = a.ctr + C_ATT + bk;
        int old = 0;
        if (tid() == 0) old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_sched_barrier(0);
        if (defer && sg + 1 < nsg && wave < sh.seg[sg + 1][3]) {
          load_block((size_t)(sh.seg[sg + 1][0] * NKV + sh.seg[sg + 1][1]) * a.cap * HD,
                     (sh.seg[sg + 1][2] + wave) * 32);
          pre = true;
        }
        if (tid() == 0) {
          const int last = old == nc - 1;
          if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          sh.flag = last;
        }
        __syncthreads();
        if (sg == 0) STEP_TRACE(p, 8);          // arrival counted
        if (sh.flag) {
          if (DD_ATT_CMB_1R && NQT > 1) attn_combine_1r(a, sh, layer, b, kvh, S, fw, lw, P, gx);
          else attn_combine(a, sh, layer, b, kvh, S, fw, lw, P, gx);
        }
        if (sg == 0) STEP_TRACE(p, 10);
      }
      __syncthreads();
    }
    i = inext;
  }
  STEP_TRACE(p, 6);
}

// ---------------------------------------------------------------------------------------------
// embedding gather: workgroup c copies the same columns of every row that it owns in the O and
// down phases, and stores their sums of squares ss[0][c][m]
template <int NM>
__device__ __forceinline__ void embed_phase(const Args& a, Shared& sh) {
  const int M = a.M;
  const int t = tid();
  if (t >= 256) return;
  const int c0 = part_lo(a.H, gridDim.x, blockIdx.x), nc = part_lo(a.H, gridDim.x, blockIdx.x + 1) - c0;
  const rsrc_t hr = make_rsrc(h_slot(a, 0), (unsigned)((size_t)M * a.H * 2));
  const rsrc_t ssr = make_rsrc(ss_slot<NM>(a, 0), (unsigned)(gridDim.x * 16 * NM * 4));
#pragma unroll
  for (int n = 0; n < NM; ++n) {
    const int m = 16 * n + (t >> 4), j = t & 15;
    float s = 0.f;
    if (m < M && j < nc) {
      int64_t tk = a.tok[m];
      if (tk < 0 || tk >= a.V) {
        if (j == 0) atomicOr(a.err, E_TOKEN);
        tk = 0;
      }
      const bf16 v = a.embed[(size_t)tk * a.H + c0 + j];
      stc_b16(hr, xoff(m, c0 + j, M) * 2, v);
      s = bf2f(v) * bf2f(v);
    }
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (j == 0) stc_f32(ssr, (unsigned)(blockIdx.x * 16 * NM + m) * 4, s);
  }
}

// NM: 16-row activation tiles (1: decode, M <= 16; 5: verify, M <= 80)
template <int NM>
__global__ void __launch_bounds__(NTHR, 1) decode_step_kernel(Args a_in) {
  constexpr int MS = 16 * NM, NQT = NM == 1 ? 1 : 2;
  Args a = a_in;
  extern __shared__ unsigned char smem_raw[];
  Shared& sh = *(Shared*)smem_raw;
  if (tid() < MS) {
    sh.bestv[tid()] = -INFINITY;
    sh.besti[tid()] = 0x7fffffff;
  }
  if (tid() == 0) sh.bail = 0;
  if (tid() < a.B) sh.pseq[tid()] = a.pos[tid()];
  for (int e = tid(); e < a.L * LFIELDS; e += NTHR)
    sh.ltab[e / LFIELDS][e % LFIELDS] = a.layers[(size_t)(e / LFIELDS) * NFIELD + e % LFIELDS];
  __syncthreads();
  {
    // attention phases are p = 2 + 5l: position errors are flagged when one of them runs
    const int l0 = a.phase_begin <= 2 ? 0 : (a.phase_begin - 2 + 4) / 5;
    attn_partition<NM>(a, sh, l0 < a.L && 2 + 5 * l0 < a.phase_end);
  }
  const int nqkv = (a.NH + 2 * a.NKV) * HD;
  // The phases run in their fixed order (embedding; per layer QKV, attention, O, gate/up, down;
  // lm_head), written out in that order rather than dispatched per phase index (measured: 1.6%
  // faster per step at B = 16). Phase q runs when phase_begin <= q < phase_end and waits at a
  // barrier (epoch q - phase_begin) unless it is the launch's first phase.
  auto in_range = [&](int q) { return q >= a.phase_begin && q < a.phase_end; };
  auto epoch_of = [&](int q) { return (unsigned)(q - a.phase_begin); };
#ifdef DD_STEP_TRACE
#define SET_PHASE(q) (a.phase_cur = (q))
#else
#define SET_PHASE(q) ((void)0)
#endif
  if (in_range(0)) {                          // the embedding (phase 0) never waits
    SET_PHASE(0);
    STEP_TRACE(0, 0);
    STEP_TRACE(0, 1);
    embed_phase<NM>(a, sh);
    STEP_TRACE(0, 3);
  }
  const int l0 = a.phase_begin <= 1 ? 0 : (a.phase_begin - 1) / 5;
  for (int layer = l0; layer < a.L; ++layer) {
    const int q0 = 1 + 5 * layer;             // this layer's QKV phase
    if (q0 >= a.phase_end) break;
    const long long* lp = sh.ltab[layer];
    if (in_range(q0)) {
      SET_PHASE(q0);
      run_gemv<M_QKV, NM, true, EPI_QKV>(a, sh, q0, q0 > a.phase_begin, epoch_of(q0),
                                         uniform_ptr<const bf16>(lp[F_WQKV]), nqkv, a.H,
                                         h_slot(a, 2 * layer), uniform_ptr<const bf16>(lp[F_LN1]),
                                         ss_slot<NM>(a, 2 * layer), layer);
    }
    if (in_range(q0 + 1)) {
      SET_PHASE(q0 + 1);
      const bool sync = q0 + 1 > a.phase_begin;
      STEP_TRACE(q0 + 1, 0);
      if (sync) bar_arrive(a, epoch_of(q0 + 1));
      attention_phase<NQT>(a, sh, layer, q0 + 1, sync, epoch_of(q0 + 1));
      STEP_TRACE(q0 + 1, 3);
    }
    if (in_range(q0 + 2)) {
      SET_PHASE(q0 + 2);
      if (NM > 1 && DD_SPL_O && res_split_ok(a.NH * HD))
        run_res_split<M_O, NM>(a, sh, q0 + 2, q0 + 2 > a.phase_begin, epoch_of(q0 + 2),
                           uniform_ptr<const bf16>(lp[F_WO]), a.H, a.NH * HD, attn_slot(a, layer),
                           2 * layer + 1);
      else
        run_gemv<M_O, NM, false, EPI_RES>(a, sh, q0 + 2, q0 + 2 > a.phase_begin, epoch_of(q0 + 2),
                                          uniform_ptr<const bf16>(lp[F_WO]), a.H, a.NH * HD,
                                          attn_slot(a, layer), nullptr, nullptr, 2 * layer + 1);
    }
    if (in_range(q0 + 3)) {
      SET_PHASE(q0 + 3);
      run_gemv<M_GU, NM, true, EPI_SILU>(a, sh, q0 + 3, q0 + 3 > a.phase_begin, epoch_of(q0 + 3),
                                         uniform_ptr<const bf16>(lp[F_WGU]), a.I, a.H,
                                         h_slot(a, 2 * layer + 1), uniform_ptr<const bf16>(lp[F_LN2]),
                                         ss_slot<NM>(a, 2 * layer + 1), layer);
    }
    if (in_range(q0 + 4)) {
      SET_PHASE(q0 + 4);
      if ((NM > 1 || a.B >= DD_SPL_MINM) && res_split_ok(a.I))
        run_res_split<M_D, NM>(a, sh, q0 + 4, q0 + 4 > a.phase_begin, epoch_of(q0 + 4),
                           uniform_ptr<const bf16>(lp[F_WD]), a.H, a.I, m_slot(a, layer),
                           2 * layer + 2);
      else
        run_gemv<M_D, NM, false, EPI_RES>(a, sh, q0 + 4, q0 + 4 > a.phase_begin, epoch_of(q0 + 4),
                                          uniform_ptr<const bf16>(lp[F_WD]), a.H, a.I,
                                          m_slot(a, layer), nullptr, nullptr, 2 * layer + 2);
    }
  }
  const int qlm = 1 + 5 * a.L;
  if (in_range(qlm)) {
    SET_PHASE(qlm);
    if (NM > 1 && DD_V_LM_WIDE)
      run_lm_wide<NM>(a, sh, qlm, qlm > a.phase_begin, epoch_of(qlm));
    else
      run_gemv<M_LM, NM, true, EPI_LOGITS>(a, sh, qlm, qlm > a.phase_begin, epoch_of(qlm), a.lm_t, a.V,
                                           a.H, h_slot(a, 2 * a.L), a.fnorm, ss_slot<NM>(a, 2 * a.L), 0);
    // argmax over the workgroups' candidates; the last workgroup writes the tokens and, for a
    // decode step (W = 1), advances the positions
    const rsrc_t cr = make_rsrc(a.ws + a.off_am, (unsigned)(gridDim.x * MS * 2 * 4));
    if (tid() < (unsigned)a.M) {
      stc_f32(cr, (unsigned)((blockIdx.x * MS + tid()) * 2) * 4, sh.bestv[tid()]);
      stc_u32(cr, (unsigned)((blockIdx.x * MS + tid()) * 2 + 1) * 4, (unsigned)sh.besti[tid()]);
    }
    if (arrive_last(a.ctr + C_AM, gridDim.x, &sh.flag)) {
      // one wave per row: lanes scan the workgroups' candidates, then a wave reduction
      const int lane = tid() & 63;
      for (int m = wave_id(); m < a.M; m += NWAVE) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
        for (int w = lane; w < (int)gridDim.x; w += 64) {
          const float v = ldc_f32(cr, (unsigned)((w * MS + m) * 2) * 4);
          const int i = (int)ldc_u32(cr, (unsigned)((w * MS + m) * 2 + 1) * 4);
          if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          const float ov = __shfl_xor(bv, o, 64);
          const int oi = __shfl_xor(bi, o, 64);
          if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        }
        if (lane == 0) {
          a.otok[m] = bi;
          if (a.W == 1) a.pos[m] = sh.pseq[m] + 1;
        }
      }
    }
  }
#undef SET_PHASE
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
// Weight re-layout for the step (one thread per 16 source bytes). Matrix `kind` is split into
// units (rows; gate/up: features, unit u = gate row u and up row gate_up_I + u) over G
// workgroups exactly as the step's GEMV phases split it; workgroup c's units are stored from
// unit u0(c) on (so its region starts at byte u0 * UPR * K * 2), in chunks of up to CAPU units;
// a chunk of `rows` weight rows (gate rows, then up rows) is k-step-major: row j of k-step ks
// (32 columns, 64 bytes) at chunk byte (ks * rows + j) * 64. QKV rows are taken in head-grouped
// order (aux = NKV kv heads): row r of kv head h = r / per (per = N / NKV rows) is q row
// h G HD + t for t = r % per < G HD, else k row (NH + h) HD + t - G HD, else v row
// (NH + NKV + h) HD + t - (G + 1) HD of cat(q, k, v). Gate/up: aux = I.
__global__ void tile_weight_kernel(const bf16* __restrict__ src, bf16* __restrict__ dst, int N, int K,
                                   int kind, int aux, int G) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  const int q8 = K >> 3;
  if (idx >= (size_t)N * q8) return;
  const int r = (int)(idx / q8), q = (int)(idx - (size_t)r * q8);
  int sr = r;                                               // source row of tiled-order row r
  if (kind == M_QKV) {
    const int per = N / aux, Gq = per / HD - 2, h = r / per, t = r - h * per, NHq = aux * Gq;
    sr = t < Gq * HD ? h * Gq * HD + t
       : t < (Gq + 1) * HD ? (NHq + h) * HD + t - Gq * HD
                           : (NHq + aux + h) * HD + t - (Gq + 1) * HD;
  }
  const int gate_up_I = kind == M_GU ? aux : 0;
  const int UPR = kind == M_GU ? 2 : 1;
  const int CAPU = kind == M_QKV ? mat_CAPU(M_QKV) : kind == M_O ? mat_CAPU(M_O)
                 : kind == M_GU ? mat_CAPU(M_GU) : kind == M_D ? mat_CAPU(M_D) : mat_CAPU(M_LM);
  const bool gu = kind == M_GU;
  const int half = gu && r >= gate_up_I;
  const int u = gu ? (half ? r - gate_up_I : r) : r / UPR;   // unit of row r
  const int nunits = gu ? gate_up_I : N / UPR;
  const int c = (int)(((unsigned)(u + 1) * (unsigned)G - 1) / (unsigned)nunits);
  const int u0 = part_lo(nunits, G, c), u1 = part_lo(nunits, G, c + 1);
  const int ch = (u - u0) / CAPU;
  const int ua = u0 + ch * CAPU;
  const int nu = min(CAPU, u1 - ua);
  const int rows = nu * UPR;
  const int j = gu ? (u - ua) + (half ? nu : 0) : r - ua * UPR;
  const int ks = q >> 2, kq = q & 3;
  const size_t d = (size_t)ua * UPR * K + ((size_t)ks * rows + j) * 32 + kq * 8;
  *(u32x4*)(dst + d) = *(const u32x4*)(src + (size_t)sr * K + q * 8);
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
    if (hipFuncSetAttribute((const void*)decode_step_kernel<1>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(Shared)) !=
            hipSuccess ||
        hipFuncSetAttribute((const void*)decode_step_kernel<5>,
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)sizeof(Shared)) !=
            hipSuccess)
      return (int)hipErrorInvalidConfiguration;
    attr_set = true;
  }
  // every workgroup of the grid must be resident at once (the phases meet at grid barriers):
  // one workgroup per CU fits, for both instantiations
  int occ1 = 0, occ5 = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ1, decode_step_kernel<1>, NTHR, sizeof(Shared)) !=
          hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ5, decode_step_kernel<5>, NTHR, sizeof(Shared)) !=
          hipSuccess ||
      occ1 < 1 || occ5 < 1)
    return (int)hipErrorInvalidConfiguration;
  *G_out = cus & ~7;   // barrier groups workgroups by XCD (8 per device)
  if (*G_out < 8 || *G_out > MAXG) return (int)hipErrorInvalidConfiguration;
  return 0;
}

// activation tiles of a launch with W tokens per sequence: decode (W = 1, M <= 16) or verify
// a launch of B sequences with W tokens each runs the 16-row instantiation when its rows fit one
// 16-row MFMA tile (B W <= 16) and each (sequence, kv head) pair's query rows one 16-column
// query tile (W G <= 16): decode steps, and the small verify steps of speculation at B <= 4;
// wider verify steps run the 80-row one
static int step_nm(int B, int W, int G_heads) { return B * W <= 16 && W * G_heads <= 16 ? 1 : 5; }
// workspace sizing for any B: the 80-row instantiation's layout bounds the 16-row one's
static int ws_nm(int W) { return W == 1 ? 1 : 5; }

struct WsLayout { size_t ss, att, am, spl, total; };

static WsLayout ws_layout(int L, int G, int G_heads, int W, int NM) {
  const size_t MS = 16 * (size_t)NM;
  WsLayout w;
  w.ss = 0;                                                  // [2L+1][G][16 NM]
  w.att = w.ss + (size_t)(2 * L + 1) * G * MS;
  w.am = w.att + (size_t)L * G * 2 * W * G_heads * ATT_REC;  // attention: per layer, 2 slots
  w.spl = w.am + (size_t)G * MS * 2;
  w.total = w.spl + (size_t)2 * L * G * spl_floats(NM);               // split O / down partials
  return w;
}

DD_API int dd_step_grid(void) {
  int G = 0;
  return step_grid(&G) == 0 ? G : -1;
}

DD_API int dd_step_counters(void) { return C_TOTAL; }

// Zeroed counters for dd_decode_step in uncached device memory: the barrier and hand-off atomics
// and polls are served by memory directly instead of passing through the per-XCD L2s (faster
// under the decode step's streaming load). The memory is never freed: uncached memory must stay
// mapped for the life of the process once a kernel has read it.
DD_API int dd_step_counters_alloc(void** out) {
  DD_REQUIRE(out != nullptr);
  void* p = nullptr;
  hipError_t e = hipExtMallocWithFlags(&p, C_TOTAL * sizeof(int), hipDeviceMallocUncached);
  if (e != hipSuccess) return (int)e;
  e = hipMemset(p, 0, C_TOTAL * sizeof(int));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) return (int)e;
  *out = p;
  return 0;
}

// Diagnostics: copy the dd_step_counters() ints at `counters` to host memory (synchronous).
DD_API int dd_step_counters_read(const void* counters, int* host) {
  DD_REQUIRE(counters != nullptr && host != nullptr);
  return (int)hipMemcpy(host, counters, C_TOTAL * sizeof(int), hipMemcpyDeviceToHost);
}

// Diagnostics and tests: overwrite the dd_step_counters() ints at `counters` from host memory
// (waits for the device first; synchronous).
DD_API int dd_step_counters_write(void* counters, const int* host) {
  DD_REQUIRE(counters != nullptr && host != nullptr);
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemcpy(counters, host, C_TOTAL * sizeof(int), hipMemcpyHostToDevice);
  return (int)e;
}

// Zero every counter after a launch that timed out at a grid barrier (error flag 4): its
// workgroups stopped waiting, so the hand-off counters that their last arrivers reset (attention
// combines, split down pairs, argmax) may be left nonzero. Waits for the device first; not for
// use under graph capture.
DD_API int dd_step_counters_clear(void* counters) {
  DD_REQUIRE(counters != nullptr);
  hipError_t e = hipDeviceSynchronize();
  if (e == hipSuccess) e = hipMemset(counters, 0, C_TOTAL * sizeof(int));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  return (int)e;
}

DD_API size_t dd_step_ws_bytes(int L, int NH, int NKV, int W) {
  int G = 0;
  if (L < 1 || NKV < 1 || NH < NKV || W < 1 || W > MAXW || step_grid(&G) != 0) return 0;
  return ws_layout(L, G, NH / NKV, W, ws_nm(W)).total * sizeof(float);
}

DD_API size_t dd_tiled_bytes(int N, int K) { return (size_t)N * K * 2; }

DD_API int dd_tile_weight(const void* src, void* dst, int N, int K, int matrix, int aux,
                          hipStream_t stream) {
  DD_REQUIRE(src && dst && matrix >= 0 && matrix < NMAT && N >= 1 && K >= 256 && K % 256 == 0);
  DD_REQUIRE((matrix == M_GU || matrix == M_QKV) == (aux > 0));
  DD_REQUIRE(matrix != M_GU || N == 2 * aux);
  DD_REQUIRE(matrix != M_QKV || (N % aux == 0 && (N / aux) % HD == 0 && N / aux >= 3 * HD));
  DD_REQUIRE(aligned16(src) && aligned16(dst));
  DD_REQUIRE((long long)N * K < (1ll << 40));
  int G = 0;
  const int e = step_grid(&G);
  if (e != 0) return e;
  DD_REQUIRE((long long)N * G < (1ll << 32));
  const size_t n16 = (size_t)N * (K / 8);
  hipLaunchKernelGGL(tile_weight_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, stream,
                     (const bf16*)src, (bf16*)dst, N, K, matrix, aux, G);
  return launch_status();
}

// Model geometry the phases take (Qwen3 family, head_dim 128) for B sequences of W tokens;
// G > 0 also checks the split of every GEMV over that many workgroups.
static bool geometry_ok(int L, int H, int NH, int NKV, int I, int V, int B, int W, int G) {
  if (!(B >= 1 && B <= MAXB && W >= 1 && W <= MAXW && B * W <= MAXROWS && L >= 1 &&
        NKV >= 1 && NH >= NKV && NH % NKV == 0 && NH / NKV <= MAXG_HEADS &&
        ((NH / NKV) & (NH / NKV - 1)) == 0 && W * (NH / NKV) <= MAXR && L <= MAXL))
    return false;
  if (MAXB * NKV > C_AM - C_ATT) return false;            // one combine counter per (sequence, kv head)
  // every GEMV K is a whole number of 8-wave rounds of 32-column k-steps; the normalised inputs
  // (K = H) fit the LDS norm-weight window
  if (!(H % 256 == 0 && (NH * HD) % 256 == 0 && I % 256 == 0 && H <= MAXH && V >= 1 && I >= 1))
    return false;
  if (G > 0) {
    if (H > 16 * G) return false;                          // O / down: one 16-row tile per WG
    const long long units[5] = {(long long)(NH + 2 * NKV) * HD, H, I, H, V};
    for (int q = 0; q < 5; ++q)
      if (units[q] * G >= (1ll << 32)) return false;      // 32-bit partition arithmetic
    // decode: a workgroup's chunks before its last fit the LDS staging: (chunks - 1) x chunk
    // units <= LGS_ROWS for QKV, gate/up and lm_head (O and down have one chunk)
    const int stq[3] = {M_QKV, M_GU, M_LM};
    for (int q = 0; q < 3 && step_nm(B, W, NH / NKV) == 1; ++q) {
      const long long cap = mat_CAPU(stq[q]);
      const long long nu = (units[stq[q]] + G - 1) / G;          // most units of a workgroup
      if (((nu + cap - 1) / cap - 1) * cap > LGS_ROWS) return false;
    }
    // a workgroup's weight region stays below 2^31 bytes (32-bit buffer offsets)
    if ((long long)((V + G - 1) / G) * H * 2 >= (1ll << 31)) return false;
    if ((long long)((I + G - 1) / G) * 2 * H * 2 >= (1ll << 31)) return false;
  }
  return true;
}

DD_API int dd_step_supported(int L, int H, int NH, int NKV, int I, int V, int B, int W) {
  int G = 0;
  if (step_grid(&G) != 0) return 0;
  return geometry_ok(L, H, NH, NKV, I, V, B, W, G) ? 1 : 0;
}

DD_API int dd_decode_step(const int64_t* layer_table, int L, const void* embed, const void* lm_tiled,
                          const void* final_norm, const void* cos_t, const void* sin_t,
                          int rope_rows, const int64_t* tok, int64_t* out_tok, int64_t* pos, void* h,
                          void* qkv, void* attn, void* mbuf, void* logits, void* ws, int* counters,
                          int* err, int B, int W, int H, int NH, int NKV, int I, int V, int cap,
                          float eps, int phase_begin, int phase_end, hipStream_t stream) {
  DD_REQUIRE(layer_table && embed && lm_tiled && final_norm && cos_t && sin_t && tok && out_tok && pos);
  DD_REQUIRE(h && qkv && attn && mbuf && logits && ws && counters && err);
  DD_REQUIRE(geometry_ok(L, H, NH, NKV, I, V, B, W, 0));
  DD_REQUIRE(cap >= 1 && rope_rows >= 1 && rope_rows <= (1 << 23));   // cos/sin byte ranges < 2^31
  DD_REQUIRE(phase_begin >= 0 && phase_begin < phase_end && phase_end <= 2 + 5 * L);
  int G = 0;
  const int e = step_grid(&G);
  if (e != 0) return e;
  DD_REQUIRE(geometry_ok(L, H, NH, NKV, I, V, B, W, G));
  // attention partition units (32-bit arithmetic in the kernel)
  DD_REQUIRE((long long)MAXB * NKV * (ATT_OVH_MAX + cap / 32 + 1) * (G + 1) < (1ll << 31));
  // K/V cache byte ranges (32-bit buffer offsets)
  DD_REQUIRE((long long)B * NKV * cap * HD * 2 < (1ll << 32));
  const int NM = step_nm(B, W, NH / NKV);
  const WsLayout w = ws_layout(L, G, NH / NKV, W, NM);   // within dd_step_ws_bytes(L, NH, NKV, W)
  Args a;
  a.layers = layer_table;
  a.embed = (const bf16*)embed;
  a.lm_t = (const bf16*)lm_tiled;
  a.fnorm = (const bf16*)final_norm;
  a.cos_t = (const bf16*)cos_t;
  a.sin_t = (const bf16*)sin_t;
  a.tok = tok;
  a.otok = out_tok;
  a.pos = pos;
  a.h = (bf16*)h;
  a.qkv = (bf16*)qkv;
  a.attn = (bf16*)attn;
  a.mbuf = (bf16*)mbuf;
  a.logits = (bf16*)logits;
  a.ws = (float*)ws;
  a.ctr = counters;
  a.err = err;
  a.L = L; a.B = B; a.W = W; a.M = B * W; a.H = H; a.NH = NH; a.NKV = NKV; a.I = I; a.V = V;
  a.cap = cap; a.rope_rows = rope_rows; a.eps = eps;
  a.phase_begin = phase_begin;
  a.phase_end = phase_end;
  a.off_ss = (unsigned)w.ss;
  a.off_att = (unsigned)w.att;
  a.off_am = (unsigned)w.am;
  a.off_spl = (unsigned)w.spl;
  if (NM == 1)
    hipLaunchKernelGGL(decode_step_kernel<1>, dim3(G), dim3(NTHR), sizeof(Shared), stream, a);
  else
    hipLaunchKernelGGL(decode_step_kernel<5>, dim3(G), dim3(NTHR), sizeof(Shared), stream, a);
  return launch_status();
}

#ifdef DD_STEP_TRACE
// Profiling builds only: copy the timing trace ([1024][192][12] u64) to host memory.
DD_API int dd_step_trace(void* host, size_t bytes) {
  return (int)hipMemcpyFromSymbol(host, HIP_SYMBOL(g_trace), bytes, 0, hipMemcpyDeviceToHost);
}
#endif
