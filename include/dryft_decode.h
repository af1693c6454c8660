/* dryft_decode.h -- C ABI of the MI355X (gfx950) decode-step kernels.
 *
 * Drop-in boundary for the decode hot path of KrishP147/Dryft-Challenge-HTN-2026: each entry
 * point replaces one method of the reference's ops object (``TritonOps`` in engine/fused.py,
 * whose reference arithmetic is ``_TorchOps`` in engine/engine.py) or one step of
 * ``Engine._forward`` / ``_decode_body``. The Python host (hipops.py) binds these with ctypes
 * exactly where the reference launches its Triton kernels.
 *
 * Conventions
 *  - All tensors are device pointers to contiguous row-major memory on the current HIP device.
 *    bf16 tensors are passed as ``const void*`` / ``void*`` (16-bit patterns); fp32 workspaces
 *    as ``void*``; positions and token ids as int64 (torch.long).
 *  - The kernel entry points (everything that takes a ``stream``) are asynchronous on it and
 *    capture-safe: no device allocation, no host sync, positions are read from device memory.
 *    dd_gemm_bf16 keeps that contract too; its first call of a shape creates hipBLASLt
 *    descriptors on the host. The exceptions are set-up and diagnostics calls, marked where
 *    they are declared: dd_step_counters_alloc (allocates), dd_step_counters_read / _write /
 *    _clear (synchronous) and dd_attn_decode_noalloc's first call on a device (a synchronous
 *    clear of its static counters).
 *  - Return value: 0 on success; hipErrorInvalidValue (1) when an argument fails validation
 *    (nothing is launched then); otherwise the hipError_t reported by the launch. Nothing throws
 *    across the ABI.
 *  - ``err`` (optional, may be NULL) is a device int that kernels OR flags into instead of
 *    faulting: 1 = token id out of range (row 0 used), 2 = position outside cache/rope table
 *    (row skipped).
 *  - ``counters`` are caller-owned device ints that must be zero before the first call; every
 *    call leaves them zero again (the last workgroup to arrive resets them), so one zeroed
 *    buffer serves any number of calls on one stream. Calls that overlap in time must not share
 *    counters or workspaces.
 */
#ifndef DRYFT_DECODE_H
#define DRYFT_DECODE_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version (bumped on any signature change). */
int dd_abi_version(void);

/* y[m] = rmsnorm(x[m]) * w, m < M, row length N (N <= 4096).
 * Replaces TritonOps.rms (fused.py:894-895; kernel fused.py:152-172), reference
 * _TorchOps.rms / _rms (engine.py:107-110, 134-135). */
int dd_rmsnorm(const void* x, const void* w, void* y, int M, int N, float eps, hipStream_t stream);

/* hn = bf16(x + d); y = rmsnorm(hn) * w.
 * Replaces TritonOps.add_rms (fused.py:897-898; kernel fused.py:152-172 with HAS_ADD). */
int dd_add_rmsnorm(const void* x, const void* d, const void* w, void* hn, void* y, int M, int N,
                   float eps, hipStream_t stream);

/* y[M,N] = x[M,K] . W[N,K]^T (bf16 out, fp32 accumulate), 1 <= M <= 16, K % 8 == 0,
 * x and W 16-byte aligned. splitk <= 0 picks the library's choice (dd_gemv_splitk); with more
 * than one split, ws must hold dd_gemv_ws_bytes and counters dd_gemv_counters(N) zeroed ints
 * (the split-K sum happens in the same launch).
 * Replaces TritonOps.linear (fused.py:989-1014; kernels fused.py:568-628), reference
 * _TorchOps.linear = F.linear (engine.py:131-132). */
int dd_gemv(const void* x, const void* W, void* y, int M, int N, int K, int splitk, void* ws,
            int* counters, hipStream_t stream);

/* The split-K factor dd_gemv / dd_gemv_add_rmsnorm use for this shape when splitk <= 0.
 * Replaces the shape-keyed tile table GEMM_CFG (fused.py:711-718, 773-789). */
int dd_gemv_splitk(int M, int N, int K);
size_t dd_gemv_ws_bytes(int M, int N, int K, int splitk);
int dd_gemv_counters(int N);

/* hn = bf16(h + bf16(x . W^T)); y = rmsnorm(hn) * lnw, in one launch (split-K partials, the
 * residual and the row norm are finished by the last workgroups to arrive).
 * ws: dd_gemv_add_rmsnorm_ws_bytes; counters: dd_gemv_counters(N) zeroed ints.
 * Replaces TritonOps.linear_add_norm (fused.py:1034-1059; kernels fused.py:568-618, 685-709),
 * reference _TorchOps.linear_add_norm (engine.py:140-142). */
int dd_gemv_add_rmsnorm(const void* x, const void* W, const void* h, const void* lnw, void* hn,
                        void* y, int M, int N, int K, float eps, int splitk, void* ws,
                        int* counters, hipStream_t stream);
size_t dd_gemv_add_rmsnorm_ws_bytes(int M, int N, int K, int splitk);

/* out[M,I] = bf16(bf16(silu(g)) * u), [g | u] = x . Wgu^T, Wgu = [gate; up] of shape [2I, K].
 * Replaces TritonOps.gate_up_silu (fused.py:1016-1032; kernel fused.py:631-682), reference
 * _TorchOps.gate_up_silu (engine.py:137-138, 144-146). */
int dd_gate_up_silu(const void* x, const void* Wgu, void* out, int M, int I, int K,
                    hipStream_t stream);

/* out[M,I] = bf16(bf16(silu(g)) * u) with gu[M, 2I] = [g | u].
 * Replaces TritonOps.silu_mul (fused.py:900-906; kernel fused.py:175-188). */
int dd_silu_mul(const void* gu, void* out, int M, int I, hipStream_t stream);

/* Decode qkv_post: per-head q/k RMSNorm (qn/kn), RoPE at position pos[b*pos_stride] + s,
 * k and v written to kc/vc[b, h, position], q written as [B, NKV, S, G, HD].
 * qkv: [B*S, (NH + 2*NKV) * HD]; cos/sin: [rope_rows, HD] bf16 tables; HD must be 128.
 * Replaces TritonOps.qkv_post with pos given (fused.py:932-941; kernel fused.py:415-475),
 * reference _TorchOps.qkv_post decode branch (engine.py:166-187). */
int dd_qkv_post_decode(const void* qkv, const void* qn, const void* kn, const void* cos_t,
                       const void* sin_t, int rope_rows, const int64_t* pos, int pos_stride,
                       void* q, void* kc, void* vc, int B, int S, int NH, int NKV, int HD, int cap,
                       float eps, int* err, hipStream_t stream);

/* Split-KV GQA decode attention with log-sum-exp combine.
 * q: [B, NKV, W, G, HD] (dd_qkv_post_decode layout); kc/vc: [B, NKV, cap, HD] (zero-initialised);
 * query row (b, s) sees keys 0 .. pos[b*pos_stride] + s. out: [B*W, NH*HD].
 * chunk: keys per split (multiple of 32; <= 0 picks dd_attn_chunk). ws: dd_attn_ws_bytes bytes;
 * counters: B*NKV ints, zero before the first call (kernels leave them zero).
 * HD must be 128 and W*G <= 32.
 * Replaces TritonOps.attn_decode (fused.py:961-987; kernels fused.py:478-565), reference
 * _TorchOps.attn_decode (engine.py:154-164). */
int dd_attn_decode(const void* q, const void* kc, const void* vc, const int64_t* pos,
                   int pos_stride, void* out, void* ws, int* counters, int B, int W, int NH,
                   int NKV, int HD, int cap, int chunk, hipStream_t stream);
int dd_attn_chunk(int B, int NKV, int cap);
size_t dd_attn_ws_bytes(int B, int W, int NH, int NKV, int HD, int cap, int chunk);

/* dd_attn_decode without workspace arguments: it allocates nothing and takes no caller memory
 * beyond its inputs and output. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under graph capture with a fixed pool, serving loops or harnesses
 * that forbid hipMalloc). The split partials and the combine counters live in a static device
 * array of 24 MiB + 16 KiB per GPU, held until the process ends; the key chunk is always
 * dd_attn_chunk(B, NKV, cap). Shapes whose dd_attn_ws_bytes exceeds 24 MiB, or with
 * B * NKV > 4096, return hipErrorOutOfMemory (2) and launch nothing. The first call on a device
 * looks the array up and clears its counters (a fill kernel on `stream`, then a wait for the
 * stream), so it must not be made under graph capture: there it returns
 * hipErrorStreamCaptureUnsupported and launches nothing; make one call outside capture first.
 * Every call leaves the counters zero. All calls on one GPU share the array: calls that overlap in time on one GPU race. The
 * output equals dd_attn_decode's with the same chunk, bit for bit. */
int dd_attn_decode_noalloc(const void* q, const void* kc, const void* vc, const int64_t* pos,
                           int pos_stride, void* out, int B, int W, int NH, int NKV, int HD,
                           int cap, hipStream_t stream);

/* Prefill qkv_post over a packed ("varlen") batch: prompt b holds packed tokens
 * seq_start[b] .. seq_start[b+1]-1 (seq_start: B+1 ascending device ints, seq_start[B] = T) at
 * positions 0 .. len_b-1. Per-head q/k RMSNorm + RoPE at the token's position; k and v written
 * to kc/vc[b, h, position]; q written token-major [T, NH, HD], or with last_only != 0 only each
 * prompt's last token, at row b of [B, NH, HD]. qkv: [T, (NH + 2*NKV) * HD]; HD must be 128.
 * A token whose position is not below cap and rope_rows (or offsets that do not cover it) is
 * not written and sets bit 1 (value 2) of *err.
 * Replaces TritonOps.qkv_post with pos = None (fused.py:912-931; kernels fused.py:221-298,
 * 347-412), reference _TorchOps.qkv_post prefill branch (engine.py:166-181); the reference takes
 * B prompts of one length S, which is seq_start[b] = b*S. */
int dd_qkv_post_prefill(const void* qkv, const void* qn, const void* kn, const void* cos_t,
                        const void* sin_t, int rope_rows, const int* seq_start, int B, int T,
                        int last_only, void* q_out, void* kc, void* vc, int NH, int NKV, int HD,
                        int cap, float eps, int* err, hipStream_t stream);

/* Causal GQA flash attention for prefill over a packed batch (seq_start as dd_qkv_post_prefill).
 * Token at position p of prompt b attends to kc/vc[b, h/G, 0..p]. q: [T, NH, HD] token-major,
 * out: [T, NH*HD]; with last_only != 0, q and out are [B, NH, HD] / [B, NH*HD] and only each
 * prompt's last token is computed. P is rounded to bf16 before P.V; scale HD^-0.5 in the log2
 * domain. HD must be 128, NH/NKV one of 1, 2, 4, 8, q/kc/vc 16-byte aligned.
 * Replaces TritonOps.attn_prefill (fused.py:943-959; kernel fused.py:301-343), reference
 * _TorchOps.attn_prefill (engine.py:148-152). */
int dd_attn_prefill(const void* q, const void* kc, const void* vc, const int* seq_start, int B,
                    int T, int last_only, void* out, int NH, int NKV, int HD, int cap,
                    hipStream_t stream);

/* Prefill GEMM: y[M,N] = x[M,K] . W[N,K]^T, bf16 in and out, fp32 accumulation, on hipBLASLt.
 * solution >= 0 names the hipBLASLt solution to run (an index from dd_gemm_bf16_solutions,
 * stable for one hipBLASLt build); when it does not support this problem within ws_bytes, or
 * solution < 0, the heuristic's first candidate runs. The choice depends only on the arguments,
 * so the same operands give the same bits in every process. No timing, no device allocation, no
 * host sync (the first call of a shape creates hipBLASLt descriptors on the host); safe under
 * graph capture. ws: at least dd_gemm_ws_bytes() bytes of device memory (hipBLASLt workspace).
 * Replaces the prefill's F.linear of _TorchOps.linear (engine.py:131-132) in Engine._forward
 * over all prompt tokens (engine.py:459-503). */
int dd_gemm_bf16(const void* x, const void* w, void* y, int M, int N, int K, void* ws,
                 size_t ws_bytes, int solution, hipStream_t stream);
/* The solution indices of hipBLASLt's heuristic candidates for the product (up to max of them,
 * in the heuristic's order, those that fit ws_bytes), written to out; returns their number, or
 * -1. For the offline tuning tool that builds the host's solution table (tune_gemm.py). */
int dd_gemm_bf16_solutions(int M, int N, int K, size_t ws_bytes, int* out, int max);
/* 1 when hipBLASLt solution `solution` supports the product within ws_bytes (dd_gemm_bf16 then
 * runs it), else 0. For the tuning tool. */
int dd_gemm_bf16_supported(int M, int N, int K, size_t ws_bytes, int solution);
size_t dd_gemm_ws_bytes(void);

/* Tensorwise fp8 quantisation of a prefill GEMM input: x [n] bf16 (n a multiple of 8, x 16-byte
 * aligned, out 8-byte aligned); amax = max(max |x|, 1e-6); *scale = amax / 448 (fp32, device);
 * out[i] = float8_e4m3fn(x[i] * (448 / amax)) (OCP e4m3, round to nearest even). ws:
 * dd_fp8_quant_ws_bytes(n) bytes. The fp8 GEMM itself is a plain library GEMM (hipBLASLt).
 * Replaces quant_fp8_tensorwise (fused.py:130-149) of the reference's fp8 prefill GEMMs
 * (engine.py:451-457). */
int dd_fp8_quant(const void* x, size_t n, void* out, float* scale, void* ws, hipStream_t stream);
size_t dd_fp8_quant_ws_bytes(size_t n);

/* h[m] = embed[tok[m]]; y = rmsnorm(h) * w. embed: [V, N].
 * Replaces the embedding gather + first ops.rms of Engine._forward (engine.py:467-468). */
int dd_embed_rmsnorm(const int64_t* tok, const void* embed, int V, const void* w, void* h,
                     void* y, int M, int N, float eps, int* err, hipStream_t stream);

/* tok[m] = argmax(logits[m]) (first index on ties, NaN largest); then pos[i] += 1 for
 * i < npos when pos is not NULL. ws: dd_argmax_ws_bytes; counters: M zeroed ints.
 * Replaces logits.argmax(-1) and st.pos.add_(1) (engine.py:503, 538-540). */
int dd_argmax(const void* logits, int M, int V, int64_t* tok, int64_t* pos, int npos, void* ws,
              int* counters, hipStream_t stream);
size_t dd_argmax_ws_bytes(int M, int V);

/* ---- whole decode step in one persistent launch ------------------------------------------
 * One launch runs Engine._decode_body for M <= 16 rows, one token each: embedding, every layer
 * (QKV + q/k RMSNorm + RoPE + K/V write, attention, O + residual, gate/up + SiLU, down +
 * residual), final RMSNorm, lm_head, argmax, pos += 1. Replaces the body of
 * Engine._forward(pos=...) + _decode_body (engine.py:459-503, 538-540) that the reference
 * captures into one CUDA graph (engine.py:380-396) and replays per token (engine.py:722).
 *
 * The launch has dd_step_grid() workgroups that must all be resident at once (one per CU, the
 * device to itself); they meet at grid barriers between phases, each wait bounded by a 200 ms
 * timeout that sets err flag 4 instead of hanging.
 *
 * Weights are streamed from a tiled copy made once per matrix by dd_tile_weight (the natural
 * row-major matrices stay the interface). matrix: 0 wqkv (aux = NKV; rows taken head-grouped:
 * per kv head h its NH / NKV q heads' rows, then k row block h, then v row block h, of cat(q, k,
 * v)), 1 wo, 2 wgu (aux = I, N = 2 I), 3 wd, 4 lm_head (aux = 0 for 1, 3, 4). The matrix is split
 * into units (rows; wgu: features, unit u = gate row u and up row I + u) over the
 * dd_step_grid() workgroups, workgroup c taking units
 * [floor(n c / G), floor(n (c + 1) / G)); a workgroup's units are stored in order from byte
 * u0 * rows_per_unit * K * 2 on, in chunks of up to 32 / 16 / 40 / 16 / 128 units (per matrix as
 * listed); a chunk of R weight rows (wgu: its gate rows, then its up rows) is k-step-major: the
 * 32 columns s*32 .. +32 of chunk row j at chunk byte (s * R + j) * 64. K must be a multiple of
 * 256. dst holds dd_tiled_bytes(N, K); the layout depends on the device's workgroup count. */
int dd_step_grid(void);
/* 1 when dd_decode_step takes this model geometry for B sequences of W tokens on the current
 * device (head_dim 128; hidden, heads * 128 and intermediate multiples of 256; hidden <= 4096
 * and <= 16 * dd_step_grid(); B <= 16; W = 1, or W <= 5 with B * W <= 80 and W * NH / NKV
 * <= 32), else 0. */
int dd_step_supported(int L, int H, int NH, int NKV, int I, int V, int B, int W);
int dd_step_counters(void);
/* Allocates dd_step_counters() zeroed ints for dd_decode_step in uncached device memory (the
 * barrier and hand-off atomics and polls are then served by memory directly, not through the
 * per-XCD L2s) and stores the device pointer in *out. The memory is never freed (uncached memory
 * must stay mapped for the life of the process once a kernel has read it). No counterpart in the
 * reference: the caller-owned counters of the persistent step. */
int dd_step_counters_alloc(void** out);
/* Diagnostics: synchronous copy of the dd_step_counters() ints at `counters` to `host`. */
int dd_step_counters_read(const void* counters, int* host);
/* Diagnostics and tests: synchronous copy of dd_step_counters() ints from `host` to
 * `counters` (waits for the device first). No counterpart in the reference. */
int dd_step_counters_write(void* counters, const int* host);
/* Zeroes every counter (waits for the device first; synchronous; not under graph capture).
 * Needed after a launch that set error flag 4 (a grid barrier timed out): its workgroups stopped
 * waiting, so hand-off counters their last arrivers would have reset may be left nonzero. No
 * counterpart in the reference: recovery of the persistent step's caller-owned counters. */
int dd_step_counters_clear(void* counters);
size_t dd_step_ws_bytes(int L, int NH, int NKV, int W);
size_t dd_tiled_bytes(int N, int K);
int dd_tile_weight(const void* src, void* dst, int N, int K, int matrix, int aux,
                   hipStream_t stream);

/* One decode step (W = 1) or one verify-shaped step (W > 1) of B sequences in one launch.
 * Replaces Engine._decode_body (engine.py:538-540) over _forward (engine.py:459-503) for W = 1,
 * and the multi-query forward of _spec_body (engine.py:542-547; fused.py:438-441, 492-503) for
 * W > 1: row m = b W + s is token s of sequence b, at position pos[b] + s, attending keys
 * 0 .. pos[b] + s of its sequence's cache (causal within the W rows); K/V are written at
 * pos[b] .. pos[b] + W - 1.
 * layer_table: [L][16] int64 device pointers per layer: 0 wqkv (tiled), 1 wo (tiled),
 * 2 wgu (tiled), 3 wd (tiled), 4 input_layernorm, 5 post_attention_layernorm, 6 q_norm,
 * 7 k_norm, 8 K cache, 9 V cache ([B, NKV, cap, 128] each); 10..15 unused.
 * tok: [B W] int64 tokens in; out_tok: [B W] the argmax of every row's logits (first index on
 * ties; may be tok itself); pos: [B] int64 positions, advanced by one when W = 1 (a decode
 * step), left as they are when W > 1.
 * Activation buffers (bf16, M = B W rows), written once per launch (one slot per producing
 * phase, so they are read with plain cached loads): h [2L+1] slots of M x H (slot 0 embedding,
 * 2l+1 after layer l's O projection, 2l+2 after its down projection), qkv [L, M, (NH + 2 NKV) *
 * 128] (raw q|k|v projection, row-major, head-grouped: [NKV][NH / NKV + 2][128] per row, a kv
 * head's q heads then its k and v), attn [L] slots of M x NH*128, mbuf [L] slots of M x I; the
 * h, attn and mbuf slots are k-step-major: element (m, k) of a slot at ((k / 32) * M + m) * 32 +
 * k % 32. logits [M, V] (row-major) hold the step's lm_head output afterwards.
 * ws: dd_step_ws_bytes(L, NH, NKV, W); counters: dd_step_counters() zeroed ints.
 * phase_begin/phase_end select a sub-range of the 2 + 5L phases (0 embedding, 1 + 5l + {0 QKV,
 * 1 attention, 2 O, 3 gate/up, 4 down}, 1 + 5L lm_head/argmax); a full step is 0 .. 2 + 5L. */
int dd_decode_step(const int64_t* layer_table, int L, const void* embed, const void* lm_tiled,
                   const void* final_norm, const void* cos_t, const void* sin_t, int rope_rows,
                   const int64_t* tok, int64_t* out_tok, int64_t* pos, void* h, void* qkv,
                   void* attn, void* mbuf, void* logits, void* ws, int* counters, int* err, int B,
                   int W, int H, int NH, int NKV, int I, int V, int cap, float eps,
                   int phase_begin, int phase_end, hipStream_t stream);

/* In-graph speculative decoding around the verify-shaped step (W > 1), with exact greedy
 * acceptance. Replaces the gpu-mode speculation of the reference: the table drafter and
 * acceptance of _gspec_body (engine.py:889-943) and the table seeding of _generate_gspec
 * (engine.py:952-975), with the margin acceptance (engine.py:923-929) left out: a draft is kept
 * only when it equals the model's argmax. T: [B, V] int32 token-recycling table (T[b, v]: the
 * model's latest prediction after token v in sequence b).
 * dd_spec_seed: T must be zero; T[b, ids[i]] = ids[i+1] over prompt b (packed ids, seq_start as
 *   dd_qkv_post_prefill; a later occurrence wins), then T[b, last prompt id] = first[b].
 * dd_spec_draft: rows[b, 0] = tok[b], rows[b, j] = T[b, rows[b, j-1]] (rows: [B, W], the verify
 *   step's tok); pos[b] = gpos[b] (the verify step's pos).
 * dd_spec_accept: out = the verify step's out_tok [B, W]; acc = longest prefix with
 *   rows[b, j+1] == out[b, j]; T[b, rows[b, j]] = out[b, j] for j = 0 .. W-1 in order;
 *   tok[b] = out[b, acc]; gpos[b] = min(gpos[b] + acc + 1, limit[b]); rec (B W + B + 1 int64) =
 *   out, then acc, then the step's error word *err.
 * Ids outside [0, V) are never used as table indices (bit 0 of *err is set for a bad tok/ids). */
int dd_spec_seed(void* T, int V, const int64_t* ids, const int* seq_start, int B,
                 const int64_t* first, int* err, hipStream_t stream);
int dd_spec_draft(const void* T, int V, const int64_t* tok, const int64_t* gpos, int B, int W,
                  int64_t* rows, int64_t* pos, int* err, hipStream_t stream);
int dd_spec_accept(const int64_t* rows, const int64_t* out, void* T, int V, int B, int W,
                   int64_t* tok, int64_t* gpos, const int64_t* limit, int64_t* rec,
                   const int* err, hipStream_t stream);

/* Measurement helper, no counterpart in the reference: streams `bytes` from p (16-byte words,
 * nontemporal loads) with the given launch shape; used to measure the achievable HBM read
 * bandwidth that decode-step throughput is reported against. */
int dd_stream_read(const void* p, size_t bytes, int grid, int block, unsigned* sink,
                   hipStream_t stream);

/* Measurement helper, no counterpart in the reference: reads the K and V cache rows 0 ..
 * lens[b] - 1 of every (sequence, kv head) of a [B, NKV, cap, 128] cache, one 32-key block per
 * wave, with the decode attention's access pattern (mode 0) or 1 KB contiguous wave loads (mode
 * 1); used to check that the cache layout costs the attention no bandwidth. */
int dd_kv_read(const void* kc, const void* vc, const int64_t* lens, int B, int NKV, int cap,
               int mode, unsigned* sink, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* DRYFT_DECODE_H */
