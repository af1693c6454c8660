// Shared device helpers for the gfx950 decode-step kernels.
//
// Conventions
//  * bf16 tensors are passed as raw 16-bit patterns (uint16_t); arithmetic is fp32.
//  * fp32 -> bf16 conversion is round-to-nearest-even (the rounding torch and the reference's
//    kernels use at every bf16 cast point).
//  * wave64 everywhere; MFMA tiles are v_mfma_f32_16x16x32_bf16 with the gfx950 operand layout
//      A (16x32): lane l holds A[l%16][(l/16)*8 + i], i = 0..7
//      B (32x16): lane l holds B[(l/16)*8 + i][l%16]
//      D (16x16): lane l holds D[(l/16)*4 + i][l%16], i = 0..3
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dd {

typedef uint16_t bf16;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned u32x2;

__device__ __forceinline__ float bf2f(bf16 v) { return __uint_as_float(((unsigned)v) << 16); }

// Round-to-nearest-even fp32 -> bf16; NaN stays NaN (quietened). gfx950 converts in hardware
// (v_cvt_pk_bf16_f32), two values per instruction when they are packed together.
__device__ __forceinline__ bf16 f2bf(float f) { return __builtin_bit_cast(bf16, (__bf16)f); }

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
// two fp32 -> packed bf16 pair (lo in bits 0..15)
__device__ __forceinline__ unsigned pk_bf16(float lo, float hi) {
  return __builtin_bit_cast(unsigned, bf16x2_t{(__bf16)lo, (__bf16)hi});
}

// Round an fp32 value to the nearest bf16 value, returned as fp32.
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// low / high bf16 of a packed 32-bit word
__device__ __forceinline__ float lo_bf(unsigned w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(unsigned w) { return __uint_as_float(w & 0xffff0000u); }

__device__ __forceinline__ bf16x8_t as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8_t, v); }

__device__ __forceinline__ f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a), as_bf16x8(b), c, 0, 0, 0);
}

// Global-memory pointers. Device pointers read from memory (layer tables) have no address space
// the compiler can infer; without one it emits flat loads, which also count in lgkmcnt, so every
// LDS wait would wait for the whole weight stream. These casts keep loads global (vmcnt only).
typedef __attribute__((address_space(1))) const u32x4 gu32x4;

// 16-byte global load; the pointer must be 16-byte aligned.
__device__ __forceinline__ u32x4 ld16(const void* p) { return *(gu32x4*)p; }
// 16-byte global load that streams past the caches (weights are read once per step).
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load((gu32x4*)p);
}

// Wave-wide reductions (64 lanes). xor-shuffles give every lane the full result.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Sum over a workgroup of NW waves; deterministic order (wave partials added in wave order).
// `red` must hold at least NW floats of shared memory. Every thread gets the result.
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int i = 0; i < NW; ++i) t += red[i];
  __syncthreads();
  return t;
}

// 1/sqrt with IEEE sqrt and IEEE divide (torch.rsqrt on the CPU is 1/sqrt in fp32).
__device__ __forceinline__ float rsqrt_ieee(float x) { return 1.0f / __builtin_sqrtf(x); }

// 2^x by the hardware's v_exp_f32 alone. The library exp2f is the same instruction for
// x >= -126 and rescales smaller arguments so that results below 2^-126 come out as denormals
// instead of zero (5 VALU instructions per call instead of 1). The softmax weights it computes
// are exp2(s - max) of a row, so the only values that differ are weights under 2^-126 (1e-38)
// next to a weight of 1.
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// ---- cross-workgroup hand-off without cache-wide fences ---------------------------------------
// The L2 is per XCD and not coherent across XCDs. A device-scope fence writes back / invalidates
// the whole L2 (measured: a fence-based grid barrier costs 16-45 us on MI355X), so data handed
// from one workgroup to another within a launch goes through sc1 accesses instead, which are
// served at the device coherence point rather than from a (possibly stale) L2 line:
//   producer: stc_*() its data; arrive_last() (waits for its stores, then bumps a counter);
//   consumer: the workgroup that completes the count ldc_*()s the data.
// Buffer (not flat) accesses are used so the compiler can keep many sc1 loads in flight (it
// serialises atomic loads), and a buffer's byte range is checked by the hardware: an access
// past `nbytes` reads 0 / writes nothing instead of faulting.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr int CP_SC1 = 16;  // buffer cache-policy bit sc1 (gfx94x/gfx950)

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, unsigned nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)nbytes,
                                           0x00020000);
}
__device__ __forceinline__ float ldc_f32(rsrc_t r, unsigned off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CP_SC1));
}
__device__ __forceinline__ unsigned ldc_u32(rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CP_SC1);
}
__device__ __forceinline__ u32x4 ldc_b128(rsrc_t r, unsigned off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP_SC1);
}
__device__ __forceinline__ void stc_f32(rsrc_t r, unsigned off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, CP_SC1);
}
__device__ __forceinline__ void stc_b128(rsrc_t r, unsigned off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, CP_SC1);
}
__device__ __forceinline__ void stc_u32(rsrc_t r, unsigned off, unsigned v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, CP_SC1);
}
__device__ __forceinline__ void stc_b16(rsrc_t r, unsigned off, unsigned short v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, CP_SC1);
}

// Every thread of the workgroup calls this after its stc_* stores. Returns true (in every
// thread) for the workgroup whose arrival completes `expected` arrivals on `counter`; that
// workgroup resets the counter to 0 for the next use. `sflag` is a shared int.
__device__ __forceinline__ bool arrive_last(int* counter, int expected, int* sflag) {
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = old == expected - 1;
    if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *sflag = last;
  }
  __syncthreads();
  return *sflag != 0;
}

}  // namespace dd
