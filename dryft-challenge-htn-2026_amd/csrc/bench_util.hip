// Measurement helper: a streaming-read kernel that gives the achievable HBM read bandwidth of
// the device (the "measured roofline" the decode step is compared with). Not part of the
// decode path.
#include "common.h"

namespace dd {

// Each thread streams 16-byte words with 4 loads in flight per iteration; the XOR of everything
// read is stored only if it hits an impossible value, so the loads cannot be dropped.
__global__ void __launch_bounds__(512) stream_read_kernel(const u32x4* __restrict__ p, size_t n16,
                                                          unsigned* __restrict__ sink) {
  size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  unsigned acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(p + i);
    const u32x4 b = __builtin_nontemporal_load(p + i + stride);
    const u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(p + i + 3 * stride);
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const u32x4 a = p[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9e3779b9u && sink != nullptr) sink[0] = acc;
}

}  // namespace dd

#include "api.h"

using namespace dd;

DD_API int dd_stream_read(const void* p, size_t bytes, int grid, int block, unsigned* sink,
                          hipStream_t stream) {
  DD_REQUIRE(p && aligned16(p) && bytes >= 16 && grid >= 1 && (block == 256 || block == 512));
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(block), 0, stream, (const u32x4*)p,
                     bytes / 16, sink);
  return launch_status();
}
