// Kernels that measure what one MI355X allows a layer, against which the layer kernels are judged: how fast HBM
// streams a large buffer, how long one launch takes to read a layer's worth of bytes once, and what an empty launch
// costs in a graph. No reference counterpart: they are measurement, not part of the layer.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/drama3_moe.h"

namespace d3 {
int fail(const std::string& msg);
int hip_fail(hipError_t err, const char* what);

// Every thread reads 16-byte words i, i + stride, ... of src (stride = all threads of the grid), four loads in
// flight per round, and folds them with xor. The fold is stored only when it equals a value no input makes likely,
// so the loads cannot be dropped and the kernel writes nothing in practice. Only in-bounds words are read: the
// unrolled rounds stop while four whole strides remain, the tail loop takes the rest.
__global__ void __launch_bounds__(256) stream_read_kernel(const uint4* __restrict__ src, int64_t n16, uint32_t* sink) {
  const int64_t stride = (int64_t)gridDim.x * 256;
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= a.x ^ a.y ^ a.z ^ a.w ^ b.x ^ b.y ^ b.z ^ b.w ^ c.x ^ c.y ^ c.z ^ c.w ^ d.x ^ d.y ^ d.z ^ d.w;
  }
  for (; i < n16; i += stride) {
    const uint4 a = src[i];
    acc ^= a.x ^ a.y ^ a.z ^ a.w;
  }
  if (acc == 0x9E3779B9u) sink[0] = acc;
}

__global__ void __launch_bounds__(256) empty_kernel() {}

}  // namespace d3

extern "C" {

int d3_stream_read(const void* src, int64_t bytes, uint32_t* sink, int32_t grid, void* stream) {
  using namespace d3;
  if (!src || !sink) return fail("d3_stream_read: null pointer");
  if (bytes < 16 || bytes % 16) return fail("d3_stream_read: bytes must be a positive multiple of 16");
  if (grid < 1 || grid > (1 << 20)) return fail("d3_stream_read: grid must be 1 .. 2^20 workgroups");
  hipLaunchKernelGGL(stream_read_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, (const uint4*)src, bytes / 16,
                     sink);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_fail(e, "d3_stream_read launch");
}

int d3_empty_launch(int32_t grid, void* stream) {
  using namespace d3;
  if (grid < 1 || grid > (1 << 20)) return fail("d3_empty_launch: grid must be 1 .. 2^20 workgroups");
  hipLaunchKernelGGL(empty_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_fail(e, "d3_empty_launch launch");
}

}  // extern "C"
