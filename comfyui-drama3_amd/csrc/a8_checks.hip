// The fused layer's inner operations on their own, for exact checks: a bank's rows against given activations, one
// 128-column group at a time (the int32 sums the MFMA produces), and the unpacked W4 / W6 codes. They run the same
// load_step / operand_i8 / step_* functions as moe_a8_kernel.
#include "formats.hpp"
#include "../../include/drama3_moe.h"

#include <string>

namespace d3 {
int fail(const std::string& msg);
int hip_fail(hipError_t err, const char* what);

// One wave per 16 rows. act [C, K] in column order is staged into LDS in the format's storage order.
template <int F>
__global__ void __launch_bounds__(64) gemv_groups_kernel(const uint8_t* rows, int K, const uint8_t* act, int C, void* acc) {
  extern __shared__ __attribute__((aligned(16))) uint8_t xs[];
  const int lane = threadIdx.x, q = lane >> 4, col = lane & 15;
  for (int i = lane; i < C * K; i += 64) {
    const int c = i / K, k = i % K;
    const int pos = F == FMT_W4 ? (k & ~7) + act_pos_w4(k & 7) : k;
    xs[c * K + pos] = act[i];
  }
  __syncthreads();
  const int rb = row_bytes(F, K), groups = K / 128;
  const int row = blockIdx.x * 16 + (lane & 15);
  const uint8_t* wp = rows + (size_t)row * rb;
  for (int s = 0; s < groups; s++) {
    Raw<F> raw;
    load_step<F>(raw, wp, s, q);
    i32x4 xlo = {0, 0, 0, 0}, xhi = {0, 0, 0, 0};
    if (col < C) {
      xlo = *(const i32x4*)(xs + col * K + 128 * s + 32 * q);
      xhi = *(const i32x4*)(xs + col * K + 128 * s + 32 * q + 16);
    }
    if constexpr (F == FMT_F8) {
      const i32x8 fa = f8_operand(raw), fb = f8_operand(xlo, xhi);
      const f32x4 f = mfma_f8_chain<1>(&fa, &fb);
      if (col < C)
        for (int i = 0; i < 4; i++)
          ((float*)acc)[((size_t)(blockIdx.x * 16 + 4 * q + i) * groups + s) * C + col] = f[i];
    } else {
      const i32x4 g = step_i8<F>(raw, xlo, xhi, i32x4{0, 0, 0, 0});
      if (col < C)
        for (int i = 0; i < 4; i++)
          ((int*)acc)[((size_t)(blockIdx.x * 16 + 4 * q + i) * groups + s) * C + col] = g[i] >> unpack_shift(F);
    }
  }
}

// One thread per (row, step, lane group): the 32 codes it feeds the MFMA, back in column order.
template <int F>
__global__ void unpack_kernel(const uint8_t* rows, int R, int K, int8_t* codes) {
  const int groups = K / 128;
  const size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
  if (i >= (size_t)R * groups * 4) return;
  const int q = (int)(i & 3), s = (int)((i >> 2) % groups);
  const size_t row = (i >> 2) / groups;
  Raw<F> raw;
  load_step<F>(raw, rows + row * row_bytes(F, K), s, q);
  i32x4 lo, hi;
  operand_i8<F>(raw, lo, hi);
  const int8_t* b[2] = {(const int8_t*)&lo, (const int8_t*)&hi};
  for (int h = 0; h < 2; h++)
    for (int j = 0; j < 16; j++) {
      const int within = j & 7, block = j >> 3;
      const int c = F == FMT_W4 ? 8 * block + (within < 4 ? 2 * within : 2 * (within - 4) + 1) : j;
      codes[row * K + 128 * s + 32 * q + 16 * h + c] = (int8_t)(b[h][j] >> unpack_shift(F));
    }
}

}  // namespace d3

namespace d3 {
// float -> e4m3fn codes, pairs per thread, by the hardware converter (1) or the format-definition one (0)
// (both halves of the packed converter: a pair into the low half-word, the next pair into the high one)
__global__ void __launch_bounds__(256) cvt_fp8_kernel(const float* in, int quads, uint8_t* out, int hardware) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= quads) return;
  const float a = in[4 * i], b = in[4 * i + 1], c = in[4 * i + 2], d = in[4 * i + 3];
  const uint32_t r = hardware ? f32x4_to_fp8x4(a, b, c, d)
                              : (f32_to_fp8(a) | (f32_to_fp8(b) << 8) | (f32_to_fp8(c) << 16) | (f32_to_fp8(d) << 24));
  for (int j = 0; j < 4; j++) out[4 * i + j] = (uint8_t)(r >> (8 * j));
}
}  // namespace d3

extern "C" {

int d3_gemv_a8_groups(int32_t format, const void* rows, int32_t R, int32_t K, const void* act, int32_t C, void* acc,
                      void* stream) {
  using namespace d3;
  if (!rows || !act || !acc) return fail("d3_gemv_a8_groups: null pointer");
  if (R < 16 || R % 16 || K < 128 || K % 128 || K > 4096 || C < 1 || C > 16)
    return fail("d3_gemv_a8_groups: R % 16, K % 128 (<= 4096), C 1..16");
  const size_t lds = (size_t)C * K;
  hipStream_t s = (hipStream_t)stream;
  const uint8_t* r = (const uint8_t*)rows;
  const uint8_t* x = (const uint8_t*)act;
  switch (format) {
    case FMT_I8: hipLaunchKernelGGL(gemv_groups_kernel<FMT_I8>, dim3(R / 16), dim3(64), lds, s, r, K, x, C, acc); break;
    case FMT_W4: hipLaunchKernelGGL(gemv_groups_kernel<FMT_W4>, dim3(R / 16), dim3(64), lds, s, r, K, x, C, acc); break;
    case FMT_W6: hipLaunchKernelGGL(gemv_groups_kernel<FMT_W6>, dim3(R / 16), dim3(64), lds, s, r, K, x, C, acc); break;
    case FMT_F8: hipLaunchKernelGGL(gemv_groups_kernel<FMT_F8>, dim3(R / 16), dim3(64), lds, s, r, K, x, C, acc); break;
    default: return fail("d3_gemv_a8_groups: unknown format");
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_fail(e, "d3_gemv_a8_groups launch");
}

int d3_unpack_rows(int32_t format, const void* rows, int32_t R, int32_t K, void* codes, void* stream) {
  using namespace d3;
  if (!rows || !codes) return fail("d3_unpack_rows: null pointer");
  if (R < 1 || K < 128 || K % 128) return fail("d3_unpack_rows: K % 128");
  const size_t threads = (size_t)R * (K / 128) * 4;
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  switch (format) {
    case FMT_W4: hipLaunchKernelGGL(unpack_kernel<FMT_W4>, grid, dim3(256), 0, s, (const uint8_t*)rows, R, K, (int8_t*)codes); break;
    case FMT_W6: hipLaunchKernelGGL(unpack_kernel<FMT_W6>, grid, dim3(256), 0, s, (const uint8_t*)rows, R, K, (int8_t*)codes); break;
    default: return fail("d3_unpack_rows: format must be W4 or W6");
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_fail(e, "d3_unpack_rows launch");
}

int d3_cvt_fp8(const float* in, int32_t n, void* out, int32_t hardware, void* stream) {
  using namespace d3;
  if (!in || !out) return fail("d3_cvt_fp8: null pointer");
  if (n < 4 || n % 4) return fail("d3_cvt_fp8: n a positive multiple of 4");
  hipLaunchKernelGGL(cvt_fp8_kernel, dim3((n / 4 + 255) / 256), dim3(256), 0, (hipStream_t)stream, in, n / 4,
                     (uint8_t*)out, hardware);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_fail(e, "d3_cvt_fp8 launch");
}

}  // extern "C"
