// FP8 GEMV with one bf16 scale per output row, on bf16 activations: out[r, n] = bf16( sum_k x[r, k] * wd[n, k] ),
// wd[n, k] = bf16( e4m3(W[n, k]) * s[n] ). This is the reference's CPU path for an FP8 expert weight, dequantize then
// matmul in bf16 (drama3/offload.py:163-167 dequantize_fp8, then nn.functional.linear as offload.py:192-199
// experts_decode and 797-802 FP8Experts.forward run it), with the scale per output row (absmax / 448) instead of per
// 128 x 128 block. Each weight is rounded to bf16 after its scale, as the dequantized matrix holds it; the products
// and sums run in float32.
//
// HBM-bound (one byte per weight). A wave owns a row at a time: lane l reads the row's bytes 8 l + 512 c (one 512-byte
// run per instruction and chunk c), decodes them with the hardware e4m3 converter, scales and rounds them, and
// multiplies them against its slice of x, which it keeps in registers for every row it takes; the wave's sum goes
// through DPP. Rows are dealt to the waves of the grid in turn, so a launch covers any number of rows (stacked experts:
// experts_decode's gate_up is one [k * 2I, H] matrix against one row).
#include "common.hpp"
#include "../../include/drama3_moe.h"

#include <string>

namespace d3 {
int fail(const std::string& msg);
int hip_fail(hipError_t err, const char* what);

// float -> float on the bf16 grid, to nearest, ties to even (the products here are finite: quantized e4m3 codes
// never hold the two NaN codes)
D3_INLINE float round_to_bf16(float v) {
  uint32_t b = __float_as_uint(v);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return __uint_as_float(b & 0xFFFF0000u);
}

template <int KC, int R>  // K = 512 KC columns; R rows of x (1 .. 4)
__global__ void __launch_bounds__(256) gemv_fp8_rows_kernel(const uint16_t* __restrict__ x, const uint8_t* __restrict__ w,
                                                            const uint16_t* __restrict__ scale, uint16_t* __restrict__ out,
                                                            int N) {
  constexpr int K = 512 * KC;
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6), waves = gridDim.x * 4;
  // this lane's 8 KC columns of every row of x (columns 512 c + 8 l .. + 7), as floats
  float xv[R][KC][8];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int c = 0; c < KC; c++) {
      const i32x4 v = *(const i32x4*)(x + (size_t)r * K + 512 * c + 8 * lane);
      const uint32_t u[4] = {(uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        xv[r][c][2 * j] = bf16_to_f32(u[j] & 0xFFFFu);
        xv[r][c][2 * j + 1] = bf16_to_f32(u[j] >> 16);
      }
    }
  for (int n = wave; n < N; n += waves) {
    const uint8_t* row = w + (size_t)n * K;
    i32x2 raw[KC];
#pragma unroll
    for (int c = 0; c < KC; c++) raw[c] = *(const i32x2*)(row + 512 * c + 8 * lane);
    const float s = bf16_to_f32(scale[n]);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.0f;
#pragma unroll
    for (int c = 0; c < KC; c++) {
      const f32x2 a = fp8x2_to_f32<false>((uint32_t)raw[c].x), b = fp8x2_to_f32<true>((uint32_t)raw[c].x);
      const f32x2 d = fp8x2_to_f32<false>((uint32_t)raw[c].y), e = fp8x2_to_f32<true>((uint32_t)raw[c].y);
      const float wd[8] = {round_to_bf16(a.x * s), round_to_bf16(a.y * s), round_to_bf16(b.x * s), round_to_bf16(b.y * s),
                           round_to_bf16(d.x * s), round_to_bf16(d.y * s), round_to_bf16(e.x * s), round_to_bf16(e.y * s)};
#pragma unroll
      for (int r = 0; r < R; r++)
#pragma unroll
        for (int j = 0; j < 8; j++) acc[r] = fmaf(xv[r][c][j], wd[j], acc[r]);
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      const float total = wave_sum_f32(acc[r]);
      if (lane == 0) out[(size_t)r * N + n] = (uint16_t)f32_to_bf16(total);
    }
  }
}

template <int KC>
void launch_rows(dim3 grid, hipStream_t s, const uint16_t* x, int rows, const uint8_t* w, const uint16_t* scale,
                 uint16_t* out, int N) {
  switch (rows) {
    case 1: hipLaunchKernelGGL((gemv_fp8_rows_kernel<KC, 1>), grid, dim3(256), 0, s, x, w, scale, out, N); break;
    case 2: hipLaunchKernelGGL((gemv_fp8_rows_kernel<KC, 2>), grid, dim3(256), 0, s, x, w, scale, out, N); break;
    case 3: hipLaunchKernelGGL((gemv_fp8_rows_kernel<KC, 3>), grid, dim3(256), 0, s, x, w, scale, out, N); break;
    default: hipLaunchKernelGGL((gemv_fp8_rows_kernel<KC, 4>), grid, dim3(256), 0, s, x, w, scale, out, N); break;
  }
}

}  // namespace d3

extern "C" int d3_gemv_fp8_rows(const void* x, int32_t rows, const void* weight, const void* scale, void* out, int32_t N,
                                int32_t K, void* stream) {
  using namespace d3;
  if (!x || !weight || !scale || !out) return fail("d3_gemv_fp8_rows: null pointer");
  if (rows < 1 || rows > 4) return fail("d3_gemv_fp8_rows: rows must be 1..4");
  if (N < 1) return fail("d3_gemv_fp8_rows: N must be positive");
  if (((uintptr_t)x & 15u) || ((uintptr_t)weight & 7u)) return fail("d3_gemv_fp8_rows: x must be 16-byte aligned, weight 8-byte");
  // one row per wave, every wave of the grid resident at once up to about 8 workgroups per CU; more rows loop
  const int waves = N < 8192 ? N : 8192;
  const dim3 grid((waves + 3) / 4);
  const hipStream_t s = (hipStream_t)stream;
  const uint16_t* xb = (const uint16_t*)x;
  const uint8_t* wb = (const uint8_t*)weight;
  const uint16_t* sb = (const uint16_t*)scale;
  uint16_t* ob = (uint16_t*)out;
  switch (K) {
    case 512: launch_rows<1>(grid, s, xb, rows, wb, sb, ob, N); break;
    case 1024: launch_rows<2>(grid, s, xb, rows, wb, sb, ob, N); break;
    case 1536: launch_rows<3>(grid, s, xb, rows, wb, sb, ob, N); break;
    case 2048: launch_rows<4>(grid, s, xb, rows, wb, sb, ob, N); break;
    default: return fail("d3_gemv_fp8_rows: K must be 512, 1024, 1536 or 2048");
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : hip_fail(e, "d3_gemv_fp8_rows launch");
}
