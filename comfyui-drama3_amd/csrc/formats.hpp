// Weight formats of the A8 expert banks and their MFMA step.
//
// A bank is [E * N, row_bytes] (expert e's N rows in turn), one row per output channel, packed along K:
//   I8  int8, one bf16 scale per row                                       row_bytes = K
//   W4  signed int4, two per byte (byte b: column 2b in the low nibble, 2b + 1 in the high one), one bf16 scale
//       per 128-column group                                               row_bytes = K / 2
//   W6  signed 6-bit, 16 columns per 12-byte unit (below), one bf16 scale per 128-column group
//                                                                          row_bytes = 3K / 4
//   F8  float8 e4m3fn, one bf16 scale per row                              row_bytes = K
//
// W6 unit (columns c0..c15 of codes q_j, 6-bit two's complement): byte i (0..11) holds q_i in its low 6 bits; its top
// two bits hold bits 2*(i >> 2) .. 2*(i >> 2) + 1 of q_{12 + (i & 3)}. So q_12..q_15 are spread over bytes 0-3 (bits
// 0-1), 4-7 (bits 2-3) and 8-11 (bits 4-5), and a unit unpacks with masks and three shifts.
//
// A "step" is 128 columns. In a step the 16 rows of an MFMA tile are split over the wave's lanes: lane l reads row
// l % 16, and its lane group q = l / 16 covers columns [32q, 32q + 32) of the step. The int8 MFMA consumes 16 columns
// per lane per instruction, so a step is two i32_16x16x64_i8 (I8, W4, W6) or one f32_16x16x128_f8f6f4 (F8). The
// activation operand uses the same lane -> column map, which is all the MFMA needs: it pairs A and B by lane group and
// byte, whatever the hardware's k order is.
//
// Unpacking keeps the sign without a correction term: a 4-bit code shifted to the top of its byte is 16q as an int8,
// a 6-bit one shifted by 2 is 4q, so the MFMA's int32 sum is exactly 16 (or 4) times the true one.
#pragma once
#include "common.hpp"

namespace d3 {

enum Format : int { FMT_I8 = 0, FMT_W4 = 1, FMT_W6 = 2, FMT_F8 = 3 };

__host__ __device__ constexpr int row_bytes(int fmt, int K) {
  return fmt == FMT_W4 ? K / 2 : fmt == FMT_W6 ? K * 3 / 4 : K;
}
// bytes of one row in one 128-column step, and one lane's share of them
__host__ __device__ constexpr int step_row_bytes(int fmt) { return row_bytes(fmt, 128); }
__host__ __device__ constexpr int lane_step_bytes(int fmt) { return step_row_bytes(fmt) / 4; }
__host__ __device__ constexpr bool group_scaled(int fmt) { return fmt == FMT_W4 || fmt == FMT_W6; }
// log2 of the factor the unpacked int8 operand carries (16q or 4q)
__host__ __device__ constexpr int unpack_shift(int fmt) { return fmt == FMT_W4 ? 4 : fmt == FMT_W6 ? 2 : 0; }

template <int F> struct Raw { uint32_t d[lane_step_bytes(F) / 4]; };

// one lane's bytes of `step` of a row
template <int F> D3_INLINE void load_step(Raw<F>& r, const uint8_t* row, int step, int q) {
  const uint8_t* p = row + step * step_row_bytes(F) + q * lane_step_bytes(F);
  if constexpr (F == FMT_W6) {
    // 24 bytes at 8-byte alignment
    const i32x2* v = (const i32x2*)p;
    i32x2 a = v[0], b = v[1], c = v[2];
    r.d[0] = a.x; r.d[1] = a.y; r.d[2] = b.x; r.d[3] = b.y; r.d[4] = c.x; r.d[5] = c.y;
  } else {
    const i32x4* v = (const i32x4*)p;
#pragma unroll
    for (int i = 0; i < lane_step_bytes(F) / 16; i++) {
      i32x4 x = v[i];
      r.d[4 * i] = x.x; r.d[4 * i + 1] = x.y; r.d[4 * i + 2] = x.z; r.d[4 * i + 3] = x.w;
    }
  }
}

// W4: 8 nibbles of a word -> [16 c0, 16 c2, 16 c4, 16 c6] and [16 c1, 16 c3, 16 c5, 16 c7] as int8 bytes
D3_INLINE void unpack_w4_word(uint32_t d, uint32_t& even, uint32_t& odd) {
  even = (d << 4) & 0xF0F0F0F0u;
  odd = d & 0xF0F0F0F0u;
}
// W6: one 12-byte unit (3 words) -> 16 bytes 4 q_0 .. 4 q_15 in column order
D3_INLINE i32x4 unpack_w6_unit(uint32_t d0, uint32_t d1, uint32_t d2) {
  i32x4 o;
  o.x = (int)((d0 << 2) & 0xFCFCFCFCu);
  o.y = (int)((d1 << 2) & 0xFCFCFCFCu);
  o.z = (int)((d2 << 2) & 0xFCFCFCFCu);
  o.w = (int)(((d0 >> 4) & 0x0C0C0C0Cu) | ((d1 >> 2) & 0x30303030u) | (d2 & 0xC0C0C0C0u));
  return o;
}

// The int8 operand halves (16 columns each) of a step: columns [32q, 32q+16) and [32q+16, 32q+32). W4 halves hold
// each 8 columns as [0,2,4,6,1,3,5,7], so the activations are stored in that order for W4 (see act_perm_w4).
template <int F> D3_INLINE void operand_i8(const Raw<F>& r, i32x4& lo, i32x4& hi) {
  if constexpr (F == FMT_I8) {
    lo = i32x4{(int)r.d[0], (int)r.d[1], (int)r.d[2], (int)r.d[3]};
    hi = i32x4{(int)r.d[4], (int)r.d[5], (int)r.d[6], (int)r.d[7]};
  } else if constexpr (F == FMT_W4) {
    uint32_t e0, o0, e1, o1, e2, o2, e3, o3;
    unpack_w4_word(r.d[0], e0, o0);
    unpack_w4_word(r.d[1], e1, o1);
    unpack_w4_word(r.d[2], e2, o2);
    unpack_w4_word(r.d[3], e3, o3);
    lo = i32x4{(int)e0, (int)o0, (int)e1, (int)o1};
    hi = i32x4{(int)e2, (int)o2, (int)e3, (int)o3};
  } else {
    lo = unpack_w6_unit(r.d[0], r.d[1], r.d[2]);
    hi = unpack_w6_unit(r.d[3], r.d[4], r.d[5]);
  }
}

// A step against 32 activation bytes (int8, or e4m3 for F8) of this lane's column.
//   I8: acc (int32) += the step's dot products.
//   W4/W6: returns the step's int32 dot products scaled by 16 / 4 (the caller applies the group scale).
D3_INLINE i32x4 mfma_i8(i32x4 a, i32x4 b, i32x4 c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }

template <int F> D3_INLINE i32x4 step_i8(const Raw<F>& r, const i32x4& xlo, const i32x4& xhi, i32x4 acc) {
  i32x4 lo, hi;
  operand_i8<F>(r, lo, hi);
  acc = mfma_i8(lo, xlo, acc);
  return mfma_i8(hi, xhi, acc);
}
// F8: e4m3 x e4m3 -> float32 on the f8f6f4 MFMA (16 x 16 x 128 per step), acc = sum over steps k of A[k] . B[k] (A: 8
// registers of a weight row's 32 columns per lane group, B: the activations', lane layout as the int8 MFMA). The whole
// chain is one asm statement: every A and B operand keeps its registers until the chain has finished and the
// accumulator is both source and destination. With the compiler's own register choices for this instruction (an
// accumulator overlapping an operand or another accumulator, operand registers rewritten right after issue while the
// 16-pass instruction still reads its 8-register operands) layer outputs came out wrong on MI355X, depending on the
// surrounding code. The wait states before (operands written just before) and after (the result read just after)
// cover the instruction's own hazards, which the compiler does not see inside the statement.
template <int N> D3_INLINE f32x4 mfma_f8_chain(const i32x8* A, const i32x8* B);
template <> D3_INLINE f32x4 mfma_f8_chain<1>(const i32x8* A, const i32x8* B) {
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int one = 127;  // E8M0 block scale 2^0: a plain e4m3 x e4m3 product
  asm volatile(
      "s_nop 4\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %2, %0, %3, %3 op_sel_hi:[0,0,0]\n"
      "s_nop 7\n s_nop 7\n s_nop 7\n"
      : "+v"(acc)
      : "v"(A[0]), "v"(B[0]), "v"(one));
  return acc;
}
template <> D3_INLINE f32x4 mfma_f8_chain<2>(const i32x8* A, const i32x8* B) {
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int one = 127;  // E8M0 block scale 2^0: a plain e4m3 x e4m3 product
  asm volatile(
      "s_nop 4\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %3, %0, %5, %5 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %2, %4, %0, %5, %5 op_sel_hi:[0,0,0]\n"
      "s_nop 7\n s_nop 7\n s_nop 7\n"
      : "+v"(acc)
      : "v"(A[0]), "v"(A[1]), "v"(B[0]), "v"(B[1]), "v"(one));
  return acc;
}
template <> D3_INLINE f32x4 mfma_f8_chain<3>(const i32x8* A, const i32x8* B) {
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int one = 127;  // E8M0 block scale 2^0: a plain e4m3 x e4m3 product
  asm volatile(
      "s_nop 4\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %4, %0, %7, %7 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %2, %5, %0, %7, %7 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %3, %6, %0, %7, %7 op_sel_hi:[0,0,0]\n"
      "s_nop 7\n s_nop 7\n s_nop 7\n"
      : "+v"(acc)
      : "v"(A[0]), "v"(A[1]), "v"(A[2]), "v"(B[0]), "v"(B[1]), "v"(B[2]), "v"(one));
  return acc;
}
template <> D3_INLINE f32x4 mfma_f8_chain<4>(const i32x8* A, const i32x8* B) {
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int one = 127;  // E8M0 block scale 2^0: a plain e4m3 x e4m3 product
  asm volatile(
      "s_nop 4\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %5, %0, %9, %9 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %2, %6, %0, %9, %9 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %3, %7, %0, %9, %9 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %4, %8, %0, %9, %9 op_sel_hi:[0,0,0]\n"
      "s_nop 7\n s_nop 7\n s_nop 7\n"
      : "+v"(acc)
      : "v"(A[0]), "v"(A[1]), "v"(A[2]), "v"(A[3]), "v"(B[0]), "v"(B[1]), "v"(B[2]), "v"(B[3]), "v"(one));
  return acc;
}
template <> D3_INLINE f32x4 mfma_f8_chain<6>(const i32x8* A, const i32x8* B) {
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const int one = 127;  // E8M0 block scale 2^0: a plain e4m3 x e4m3 product
  asm volatile(
      "s_nop 4\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %1, %7, %0, %13, %13 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %2, %8, %0, %13, %13 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %3, %9, %0, %13, %13 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %4, %10, %0, %13, %13 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %5, %11, %0, %13, %13 op_sel_hi:[0,0,0]\n"
      "v_mfma_scale_f32_16x16x128_f8f6f4 %0, %6, %12, %0, %13, %13 op_sel_hi:[0,0,0]\n"
      "s_nop 7\n s_nop 7\n s_nop 7\n"
      : "+v"(acc)
      : "v"(A[0]), "v"(A[1]), "v"(A[2]), "v"(A[3]), "v"(A[4]), "v"(A[5]), "v"(B[0]), "v"(B[1]), "v"(B[2]), "v"(B[3]), "v"(B[4]), "v"(B[5]), "v"(one));
  return acc;
}
D3_INLINE i32x8 f8_operand(const Raw<FMT_F8>& r) {
  return i32x8{(int)r.d[0], (int)r.d[1], (int)r.d[2], (int)r.d[3], (int)r.d[4], (int)r.d[5], (int)r.d[6], (int)r.d[7]};
}
D3_INLINE i32x8 f8_operand(const i32x4& lo, const i32x4& hi) {
  return i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

// Activation storage order: W4 keeps each 8 columns as [0,2,4,6,1,3,5,7]; the others keep column order. Position of
// column c (within its 8) in storage:
__host__ __device__ constexpr int act_pos_w4(int c) { return (c & 1) ? 4 + (c >> 1) : (c >> 1); }

// Activations are quantized per row: int8 at absmax / 127 (I8, W4, W6) or e4m3 at absmax / 448 (F8).
template <int F> __host__ __device__ constexpr float act_qmax() { return F == FMT_F8 ? 448.0f : 127.0f; }

// quantize 8 activations with `inv`, store them in the format's storage order
template <int F> D3_INLINE void store_act8(uint8_t* dst, const float* v, float inv) {
  if constexpr (F == FMT_F8) {  // |v * inv| <= 448 (inv = 448 / amax): the packed converter, exact on that range
    const uint32_t lo = f32x4_to_fp8x4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
    const uint32_t hi = f32x4_to_fp8x4(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
    *(i32x2*)dst = i32x2{(int)lo, (int)hi};
    return;
  }
  uint32_t b[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    float r = rintf(v[i] * inv);
    r = fminf(fmaxf(r, -127.0f), 127.0f);
    b[i] = (uint32_t)((int)r) & 0xFFu;
  }
  uint32_t lo, hi;
  if constexpr (F == FMT_W4) {
    lo = b[0] | (b[2] << 8) | (b[4] << 16) | (b[6] << 24);
    hi = b[1] | (b[3] << 8) | (b[5] << 16) | (b[7] << 24);
  } else {
    lo = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    hi = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
  }
  *(i32x2*)dst = i32x2{(int)lo, (int)hi};
}

// one activation quantized as store_act8 does it, and the byte offset store_act8 gives column c of a row
template <int F> D3_INLINE uint32_t act8_byte(float v, float inv) {
  if constexpr (F == FMT_F8) return f32x2_to_fp8x2(v * inv, 0.0f) & 0xFFu;
  const float r = fminf(fmaxf(rintf(v * inv), -127.0f), 127.0f);
  return (uint32_t)((int)r) & 0xFFu;
}
template <int F> __host__ __device__ constexpr int act8_pos(int c) {
  return F == FMT_W4 ? (c & ~7) + ((c & 1) ? 4 : 0) + ((c & 7) >> 1) : c;
}

}  // namespace d3
