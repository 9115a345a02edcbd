// Kernels of the reference's own expert formats, behind drama3/kernels.py's call surface (kernels.py:590-724):
// routing, the ConvRot rotation, the weighted sum, and the decode GEMVs / prefill grouped products over int8 ConvRot
// banks (per-row float scale), FP8 banks (float scale per 128 x 128 block) and W4A8 / W6A8 code banks (nibble plane,
// 2-bit high plane for 6 bits, e4m3 scale per 16 columns, float scale per row, 16-entry codebook for 4 bits).
// Activations stay float32, as in the reference. The slot-cache semantics of the decode GEMVs are kept: plan[e] =
// (slot, code), code 0 reads the slot, 1 reads the bank (host memory) and fills the slot if it has one, 2 is the CPU's
// (zeros, or, with `late` and took_over set, read from the bank) (kernels.py:274-314).
//
// Design for gfx950, not a translation: a wave holds a row's columns across its 64 lanes (each lane a fixed slice, so
// the activation slice stays in registers across rows), int8 bytes become floats through one unsigned conversion after
// flipping the sign bit (sum u x - 128 sum x), FP8 bytes through the hardware e4m3 converter with the block scale
// folded into the activation slice, and wave sums go through DPP. The rotation runs in registers: H256 is the 4-fold
// Kronecker power of h4, whose row r is +1 except -1 at column 3 - r, so each of the four base-4 digits of the column
// index is one step y = (sum of the 4 values) - 2 * (the value at the mirrored digit), exchanged within a lane, a quad
// (DPP), a row (DPP rotate / mirror) and the wave (shuffles). Many rows (a prompt) run on the matrix cores: int8 and
// the codes on the int8 cores against the rows as three int8 planes with a power-of-two scale (grouped_i8_kernel),
// FP8 on the bf16 cores against exact bf16 planes (grouped_fp8_kernel), each weight read once per 32-row pass.
#include "common.hpp"
#include "../../include/drama3_moe.h"

#include <algorithm>
#include <string>

namespace d3 {
int fail(const std::string& msg);
int hip_fail(hipError_t err, const char* what);

constexpr int RPB = 16;  // output rows per workgroup of the GEMVs (kernels.py:590 ROWS_PER_BLOCK: N % 16 == 0)

template <int CTRL> D3_INLINE float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// ---------------------------------------------------------------------------------------------------------- route
// kernels.py:39-67: the k (<= 32) largest of n (<= 1024) bf16 logits, descending, ties to the lower index; weights
// softmax over those k, rounded to bf16. One wave per row.
template <int KPL>  // logits per lane: n <= 64 * KPL
__global__ void __launch_bounds__(256) route_kernel(const uint16_t* logits, int rows, int n, int k, int64_t* ids,
                                                    float* weights) {
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const uint16_t* lg = logits + (size_t)row * n;
  uint32_t raw[KPL], key[KPL];
#pragma unroll
  for (int j = 0; j < KPL; j++) raw[j] = lg[min(lane + 64 * j, n - 1)];  // branch-free: all loads in flight together
#pragma unroll
  for (int j = 0; j < KPL; j++) {
    const int e = lane + 64 * j;
    key[j] = e < n ? route_key(raw[j], e) : 0u;
  }
  float top[32];
  int id[32];
#pragma unroll
  for (int r = 0; r < 32; r++) {
    top[r] = 0.0f;
    id[r] = 0;
    if (r < k) {
      uint32_t m = key[0];
#pragma unroll
      for (int j = 1; j < KPL; j++) m = max(m, key[j]);
      m = wave_max_u32_v(m);  // on the vector unit: the k rounds form one dependent chain
#pragma unroll
      for (int j = 0; j < KPL; j++) key[j] = key[j] == m ? 0u : key[j];
      id[r] = route_key_index(m);
      top[r] = route_key_value(m);
    }
  }
  float total = 0.0f;
#pragma unroll
  for (int r = 0; r < 32; r++)
    if (r < k) total += expf(top[r] - top[0]);
#pragma unroll
  for (int r = 0; r < 32; r++) {
    if (r < k && lane == r) {
      ids[(size_t)row * k + r] = id[r];
      weights[(size_t)row * k + r] = bf16_round(expf(top[r] - top[0]) / total);
    }
  }
}

// -------------------------------------------------------------------------------------------------- weighted sum
// kernels.py:69-76: out[h] = bf16(sum_e parts[e, h] * w[e]), e in order.
__global__ void __launch_bounds__(256) weighted_sum_kernel(const float* parts, const float* w, int k, int H,
                                                           uint16_t* out) {
  const int h = blockIdx.x * 256 + threadIdx.x;
  if (h >= H) return;
  float acc = 0.0f;
  for (int e = 0; e < k; e++) acc = fmaf(parts[(size_t)e * H + h], w[e], acc);
  out[h] = (uint16_t)f32_to_bf16(acc);
}

// -------------------------------------------------------------------------------------------------------- rotate
// H256 / 16 of one 256-column chunk held by a wave, lane l holding columns 4l .. 4l + 3 (all 64 lanes active).
D3_INLINE void fwht256(float* v) {
  // digit 0: the lane's own four columns
  {
    const float s = (v[0] + v[1]) + (v[2] + v[3]);
    const float y0 = s - 2.0f * v[3], y1 = s - 2.0f * v[2], y2 = s - 2.0f * v[1], y3 = s - 2.0f * v[0];
    v[0] = y0; v[1] = y1; v[2] = y2; v[3] = y3;
  }
#pragma unroll
  for (int j = 0; j < 4; j++) {
    // digit 1: the four lanes of a quad; mirrored digit = lane ^ 3
    float s = v[j] + dpp_f32<0xB1>(v[j]);
    s = s + dpp_f32<0x4E>(s);
    v[j] = s - 2.0f * dpp_f32<0x1B>(v[j]);
    // digit 2: the four quads of a row (rotate by 8 and 4); mirrored digit = lane ^ 12 (row mirror, then quad mirror)
    s = v[j] + dpp_f32<0x128>(v[j]);
    s = s + dpp_f32<0x124>(s);
    v[j] = s - 2.0f * dpp_f32<0x1B>(dpp_f32<0x140>(v[j]));
    // digit 3: the four rows of the wave; mirrored digit = lane ^ 48
    s = v[j] + __shfl_xor(v[j], 16);
    s = s + __shfl_xor(s, 32);
    v[j] = (s - 2.0f * __shfl_xor(v[j], 48)) * 0.0625f;
  }
}

// kernels.py:222-258: per row, optional SwiGLU (float [rows, 2K] gate | up), then H256 on every 256 columns, / 16.
// MODE 0: float rows, 1: bf16 rows, 2: SwiGLU. Does nothing unless only_if[0].
template <int MODE>
__global__ void __launch_bounds__(256) rotate_kernel(const void* x, int K, float* out, const int* only_if) {
  if (!only_if[0]) return;
  const int row = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int g = w; g < K / 256; g += 4) {
    const int c0 = 256 * g + 4 * lane;
    float v[4];
    if constexpr (MODE == 0) {
      const f32x4 a = *(const f32x4*)((const float*)x + (size_t)row * K + c0);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    } else if constexpr (MODE == 1) {
      const i32x2 a = *(const i32x2*)((const uint16_t*)x + (size_t)row * K + c0);
      v[0] = bf16_to_f32((uint32_t)a.x & 0xFFFFu); v[1] = bf16_to_f32((uint32_t)a.x >> 16);
      v[2] = bf16_to_f32((uint32_t)a.y & 0xFFFFu); v[3] = bf16_to_f32((uint32_t)a.y >> 16);
    } else {
      const float* f = (const float*)x + (size_t)row * 2 * K;
      const f32x4 gt = *(const f32x4*)(f + c0), up = *(const f32x4*)(f + K + c0);
      const float gg[4] = {gt.x, gt.y, gt.z, gt.w}, uu[4] = {up.x, up.y, up.z, up.w};
#pragma unroll
      for (int j = 0; j < 4; j++) v[j] = gg[j] / (1.0f + __expf(-gg[j])) * uu[j];
    }
    fwht256(v);
    *(f32x4*)(out + (size_t)row * K + c0) = f32x4{v[0], v[1], v[2], v[3]};
  }
}

// ---------------------------------------------------------------------------------------------------- decode GEMVs
// Which source an expert's rows come from, and whether this launch computes them at all (kernels.py:284-295).
struct Source {
  bool zero, fill;
  int slot;
  size_t id;
};
D3_INLINE Source source_of(const int64_t* ids, const int* plan, const int* took_over, int late, int e, bool cpu_code) {
  Source s;
  const int code = plan[2 * e + 1];
  s.slot = plan[2 * e];
  s.id = (size_t)ids[e];
  s.zero = cpu_code && (late ? (code != 2 || !took_over[0]) : code == 2);
  s.fill = code == 1 && s.slot >= 0;
  return s;
}

// lane's CPL activation floats (columns lane * CPL ..), and their sum
template <int CPL> D3_INLINE float load_slice(const float* xr, int lane, float* xv) {
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL / 4; i++) {
    const f32x4 a = *(const f32x4*)(xr + lane * CPL + 4 * i);
    xv[4 * i] = a.x; xv[4 * i + 1] = a.y; xv[4 * i + 2] = a.z; xv[4 * i + 3] = a.w;
    sum += (a.x + a.y) + (a.z + a.w);
  }
  return sum;
}

// sum over the lane's int8 columns of w * x, with w's sign bit flipped into an unsigned byte: sum (w + 128) x - 128 sum x
template <int CPL> D3_INLINE float dot_i8(const uint32_t* wd, const float* xv, float xsum) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL / 4; i++) {
    const uint32_t u = wd[i] ^ 0x80808080u;
#pragma unroll
    for (int b = 0; b < 4; b++) acc = fmaf((float)((u >> (8 * b)) & 0xFFu), xv[4 * i + b], acc);
  }
  return fmaf(-128.0f, xsum, acc);
}

template <int CPL> D3_INLINE float dot_f8(const uint32_t* wd, const float* xv) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL / 4; i++) {
    const f32x2 lo = fp8x2_to_f32<false>(wd[i]), hi = fp8x2_to_f32<true>(wd[i]);
    acc = fmaf(lo.x, xv[4 * i], acc);
    acc = fmaf(lo.y, xv[4 * i + 1], acc);
    acc = fmaf(hi.x, xv[4 * i + 2], acc);
    acc = fmaf(hi.y, xv[4 * i + 3], acc);
  }
  return acc;
}

template <int CPL> D3_INLINE void load_words(const uint8_t* p, uint32_t* wd) {
#pragma unroll
  for (int i = 0; i < CPL / 4; i++) wd[i] = ((const uint32_t*)p)[i];
}
template <int CPL> D3_INLINE void store_words(uint8_t* p, const uint32_t* wd) {
#pragma unroll
  for (int i = 0; i < CPL / 4; i++) ((uint32_t*)p)[i] = wd[i];
}

// kernels.py:274-314: out[e, n] = (int8 row n of expert e) . x[e or 0] * row scale. Grid (N / 16, k), 256 threads.
template <int K>
__global__ void __launch_bounds__(256) gemv_int8_kernel(const float* x, int x_rows, const int64_t* ids, const int* plan,
                                                        const int* took_over, int late, uint8_t* slot_w, float* slot_s,
                                                        const uint8_t* host_w, const float* host_s, float* out, int N) {
  constexpr int CPL = K / 64;
  const int e = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6, n0 = blockIdx.x * RPB;
  const Source src = source_of(ids, plan, took_over, late, e, true);
  if (src.zero) {
    if (threadIdx.x < RPB) out[(size_t)e * N + n0 + threadIdx.x] = 0.0f;
    return;
  }
  const bool host = plan[2 * e + 1] != 0;
  float xv[CPL];
  const float xsum = load_slice<CPL>(x + (size_t)(x_rows == 1 ? 0 : e) * K, lane, xv);
  const uint8_t* wsrc = host ? host_w + src.id * N * K : slot_w + (size_t)src.slot * N * K;
  const float* ssrc = host ? host_s + src.id * N : slot_s + (size_t)src.slot * N;
#pragma unroll
  for (int r = 0; r < RPB / 4; r++) {
    const int n = n0 + w * (RPB / 4) + r;
    uint32_t wd[CPL / 4];
    load_words<CPL>(wsrc + (size_t)n * K + lane * CPL, wd);
    if (src.fill) store_words<CPL>(slot_w + ((size_t)src.slot * N + n) * K + lane * CPL, wd);
    const float acc = wave_sum_f32(dot_i8<CPL>(wd, xv, xsum));
    if (lane == 0) {
      const float s = ssrc[n];
      out[(size_t)e * N + n] = acc * s;
      if (src.fill) slot_s[(size_t)src.slot * N + n] = s;
    }
  }
}

// kernels.py:316-363: out[e, n] = (e4m3 row n) . x with the 128 x 128 block scales [N / 128, K / 128] folded into the
// activation slice of the block's rows.
template <int K>
__global__ void __launch_bounds__(256) gemv_fp8_kernel(const float* x, int x_rows, const int64_t* ids, const int* plan,
                                                       uint8_t* slot_w, float* slot_s, const uint8_t* host_w,
                                                       const float* host_s, float* out, int N) {
  constexpr int CPL = K / 64, SC = K / 128;
  const int e = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6, n0 = blockIdx.x * RPB;
  const int slot = plan[2 * e];
  const bool host = plan[2 * e + 1] != 0, fill = host && slot >= 0;
  const size_t id = (size_t)ids[e];
  const size_t srows = (size_t)(N / 128) * SC;
  const float* sblock = (host ? host_s + id * srows : slot_s + (size_t)slot * srows) + (size_t)(n0 / 128) * SC;
  if (fill && n0 % 128 == 0 && threadIdx.x < SC) slot_s[(size_t)slot * srows + (size_t)(n0 / 128) * SC + threadIdx.x] = sblock[threadIdx.x];
  float xv[CPL];
  load_slice<CPL>(x + (size_t)(x_rows == 1 ? 0 : e) * K, lane, xv);
#pragma unroll
  for (int j = 0; j < CPL; j++) xv[j] *= sblock[(lane * CPL + j) / 128];
  const uint8_t* wsrc = host ? host_w + id * N * K : slot_w + (size_t)slot * N * K;
#pragma unroll
  for (int r = 0; r < RPB / 4; r++) {
    const int n = n0 + w * (RPB / 4) + r;
    uint32_t wd[CPL / 4];
    load_words<CPL>(wsrc + (size_t)n * K + lane * CPL, wd);
    if (fill) store_words<CPL>(slot_w + ((size_t)slot * N + n) * K + lane * CPL, wd);
    const float acc = wave_sum_f32(dot_f8<CPL>(wd, xv));
    if (lane == 0) out[(size_t)e * N + n] = acc;
  }
}

// W4A8 / W6A8 code decoding to the int8 grid (kernels.py:466-483): 16 columns (group v) of a row; code = nibble (and
// two high bits from the plane after the K/2 nibble bytes at 6 bits); value = codebook[code] or code - 32; q =
// clamp(rint(value * e4m3(scale byte)), -127, 127).
template <int BITS>
D3_INLINE void decode_group(uint32_t lo, uint32_t hi, uint32_t high, uint32_t scale_byte, const float* lut, float* q) {
  const float s = fp8x2_to_f32<false>(scale_byte).x;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const uint32_t code = ((j < 8 ? lo : hi) >> (4 * (j & 7))) & 0xFu;
    float value;
    if constexpr (BITS == 6) value = (float)(code | (((high >> (2 * j)) & 3u) << 4)) - 32.0f;
    else value = lut[code];
    q[j] = fminf(fmaxf(rintf(value * s), -127.0f), 127.0f);
  }
}

// W4 through tables: a 16-column group's codes all share one e4m3 scale byte, so the int8-grid values of the 16 codes at
// each of the 256 scale bytes make a 4 KB table (decode_group's own arithmetic, entry by entry), kept in LDS as bytes
// q + 128. A group then costs one 16-byte table read, and four of its codes become four bytes through two byte
// permutes and a byte mask, instead of a codebook read, a product, a rounding and a clamp per value.
constexpr int QTAB_WORDS = 256 * 4;  // qtab[4 sb + i]: bytes q + 128 of codes 4i .. 4i + 3 at scale byte sb
// cb: codebook[4 (threadIdx.x & 3) .. + 3], loaded by the caller (ahead of its weight rows); SIGNED: the bytes hold q
// itself (two's complement) instead of q + 128
template <bool SIGNED = false> D3_INLINE void build_qtab(uint32_t* qtab, f32x4 cb) {
  const float c[4] = {cb.x, cb.y, cb.z, cb.w};
  for (int i = threadIdx.x; i < QTAB_WORDS; i += blockDim.x) {  // i & 3 == threadIdx.x & 3: blockDim.x % 4 == 0
    const float sc = fp8x2_to_f32<false>((uint32_t)(i >> 2)).x;
    uint32_t word = 0u;
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const float q = fminf(fmaxf(rintf(c[b] * sc), -127.0f), 127.0f);
      word |= ((uint32_t)((int)q + (SIGNED ? 0 : 128)) & 0xFFu) << (8 * b);
    }
    qtab[i] = word;
  }
}

// the table bytes (t: entries 0..15, 4 per word) at the four indices held in the low nibbles of sel's bytes
D3_INLINE uint32_t lookup16(i32x4 t, uint32_t sel) {
  const uint32_t s3 = sel & 0x07070707u;
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)t.y, (uint32_t)t.x, s3);  // entries 0..7
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)t.w, (uint32_t)t.z, s3);  // entries 8..15
  // selector byte 12 gives 0x00, 13 gives 0xFF: a byte mask of the indices >= 8
  const uint32_t m = __builtin_amdgcn_perm(0u, 0u, ((sel >> 3) & 0x01010101u) | 0x0C0C0C0Cu);
  return (hi & m) | (lo & ~m);
}

// sum over one group of (q + 128) * x for its 16 codes (nibble words lo / hi, table row t), x the group's 16 floats
D3_INLINE float group_dot_w4(uint32_t lo, uint32_t hi, i32x4 t, const float* x) {
  float acc = 0.0f;
#pragma unroll
  for (int d = 0; d < 2; d++) {
    const uint32_t word = d ? hi : lo;  // values 8 d .. 8 d + 7: byte b holds value 2b (low nibble) and 2b + 1
#pragma unroll
    for (int odd = 0; odd < 2; odd++) {
      const uint32_t q = lookup16(t, (odd ? word >> 4 : word) & 0x0F0F0F0Fu);
      acc = fmaf((float)(q & 0xFFu), x[8 * d + odd], acc);
      acc = fmaf((float)((q >> 8) & 0xFFu), x[8 * d + 2 + odd], acc);
      acc = fmaf((float)((q >> 16) & 0xFFu), x[8 * d + 4 + odd], acc);
      acc = fmaf((float)((q >> 24) & 0xFFu), x[8 * d + 6 + odd], acc);
    }
  }
  return acc;
}

// kernels.py:495-536: code rows against x, times the row's channel scale. Lane l takes 16-column groups l, l + 64.
template <int K, int BITS>
__global__ void __launch_bounds__(256) gemv_codes_kernel(const float* x, int x_rows, const int64_t* ids, const int* plan,
                                                         uint8_t* slot_w, uint8_t* slot_r, float* slot_c,
                                                         const uint8_t* host_w, const uint8_t* host_r, const float* host_c,
                                                         const float* codebook, float* out, int N) {
  constexpr int RB = K * BITS / 8, G = K / 16, GPL = (G + 63) / 64;
  __shared__ float xs[K];
  __shared__ float lut[16];
  const int e = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6, n0 = blockIdx.x * RPB;
  const float* xr = x + (size_t)(x_rows == 1 ? 0 : e) * K;
  for (int i = threadIdx.x; i < K; i += 256) xs[i] = xr[i];
  if (BITS == 4 && threadIdx.x < 16) lut[threadIdx.x] = codebook[threadIdx.x];
  __syncthreads();
  const int slot = plan[2 * e];
  const bool host = plan[2 * e + 1] != 0, fill = host && slot >= 0;
  const size_t id = (size_t)ids[e];
  const uint8_t* wsrc = host ? host_w + id * N * RB : slot_w + (size_t)slot * N * RB;
  const uint8_t* rsrc = host ? host_r + id * N * G : slot_r + (size_t)slot * N * G;
  const float* csrc = host ? host_c + id * N : slot_c + (size_t)slot * N;
#pragma unroll
  for (int r = 0; r < RPB / 4; r++) {
    const int n = n0 + w * (RPB / 4) + r;
    const uint8_t* row = wsrc + (size_t)n * RB;
    const uint8_t* rs = rsrc + (size_t)n * G;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < GPL; i++) {
      const int v = lane + 64 * i;
      if (v < G) {
        const i32x2 lw = *(const i32x2*)(row + 8 * v);
        const uint32_t high = BITS == 6 ? *(const uint32_t*)(row + K / 2 + 4 * v) : 0u;
        const uint32_t sb = rs[v];
        if (fill) {
          uint8_t* drow = slot_w + ((size_t)slot * N + n) * RB;
          *(i32x2*)(drow + 8 * v) = lw;
          if (BITS == 6) *(uint32_t*)(drow + K / 2 + 4 * v) = high;
          slot_r[((size_t)slot * N + n) * G + v] = (uint8_t)sb;
        }
        float q[16];
        decode_group<BITS>((uint32_t)lw.x, (uint32_t)lw.y, high, sb, lut, q);
#pragma unroll
        for (int j = 0; j < 16; j++) acc = fmaf(q[j], xs[16 * v + j], acc);
      }
    }
    acc = wave_sum_f32(acc);
    if (lane == 0) {
      const float c = csrc[n];
      out[(size_t)e * N + n] = acc * c;
      if (fill) slot_c[(size_t)slot * N + n] = c;
    }
  }
}

// ---------------------------------------------------------------------------------------------- grouped (prefill)
// kernels.py:365-464,538-587: rows of x sorted by expert; group g = (expert, slot, fill, first, rows); out[t, n] = row
// n of the group's expert . x[t] (* its scale). The group reads its slot, or the bank when it has no slot or fills it.
// Each wave holds 4 weight rows in registers and walks the group's activation rows.
template <int KIND, int K>  // KIND 0 int8, 1 fp8, 4 / 6 codes
__global__ void __launch_bounds__(256) grouped_kernel(const float* x, const int* groups, uint8_t* slot_w, void* slot_s,
                                                      void* slot_c, const uint8_t* host_w, const void* host_s,
                                                      const void* host_c, const float* codebook, float* out, int N) {
  constexpr int CPL = K / 64;  // int8 / fp8: bytes per lane per row
  const int* gp = groups + 5 * blockIdx.y;
  const int expert = gp[0], slot = gp[1], fill = gp[2], first = gp[3], rows = gp[4];
  const bool host = slot < 0 || fill;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, n0 = blockIdx.x * RPB;
  __shared__ float lut[16];
  if (KIND == 4 && threadIdx.x < 16) lut[threadIdx.x] = codebook[threadIdx.x];
  __syncthreads();
  if (rows <= 0) return;  // an empty group reads nothing (groups built on the device list every expert)
  if constexpr (KIND == 0 || KIND == 1) {
    const uint8_t* wsrc = host ? host_w + (size_t)expert * N * K : slot_w + (size_t)slot * N * K;
    uint32_t wd[RPB / 4][CPL / 4];
    float rs[RPB / 4];
    float sb[CPL];  // fp8: block scale of each of the lane's columns
    const int SC = K / 128;
    const size_t srows = (size_t)(N / 128) * SC;
    if constexpr (KIND == 1) {
      const float* s = (const float*)host_s;
      const float* sblock = (host ? s + (size_t)expert * srows : (const float*)slot_s + (size_t)slot * srows) + (size_t)(n0 / 128) * SC;
      if (fill && n0 % 128 == 0 && threadIdx.x < SC) ((float*)slot_s)[(size_t)slot * srows + (size_t)(n0 / 128) * SC + threadIdx.x] = sblock[threadIdx.x];
#pragma unroll
      for (int j = 0; j < CPL; j++) sb[j] = sblock[(lane * CPL + j) / 128];
    }
#pragma unroll
    for (int r = 0; r < RPB / 4; r++) {
      const int n = n0 + w * (RPB / 4) + r;
      load_words<CPL>(wsrc + (size_t)n * K + lane * CPL, wd[r]);
      if (fill) store_words<CPL>(slot_w + ((size_t)slot * N + n) * K + lane * CPL, wd[r]);
      if constexpr (KIND == 0) {
        const float* s = host ? (const float*)host_s + (size_t)expert * N : (const float*)slot_s + (size_t)slot * N;
        rs[r] = s[n];
        if (fill && lane == 0) ((float*)slot_s)[(size_t)slot * N + n] = rs[r];
      }
    }
    for (int t = first; t < first + rows; t++) {
      float xv[CPL];
      const float xsum = load_slice<CPL>(x + (size_t)t * K, lane, xv);
      if constexpr (KIND == 1) {
#pragma unroll
        for (int j = 0; j < CPL; j++) xv[j] *= sb[j];
      }
#pragma unroll
      for (int r = 0; r < RPB / 4; r++) {
        const int n = n0 + w * (RPB / 4) + r;
        float acc = KIND == 0 ? dot_i8<CPL>(wd[r], xv, xsum) : dot_f8<CPL>(wd[r], xv);
        acc = wave_sum_f32(acc);
        if (lane == 0) out[(size_t)t * N + n] = KIND == 0 ? acc * rs[r] : acc;
      }
    }
  } else {
    constexpr int BITS = KIND, RB = K * BITS / 8, G = K / 16, GPL = (G + 63) / 64;
    const uint8_t* wsrc = host ? host_w + (size_t)expert * N * RB : slot_w + (size_t)slot * N * RB;
    const uint8_t* rsrc = host ? (const uint8_t*)host_s + (size_t)expert * N * G : (const uint8_t*)slot_s + (size_t)slot * N * G;
    const float* csrc = host ? (const float*)host_c + (size_t)expert * N : (const float*)slot_c + (size_t)slot * N;
    // decoded int8-grid rows, packed 4 per word as (q + 128) bytes, and each row's channel scale
    uint32_t qd[RPB / 4][GPL * 4];
    float cs[RPB / 4];
#pragma unroll
    for (int r = 0; r < RPB / 4; r++) {
      const int n = n0 + w * (RPB / 4) + r;
      const uint8_t* row = wsrc + (size_t)n * RB;
#pragma unroll
      for (int i = 0; i < GPL; i++) {
        const int v = lane + 64 * i;
#pragma unroll
        for (int c = 0; c < 4; c++) qd[r][4 * i + c] = 0x80808080u;
        if (v < G) {
          const i32x2 lw = *(const i32x2*)(row + 8 * v);
          const uint32_t high = BITS == 6 ? *(const uint32_t*)(row + K / 2 + 4 * v) : 0u;
          const uint32_t sbyte = rsrc[(size_t)n * G + v];
          if (fill) {
            uint8_t* drow = slot_w + ((size_t)slot * N + n) * RB;
            *(i32x2*)(drow + 8 * v) = lw;
            if (BITS == 6) *(uint32_t*)(drow + K / 2 + 4 * v) = high;
            ((uint8_t*)slot_s)[((size_t)slot * N + n) * G + v] = (uint8_t)sbyte;
          }
          float q[16];
          decode_group<BITS>((uint32_t)lw.x, (uint32_t)lw.y, high, sbyte, lut, q);
#pragma unroll
          for (int c = 0; c < 4; c++) {
            uint32_t word = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) word |= ((uint32_t)((int)q[4 * c + b] + 128) & 0xFFu) << (8 * b);
            qd[r][4 * i + c] = word;
          }
        }
      }
      cs[r] = csrc[n];
      if (fill && lane == 0) ((float*)slot_c)[(size_t)slot * N + n] = cs[r];
    }
    for (int t = first; t < first + rows; t++) {
      const float* xr = x + (size_t)t * K;
      float acc[RPB / 4];
#pragma unroll
      for (int r = 0; r < RPB / 4; r++) acc[r] = 0.0f;
#pragma unroll
      for (int i = 0; i < GPL; i++) {
        const int v = lane + 64 * i;
        if (v < G) {
          float xv[16];
          float xsum = 0.0f;
#pragma unroll
          for (int c = 0; c < 4; c++) {
            const f32x4 a = *(const f32x4*)(xr + 16 * v + 4 * c);
            xv[4 * c] = a.x; xv[4 * c + 1] = a.y; xv[4 * c + 2] = a.z; xv[4 * c + 3] = a.w;
            xsum += (a.x + a.y) + (a.z + a.w);
          }
#pragma unroll
          for (int r = 0; r < RPB / 4; r++) {
            float part = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
              for (int b = 0; b < 4; b++) part = fmaf((float)((qd[r][4 * i + c] >> (8 * b)) & 0xFFu), xv[4 * c + b], part);
            acc[r] += fmaf(-128.0f, xsum, part);
          }
        }
      }
#pragma unroll
      for (int r = 0; r < RPB / 4; r++) {
        const float s = wave_sum_f32(acc[r]);
        if (lane == 0) out[(size_t)t * N + n0 + w * (RPB / 4) + r] = s * cs[r];
      }
    }
  }
}

// -------------------------------------------------------------------------- grouped (prefill) on the matrix cores
// grouped_kernel's products (kernels.py:365-464,538-587) on the bf16 MFMA. Every weight of these formats is a bf16
// value exactly (int8 and the codes' int8 grid are integers |q| <= 127; e4m3 has 3 mantissa bits). The float32
// activations are split once, before the products, into three bf16 planes x = hi + mid + lo (split3_kernel: hi =
// bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid); what is left is below 2^-24 |x|), so every product w * term
// is exact and the MFMA's float32 sums keep float32 accuracy, as the vector unit's FMAs would.
// Work: grouped_plan_kernel cuts every group into passes of up to 64 rows, the passes with most rows first; a
// workgroup takes one pass against 64 RA weight rows. Wave w holds RA tiles of 16 rows, n0 + 16 RA w + 16 a + (l & 15)
// for lane l, as the MFMA's A rows. Per 128-column chunk the workgroup stages the pass's activation rows (all three
// planes) in LDS, the next chunk's rows and weight bytes loading meanwhile; lane group q = l >> 4 takes columns
// 32 q .. 32 q + 31 of the chunk in 4 steps of 8, decodes its rows' 32 weights once and runs them against the pass's
// 16-row tiles as the B columns (lane l: row l & 15 of the tile, the same 32 columns of each plane). A and B take a
// step's columns in the same lane order, so each sum pairs the right weight and activation whatever order the MFMA
// adds them in. fp8: the 128 x 128 block scale multiplies each chunk's sums, as the reference's block sums are
// scaled. A pass's rows past a multiple of 16 read its last row and are not stored.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int GM_ROWS = 32;   // activation rows per pass (2 tiles of 16)
constexpr int GM_PAD = 136;   // LDS row stride in bf16: 128 columns + 8, so the 16 rows of a tile start 4 banks apart

// x [n] float32 (n % 8 == 0) -> planes hi, mid, lo [n] bf16, x == hi + mid + lo to within 2^-24 |x|
__global__ void __launch_bounds__(256) split3_kernel(const float* x, int64_t n8, bf16x8* hi, bf16x8* mid, bf16x8* lo) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n8; i += (int64_t)gridDim.x * 256) {
    const f32x4 a = ((const f32x4*)x)[2 * i], b = ((const f32x4*)x)[2 * i + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    bf16x8 h, m, l;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      h[j] = (__bf16)v[j];
      const float r = v[j] - (float)h[j];
      m[j] = (__bf16)r;
      l[j] = (__bf16)(r - (float)m[j]);
    }
    hi[i] = h;
    mid[i] = m;
    lo[i] = l;
  }
}

// work [2 + 2 cap] int32: [0] the number of passes, [1] how many of them are first passes (a group's rows
// 0 .. GM_ROWS - 1), then (group, first row of the pass) per pass: the first passes, then the others; within each,
// the passes with most tiles first. Groups that are empty or whose rows lie outside [0, T) get none; no more than cap
// passes are listed; the products skip a place whose group is -1. One workgroup.
// The plan in three steps for a workgroup: every group counted into its buckets (plan_count), the buckets' offsets
// by one thread (plan_offsets), every group's passes put in place (plan_put), a barrier between the steps. count /
// cursor: 8 LDS ints, bucket 4 - tiles (first passes), 8 - tiles (later passes).
static_assert(GM_ROWS % 16 == 0 && GM_ROWS <= 64, "passes of 1 to 4 tiles");
D3_INLINE int plan_tiles(int n) { return (min(n, GM_ROWS) + 15) / 16; }
D3_INLINE bool plan_valid(int first, int rows, int T) { return rows > 0 && first >= 0 && rows <= T - first; }
D3_INLINE void plan_count(int first, int rows, int T, int* count) {
  if (!plan_valid(first, rows, T)) return;
  atomicAdd(&count[4 - plan_tiles(rows)], 1);
  if (rows > GM_ROWS) {
    atomicAdd(&count[8 - GM_ROWS / 16], (rows - GM_ROWS) / GM_ROWS);
    if (rows % GM_ROWS) atomicAdd(&count[8 - plan_tiles(rows % GM_ROWS)], 1);
  }
}
D3_INLINE void plan_offsets(const int* count, int* cursor, int* work, int cap) {
  int at = 0;
  for (int b = 0; b < 8; b++) {
    cursor[b] = at;
    at += count[b];
    if (b == 3) work[1] = min(at, cap);
  }
  work[0] = min(at, cap);
}
D3_INLINE void plan_put(int g, int first, int rows, int T, int* cursor, int* work, int cap) {
  if (!plan_valid(first, rows, T)) return;
  auto put = [&](int bucket, int m0) {
    const int at = atomicAdd(&cursor[bucket], 1);
    if (at < cap) {
      work[2 + 2 * at] = g;
      work[3 + 2 * at] = m0;
    }
  };
  put(4 - plan_tiles(rows), 0);
  for (int m0 = GM_ROWS; m0 < rows; m0 += GM_ROWS) put(8 - plan_tiles(rows - m0), m0);
}

__global__ void __launch_bounds__(256) grouped_plan_kernel(const int* groups, int n_groups, int T, int* work, int cap) {
  __shared__ int count[8], cursor[8];
  if (threadIdx.x < 8) count[threadIdx.x] = 0;
  __syncthreads();
  for (int g = threadIdx.x; g < n_groups; g += 256) plan_count(groups[5 * g + 3], groups[5 * g + 4], T, count);
  __syncthreads();
  if (threadIdx.x == 0) plan_offsets(count, cursor, work, cap);
  __syncthreads();
  for (int g = threadIdx.x; g < n_groups; g += 256)
    plan_put(g, groups[5 * g + 3], groups[5 * g + 4], T, cursor, work, cap);
}

// ------------------------------------------------------------------------------- a prompt's pairs and rows
// The prompt's (token, k) pairs grouped by expert (offload.py:140-143 sorts them and counts each expert's rows): one
// workgroup counts the experts' pairs in LDS, takes the exclusive prefix as each group's first row, and deals every
// pair a place in its expert's range. Within a group the pairs' order is the order of their atomic adds: every output
// row is computed from its own activation row alone, so no result depends on it. ids outside [0, E) take the places
// after every group, inverse -1. With `work`, the same workgroup also plans the grouped products' passes over the
// groups (grouped_plan_kernel's plan, from the counts it holds), so that takes no launch of its own.
constexpr int GROUPS_MAX_E = 1024;
D3_INLINE void expert_groups_body(const int64_t* ids, int P, int E, int64_t* order, int* inverse, int* groups,
                                  int* work, int cap) {
  __shared__ int count[GROUPS_MAX_E + 1], cursor[GROUPS_MAX_E + 1], wave_total[16], pcount[8], pcursor[8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int e = tid; e <= E; e += 1024) count[e] = 0;
  if (tid < 8) pcount[tid] = 0;
  __syncthreads();
  for (int p = tid; p < P; p += 1024) {
    const int64_t e = ids[p];
    atomicAdd(&count[e >= 0 && e < E ? (int)e : E], 1);
  }
  __syncthreads();
  // exclusive prefix over count[0 .. E] (E + 1 <= 1025 entries: thread t takes entry t, thread 0 also entry 1024)
  const int v = tid <= E ? count[tid] : 0;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int u = __shfl_up(incl, d);
    if (lane >= d) incl += u;
  }
  if (lane == 63) wave_total[w] = incl;
  __syncthreads();
  int before = 0;
  for (int i = 0; i < w; i++) before += wave_total[i];
  const int first = before + incl - v;
  if (tid <= E) cursor[tid] = first;
  if (tid < E) {
    int* gp = groups + 5 * tid;
    gp[0] = tid;
    gp[1] = tid;
    gp[2] = 0;
    gp[3] = first;
    gp[4] = v;
  }
  if (E == GROUPS_MAX_E && tid == 0) {  // entry 1024: after all 1024 threads' entries
    int all = 0;
    for (int i = 0; i < 16; i++) all += wave_total[i];
    cursor[E] = all;
  }
  if (work) {  // thread e < E holds group e's (first, rows)
    if (tid < E) plan_count(first, v, P, pcount);
    __syncthreads();
    if (tid == 0) plan_offsets(pcount, pcursor, work, cap);
    __syncthreads();
    if (tid < E) plan_put(tid, first, v, P, pcursor, work, cap);
  }
  __syncthreads();
  for (int p = tid; p < P; p += 1024) {
    const int64_t e = ids[p];
    const bool valid = e >= 0 && e < E;
    const int at = atomicAdd(&cursor[valid ? (int)e : E], 1);
    order[at] = p;
    inverse[p] = valid ? at : -1;
  }
}

__global__ void __launch_bounds__(1024) expert_groups_kernel(const int64_t* ids, int P, int E, int64_t* order,
                                                             int* inverse, int* groups, int* work, int cap) {
  expert_groups_body(ids, P, E, order, inverse, groups, work, cap);
}

// columns c0 .. c0 + 3 of row `row` of x as float (SRC as for prep_planes_kernel)
template <int SRC> D3_INLINE void load_row4(const void* x, size_t row, int K, int c0, float* v) {
  if constexpr (SRC == 0) {
    const f32x4 a = *(const f32x4*)((const float*)x + row * K + c0);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  } else if constexpr (SRC == 1) {
    const i32x2 a = *(const i32x2*)((const uint16_t*)x + row * K + c0);
    v[0] = bf16_to_f32((uint32_t)a.x & 0xFFFFu); v[1] = bf16_to_f32((uint32_t)a.x >> 16);
    v[2] = bf16_to_f32((uint32_t)a.y & 0xFFFFu); v[3] = bf16_to_f32((uint32_t)a.y >> 16);
  } else {
    const float* f = (const float*)x + row * 2 * K;
    const f32x4 gt = *(const f32x4*)(f + c0), up = *(const f32x4*)(f + K + c0);
    const float gg[4] = {gt.x, gt.y, gt.z, gt.w}, uu[4] = {up.x, up.y, up.z, up.w};
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = gg[j] / (1.0f + __expf(-gg[j])) * uu[j];
  }
}

// Planes hi, mid, lo [P, K] of the rows the grouped products read (split3_kernel's split): row p is x's row
// order[p] / k (x's row p without order); SRC 0 float32 rows [., K], 1 bf16 rows, 2 float32 gate | up rows [., 2K]
// through SiLU(gate) * up (kernels.py:222-258's SwiGLU); ROT: in the ConvRot basis (H256 on every 256 columns, / 16).
template <int SRC, bool ROT, int PL>
__global__ void __launch_bounds__(256) prep_planes_kernel(const void* x, const int64_t* order, int k, int K,
                                                          __bf16* planes, int64_t plane) {
  const int p = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const size_t row = order ? (size_t)(order[p] / k) : (size_t)p;
  for (int g = w; g < K / 256; g += 4) {
    const int c0 = 256 * g + 4 * lane;
    float v[4];
    load_row4<SRC>(x, row, K, c0, v);
    if constexpr (ROT) fwht256(v);
    typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
    bf16x4 h, m, l;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      h[j] = (__bf16)v[j];
      const float r = v[j] - (float)h[j];
      m[j] = (__bf16)r;
      l[j] = (__bf16)(r - (float)m[j]);
    }
    const size_t at = (size_t)p * K + c0;
    *(bf16x4*)(planes + at) = h;
    if constexpr (PL == 3) {
      *(bf16x4*)(planes + plane + at) = m;
      *(bf16x4*)(planes + 2 * plane + at) = l;
    }
  }
}

// The same rows (SRC, ROT as for prep_planes_kernel) as three int8 planes a0, a1, a2 [P, K] and a row scale S
// (scales[p]) for the products on the int8 matrix cores: S is the smallest power of two with max |v| <= 127 S, and
//   v / S = a0 + a1 / 254 + a2 / 254^2 + r,  every a in [-127, 127], |r| <= 0.5 / 254^2 + 2^-24
// (v / S and d = v / S - a0 are exact; a1 = rint(254 d rounded), a2 = rint(254 (254 d - a1) rounded), the inner
// difference from the exact product, rounded once). So the planes hold v to within (0.5 / 254^2 + 2^-24) S <
// 1.25e-7 max |v|, and a row of integers times a power of two (such as a one-hot row) exactly in a0. An all-zero row
// gets S = 0, a row holding a non-finite value S = NaN (planes 0 both ways); below 2^-143, S stays 2^-149.
constexpr float I8_RATIO = 254.0f;  // the int8 planes' ratio

// Row p of the planes by the row's 4 waves (w = 0 .. 3 of them, lane within the wave, tid0: the row's first thread;
// wmax: 4 LDS words of the row); valid false: a row past the planes' end, which only joins the barrier. Every
// thread of the workgroup takes the one barrier inside.
template <int SRC, bool ROT>
D3_INLINE void prep_i8_row(const void* x, const int64_t* order, int k, int K, int8_t* planes, int64_t plane,
                           float* scales, int p, bool valid, int w, int lane, bool tid0, uint32_t* wmax) {
  const size_t row = !valid ? 0 : order ? (size_t)(order[p] / k) : (size_t)p;
  float v[2][4];  // wave w's columns 256 g + 4 lane .. + 3 of g = w, w + 4 (K <= 2048)
  uint32_t m = 0u;  // the bits of max |v|: non-negative floats order as their bits, inf and NaN above every finite
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int g = w + 4 * i;
    if (valid && g < K / 256) {
      load_row4<SRC>(x, row, K, 256 * g + 4 * lane, v[i]);
      if constexpr (ROT) fwht256(v[i]);
#pragma unroll
      for (int j = 0; j < 4; j++) m = max(m, __float_as_uint(v[i][j]) & 0x7FFFFFFFu);
    }
  }
  m = wave_max_u32(m);
  if (lane == 0) wmax[w] = m;
  __syncthreads();
  if (!valid) return;
  m = max(max(wmax[0], wmax[1]), max(wmax[2], wmax[3]));
  const bool split = m != 0u && m < 0x7F800000u;
  int e = 0;  // S = 2^e
  if (split) {
    const float mf = __uint_as_float(m);
    e = max(ilogbf(mf) - 6, -149);  // mf / 2^e in [64, 128) (or below 64 for tiny rows)
    if (mf > ldexpf(127.0f, e)) e += 1;
  }
  if (tid0) scales[p] = split ? ldexpf(1.0f, e) : m == 0u ? 0.0f : __uint_as_float(0x7FC00000u);
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int g = w + 4 * i;
    if (g < K / 256) {
      uint32_t q0 = 0u, q1 = 0u, q2 = 0u;
      if (split) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
          // explicit roundings (no contraction to choose them): a1 from the rounded 254 d, the remainder of the exact
          // product after a1 by one fused step
          const float a = ldexpf(v[i][j], -e), a0 = rintf(a), d = a - a0;
          const float a1 = rintf(__fmul_rn(d, I8_RATIO)), a2 = rintf(__fmul_rn(fmaf(d, I8_RATIO, -a1), I8_RATIO));
          q0 |= ((uint32_t)(int)a0 & 0xFFu) << (8 * j);
          q1 |= ((uint32_t)(int)a1 & 0xFFu) << (8 * j);
          q2 |= ((uint32_t)(int)a2 & 0xFFu) << (8 * j);
        }
      }
      uint32_t* d = (uint32_t*)(planes + (size_t)p * K + 256 * g + 4 * lane);
      d[0] = q0;
      d[plane / 4] = q1;
      d[plane / 2] = q2;
    }
  }
}

template <int SRC, bool ROT>
__global__ void __launch_bounds__(256) prep_i8_kernel(const void* x, const int64_t* order, int k, int K,
                                                      int8_t* planes, int64_t plane, float* scales) {
  __shared__ uint32_t wmax[4];
  prep_i8_row<SRC, ROT>(x, order, k, K, planes, plane, scales, blockIdx.x, true, threadIdx.x >> 6,
                        threadIdx.x & 63, threadIdx.x == 0, wmax);
}

// The grouping (workgroup 0, expert_groups_kernel's) and the token rows' int8 planes (prep_i8_kernel's, 4 rows per
// later workgroup) in one launch: neither waits for the other, so the planes cost no launch of their own.
template <int SRC, bool ROT>
__global__ void __launch_bounds__(1024) groups_prep_kernel(const int64_t* ids, int P, int E, int64_t* order,
                                                           int* inverse, int* groups, int* work, int cap,
                                                           const void* x, int T, int K, int8_t* planes,
                                                           float* scales) {
  if (blockIdx.x == 0) {
    expert_groups_body(ids, P, E, order, inverse, groups, work, cap);
    return;
  }
  __shared__ uint32_t wmax[4][4];
  const int tid = threadIdx.x, r = tid >> 8, p = 4 * ((int)blockIdx.x - 1) + r;
  prep_i8_row<SRC, ROT>(x, nullptr, 1, K, planes, (int64_t)T * K, scales, p, p < T, (tid >> 6) & 3, tid & 63,
                        (tid & 255) == 0, wmax[r]);
}

// out[t, h] = sum over j in order of w[t, j] * sorted_out[inverse[t k + j], h] (pairs with inverse -1 left out), in
// float32, stored as float32 / bf16 / fp16 (out_type 0 / 1 / 2): offload.py:144-149's weighted sum over k.
template <bool WBF16>
__global__ void __launch_bounds__(256) combine_rows_kernel(const float* sorted_out, const int* inverse,
                                                           const void* weights, int k, int H, void* out, int out_type) {
  const int t = blockIdx.y, h = 4 * (blockIdx.x * 256 + threadIdx.x);
  if (h >= H) return;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int j = 0; j < k; j++) {
    const int at = inverse[(size_t)t * k + j];
    if (at < 0) continue;
    const float wj = WBF16 ? bf16_to_f32(((const uint16_t*)weights)[(size_t)t * k + j])
                           : ((const float*)weights)[(size_t)t * k + j];
    const f32x4 y = *(const f32x4*)(sorted_out + (size_t)at * H + h);
    acc.x = fmaf(y.x, wj, acc.x);
    acc.y = fmaf(y.y, wj, acc.y);
    acc.z = fmaf(y.z, wj, acc.z);
    acc.w = fmaf(y.w, wj, acc.w);
  }
  const size_t o = (size_t)t * H + h;
  if (out_type == 0) {
    *(f32x4*)((float*)out + o) = acc;
  } else if (out_type == 1) {
    uint16_t* d = (uint16_t*)out + o;
    const uint32_t lo = f32_to_bf16(acc.x) | (f32_to_bf16(acc.y) << 16), hi = f32_to_bf16(acc.z) | (f32_to_bf16(acc.w) << 16);
    *(i32x2*)d = i32x2{(int)lo, (int)hi};
  } else {
    _Float16* d = (_Float16*)out + o;
    d[0] = (_Float16)acc.x; d[1] = (_Float16)acc.y; d[2] = (_Float16)acc.z; d[3] = (_Float16)acc.w;
  }
}

// a lane's 32 weights of one row in a chunk as they come from memory (int8 / fp8: 32 bytes in b0, b1; codes: b0 the
// 16 nibble bytes, b1.x / b1.y the W6 high plane's 8 bytes, sb0 / sb1 the two group scale bytes)
struct ChunkBytes {
  i32x4 b0, b1;
  uint32_t sb0, sb1;
};

// eight e4m3 weights (two words, byte i = column i) as bf16: exact, e4m3 has 3 mantissa bits
D3_INLINE bf16x8 fp8x8_to_bf16(uint32_t w0, uint32_t w1) {
  const f32x2 p0 = fp8x2_to_f32<false>(w0), p1 = fp8x2_to_f32<true>(w0);
  const f32x2 p2 = fp8x2_to_f32<false>(w1), p3 = fp8x2_to_f32<true>(w1);
  bf16x8 a;
  a[0] = (__bf16)p0.x; a[1] = (__bf16)p0.y; a[2] = (__bf16)p1.x; a[3] = (__bf16)p1.y;
  a[4] = (__bf16)p2.x; a[5] = (__bf16)p2.y; a[6] = (__bf16)p3.x; a[7] = (__bf16)p3.y;
  return a;
}

// The row of the planes that row p of the passes reads: p itself, or with `order` x's row order[p] / k (the rows of
// a prompt's pairs taken from its token rows, so no gathered copy is made), kept within the planes' xrows rows.
D3_INLINE size_t plane_row(const int64_t* order, int k, int xrows, int p) {
  return order ? (size_t)min(max((int)order[p], 0) / k, xrows - 1) : (size_t)p;
}

// The fp8 grouped products on the bf16 matrix cores, over PL bf16 planes of the rows (1: bf16 rows as they are).
// grid (N / (64 RA), a multiple of 8 rows): the workgroups of one pass run on one XCD (the dispatcher deals
// workgroup i to XCD i % 8), where its activation rows stay in that XCD's L2. PHASE 2 runs every pass of the plan;
// PHASE 0 the first passes, PHASE 1 the others, a filled group's then read from its slot (the first passes filled it).
template <int K, int RA, int PL>  // RA row tiles per wave; PL planes
__global__ void __launch_bounds__(256, 2) grouped_fp8_kernel(const __bf16* xs, int64_t plane, const int64_t* order,
                                                             int k_order, int xrows, const int* groups,
                                                             const int* work, int phase, uint8_t* slot_w,
                                                             float* slot_s, const uint8_t* host_w,
                                                             const float* host_s, float* out, int N) {
  constexpr int CHUNKS = K / 128, MT = GM_ROWS / 16;
  constexpr int STAGE = MT * PL;   // 16-byte pieces each thread stages per chunk
  // chunks whose weights are on their way while one is multiplied (more gain nothing: the loads complete in order,
  // and each chunk waits for the next chunk's rows, requested after the weights one chunk ahead)
  constexpr int GM_AHEAD = 2;
  static_assert(CHUNKS % GM_AHEAD == 0, "K a multiple of 256");
  __shared__ __attribute__((aligned(16))) __bf16 bt[MT * PL * 16 * GM_PAD];
  // XCD-aware order: workgroup i of the launch runs on XCD i % 8; passes p with p % 8 == xcd are dealt to it
  const int nx = gridDim.x, lin = blockIdx.x + nx * blockIdx.y, xcd = lin & 7, k = lin >> 3;
  const int item = (k / nx) * 8 + xcd + (phase == 1 ? work[1] : 0), xb = k % nx;
  if (item >= work[phase == 0 ? 1 : 0]) return;
  const int g = work[2 + 2 * item], m0 = work[3 + 2 * item];
  if (g < 0) return;  // an empty place of the list
  const int* gp = groups + 5 * g;
  const int expert = gp[0], slot = gp[1], fill = gp[2] && phase != 1, first = gp[3], rows = gp[4];
  const bool host = slot < 0 || fill, filler = fill && m0 == 0;  // the group's first pass copies it into its slot
  const int tiles = min(MT, (rows - m0 + 15) / 16);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, q = lane >> 4, c = lane & 15;
  const int nw = xb * 64 * RA + 16 * RA * w;  // the wave's first row
  const size_t src = host ? (size_t)expert : (size_t)slot;  // the expert's index in the fields it is read from
  const uint8_t* arow = (host ? host_w : slot_w) + (src * N + nw + c) * K;      // this lane's row of tile 0
  uint8_t* frow = filler ? slot_w + ((size_t)slot * N + nw + c) * K : slot_w;  // its slot row (fill)
  auto load_chunk = [&](int ch, ChunkBytes (&cb)[RA]) {
    const int k0 = 128 * ch + 32 * q;
#pragma unroll
    for (int a = 0; a < RA; a++) {
      const uint8_t* r = arow + (size_t)16 * a * K;
      cb[a].b0 = *(const i32x4*)(r + k0);
      cb[a].b1 = *(const i32x4*)(r + k0 + 16);
    }
  };
  // staging: piece j of thread tid is tile j / PL, plane j % PL, row (tid >> 4) & 15, the 16 bytes at column
  // 8 (tid & 15)
  const int srow_t = (tid >> 4) & 15, sseg = tid & 15;
  size_t xr[MT];  // where each tile's staged row starts in a plane
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
    xr[mt] = plane_row(order, k_order, xrows, first + min(m0 + 16 * mt + srow_t, rows - 1)) * K + 8 * sseg;
  i32x4 stg[STAGE];
  auto stage_load = [&](int ch) {
#pragma unroll
    for (int j = 0; j < STAGE; j++) {
      const int mt = j / PL, t = j % PL;
      if (mt < tiles) stg[j] = *(const i32x4*)(xs + t * plane + xr[mt] + 128 * ch);
    }
  };
  auto stage_store = [&]() {
#pragma unroll
    for (int j = 0; j < STAGE; j++) {
      if (j < PL * tiles) *(i32x4*)(bt + (j * 16 + srow_t) * GM_PAD + 8 * sseg) = stg[j];
    }
  };
  // the 128 x 128 block scales of the wave's row block (its 16 RA <= 64 rows lie in one), one per chunk
  const size_t srows = (size_t)(N / 128) * CHUNKS, boff = (size_t)(nw / 128) * CHUNKS;
  const float* sblk = (host ? host_s : slot_s) + src * srows + boff;
  if (filler && nw % 128 == 0 && lane < CHUNKS) slot_s[(size_t)slot * srows + boff + lane] = sblk[lane];
  f32x4 acc[RA][MT];
#pragma unroll
  for (int a = 0; a < RA; a++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[a][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  // one chunk: its weights (loaded GM_AHEAD chunks ahead into `bytes`, which then take chunk ch + GM_AHEAD's)
  // widened, the slot filled, the next chunk's rows on their way, the products from LDS scaled by the chunk's block
  // scale, then the next chunk's rows into LDS
  auto chunk = [&](int ch, ChunkBytes (&bytes)[RA]) {
    const int k0 = 128 * ch + 32 * q;
    if (filler) {  // the expert's bytes copied into its slot as they are read
#pragma unroll
      for (int a = 0; a < RA; a++) {
        uint8_t* f = frow + (size_t)16 * a * K;
        *(i32x4*)(f + k0) = bytes[a].b0;
        *(i32x4*)(f + k0 + 16) = bytes[a].b1;
      }
    }
    bf16x8 wa[RA][4];
#pragma unroll
    for (int a = 0; a < RA; a++) {
      wa[a][0] = fp8x8_to_bf16((uint32_t)bytes[a].b0.x, (uint32_t)bytes[a].b0.y);
      wa[a][1] = fp8x8_to_bf16((uint32_t)bytes[a].b0.z, (uint32_t)bytes[a].b0.w);
      wa[a][2] = fp8x8_to_bf16((uint32_t)bytes[a].b1.x, (uint32_t)bytes[a].b1.y);
      wa[a][3] = fp8x8_to_bf16((uint32_t)bytes[a].b1.z, (uint32_t)bytes[a].b1.w);
    }
    if (ch + GM_AHEAD < CHUNKS) load_chunk(ch + GM_AHEAD, bytes);
    if (ch + 1 < CHUNKS) stage_load(ch + 1);
    f32x4 part[RA][MT];  // this chunk's sums before its block scale
#pragma unroll
    for (int a = 0; a < RA; a++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) part[a][mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < 4; st++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        if (mt < tiles) {
          const __bf16* bp = bt + (mt * PL * 16 + c) * GM_PAD + 32 * q + 8 * st;
          bf16x8 b[PL];
#pragma unroll
          for (int t = 0; t < PL; t++) b[t] = *(const bf16x8*)(bp + 16 * t * GM_PAD);
#pragma unroll
          for (int a = 0; a < RA; a++)
#pragma unroll
            for (int t = 0; t < PL; t++)
              part[a][mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(wa[a][st], b[t], part[a][mt], 0, 0, 0);
        }
      }
    const float sc = sblk[ch];
#pragma unroll
    for (int a = 0; a < RA; a++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[a][mt][i] = fmaf(sc, part[a][mt][i], acc[a][mt][i]);
    if (ch + 1 < CHUNKS) {
      __syncthreads();  // every wave is done with this chunk's rows
      stage_store();
      __syncthreads();
    }
  };
  ChunkBytes ring[GM_AHEAD][RA];  // chunk ch's weight bytes in ring[ch % GM_AHEAD]
#pragma unroll
  for (int d = 0; d < GM_AHEAD; d++) load_chunk(d, ring[d]);
  stage_load(0);
  stage_store();
  __syncthreads();
  for (int ch = 0; ch < CHUNKS; ch += GM_AHEAD) {
#pragma unroll
    for (int d = 0; d < GM_AHEAD; d++) chunk(ch + d, ring[d]);
  }
  // lane l holds rows nw + 16 a + 4 q .. + 3 of activation row m0 + 16 mt + (l & 15)
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const int r = m0 + 16 * mt + c;
    if (mt < tiles && r < rows) {
#pragma unroll
      for (int a = 0; a < RA; a++) *(f32x4*)(out + (size_t)(first + r) * N + nw + 16 * a + 4 * q) = acc[a][mt];
    }
  }
}

// ----------------------------------------------------------------------------- grouped products on the int8 cores
// The grouped products of the formats whose weights are integers |q| <= 127 before their row or channel scale (int8
// ConvRot, W4 and W6 codes on the int8 grid) on the int8 matrix cores, v_mfma_i32_16x16x64_i8 (twice the bf16 rate
// and 64 columns a step), against the rows as three int8 planes (prep_i8_kernel). The weight bytes go in as they are
// (int8) or as decoded bytes (codes); each plane's sums are exact int32 (|sum| <= 2048 * 127 * 127 < 2^25), and the
// epilogue adds the planes in float32: out = es * (S * (A0 + (A1 + A2 / 254) / 254)). The work list, placement,
// slot fill and weight ring are grouped_fp8_kernel's; lane group q takes columns 32 q .. 32 q + 31 of each
// 128-column chunk in 2 steps of 16 bytes, weights and rows alike.

// W4: one 16-code group's int8-grid values as bytes in column order (word d: codes 4d .. 4d + 3) through the
// group's scale-byte row t of a signed table (build_qtab<true>); lo / hi: the nibble words of codes 0-7 / 8-15
// (code j's nibble at bits 4 (j & 7))
D3_INLINE i32x4 w4_group_i8(uint32_t lo, uint32_t hi, i32x4 t) {
  const uint32_t e0 = lookup16(t, lo), o0 = lookup16(t, lo >> 4);  // codes 0, 2, 4, 6 / 1, 3, 5, 7
  const uint32_t e1 = lookup16(t, hi), o1 = lookup16(t, hi >> 4);  // codes 8, 10, 12, 14 / 9, 11, 13, 15
  return i32x4{(int)__builtin_amdgcn_perm(o0, e0, 0x05010400u), (int)__builtin_amdgcn_perm(o0, e0, 0x07030602u),
               (int)__builtin_amdgcn_perm(o1, e1, 0x05010400u), (int)__builtin_amdgcn_perm(o1, e1, 0x07030602u)};
}

// W6: one 16-code group's int8-grid values (decode_group<6>'s arithmetic: clamp(rint((code - 32) * s), +-127), with
// (code - 32) * s formed exactly as code * s - 32 s) as bytes in column order. lo / hi: the nibble words of codes
// 0-7 / 8-15 (code j's low nibble at bits 4 (j & 7)); high: code j's top two bits at bits 2j. Codes k, k + 4, k + 8,
// k + 12 are assembled together, one per byte: their nibbles by one byte permute, their top bits by a shift. rint(t)
// for |t| < 2^22 is the low mantissa bits of t + 1.5 * 2^23 (round to nearest even, as rintf), two's complement; the
// clamp to +-127 happens on the biased value (a NaN scale gives -127, as fmaxf / fminf do).
D3_INLINE i32x4 w6_group_i8(uint32_t lo, uint32_t hi, uint32_t high, float s) {
  constexpr float MAGIC = 12582912.0f;
  const float ms = -32.0f * s;
  uint32_t u[4][4];  // u[k][b]: code k + 4b
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t h = k >> 1, sel = h | ((h + 2) << 8) | ((h + 4) << 16) | ((h + 6) << 24);
    const uint32_t p = __builtin_amdgcn_perm(hi, lo, sel);
    const uint32_t code = ((k & 1 ? p >> 4 : p) & 0x0F0F0F0Fu) | (((high >> (2 * k)) & 0x03030303u) << 4);
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const float t = fmaf((float)((code >> (8 * b)) & 0xFFu), s, ms) + MAGIC;
      u[k][b] = __float_as_uint(fminf(fmaxf(t, MAGIC - 127.0f), MAGIC + 127.0f));
    }
  }
  i32x4 r;
#pragma unroll
  for (int d = 0; d < 4; d++) {
    const uint32_t p01 = __builtin_amdgcn_perm(u[1][d], u[0][d], 0x0C0C0400u);  // bytes u0, u1, 0, 0
    const uint32_t p23 = __builtin_amdgcn_perm(u[3][d], u[2][d], 0x04000C0Cu);  // bytes 0, 0, u2, u3
    r[d] = (int)(p01 | p23);
  }
  return r;
}

constexpr int GI_SC = 2;                   // chunks staged together: 256 columns of each row per stage
constexpr int GI_PITCH = 128 * GI_SC + 16;  // LDS row stride in bytes: the 16 rows of a tile start 4 banks apart

template <int KIND, int K, int RA>  // KIND 0 int8, 4 / 6 codes; RA row tiles per wave
__global__ void __launch_bounds__(256, 2) grouped_i8_kernel(const int8_t* xs, int64_t plane, const float* xscale,
                                                            const int64_t* order, int k_order, int xrows,
                                                            const int* groups, const int* work, int phase,
                                                            uint8_t* slot_w, void* slot_s, void* slot_c,
                                                            const uint8_t* host_w, const void* host_s,
                                                            const void* host_c, const float* codebook, float* out,
                                                            int N) {
  static_assert(KIND == 0 || KIND == 4 || KIND == 6, "integer formats");
  constexpr int RB = KIND == 0 ? K : K * KIND / 8;  // row bytes
  constexpr int G = K / 16;                          // codes: 16-column scale groups per row
  constexpr int CHUNKS = K / 128, MT = GM_ROWS / 16, PL = 3;
  static_assert(GI_SC == 2, "a stage's row of 256 bytes is 16 threads' 16-byte pieces");
  constexpr int STAGE = MT * PL;  // 16-byte pieces each thread stages per stage: tile-plane j, row tid >> 4
  // chunks of weights on their way while one is multiplied: one stage. Each stage's rows are requested before the
  // weights, so the wait for them at the stage's end leaves the weights in flight (deeper measured no faster).
  constexpr int AHEAD = GI_SC;
  static_assert(CHUNKS % GI_SC == 0, "K a multiple of 256");
  __shared__ uint32_t qtab[KIND == 4 ? QTAB_WORDS : 1];
  __shared__ __attribute__((aligned(16))) int8_t bt[MT * PL * 16 * GI_PITCH];
  // XCD-aware order: workgroup i of the launch runs on XCD i % 8; passes p with p % 8 == xcd are dealt to it
  const int nx = gridDim.x, lin = blockIdx.x + nx * blockIdx.y, xcd = lin & 7, k = lin >> 3;
  const int item = (k / nx) * 8 + xcd + (phase == 1 ? work[1] : 0), xb = k % nx;
  if (item >= work[phase == 0 ? 1 : 0]) return;
  const int g = work[2 + 2 * item], m0 = work[3 + 2 * item];
  if (g < 0) return;  // an empty place of the list
  const int* gp = groups + 5 * g;
  const int expert = gp[0], slot = gp[1], fill = gp[2] && phase != 1, first = gp[3], rows = gp[4];
  const bool host = slot < 0 || fill, filler = fill && m0 == 0;  // the group's first pass copies it into its slot
  const int tiles = min(MT, (rows - m0 + 15) / 16);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, q = lane >> 4, c = lane & 15;
  const int nw = xb * 64 * RA + 16 * RA * w;  // the wave's first row
  if constexpr (KIND == 4) build_qtab<true>(qtab, *(const f32x4*)(codebook + 4 * (tid & 3)));
  const size_t src = host ? (size_t)expert : (size_t)slot;  // the expert's index in the fields it is read from
  const uint8_t* arow = (host ? host_w : slot_w) + (src * N + nw + c) * RB;      // this lane's row of tile 0
  uint8_t* frow = filler ? slot_w + ((size_t)slot * N + nw + c) * RB : slot_w;  // its slot row (fill)
  const uint8_t* srow = nullptr;                                                 // codes: its scale bytes
  if constexpr (KIND >= 4) srow = (const uint8_t*)(host ? host_s : slot_s) + (src * N + nw + c) * G;
  auto load_chunk = [&](int ch, ChunkBytes (&cb)[RA]) {
    const int k0 = 128 * ch + 32 * q;
#pragma unroll
    for (int a = 0; a < RA; a++) {
      const uint8_t* r = arow + (size_t)16 * a * RB;
      if constexpr (KIND == 0) {
        cb[a].b0 = *(const i32x4*)(r + k0);
        cb[a].b1 = *(const i32x4*)(r + k0 + 16);
      } else {
        cb[a].b0 = *(const i32x4*)(r + k0 / 2);
        cb[a].b1 = i32x4{0, 0, 0, 0};
        if constexpr (KIND == 6) {
          const i32x2 hw = *(const i32x2*)(r + K / 2 + k0 / 4);
          cb[a].b1.x = hw.x;
          cb[a].b1.y = hw.y;
        }
        cb[a].sb0 = srow[16 * a * G + k0 / 16];
        cb[a].sb1 = srow[16 * a * G + k0 / 16 + 1];
      }
    }
  };
  // staging: piece j of thread tid is tile j / PL, plane j % PL, row tid >> 4, the 16 bytes at column 16 (tid & 15)
  // of the stage's 256
  const int srow_t = tid >> 4, sseg = tid & 15;
  size_t xr[MT];  // where each tile's staged row starts in a plane
#pragma unroll
  for (int mt = 0; mt < MT; mt++)
    xr[mt] = plane_row(order, k_order, xrows, first + min(m0 + 16 * mt + srow_t, rows - 1)) * K + 16 * sseg;
  i32x4 stg[STAGE];
  auto stage_load = [&](int s) {
#pragma unroll
    for (int j = 0; j < STAGE; j++) {
      const int mt = j / PL, t = j % PL;
      if (mt < tiles) stg[j] = *(const i32x4*)(xs + t * plane + xr[mt] + 128 * GI_SC * s);
    }
  };
  auto stage_store = [&]() {
#pragma unroll
    for (int j = 0; j < STAGE; j++) {
      if (j < PL * tiles) *(i32x4*)(bt + (j * 16 + srow_t) * GI_PITCH + 16 * sseg) = stg[j];
    }
  };
  // the epilogue's scales of rows nw + 16 a + 4 q .. + 3: int8 row scales, codes channel scales
  float es[RA][4];
  {
    const float* s = (const float*)(KIND == 0 ? (host ? host_s : slot_s) : (host ? host_c : slot_c)) + src * N;
    float* fs = (float*)(KIND == 0 ? slot_s : slot_c) + (size_t)slot * N;
#pragma unroll
    for (int a = 0; a < RA; a++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        es[a][r] = s[nw + 16 * a + 4 * q + r];
        if (filler && c == 0) fs[nw + 16 * a + 4 * q + r] = es[a][r];
      }
  }
  i32x4 acc[RA][MT][PL];
#pragma unroll
  for (int a = 0; a < RA; a++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int t = 0; t < PL; t++) acc[a][mt][t] = i32x4{0, 0, 0, 0};
  // one chunk (half `h` of its stage): its weights (loaded AHEAD chunks ahead into `bytes`, which then take chunk
  // ch + AHEAD's) as int8 operands, the slot filled, the products from LDS; after the stage's second chunk the next
  // stage's rows (requested with the first chunk) go into LDS
  auto chunk = [&](int ch, int h, ChunkBytes (&bytes)[RA]) {
    const int k0 = 128 * ch + 32 * q;
    if (filler) {  // the expert's bytes copied into its slot as they are read
#pragma unroll
      for (int a = 0; a < RA; a++) {
        uint8_t* f = frow + (size_t)16 * a * RB;
        if constexpr (KIND == 0) {
          *(i32x4*)(f + k0) = bytes[a].b0;
          *(i32x4*)(f + k0 + 16) = bytes[a].b1;
        } else {
          *(i32x4*)(f + k0 / 2) = bytes[a].b0;
          if constexpr (KIND == 6) *(i32x2*)(f + K / 2 + k0 / 4) = i32x2{bytes[a].b1.x, bytes[a].b1.y};
          uint8_t* fsb = (uint8_t*)slot_s + ((size_t)slot * N + nw + 16 * a + c) * G;
          fsb[k0 / 16] = (uint8_t)bytes[a].sb0;
          fsb[k0 / 16 + 1] = (uint8_t)bytes[a].sb1;
        }
      }
    }
    i32x4 wa[RA][2];
#pragma unroll
    for (int a = 0; a < RA; a++) {
      if constexpr (KIND == 0) {
        wa[a][0] = bytes[a].b0;
        wa[a][1] = bytes[a].b1;
      } else if constexpr (KIND == 4) {
        wa[a][0] = w4_group_i8((uint32_t)bytes[a].b0.x, (uint32_t)bytes[a].b0.y, *(const i32x4*)(qtab + 4 * bytes[a].sb0));
        wa[a][1] = w4_group_i8((uint32_t)bytes[a].b0.z, (uint32_t)bytes[a].b0.w, *(const i32x4*)(qtab + 4 * bytes[a].sb1));
      } else {
        wa[a][0] = w6_group_i8((uint32_t)bytes[a].b0.x, (uint32_t)bytes[a].b0.y, (uint32_t)bytes[a].b1.x,
                               fp8x2_to_f32<false>(bytes[a].sb0).x);
        wa[a][1] = w6_group_i8((uint32_t)bytes[a].b0.z, (uint32_t)bytes[a].b0.w, (uint32_t)bytes[a].b1.y,
                               fp8x2_to_f32<false>(bytes[a].sb1).x);
      }
    }
    if (h == 0 && ch + GI_SC < CHUNKS) stage_load(ch / GI_SC + 1);
    if (ch + AHEAD < CHUNKS) load_chunk(ch + AHEAD, bytes);
#pragma unroll
    for (int st = 0; st < 2; st++)
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        if (mt < tiles) {
          const int8_t* bp = bt + (mt * PL * 16 + c) * GI_PITCH + 128 * h + 32 * q + 16 * st;
          i32x4 b[PL];
#pragma unroll
          for (int t = 0; t < PL; t++) b[t] = *(const i32x4*)(bp + 16 * t * GI_PITCH);
#pragma unroll
          for (int a = 0; a < RA; a++)
#pragma unroll
            for (int t = 0; t < PL; t++) acc[a][mt][t] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[a][st], b[t], acc[a][mt][t], 0, 0, 0);
        }
      }
    if (h == GI_SC - 1 && ch + 1 < CHUNKS) {
      __syncthreads();  // every wave is done with this stage's rows
      stage_store();
      __syncthreads();
    }
  };
  ChunkBytes ring[AHEAD][RA];  // chunk ch's weight bytes in ring[ch % AHEAD]
  stage_load(0);
#pragma unroll
  for (int d = 0; d < AHEAD; d++) load_chunk(d, ring[d]);
  stage_store();
  __syncthreads();
  for (int ch = 0; ch < CHUNKS; ch += AHEAD) {
#pragma unroll
    for (int d = 0; d < AHEAD; d++) chunk(ch + d, d, ring[d]);
  }
  // lane l holds rows nw + 16 a + 4 q .. + 3 of activation row m0 + 16 mt + (l & 15)
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const int r = m0 + 16 * mt + c;
    if (mt < tiles && r < rows) {
      const float sx = xscale[plane_row(order, k_order, xrows, first + r)];
#pragma unroll
      for (int a = 0; a < RA; a++) {
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float mid = (float)acc[a][mt][1][i] + (float)acc[a][mt][2][i] / I8_RATIO;
          o[i] = es[a][i] * (sx * ((float)acc[a][mt][0][i] + mid / I8_RATIO));
        }
        *(f32x4*)(out + (size_t)(first + r) * N + nw + 16 * a + 4 * q) = o;
      }
    }
  }
}

// ------------------------------------------------------------------------------------ fused resident decode
// offload.py:108-123 resident_decode in two launches instead of five (rotate, gemv, rotate(SwiGLU), gemv,
// weighted_sum): banks held whole on the device (expert e in slot e), KIND 0 int8 (ConvRot), 1 fp8 (128 x 128 block
// scales), 4 / 6 codes (ConvRot). The same arithmetic per row as the separate kernels; the rotations move into the
// products' prologues (every workgroup rotates the row it needs, from L2, which costs far less than a launch).
//
// gate_up: grid (N / 16, k), workgroup (rows n0 .. n0 + 15, expert j): its rows' bytes are loaded first, then x
// (bf16) goes into LDS as float, rotated per 256 columns unless fp8, then 4 rows per wave: gu[j, n] = row . x (* row
// scale / channel scale; fp8 block scales folded into the activation slice).
// One lane's share of a row for the row-slice products: int8 / fp8 bytes (CPL per lane), or for codes the lane's
// 16-column groups (GPL of them: nibble words, 2-bit plane word, e4m3 scale byte). Loaded before anything the
// products wait for, so the weight stream starts at once.
template <int KIND, int K> struct RowBytes {
  static constexpr int CPL = K / 64, G = K / 16, GPL = (G + 63) / 64;
  uint32_t wd[KIND <= 1 ? CPL / 4 : 1];
  i32x2 lw[KIND <= 1 ? 1 : GPL];
  uint32_t high[KIND <= 1 ? 1 : GPL];
  uint32_t sb[KIND <= 1 ? 1 : GPL];
};

template <int KIND, int K>
D3_INLINE void load_row(RowBytes<KIND, K>& rb, const uint8_t* bw, const uint8_t* bs, size_t row, int lane) {
  using R = RowBytes<KIND, K>;
  if constexpr (KIND <= 1) {
    load_words<R::CPL>(bw + row * K + lane * R::CPL, rb.wd);
  } else {
    constexpr int RB = K * KIND / 8;
    const uint8_t* p = bw + row * RB;
#pragma unroll
    for (int i = 0; i < R::GPL; i++) {
      // lanes past the row's groups read its last group (branch-free loads; row_dot skips them)
      const int v = min(lane + 64 * i, R::G - 1);
      rb.lw[i] = *(const i32x2*)(p + 8 * v);
      rb.high[i] = KIND == 6 ? *(const uint32_t*)(p + K / 2 + 4 * v) : 0u;
      rb.sb[i] = bs[row * R::G + v];
    }
  }
}

// row . xs (LDS, K floats) for a row loaded by load_row; fp8 block scales of the row's 128-row block in `sblock`.
template <int KIND, int K>
D3_INLINE float row_dot(const RowBytes<KIND, K>& rb, const float* xs, const float* sblock, const float* lut,
                        int lane) {
  using R = RowBytes<KIND, K>;
  if constexpr (KIND <= 1) {
    float xv[R::CPL];
    const float xsum = load_slice<R::CPL>(xs, lane, xv);
    if constexpr (KIND == 1) {
#pragma unroll
      for (int i = 0; i < R::CPL; i++) xv[i] *= sblock[(lane * R::CPL + i) / 128];
      return dot_f8<R::CPL>(rb.wd, xv);
    } else {
      return dot_i8<R::CPL>(rb.wd, xv, xsum);
    }
  } else {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < R::GPL; i++) {
      const int v = lane + 64 * i;
      if (v < R::G) {
        float q[16];
        decode_group<KIND>((uint32_t)rb.lw[i].x, (uint32_t)rb.lw[i].y, rb.high[i], rb.sb[i], lut, q);
#pragma unroll
        for (int t = 0; t < 16; t++) acc = fmaf(q[t], xs[16 * v + t], acc);
      }
    }
    return acc;
  }
}

// the row's scale applied after the sum: int8 row scale, codes channel scale, fp8 none (folded into x)
template <int KIND> D3_INLINE float row_scale(const void* bs, const float* bc, size_t row) {
  if constexpr (KIND == 0) return ((const float*)bs)[row];
  else if constexpr (KIND == 1) return 1.0f;
  else return bc[row];
}

//
// gate_up: grid (I / 8, k), workgroup (hidden units u0 .. u0 + 7 of expert j): its 8 gate rows and the 8 matching up
// rows, a gate and an up row of two units per wave, so the workgroup ends with h[j, u] = SiLU(gate) * up itself and
// the down launch reads I floats per expert instead of 2I (the same float operations as rotate_rows' SwiGLU,
// kernels.py:236, or torch's silu for fp8, offload.py:115). x (bf16) is loaded first, then the weight rows, and x is
// rotated into LDS (per 256 columns unless fp8) while the rows stream: a wave's loads return in issue order, so x
// never waits behind the weights.
// A gate_up item's rows for one wave: the gate rows of units `unit`, `unit` + 1 of expert e and the matching up rows
// (rows e 2I + unit, + 1, e 2I + I + unit, + 1), their bytes and row scales, loaded before anything waits.
template <int KIND, int K> struct GuRows {
  RowBytes<KIND, K> rb[4];
  float sc[4];
  size_t rows[4];
};
template <int KIND, int K>
D3_INLINE void gu_load(GuRows<KIND, K>& g, const uint8_t* bw, const void* bs, const float* bc, size_t e, int I,
                       int unit, int lane) {
  const size_t N = 2 * (size_t)I;
  g.rows[0] = e * N + unit;
  g.rows[1] = e * N + unit + 1;
  g.rows[2] = e * N + I + unit;
  g.rows[3] = e * N + I + unit + 1;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    load_row<KIND, K>(g.rb[r], bw, (const uint8_t*)bs, g.rows[r], lane);
    g.sc[r] = row_scale<KIND>(bs, bc, g.rows[r]);
  }
}

// x (bf16, this wave's 256-column chunks w, w + 4, ... in xr: lane l holds columns 4l .. 4l + 3 of each) into LDS as
// float, rotated per 256 columns unless fp8
template <int KIND, int K>
D3_INLINE void x_to_lds(const i32x2* xr, float* xs, int w, int lane) {
#pragma unroll
  for (int c = 0; c < K / 1024; c++) {
    float v[4] = {bf16_to_f32((uint32_t)xr[c].x & 0xFFFFu), bf16_to_f32((uint32_t)xr[c].x >> 16),
                  bf16_to_f32((uint32_t)xr[c].y & 0xFFFFu), bf16_to_f32((uint32_t)xr[c].y >> 16)};
    if constexpr (KIND != 1) fwht256(v);
    *(f32x4*)(xs + 256 * (w + 4 * c) + 4 * lane) = f32x4{v[0], v[1], v[2], v[3]};
  }
}

// The item's hidden units: lane 0 gets SiLU(gate) * up of unit `unit`, lane 1 of unit + 1 (fp8: torch's silu as
// offload.py:115 applies it; the others: rotate_rows' SwiGLU, kernels.py:236). x is in LDS (xs), and at 4 bits the
// gate_up bank's code tables (qtab).
template <int KIND, int K>
D3_INLINE float gu_hidden(const GuRows<KIND, K>& g, const float* xs, const uint32_t* qtab, const float* lut,
                          const void* bs, int lane) {
  float y[4];
  if constexpr (KIND == 4) {
    // the lane's groups v = lane + 64 i of x, once for the four rows, and their sum (values enter as q + 128)
    using R = RowBytes<KIND, K>;
    float xv[R::GPL][16];
    float xsum = 0.0f;
#pragma unroll
    for (int i = 0; i < R::GPL; i++) xsum += load_slice<16>(xs + 16 * 64 * i, lane, xv[i]);
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < R::GPL; i++) {
        const i32x4 t = *(const i32x4*)(qtab + 4 * g.rb[r].sb[i]);
        acc += group_dot_w4((uint32_t)g.rb[r].lw[i].x, (uint32_t)g.rb[r].lw[i].y, t, xv[i]);
      }
      y[r] = wave_sum_f32(fmaf(-128.0f, xsum, acc)) * g.sc[r];
    }
  } else {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const float* sblock = KIND == 1 ? (const float*)bs + (g.rows[r] / 128) * (K / 128) : nullptr;
      y[r] = wave_sum_f32(row_dot<KIND, K>(g.rb[r], xs, sblock, lut, lane)) * g.sc[r];
    }
  }
  const float gt = lane ? y[1] : y[0], up = lane ? y[3] : y[2];
  const float sig = KIND == 1 ? 1.0f + expf(-gt) : 1.0f + __expf(-gt);
  return gt / sig * up;
}

// gu_hidden computed one row at a time (the same operations per row, so the same value, bit for bit), for a caller
// that holds other registers meanwhile; the rows are loaded here
template <int KIND, int K>
D3_INLINE float gu_hidden_lean(const uint8_t* bw, const void* bs, const float* bc, size_t e, int I, int unit,
                               const float* xs, const uint32_t* qtab, const float* lut, int lane) {
  const size_t N = 2 * (size_t)I;
  float y0 = 0.0f, y1 = 0.0f, y2 = 0.0f, y3 = 0.0f;
#pragma unroll 1
  for (int r = 0; r < 4; r++) {
    const size_t row = e * N + (r >= 2 ? I : 0) + unit + (r & 1);
    RowBytes<KIND, K> rb;
    load_row<KIND, K>(rb, bw, (const uint8_t*)bs, row, lane);
    const float sc = row_scale<KIND>(bs, bc, row);
    float v;
    if constexpr (KIND == 4) {
      using R = RowBytes<KIND, K>;
      float xsum = 0.0f, acc = 0.0f;
#pragma unroll
      for (int i = 0; i < R::GPL; i++) {
        float xv[16];
        xsum += load_slice<16>(xs + 16 * 64 * i, lane, xv);
        const i32x4 t = *(const i32x4*)(qtab + 4 * rb.sb[i]);
        acc += group_dot_w4((uint32_t)rb.lw[i].x, (uint32_t)rb.lw[i].y, t, xv);
      }
      v = wave_sum_f32(fmaf(-128.0f, xsum, acc)) * sc;
    } else {
      const float* sblock = KIND == 1 ? (const float*)bs + (row / 128) * (K / 128) : nullptr;
      v = wave_sum_f32(row_dot<KIND, K>(rb, xs, sblock, lut, lane)) * sc;
    }
    if (r == 0) y0 = v;
    else if (r == 1) y1 = v;
    else if (r == 2) y2 = v;
    else y3 = v;
  }
  const float gt = lane ? y1 : y0, up = lane ? y3 : y2;
  const float sig = KIND == 1 ? 1.0f + expf(-gt) : 1.0f + __expf(-gt);
  return gt / sig * up;
}

//
// ROUTED: every wave routes the row itself (kernels.py:39-67 on logits [n <= 256] bf16: the top keys and softmax
// weights as route_kernel computes them, the same key order, the exponentials summed in rank order), running the
// rounds up to its workgroup's rank j only; workgroup (0, k - 1), which runs all k, writes ids [k] and weights [k] for
// the down launch and the caller. `ids` is then unused. This saves route's own launch for callers that pass the
// router's logits.
constexpr int ROUTED_MAX_N = 256, GU_UNITS = 8;
template <int KIND, int K, int KPL, bool ROUTED>
__global__ void __launch_bounds__(256) resident_gu_kernel(const uint16_t* x, const int64_t* ids,
                                                          const uint16_t* logits, int n, int k, int64_t* ids_out,
                                                          float* w_out, const uint8_t* bw, const void* bs,
                                                          const float* bc, const float* codebook, float* h, int I) {
  constexpr int CH = K / 256 / 4;  // 256-column chunks of x per wave
  __shared__ float xs[K];
  __shared__ float lut[1];  // (row_dot reads a codebook only at 4 bits, which go through qtab here)
  __shared__ uint32_t qtab[KIND == 4 ? QTAB_WORDS : 1];
  const int j = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int unit = blockIdx.x * GU_UNITS + 2 * w;  // this wave's units: unit, unit + 1
  i32x2 xr[CH];
#pragma unroll
  for (int c = 0; c < CH; c++) xr[c] = *(const i32x2*)(x + 256 * (w + 4 * c) + 4 * lane);
  f32x4 cb = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (KIND == 4) cb = *(const f32x4*)(codebook + 4 * (threadIdx.x & 3));
  size_t e;
  if constexpr (ROUTED) {
    uint32_t lb[KPL];
#pragma unroll
    for (int q = 0; q < KPL; q++) lb[q] = logits[min(lane + 64 * q, n - 1)];  // lanes past n masked by TopKeys
    const bool writer = blockIdx.x == 0 && j == k - 1;
    TopKeys<KPL> tk(lb, lane, n);
    tk.rounds(lane, 0, j + 1);
    e = (size_t)route_key_index((uint32_t)__builtin_amdgcn_readlane((int)tk.mine, j));
    if (writer && w == 0) {  // uniform over the wave: route_weight reads lanes 0 .. k-1
      const float wt = route_weight(tk.mine, lane, k);
      if (lane < k) {
        ids_out[lane] = route_key_index(tk.mine);
        w_out[lane] = wt;
      }
    }
  } else {
    e = (size_t)ids[j];
  }
  GuRows<KIND, K> g;
  gu_load<KIND, K>(g, bw, bs, bc, e, I, unit, lane);
  x_to_lds<KIND, K>(xr, xs, w, lane);
  if constexpr (KIND == 4) build_qtab(qtab, cb);
  __syncthreads();
  const float hv = gu_hidden<KIND, K>(g, xs, qtab, lut, bs, lane);
  if (lane < 2) h[(size_t)j * I + unit + lane] = hv;
}

// down: grid (H / 4), workgroup (output rows m0 .. m0 + 3) for all k experts, so the routing-weighted sum stays in the
// workgroup. Each wave first loads its share of the k hidden rows h_j (I floats each, 256-column chunks), then its
// output row's bytes for every expert; the hidden chunks are rotated (unless fp8) into LDS while the rows stream, and
// a row per wave gives out[m] = bf16(sum_j w_j * (row . h_j) * scale), experts in order as weighted_sum sums them.
// (8 rows per workgroup, H / 8 = 256 of them, left one workgroup per CU: int8 25.5 against 24.2 us per layer, W4A8
// 30.7 against 26.8, fp8 26.9 against 25.0; 2 rows, in workgroups of two waves that each recompute the hidden rows:
// int8 27.7, W4A8 30.3, fp8 27.6.)
constexpr int DN_ROWS = 4, MAX_K_RES = 8;
template <int KIND, int K>
__global__ void __launch_bounds__(256) resident_dn_kernel(const float* h, const int64_t* ids, const float* wts, int k,
                                                          const uint8_t* bw, const void* bs, const float* bc,
                                                          const float* codebook, uint16_t* out, int H) {
  constexpr int RW = DN_ROWS / 4, CPE = K / 256, CH = MAX_K_RES * CPE / 4;  // chunks per expert, per wave
  __shared__ float hs[MAX_K_RES][K];
  __shared__ float lut[16];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, m0 = blockIdx.x * DN_ROWS;
  // the hidden chunks first (chunk c = w + 4 i: expert c / CPE, columns 256 (c % CPE) ..; past k: the last expert's,
  // loaded but not stored), so they return ahead of the weight rows
  f32x4 hv[CH];
#pragma unroll
  for (int i = 0; i < CH; i++) {
    const int c = w + 4 * i, jj = min(c / CPE, k - 1);
    hv[i] = *(const f32x4*)(h + (size_t)jj * K + 256 * (c % CPE) + 4 * lane);
  }
  RowBytes<KIND, K> rb[RW][MAX_K_RES];
  float sc[RW][MAX_K_RES];
  size_t ex[MAX_K_RES];
  // every expert slot up to MAX_K_RES loads a valid row (the last expert's again past k), without branches, so all
  // of a wave's loads are in flight together; the products skip the slots past k
#pragma unroll
  for (int j = 0; j < MAX_K_RES; j++) ex[j] = (size_t)ids[min(j, k - 1)];
#pragma unroll
  for (int r = 0; r < RW; r++)
#pragma unroll
    for (int j = 0; j < MAX_K_RES; j++) {
      const size_t row = ex[j] * H + m0 + w * RW + r;
      load_row<KIND, K>(rb[r][j], bw, (const uint8_t*)bs, row, lane);
      sc[r][j] = row_scale<KIND>(bs, bc, row);
    }
#pragma unroll
  for (int i = 0; i < CH; i++) {
    const int c = w + 4 * i;
    if (c < k * CPE) {
      float v[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w};
      if constexpr (KIND != 1) fwht256(v);
      *(f32x4*)(&hs[c / CPE][256 * (c % CPE) + 4 * lane]) = f32x4{v[0], v[1], v[2], v[3]};
    }
  }
  if (KIND == 4 && threadIdx.x < 16) lut[threadIdx.x] = codebook[threadIdx.x];
  __syncthreads();
#pragma unroll
  for (int r = 0; r < RW; r++) {
    const int m = m0 + w * RW + r;
    float total = 0.0f;
#pragma unroll
    for (int j = 0; j < MAX_K_RES; j++) {
      if (j < k) {
        const float* sblock = KIND == 1 ? (const float*)bs + ((ex[j] * H + m) / 128) * (K / 128) : nullptr;
        const float y = wave_sum_f32(row_dot<KIND, K>(rb[r][j], hs[j], sblock, lut, lane)) * sc[r][j];
        total = fmaf(y, wts[j], total);
      }
    }
    if (lane == 0) out[m] = (uint16_t)f32_to_bf16(total);
  }
}

// down for the code formats: W4 / W6 rows are short (I / 2 or 3I / 4 bytes, I / 16 scale groups), so a row takes 16
// lanes, each holding I / 256 of its groups, and a wave covers four experts' rows of its output row at once, in two
// passes over eight experts; a 16-lane row sum is four DPP steps. The hidden rows arrive and are rotated as in
// resident_dn_kernel; W4 decodes through qtab.
template <int KIND, int K>
__global__ void __launch_bounds__(256) resident_dn_codes_kernel(const float* h, const int64_t* ids, const float* wts,
                                                                int k, const uint8_t* bw, const uint8_t* bs,
                                                                const float* bc, const float* codebook,
                                                                uint16_t* out, int H) {
  constexpr int CPE = K / 256, CH = MAX_K_RES * CPE / 4, G = K / 16, GS = G / 16, RB = K * KIND / 8;
  static_assert(DN_ROWS == 4, "one output row per wave");
  __shared__ float hs[MAX_K_RES][K];
  __shared__ uint32_t qtab[KIND == 4 ? QTAB_WORDS : 1];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, seg = lane >> 4, li = lane & 15;
  const int m = blockIdx.x * DN_ROWS + w;
  f32x4 hv[CH];
#pragma unroll
  for (int i = 0; i < CH; i++) {
    const int c = w + 4 * i, jj = min(c / CPE, k - 1);
    hv[i] = *(const f32x4*)(h + (size_t)jj * K + 256 * (c % CPE) + 4 * lane);
  }
  f32x4 cb = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (KIND == 4) cb = *(const f32x4*)(codebook + 4 * (threadIdx.x & 3));
  // pass p: this lane's expert is 4 p + seg (the last routed one again past k), its groups li + 16 i
  size_t row[2];
#pragma unroll
  for (int p = 0; p < 2; p++) row[p] = (size_t)ids[min(4 * p + seg, k - 1)] * H + m;
  i32x2 lw[2][GS];
  uint32_t high[2][GS], sb[2][GS];
  float sc[2];
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const uint8_t* r = bw + row[p] * RB;
#pragma unroll
    for (int i = 0; i < GS; i++) {
      const int v = li + 16 * i;
      lw[p][i] = *(const i32x2*)(r + 8 * v);
      high[p][i] = KIND == 6 ? *(const uint32_t*)(r + K / 2 + 4 * v) : 0u;
      sb[p][i] = bs[row[p] * G + v];
    }
    sc[p] = bc[row[p]];
  }
#pragma unroll
  for (int i = 0; i < CH; i++) {
    const int c = w + 4 * i;
    if (c < k * CPE) {
      float v[4] = {hv[i].x, hv[i].y, hv[i].z, hv[i].w};
      fwht256(v);
      *(f32x4*)(&hs[c / CPE][256 * (c % CPE) + 4 * lane]) = f32x4{v[0], v[1], v[2], v[3]};
    }
  }
  if constexpr (KIND == 4) build_qtab(qtab, cb);
  __syncthreads();
  float y[2];
#pragma unroll
  for (int p = 0; p < 2; p++) {
    const float* hr = hs[min(4 * p + seg, k - 1)];
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < GS; i++) {
      float xv[16];
      const float xsum = load_slice<16>(hr + 256 * i, li, xv);  // values 16 (li + 16 i) ..
      if constexpr (KIND == 4) {
        const i32x4 t = *(const i32x4*)(qtab + 4 * sb[p][i]);
        acc += fmaf(-128.0f, xsum, group_dot_w4((uint32_t)lw[p][i].x, (uint32_t)lw[p][i].y, t, xv));
      } else {
        float q[16];
        decode_group<KIND>((uint32_t)lw[p][i].x, (uint32_t)lw[p][i].y, high[p][i], sb[p][i], nullptr, q);
#pragma unroll
        for (int t = 0; t < 16; t++) acc = fmaf(q[t], xv[t], acc);
      }
    }
    // the row's sum over its 16 lanes, in every lane of the row
    acc += __int_as_float(dpp_i32(__float_as_int(acc), 0xB1));
    acc += __int_as_float(dpp_i32(__float_as_int(acc), 0x4E));
    acc += __int_as_float(dpp_i32(__float_as_int(acc), 0x141));
    acc += __int_as_float(dpp_i32(__float_as_int(acc), 0x140));
    y[p] = acc * sc[p];
  }
  // out[m] = bf16(sum over the routed experts, in order, of w_j * y_j)
  float total = 0.0f;
#pragma unroll
  for (int j = 0; j < MAX_K_RES; j++) {
    if (j < k) total = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(y[j / 4]), 16 * (j % 4))), wts[j], total);
  }
  if (lane == 0) out[m] = (uint16_t)f32_to_bf16(total);
}

// ----------------------------------------------------------------------------- resident decode in one launch
// d3_resident_decode_fused: the resident decode (offload.py:108-123, after route, kernels.py:39-67, when routed) in one
// launch, with the two launches' arithmetic, bit for bit.
//   Workgroup i < k I / 8 computes the gate_up item (rank i / (I / 8), units 8 (i % (I / 8)) .. + 7) as
//   resident_gu_kernel does and publishes each wave's two hidden units as tagged words (value, launch epoch), written
//   and read device-coherently (common.hpp's hand-off: no counter or flag; a word's epoch tells a current one from a
//   stale one).
//   The last H / (4 RW) workgroups of the grid then each take a down block: output rows 4 RW b .. + 4 RW - 1 of every
//   routed expert, RW per wave. A down block requests its rows' bytes, then gathers the k hidden rows (stale words
//   read again, coherently, within spin_limit polls), rotates them into LDS and writes out[m] = bf16(sum_j w_j (row .
//   h_j) scale), experts in order, as resident_dn_kernel / resident_dn_codes_kernel do.
// No wait can block forever: the down blocks come last in the grid and every workgroup before a down block is a
// producer that waits for nothing, so each has started (workgroups start in grid order) and will finish. Waits are
// bounded anyway: one that gives up (the spin limit) makes its down block compute every hidden row itself with the
// gate_up items' own code (gu_load / gu_hidden), so the output is the same bit for bit; the launch's give-up word
// stops the other waits soon, and a sticky bit records it (d3_resident_status).
struct ResidentArgs {
  const uint16_t* x;
  const int64_t* ids;     // [k] (not routed)
  const float* wts;       // [k] (not routed)
  const uint16_t* logits; // [n] (routed)
  int n, k;
  int64_t* ids_out;       // [k] (routed)
  float* w_out;           // [k] (routed)
  const uint8_t* gw;
  const void* gs;
  const float* gc;
  const float* gcb;
  const uint8_t* dw;
  const void* ds;
  const float* dc;
  const float* dcb;
  uint16_t* out;
  int H, I;
  uint64_t* hidden;       // [k, I] tagged words
  uint64_t* status;       // the launch give-up word
  uint32_t* sticky;       // bit 0: a wait gave up and the block recomputed (output exact)
  uint32_t spin_limit;    // 0: every wait gives up at once (test hook)
  int items, dn_first;    // gate_up items (k I / 8); first down block
};
// workspace: the give-up word at byte 0, the sticky bits at byte 256, the hidden words from byte RES_HEADER
constexpr int RES_HEADER = 512, RES_STICKY = 256;

// one wave's down rows for the int8 / fp8 banks: RW output rows x MAX_K_RES experts (every slot loads a valid row, the
// last routed expert's again past k)
template <int KIND, int KI, int RW> struct DnRowsRef {
  RowBytes<KIND, KI> rb[RW][MAX_K_RES];
  float sc[RW][MAX_K_RES];
};
// the code formats: 2 RW passes of four 16-lane row segments (pass p: output row p / 2, expert 4 (p % 2) + lane / 16),
// each lane KI / 256 groups of its row
template <int KIND, int KI, int RW> struct DnRowsCodes {
  static constexpr int GS = KI / 256;
  i32x2 lw[2 * RW][GS];
  uint32_t high[2 * RW][GS], sb[2 * RW][GS];
  float sc[2 * RW];
};

template <int KIND, int K, int KI, int RW, int KPL, bool ROUTED>
__global__ void __launch_bounds__(256, 3) resident_fused_kernel(ResidentArgs a) {
  constexpr int CH = K / 1024, CPE = KI / 256, HCH = MAX_K_RES * CPE / 4;  // x chunks, hidden chunks per wave
  constexpr bool CODES = KIND == 4 || KIND == 6;
  __shared__ float xs[K];
  __shared__ float lut[1];  // (row_dot reads a codebook only at 4 bits, which go through qtab here)
  __shared__ uint32_t qtab[KIND == 4 ? QTAB_WORDS : 1];
  __shared__ float hs[MAX_K_RES][KI];
  __shared__ int gave_w[4];  // per wave: its wait gave up
  const int i = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6, k = a.k;
  const int T = KI / GU_UNITS, u = i / T, unit = (i % T) * GU_UNITS + 2 * w;
  const uint32_t epoch = launch_epoch();
  const int hb = i - a.dn_first;
  const bool has_item = i < a.items, has_down = hb >= 0;
  // ---- the gate_up item (x first, so it returns ahead of the weight rows)
  i32x2 xr[CH];
#pragma unroll
  for (int c = 0; c < CH; c++) xr[c] = *(const i32x2*)(a.x + 256 * (w + 4 * c) + 4 * lane);
  f32x4 cb = {0.0f, 0.0f, 0.0f, 0.0f};
  if constexpr (KIND == 4) cb = *(const f32x4*)(a.gcb + 4 * (threadIdx.x & 3));
  size_t e = 0;
  size_t ex[MAX_K_RES];  // the routed experts and their weights (down blocks)
  float wt[MAX_K_RES];
  int e_lane = 0;        // lane l: the expert of rank min(l % 8, k - 1) (down blocks)
  if constexpr (ROUTED) {
    uint32_t lb[KPL];
#pragma unroll
    for (int q = 0; q < KPL; q++) lb[q] = a.logits[min(lane + 64 * q, a.n - 1)];  // lanes past n masked by TopKeys
    TopKeys<KPL> tk(lb, lane, a.n);
    const int ur = has_item ? u : -1;
    tk.rounds(lane, 0, has_down ? k : ur + 1);
    if (has_item) e = (size_t)route_key_index((uint32_t)__builtin_amdgcn_readlane((int)tk.mine, u));
    if (has_down) {
      const float wl = route_weight(tk.mine, lane, k);  // uniform over the wave: reads lanes 0 .. k-1
#pragma unroll
      for (int j = 0; j < MAX_K_RES; j++) {
        ex[j] = (size_t)route_key_index((uint32_t)__builtin_amdgcn_readlane((int)tk.mine, min(j, k - 1)));
        wt[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), min(j, k - 1)));
      }
      e_lane = route_key_index((uint32_t)__shfl((int)tk.mine, min(lane & 7, k - 1)));
      if (hb == 0 && w == 0 && lane < k) {
        a.ids_out[lane] = route_key_index(tk.mine);
        a.w_out[lane] = wl;
      }
    }
  } else {
    if (has_item) e = (size_t)a.ids[u];
    if (has_down) {
#pragma unroll
      for (int j = 0; j < MAX_K_RES; j++) {
        ex[j] = (size_t)a.ids[min(j, k - 1)];
        wt[j] = a.wts[min(j, k - 1)];
      }
      e_lane = (int)a.ids[min(lane & 7, k - 1)];
    }
  }
  if (has_item) {
    GuRows<KIND, K> g;
    gu_load<KIND, K>(g, a.gw, a.gs, a.gc, e, KI, unit, lane);
    x_to_lds<KIND, K>(xr, xs, w, lane);
    if constexpr (KIND == 4) build_qtab(qtab, cb);
    __syncthreads();
    const float hv = gu_hidden<KIND, K>(g, xs, qtab, lut, a.gs, lane);
    if (lane < 2) put_tagged(a.hidden + (size_t)u * KI + unit + lane, hv, epoch);
  } else {
    x_to_lds<KIND, K>(xr, xs, w, lane);  // for a recomputation
    if constexpr (KIND == 4) build_qtab(qtab, cb);
  }
  if (!has_down) return;
  // ---- the down block: this wave's rows, requested once the gate_up item is done (requested earlier, they
  // compete with the items' rows, which every down block waits for: measured slower)
  const int m0 = 4 * RW * hb + RW * w;  // this wave's output rows m0 .. m0 + RW - 1
  const int seg = lane >> 4, li = lane & 15;
  DnRowsRef<KIND, KI, RW> dr;
  DnRowsCodes<KIND, KI, RW> dc;
  auto load_down = [&]() {
    if constexpr (CODES) {
      constexpr int RB = KI * KIND / 8, G = KI / 16;
#pragma unroll
      for (int p = 0; p < 2 * RW; p++) {
        const size_t ej = (size_t)__shfl(e_lane, 4 * (p & 1) + seg);  // this segment's expert
        const size_t row = ej * a.H + m0 + (p >> 1);
        const uint8_t* r = a.dw + row * RB;
#pragma unroll
        for (int g = 0; g < DnRowsCodes<KIND, KI, RW>::GS; g++) {
          const int v = li + 16 * g;
          dc.lw[p][g] = *(const i32x2*)(r + 8 * v);
          dc.high[p][g] = KIND == 6 ? *(const uint32_t*)(r + KI / 2 + 4 * v) : 0u;
          dc.sb[p][g] = ((const uint8_t*)a.ds)[row * G + v];
        }
        dc.sc[p] = a.dc[row];
      }
    } else {
#pragma unroll
      for (int r = 0; r < RW; r++)
#pragma unroll
        for (int j = 0; j < MAX_K_RES; j++) {
          const size_t row = ex[j] * a.H + m0 + r;
          load_row<KIND, KI>(dr.rb[r][j], a.dw, (const uint8_t*)a.ds, row, lane);
          dr.sc[r][j] = row_scale<KIND>(a.ds, a.dc, row);
        }
    }
  };
  load_down();
  // ---- this wave's hidden chunks c = w + 4 q: expert c / CPE, columns 256 (c % CPE) + 4 lane .. + 3 (chunks past k
  // read the last expert's again and are not stored); values kept, tags reduced to one stale bit per word
  auto hidden_src = [&](int q) {
    const int c = w + 4 * q, jj = min(c / CPE, k - 1);
    return a.hidden + (size_t)jj * KI + 256 * (c % CPE) + 4 * lane;
  };
  float hv[HCH][4];
  uint32_t stale = 0;
#pragma unroll
  for (int q = 0; q < HCH; q++) {
    const uint64_t* src = hidden_src(q);
#pragma unroll
    for (int t = 0; t < 4; t++) {
      const uint64_t word = get_tagged_cached(src + t);
      hv[q][t] = tagged_value(word);
      stale |= tag_is(word, epoch) ? 0u : 1u << (4 * q + t);
    }
  }
  bool gave = a.spin_limit == 0u;
  if (!gave) {
    uint32_t polls = 0;
    while (!__all(stale == 0u)) {
      if (!keep_polling(polls, a.status, a.spin_limit, epoch)) {
        gave = true;
        break;
      }
#pragma unroll
      for (int q = 0; q < HCH; q++) {
        const uint64_t* src = hidden_src(q);
#pragma unroll
        for (int t = 0; t < 4; t++) {
          if (stale & (1u << (4 * q + t))) {
            const uint64_t word = get_tagged(src + t);
            hv[q][t] = tagged_value(word);
            stale &= tag_is(word, epoch) ? ~(1u << (4 * q + t)) : ~0u;
          }
        }
      }
    }
  }
  if (lane == 0) gave_w[w] = gave;
  __syncthreads();
  if (gave_w[0] | gave_w[1] | gave_w[2] | gave_w[3]) {
    // a producer did not come in time: every hidden row this block needs, computed here with the gate_up items' own
    // code (x, and at 4 bits the gate_up bank's tables, are still in LDS), raw into hs, then rotated in place
    if (threadIdx.x == 0) __hip_atomic_fetch_or(a.sticky, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll 1
    for (int j = 0; j < k; j++) {
      size_t ej = ex[0];  // (selected, not indexed: ex stays in registers)
#pragma unroll
      for (int q = 1; q < MAX_K_RES; q++) ej = j == q ? ex[q] : ej;
#pragma unroll 1
      for (int t = 0; t < T; t++) {
        const float h = gu_hidden_lean<KIND, K>(a.gw, a.gs, a.gc, ej, KI, t * GU_UNITS + 2 * w, xs, qtab, lut, lane);
        if (lane < 2) hs[j][t * GU_UNITS + 2 * w + lane] = h;
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < HCH; q++) {
      const int c = w + 4 * q;
      if (c < k * CPE) {
        float* dst = &hs[c / CPE][256 * (c % CPE) + 4 * lane];
        const f32x4 r = *(const f32x4*)dst;
        float v[4] = {r.x, r.y, r.z, r.w};
        if constexpr (KIND != 1) fwht256(v);
        *(f32x4*)dst = f32x4{v[0], v[1], v[2], v[3]};
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < HCH; q++) {
      const int c = w + 4 * q;
      if (c < k * CPE) {
        float v[4] = {hv[q][0], hv[q][1], hv[q][2], hv[q][3]};
        if constexpr (KIND != 1) fwht256(v);
        *(f32x4*)(&hs[c / CPE][256 * (c % CPE) + 4 * lane]) = f32x4{v[0], v[1], v[2], v[3]};
      }
    }
  }
  __syncthreads();  // every hidden row in hs; the gate_up bank's tables no longer read
  if constexpr (KIND == 4) {
    build_qtab(qtab, *(const f32x4*)(a.dcb + 4 * (threadIdx.x & 3)));
    __syncthreads();
  }
  // ---- the products and the weighted sum, as the two-launch down kernels compute them
  if constexpr (CODES) {
    constexpr int GS = DnRowsCodes<KIND, KI, RW>::GS;
    float y[2 * RW];
#pragma unroll
    for (int p = 0; p < 2 * RW; p++) {
      const float* hr = hs[min(4 * (p & 1) + seg, k - 1)];
      float acc = 0.0f;
#pragma unroll
      for (int g = 0; g < GS; g++) {
        float xv[16];
        const float xsum = load_slice<16>(hr + 256 * g, li, xv);
        if constexpr (KIND == 4) {
          const i32x4 t = *(const i32x4*)(qtab + 4 * dc.sb[p][g]);
          acc += fmaf(-128.0f, xsum, group_dot_w4((uint32_t)dc.lw[p][g].x, (uint32_t)dc.lw[p][g].y, t, xv));
        } else {
          float qv[16];
          decode_group<KIND>((uint32_t)dc.lw[p][g].x, (uint32_t)dc.lw[p][g].y, dc.high[p][g], dc.sb[p][g], nullptr,
                             qv);
#pragma unroll
          for (int t = 0; t < 16; t++) acc = fmaf(qv[t], xv[t], acc);
        }
      }
      acc += __int_as_float(dpp_i32(__float_as_int(acc), 0xB1));
      acc += __int_as_float(dpp_i32(__float_as_int(acc), 0x4E));
      acc += __int_as_float(dpp_i32(__float_as_int(acc), 0x141));
      acc += __int_as_float(dpp_i32(__float_as_int(acc), 0x140));
      y[p] = acc * dc.sc[p];
    }
#pragma unroll
    for (int r = 0; r < RW; r++) {
      float total = 0.0f;
#pragma unroll
      for (int j = 0; j < MAX_K_RES; j++)
        if (j < k)
          total = fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(y[2 * r + j / 4]), 16 * (j % 4))),
                       wt[j], total);
      if (lane == 0) a.out[m0 + r] = (uint16_t)f32_to_bf16(total);
    }
  } else {
#pragma unroll
    for (int r = 0; r < RW; r++) {
      float total = 0.0f;
#pragma unroll
      for (int j = 0; j < MAX_K_RES; j++) {
        if (j < k) {
          const float* sblock =
              KIND == 1 ? (const float*)a.ds + ((ex[j] * a.H + m0 + r) / 128) * (KI / 128) : nullptr;
          const float y = wave_sum_f32(row_dot<KIND, KI>(dr.rb[r][j], hs[j], sblock, lut, lane)) * dr.sc[r][j];
          total = fmaf(y, wt[j], total);
        }
      }
      if (lane == 0) a.out[m0 + r] = (uint16_t)f32_to_bf16(total);
    }
  }
}

// Check of the decodes above on their own: one thread per (row, 16-column group) writes the int8-grid values, through
// decode_group (TABLE false: the GEMVs' and grouped products' decode) or through qtab (TABLE true, 4 bits: the resident
// kernels' decode).
template <int BITS, bool TABLE>
__global__ void __launch_bounds__(256) decode_codes_kernel(const uint8_t* rows, const uint8_t* scales,
                                                           const float* codebook, int R, int K, int8_t* out) {
  __shared__ float lut[16];
  __shared__ uint32_t qtab[TABLE ? QTAB_WORDS : 1];
  if (BITS == 4 && threadIdx.x < 16) lut[threadIdx.x] = codebook[threadIdx.x];
  if constexpr (TABLE) build_qtab(qtab, *(const f32x4*)(codebook + 4 * (threadIdx.x & 3)));
  __syncthreads();
  const int G = K / 16;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)R * G) return;
  const int r = (int)(idx / G), v = (int)(idx % G);
  const uint8_t* row = rows + (size_t)r * (K * BITS / 8);
  const i32x2 lw = *(const i32x2*)(row + 8 * v);
  const uint32_t sb = scales[(size_t)r * G + v];
  int8_t* o = out + (size_t)r * K + 16 * v;
  if constexpr (TABLE) {
    const i32x4 t = *(const i32x4*)(qtab + 4 * sb);
#pragma unroll
    for (int d = 0; d < 2; d++) {
      const uint32_t word = d ? (uint32_t)lw.y : (uint32_t)lw.x;
      const uint32_t ev = lookup16(t, word & 0x0F0F0F0Fu) ^ 0x80808080u;  // values 8d + 0, 2, 4, 6 as int8
      const uint32_t od = lookup16(t, (word >> 4) & 0x0F0F0F0Fu) ^ 0x80808080u;
      *(uint32_t*)(o + 8 * d) = __builtin_amdgcn_perm(od, ev, 0x05010400u);
      *(uint32_t*)(o + 8 * d + 4) = __builtin_amdgcn_perm(od, ev, 0x07030602u);
    }
  } else {
    const uint32_t high = BITS == 6 ? *(const uint32_t*)(row + K / 2 + 4 * v) : 0u;
    float q[16];
    decode_group<BITS>((uint32_t)lw.x, (uint32_t)lw.y, high, sb, lut, q);
#pragma unroll
    for (int j = 0; j < 16; j++) o[j] = (int8_t)(int)q[j];
  }
}

}  // namespace d3

// ============================================================================================================ C ABI
using namespace d3;

namespace {
template <template <int> class KT> struct None {};

hipError_t last() { return hipGetLastError(); }
int done(const char* what) {
  const hipError_t e = last();
  return e == hipSuccess ? 0 : hip_fail(e, what);
}
bool supported_k(int K) { return K == 256 || K == 512 || K == 768 || K == 1024 || K == 1536 || K == 2048; }
}  // namespace

#define D3_K_SWITCH(K, CALL)                          \
  switch (K) {                                        \
    case 256: { constexpr int KK = 256; CALL; } break;  \
    case 512: { constexpr int KK = 512; CALL; } break;  \
    case 768: { constexpr int KK = 768; CALL; } break;  \
    case 1024: { constexpr int KK = 1024; CALL; } break; \
    case 1536: { constexpr int KK = 1536; CALL; } break; \
    case 2048: { constexpr int KK = 2048; CALL; } break; \
    default: break;                                   \
  }

extern "C" {

int d3_route(const void* logits, int32_t rows, int32_t n, int32_t k, int64_t* ids, float* weights, void* stream) {
  if (!logits || !ids || !weights) return fail("d3_route: null pointer");
  if (rows < 1 || n < 1 || n > 1024 || k < 1 || k > 32 || k > n) return fail("d3_route: n <= 1024, 1 <= k <= min(32, n)");
  const dim3 grid((rows + 3) / 4);
  const hipStream_t s = (hipStream_t)stream;
  const uint16_t* lg = (const uint16_t*)logits;
  if (n <= 64) hipLaunchKernelGGL(route_kernel<1>, grid, dim3(256), 0, s, lg, rows, n, k, ids, weights);
  else if (n <= 128) hipLaunchKernelGGL(route_kernel<2>, grid, dim3(256), 0, s, lg, rows, n, k, ids, weights);
  else if (n <= 256) hipLaunchKernelGGL(route_kernel<4>, grid, dim3(256), 0, s, lg, rows, n, k, ids, weights);
  else if (n <= 512) hipLaunchKernelGGL(route_kernel<8>, grid, dim3(256), 0, s, lg, rows, n, k, ids, weights);
  else hipLaunchKernelGGL(route_kernel<16>, grid, dim3(256), 0, s, lg, rows, n, k, ids, weights);
  return done("d3_route");
}

int d3_weighted_sum(const float* parts, const float* weights, int32_t k, int32_t H, void* out, void* stream) {
  if (!parts || !weights || !out) return fail("d3_weighted_sum: null pointer");
  if (k < 1 || H < 1) return fail("d3_weighted_sum: k, H >= 1");
  hipLaunchKernelGGL(weighted_sum_kernel, dim3((H + 255) / 256), dim3(256), 0, (hipStream_t)stream, parts, weights, k, H,
                     (uint16_t*)out);
  return done("d3_weighted_sum");
}

int d3_rotate(const void* x, int32_t mode, int32_t rows, int32_t K, float* out, const int32_t* only_if, void* stream) {
  if (!x || !out || !only_if) return fail("d3_rotate: null pointer");
  if (rows < 1 || K < 256 || K % 256 || K > 4096) return fail("d3_rotate: K % 256 == 0, K <= 4096");
  const hipStream_t s = (hipStream_t)stream;
  switch (mode) {
    case 0: hipLaunchKernelGGL(rotate_kernel<0>, dim3(rows), dim3(256), 0, s, x, K, out, only_if); break;
    case 1: hipLaunchKernelGGL(rotate_kernel<1>, dim3(rows), dim3(256), 0, s, x, K, out, only_if); break;
    case 2: hipLaunchKernelGGL(rotate_kernel<2>, dim3(rows), dim3(256), 0, s, x, K, out, only_if); break;
    default: return fail("d3_rotate: mode 0 (float), 1 (bf16) or 2 (swiglu)");
  }
  return done("d3_rotate");
}

int d3_gemv_int8(const float* x, int32_t x_rows, const int64_t* ids, const int32_t* plan, const int32_t* took_over,
                 int32_t late, void* slot_w, float* slot_s, const void* host_w, const float* host_s, float* out,
                 int32_t k, int32_t N, int32_t K, void* stream) {
  if (!x || !ids || !plan || !took_over || !slot_w || !slot_s || !host_w || !host_s || !out)
    return fail("d3_gemv_int8: null pointer");
  if (k < 1 || N < RPB || N % RPB || !supported_k(K)) return fail("d3_gemv_int8: N % 16 == 0, K in {256..2048}");
  const dim3 grid(N / RPB, k);
  D3_K_SWITCH(K, hipLaunchKernelGGL(gemv_int8_kernel<KK>, grid, dim3(256), 0, (hipStream_t)stream, x, x_rows, ids, plan,
                                    took_over, late, (uint8_t*)slot_w, slot_s, (const uint8_t*)host_w, host_s, out, N));
  return done("d3_gemv_int8");
}

int d3_gemv_fp8(const float* x, int32_t x_rows, const int64_t* ids, const int32_t* plan, void* slot_w, float* slot_s,
                const void* host_w, const float* host_s, float* out, int32_t k, int32_t N, int32_t K, void* stream) {
  if (!x || !ids || !plan || !slot_w || !slot_s || !host_w || !host_s || !out) return fail("d3_gemv_fp8: null pointer");
  if (k < 1 || N < 128 || N % 128 || !supported_k(K)) return fail("d3_gemv_fp8: N % 128 == 0, K in {256..2048}");
  const dim3 grid(N / RPB, k);
  D3_K_SWITCH(K, hipLaunchKernelGGL(gemv_fp8_kernel<KK>, grid, dim3(256), 0, (hipStream_t)stream, x, x_rows, ids, plan,
                                    (uint8_t*)slot_w, slot_s, (const uint8_t*)host_w, host_s, out, N));
  return done("d3_gemv_fp8");
}

int d3_gemv_codes(const float* x, int32_t x_rows, const int64_t* ids, const int32_t* plan, void* slot_w, void* slot_r,
                  float* slot_c, const void* host_w, const void* host_r, const float* host_c, const float* codebook,
                  int32_t bits, float* out, int32_t k, int32_t N, int32_t K, void* stream) {
  if (!x || !ids || !plan || !slot_w || !slot_r || !slot_c || !host_w || !host_r || !host_c || !out)
    return fail("d3_gemv_codes: null pointer");
  if (bits == 4 && !codebook) return fail("d3_gemv_codes: 4 bits need a codebook");
  if (k < 1 || N < RPB || N % RPB || !supported_k(K) || (bits != 4 && bits != 6))
    return fail("d3_gemv_codes: N % 16 == 0, K in {256..2048}, bits 4 or 6");
  const dim3 grid(N / RPB, k);
  const hipStream_t s = (hipStream_t)stream;
  if (bits == 4) {
    D3_K_SWITCH(K, hipLaunchKernelGGL((gemv_codes_kernel<KK, 4>), grid, dim3(256), 0, s, x, x_rows, ids, plan,
                                      (uint8_t*)slot_w, (uint8_t*)slot_r, slot_c, (const uint8_t*)host_w,
                                      (const uint8_t*)host_r, host_c, codebook, out, N));
  } else {
    D3_K_SWITCH(K, hipLaunchKernelGGL((gemv_codes_kernel<KK, 6>), grid, dim3(256), 0, s, x, x_rows, ids, plan,
                                      (uint8_t*)slot_w, (uint8_t*)slot_r, slot_c, (const uint8_t*)host_w,
                                      (const uint8_t*)host_r, host_c, codebook, out, N));
  }
  return done("d3_gemv_codes");
}

// kind: 0 int8 (scale float [E * N]), 1 fp8 (scale float [E * N / 128, K / 128]), 4 / 6 codes (scale e4m3 [E * N, K / 16],
// channel float [E * N])
int d3_grouped(int32_t kind, const float* x, const int32_t* groups, int32_t n_groups, void* slot_w, void* slot_s,
               void* slot_c, const void* host_w, const void* host_s, const void* host_c, const float* codebook,
               float* out, int32_t N, int32_t K, void* stream) {
  if (!x || !groups || !slot_w || !slot_s || !host_w || !host_s || !out) return fail("d3_grouped: null pointer");
  if ((kind == 4 || kind == 6) && (!slot_c || !host_c)) return fail("d3_grouped: codes need channel scales");
  if (kind == 4 && !codebook) return fail("d3_grouped: 4 bits need a codebook");
  if (n_groups < 1) return 0;
  if (N < RPB || N % (kind == 1 ? 128 : RPB) || !supported_k(K))
    return fail("d3_grouped: N % 16 == 0 (N % 128 == 0 for fp8), K in {256..2048}");
  const hipStream_t s = (hipStream_t)stream;
  const uint8_t* hw = (const uint8_t*)host_w;
  uint8_t* sw = (uint8_t*)slot_w;
  const dim3 grid(N / RPB, n_groups);
  switch (kind) {
    case 0: D3_K_SWITCH(K, hipLaunchKernelGGL((grouped_kernel<0, KK>), grid, dim3(256), 0, s, x, groups, sw, slot_s, slot_c, hw, host_s, host_c, codebook, out, N)); break;
    case 1: D3_K_SWITCH(K, hipLaunchKernelGGL((grouped_kernel<1, KK>), grid, dim3(256), 0, s, x, groups, sw, slot_s, slot_c, hw, host_s, host_c, codebook, out, N)); break;
    case 4: D3_K_SWITCH(K, hipLaunchKernelGGL((grouped_kernel<4, KK>), grid, dim3(256), 0, s, x, groups, sw, slot_s, slot_c, hw, host_s, host_c, codebook, out, N)); break;
    case 6: D3_K_SWITCH(K, hipLaunchKernelGGL((grouped_kernel<6, KK>), grid, dim3(256), 0, s, x, groups, sw, slot_s, slot_c, hw, host_s, host_c, codebook, out, N)); break;
    default: return fail("d3_grouped: kind 0, 1, 4 or 6");
  }
  return done("d3_grouped");
}

int d3_split_bf16x3(const float* x, int64_t n, void* planes, void* stream) {
  if (!x || !planes) return fail("d3_split_bf16x3: null pointer");
  if (n < 8 || n % 8) return fail("d3_split_bf16x3: n a positive multiple of 8");
  const int64_t n8 = n / 8;
  const int grid = (int)std::min<int64_t>((n8 + 255) / 256, 8192);
  bf16x8* p = (bf16x8*)planes;
  hipLaunchKernelGGL(split3_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, x, n8, p, p + n8, p + 2 * n8);
  return done("d3_split_bf16x3");
}

int64_t d3_grouped_mfma_work_ints(int32_t n_groups, int64_t rows) {
  const int64_t cap = (rows + GM_ROWS - 1) / GM_ROWS + std::max(n_groups, 0);
  return 2 + 2 * ((cap + 7) / 8 * 8);
}

int d3_grouped_plan(const int32_t* groups, int32_t n_groups, int64_t rows, int32_t* work, int64_t work_ints,
                    void* stream) {
  if (!groups || !work) return fail("d3_grouped_plan: null pointer");
  if (n_groups < 1 || rows < 0 || rows > INT32_MAX) return fail("d3_grouped_plan: n_groups >= 1, 0 <= rows < 2^31");
  const int64_t need = d3_grouped_mfma_work_ints(n_groups, rows);
  if (work_ints < need) return fail("d3_grouped_plan: work holds fewer than d3_grouped_mfma_work_ints ints");
  hipLaunchKernelGGL(grouped_plan_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, groups, n_groups, (int)rows,
                     work, (int)((need - 2) / 2));
  return done("d3_grouped_plan");
}

// the planes' rows and the pass rows' checks shared by d3_grouped_fp8 and d3_grouped_i8; 0 when they fit
static int check_rows(const char* what, int64_t plane, int32_t K, const int64_t* order, int32_t k, int32_t rows) {
  if (!supported_k(K) || plane < K || plane % K || plane / K > INT32_MAX)
    return fail(std::string(what) + ": K in {256..2048}, plane a multiple of K, under 2^31 rows");
  if (rows < 1 || (order ? k < 1 : rows > plane / K))
    return fail(std::string(what) + ": 1 <= rows (<= plane / K without order), k >= 1 with order");
  return 0;
}

int d3_expert_groups_prep_i8(const int64_t* ids, int32_t P, int32_t E, int64_t* order, int32_t* inverse,
                             int32_t* groups, int32_t* work, int64_t work_ints, int32_t mode, int32_t rotate,
                             const void* x, int32_t T, int32_t K, void* planes, float* scales, void* stream) {
  if (!groups || !work || (P > 0 && (!ids || !order || !inverse))) return fail("d3_expert_groups_prep_i8: null pointer");
  if (P < 0 || E < 1 || E > GROUPS_MAX_E) return fail("d3_expert_groups_prep_i8: 1 <= E <= 1024, P >= 0");
  if (T > 0 && (!x || !planes || !scales)) return fail("d3_expert_groups_prep_i8: null pointer");
  if (T < 0 || (mode != 0 && mode != 1) || !supported_k(K))
    return fail("d3_expert_groups_prep_i8: T >= 0, mode 0 (float32 rows) or 1 (bf16 rows), K in {256..2048}");
  const int64_t need = d3_grouped_mfma_work_ints(E, P);
  if (work_ints < need) return fail("d3_expert_groups_prep_i8: work holds fewer than d3_grouped_mfma_work_ints ints");
  const int cap = (int)((need - 2) / 2);
  const hipStream_t s = (hipStream_t)stream;
  const dim3 grid(1 + (T + 3) / 4);
  int8_t* pl = (int8_t*)planes;
#define D3_GP(M, R) hipLaunchKernelGGL((groups_prep_kernel<M, R>), grid, dim3(1024), 0, s, ids, P, E, order, inverse, groups, work, cap, x, T, K, pl, scales)
  switch (mode * 2 + (rotate ? 1 : 0)) {
    case 0: D3_GP(0, false); break;
    case 1: D3_GP(0, true); break;
    case 2: D3_GP(1, false); break;
    default: D3_GP(1, true); break;
  }
#undef D3_GP
  return done("d3_expert_groups_prep_i8");
}

int d3_grouped_fp8(const void* planes, int32_t n_planes, int64_t plane, const int64_t* order, int32_t k,
                   int32_t rows, const int32_t* groups, int32_t n_groups, const int32_t* work, int64_t work_ints,
                   int32_t fills_first, void* slot_w, void* slot_s, const void* host_w, const void* host_s,
                   float* out, int32_t N, int32_t K, void* stream) {
  if (!planes || !groups || !work || !slot_w || !slot_s || !host_w || !host_s || !out)
    return fail("d3_grouped_fp8: null pointer");
  if (n_planes != 1 && n_planes != 3) return fail("d3_grouped_fp8: 1 or 3 planes");
  if (n_groups < 1) return 0;
  if (N < 128 || N % 128) return fail("d3_grouped_fp8: N % 128 == 0");
  if (const int e = check_rows("d3_grouped_fp8", plane, K, order, k, rows)) return e;
  const int xrows = (int)(plane / K);
  const int64_t need = d3_grouped_mfma_work_ints(n_groups, rows);
  if (work_ints < need) return fail("d3_grouped_fp8: work holds fewer than d3_grouped_mfma_work_ints ints");
  const int cap = (int)((need - 2) / 2), firsts = (n_groups + 7) / 8 * 8;
  const hipStream_t s = (hipStream_t)stream;
  const __bf16* xs = (const __bf16*)planes;
  const uint8_t* hw = (const uint8_t*)host_w;
  uint8_t* sw = (uint8_t*)slot_w;
  float* ss = (float*)slot_s;
  const float* hs = (const float*)host_s;
  // two 16-row tiles per wave
#define D3_GF(PL, PH, Y) D3_K_SWITCH(K, hipLaunchKernelGGL((grouped_fp8_kernel<KK, 2, PL>), dim3(N / 128, Y), dim3(256), 0, s, xs, plane, order, k, xrows, groups, work, PH, sw, ss, hw, hs, out, N))
#define D3_GF_PL(PH, Y) \
  if (n_planes == 1) { D3_GF(1, PH, Y); } else { D3_GF(3, PH, Y); }
  if (fills_first) {
    D3_GF_PL(0, firsts);
    D3_GF_PL(1, cap);
  } else {
    D3_GF_PL(2, cap);
  }
#undef D3_GF_PL
#undef D3_GF
  return done("d3_grouped_fp8");
}

int d3_expert_groups(const int64_t* ids, int32_t P, int32_t E, int64_t* order, int32_t* inverse, int32_t* groups,
                     int32_t* work, int64_t work_ints, void* stream) {
  if (!groups || (P > 0 && (!ids || !order || !inverse))) return fail("d3_expert_groups: null pointer");
  if (P < 0 || E < 1 || E > GROUPS_MAX_E) return fail("d3_expert_groups: 1 <= E <= 1024, P >= 0");
  int cap = 0;
  if (work) {
    const int64_t need = d3_grouped_mfma_work_ints(E, P);
    if (work_ints < need) return fail("d3_expert_groups: work holds fewer than d3_grouped_mfma_work_ints ints");
    cap = (int)((need - 2) / 2);
  }
  hipLaunchKernelGGL(expert_groups_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, ids, P, E, order, inverse,
                     groups, work, cap);
  return done("d3_expert_groups");
}

int d3_prep_planes(int32_t mode, int32_t rotate, int32_t n_planes, const void* x, const int64_t* order, int32_t k,
                   int32_t P, int32_t K, void* planes, void* stream) {
  if (P > 0 && (!x || !planes)) return fail("d3_prep_planes: null pointer");
  if (mode < 0 || mode > 2 || P < 0 || k < 1 || !supported_k(K)) return fail("d3_prep_planes: mode 0-2, K in {256..2048}");
  if (n_planes != 3 && !(n_planes == 1 && mode == 1 && !rotate))
    return fail("d3_prep_planes: 3 planes, or 1 for bf16 rows taken as they are");
  if (P == 0) return 0;
  const hipStream_t s = (hipStream_t)stream;
  const int64_t plane = (int64_t)P * K;
  __bf16* out = (__bf16*)planes;
#define D3_PREP(M, R, PL) hipLaunchKernelGGL((prep_planes_kernel<M, R, PL>), dim3(P), dim3(256), 0, s, x, order, k, K, out, plane)
  if (n_planes == 1) {
    D3_PREP(1, false, 1);
  } else {
    switch (mode * 2 + (rotate ? 1 : 0)) {
      case 0: D3_PREP(0, false, 3); break;
      case 1: D3_PREP(0, true, 3); break;
      case 2: D3_PREP(1, false, 3); break;
      case 3: D3_PREP(1, true, 3); break;
      case 4: D3_PREP(2, false, 3); break;
      default: D3_PREP(2, true, 3); break;
    }
  }
#undef D3_PREP
  return done("d3_prep_planes");
}

int d3_prep_planes_i8(int32_t mode, int32_t rotate, const void* x, const int64_t* order, int32_t k, int32_t P,
                      int32_t K, void* planes, float* scales, void* stream) {
  if (P > 0 && (!x || !planes || !scales)) return fail("d3_prep_planes_i8: null pointer");
  if (mode < 0 || mode > 2 || P < 0 || k < 1 || !supported_k(K))
    return fail("d3_prep_planes_i8: mode 0-2, K in {256..2048}");
  if (P == 0) return 0;
  const hipStream_t s = (hipStream_t)stream;
  const int64_t plane = (int64_t)P * K;
  int8_t* out = (int8_t*)planes;
#define D3_PREP(M, R) hipLaunchKernelGGL((prep_i8_kernel<M, R>), dim3(P), dim3(256), 0, s, x, order, k, K, out, plane, scales)
  switch (mode * 2 + (rotate ? 1 : 0)) {
    case 0: D3_PREP(0, false); break;
    case 1: D3_PREP(0, true); break;
    case 2: D3_PREP(1, false); break;
    case 3: D3_PREP(1, true); break;
    case 4: D3_PREP(2, false); break;
    default: D3_PREP(2, true); break;
  }
#undef D3_PREP
  return done("d3_prep_planes_i8");
}

int d3_grouped_i8(int32_t kind, const void* planes, const float* scales, int64_t plane, const int64_t* order,
                  int32_t k, int32_t rows, const int32_t* groups, int32_t n_groups, const int32_t* work,
                  int64_t work_ints, int32_t fills_first, void* slot_w, void* slot_s, void* slot_c,
                  const void* host_w, const void* host_s, const void* host_c, const float* codebook, float* out,
                  int32_t N, int32_t K, void* stream) {
  if (!planes || !scales || !groups || !work || !slot_w || !slot_s || !host_w || !host_s || !out)
    return fail("d3_grouped_i8: null pointer");
  if (kind != 0 && kind != 4 && kind != 6) return fail("d3_grouped_i8: kind 0, 4 or 6");
  if (kind != 0 && (!slot_c || !host_c)) return fail("d3_grouped_i8: codes need channel scales");
  if (kind == 4 && !codebook) return fail("d3_grouped_i8: 4 bits need a codebook");
  if (n_groups < 1) return 0;
  if (N < 64 || N % 64) return fail("d3_grouped_i8: N % 64 == 0");
  if (const int e = check_rows("d3_grouped_i8", plane, K, order, k, rows)) return e;
  const int xrows = (int)(plane / K);
  const int64_t need = d3_grouped_mfma_work_ints(n_groups, rows);
  if (work_ints < need) return fail("d3_grouped_i8: work holds fewer than d3_grouped_mfma_work_ints ints");
  const int cap = (int)((need - 2) / 2), firsts = (n_groups + 7) / 8 * 8;
  const hipStream_t s = (hipStream_t)stream;
  const int8_t* xs = (const int8_t*)planes;
  const uint8_t* hw = (const uint8_t*)host_w;
  uint8_t* sw = (uint8_t*)slot_w;
#define D3_GI(KD, RA, PH, Y) D3_K_SWITCH(K, hipLaunchKernelGGL((grouped_i8_kernel<KD, KK, RA>), dim3(N / (64 * RA), Y), dim3(256), 0, s, xs, plane, scales, order, k, xrows, groups, work, PH, sw, slot_s, slot_c, hw, host_s, host_c, codebook, out, N))
// int8: two 16-row tiles per wave where N allows; the codes one (their decode takes the registers and the vector
// unit: more waves per SIMD hide it better)
#define D3_GI_KIND(PH, Y)                                                           \
  switch (kind) {                                                                   \
    case 0:                                                                         \
      if (N % 128 == 0) { D3_GI(0, 2, PH, Y); } else { D3_GI(0, 1, PH, Y); }         \
      break;                                                                        \
    case 4: D3_GI(4, 1, PH, Y); break;                                              \
    default: D3_GI(6, 1, PH, Y); break;                                             \
  }
  if (fills_first) {
    D3_GI_KIND(0, firsts);
    D3_GI_KIND(1, cap);
  } else {
    D3_GI_KIND(2, cap);
  }
#undef D3_GI_KIND
#undef D3_GI
  return done("d3_grouped_i8");
}

int d3_combine_rows(const float* sorted_out, const int32_t* inverse, const void* weights, int32_t weights_bf16,
                    int32_t T, int32_t k, int32_t H, void* out, int32_t out_type, void* stream) {
  if (T > 0 && (!sorted_out || !inverse || !weights || !out)) return fail("d3_combine_rows: null pointer");
  if (T < 0 || k < 1 || H < 4 || H % 4 || out_type < 0 || out_type > 2)
    return fail("d3_combine_rows: H % 4 == 0, out_type 0 float32, 1 bf16, 2 fp16");
  if (T == 0) return 0;
  const dim3 grid((H / 4 + 255) / 256, T);
  const hipStream_t s = (hipStream_t)stream;
  if (weights_bf16)
    hipLaunchKernelGGL(combine_rows_kernel<true>, grid, dim3(256), 0, s, sorted_out, inverse, weights, k, H, out, out_type);
  else
    hipLaunchKernelGGL(combine_rows_kernel<false>, grid, dim3(256), 0, s, sorted_out, inverse, weights, k, H, out, out_type);
  return done("d3_combine_rows");
}

}  // extern "C"

// Both resident entries: gate_up (routed in its prologue when `logits` is given, else on `ids`), then down on the
// ids and weights (for the routed entry, the ones gate_up wrote).
static int resident_launch(const char* name, int32_t kind, const void* x, const int64_t* ids, const float* weights,
                           const void* logits, int32_t n, int32_t k, const void* gu_w, const void* gu_s,
                           const float* gu_c, const void* dn_w, const void* dn_s, const float* dn_c,
                           const float* gu_codebook, const float* dn_codebook, float* gu, void* out, int32_t H,
                           int32_t I, void* stream) {
  if (!x || !ids || !weights || !gu_w || !gu_s || !dn_w || !dn_s || !gu || !out) return fail(std::string(name) + ": null pointer");
  if ((kind == 4 || kind == 6) && (!gu_c || !dn_c)) return fail(std::string(name) + ": codes need channel scales");
  if (kind == 4 && (!gu_codebook || !dn_codebook)) return fail(std::string(name) + ": 4 bits need codebooks");
  if (k < 1 || k > MAX_K_RES) return fail(std::string(name) + ": 1 <= k <= 8");
  if (logits && (n < k || n > ROUTED_MAX_N)) return fail(std::string(name) + ": k <= n <= 256 logits");
  if ((H != 2048 && H != 1024) || (I != 512 && I != 768 && I != 1024) || H % DN_ROWS)
    return fail(std::string(name) + ": H 1024 or 2048, I 512, 768 or 1024");
  const hipStream_t s = (hipStream_t)stream;
  const dim3 ggrid(I / GU_UNITS, k), dgrid(H / DN_ROWS);
  const uint16_t *xb = (const uint16_t*)x, *lg = (const uint16_t*)logits;
  const uint8_t *gw = (const uint8_t*)gu_w, *dw = (const uint8_t*)dn_w;
  int64_t* ids_out = const_cast<int64_t*>(ids);
  float* w_out = const_cast<float*>(weights);
  uint16_t* o = (uint16_t*)out;
#define D3_GU(KIND, K)                                                                                               \
  do {                                                                                                               \
    if (!lg) hipLaunchKernelGGL((resident_gu_kernel<KIND, K, 1, false>), ggrid, dim3(256), 0, s, xb, ids, nullptr, 0, \
                                k, nullptr, nullptr, gw, gu_s, gu_c, gu_codebook, gu, I);                            \
    else if (n <= 64) hipLaunchKernelGGL((resident_gu_kernel<KIND, K, 1, true>), ggrid, dim3(256), 0, s, xb, nullptr, \
                                         lg, n, k, ids_out, w_out, gw, gu_s, gu_c, gu_codebook, gu, I);              \
    else if (n <= 128) hipLaunchKernelGGL((resident_gu_kernel<KIND, K, 2, true>), ggrid, dim3(256), 0, s, xb,        \
                                          nullptr, lg, n, k, ids_out, w_out, gw, gu_s, gu_c, gu_codebook, gu, I);    \
    else hipLaunchKernelGGL((resident_gu_kernel<KIND, K, 4, true>), ggrid, dim3(256), 0, s, xb, nullptr, lg, n, k,   \
                            ids_out, w_out, gw, gu_s, gu_c, gu_codebook, gu, I);                                     \
  } while (0)
#define D3_DN(KERNEL, KIND, ST)                                                                                     \
  do {                                                                                                               \
    if (I == 768) hipLaunchKernelGGL((KERNEL<KIND, 768>), dgrid, dim3(256), 0, s, gu, ids, weights, k, dw, (ST)dn_s, \
                                     dn_c, dn_codebook, o, H);                                                       \
    else if (I == 512) hipLaunchKernelGGL((KERNEL<KIND, 512>), dgrid, dim3(256), 0, s, gu, ids, weights, k, dw,     \
                                          (ST)dn_s, dn_c, dn_codebook, o, H);                                        \
    else hipLaunchKernelGGL((KERNEL<KIND, 1024>), dgrid, dim3(256), 0, s, gu, ids, weights, k, dw, (ST)dn_s, dn_c,   \
                            dn_codebook, o, H);                                                                      \
  } while (0)
#define D3_RES(KIND, DN_KERNEL, ST)                                                                                  \
  do {                                                                                                               \
    if (H == 2048) D3_GU(KIND, 2048);                                                                                \
    else D3_GU(KIND, 1024);                                                                                          \
    D3_DN(DN_KERNEL, KIND, ST);                                                                                      \
  } while (0)
  switch (kind) {
    case 0: D3_RES(0, resident_dn_kernel, const void*); break;
    case 1: D3_RES(1, resident_dn_kernel, const void*); break;
    case 4: D3_RES(4, resident_dn_codes_kernel, const uint8_t*); break;
    case 6: D3_RES(6, resident_dn_codes_kernel, const uint8_t*); break;
    default: return fail(std::string(name) + ": kind 0, 1, 4 or 6");
  }
#undef D3_RES
#undef D3_DN
#undef D3_GU
  return done(name);
}

extern "C" {

int d3_resident_decode(int32_t kind, const void* x, const int64_t* ids, const float* weights, int32_t k,
                       const void* gu_w, const void* gu_s, const float* gu_c, const void* dn_w, const void* dn_s,
                       const float* dn_c, const float* gu_codebook, const float* dn_codebook, float* gu, void* out,
                       int32_t H, int32_t I, void* stream) {
  return resident_launch("d3_resident_decode", kind, x, ids, weights, nullptr, 0, k, gu_w, gu_s, gu_c, dn_w, dn_s,
                         dn_c, gu_codebook, dn_codebook, gu, out, H, I, stream);
}

int d3_resident_decode_routed(int32_t kind, const void* x, const void* logits, int32_t n, int32_t k, int64_t* ids,
                              float* weights, const void* gu_w, const void* gu_s, const float* gu_c, const void* dn_w,
                              const void* dn_s, const float* dn_c, const float* gu_codebook, const float* dn_codebook,
                              float* gu, void* out, int32_t H, int32_t I, void* stream) {
  if (!logits) return fail("d3_resident_decode_routed: null pointer");
  return resident_launch("d3_resident_decode_routed", kind, x, ids, weights, logits, n, k, gu_w, gu_s, gu_c, dn_w,
                         dn_s, dn_c, gu_codebook, dn_codebook, gu, out, H, I, stream);
}

int64_t d3_resident_workspace_bytes(int32_t k, int32_t I) {
  if (k < 1 || k > MAX_K_RES || I < 1) return -1;
  return RES_HEADER + (int64_t)k * I * 8;
}

int d3_resident_decode_fused(int32_t kind, const void* x, const void* logits, int32_t n, int32_t k, int64_t* ids,
                             float* weights, const void* gu_w, const void* gu_s, const float* gu_c, const void* dn_w,
                             const void* dn_s, const float* dn_c, const float* gu_codebook, const float* dn_codebook,
                             void* workspace, int64_t workspace_bytes, uint32_t spin_limit, int32_t block_rows,
                             int32_t recompute_all, void* out, int32_t H, int32_t I, void* stream) {
  const char* name = "d3_resident_decode_fused";
  if (!x || !ids || !weights || !gu_w || !gu_s || !dn_w || !dn_s || !workspace || !out)
    return fail(std::string(name) + ": null pointer");
  if ((kind == 4 || kind == 6) && (!gu_c || !dn_c)) return fail(std::string(name) + ": codes need channel scales");
  if (kind == 4 && (!gu_codebook || !dn_codebook)) return fail(std::string(name) + ": 4 bits need codebooks");
  if (k < 1 || k > MAX_K_RES) return fail(std::string(name) + ": 1 <= k <= 8");
  if (logits && (n < k || n > ROUTED_MAX_N)) return fail(std::string(name) + ": k <= n <= 256 logits");
  if (H != 2048 || (I != 512 && I != 768)) return fail(std::string(name) + ": H 2048, I 512 or 768");
  if (block_rows == 0) block_rows = 4;
  if (block_rows != 4 && block_rows != 8) return fail(std::string(name) + ": block_rows 4 or 8");
  if (workspace_bytes < d3_resident_workspace_bytes(k, I)) return fail(std::string(name) + ": workspace too small");
  if ((uintptr_t)workspace & 255u) return fail(std::string(name) + ": workspace must be 256-byte aligned");
  ResidentArgs a{};
  a.x = (const uint16_t*)x;
  a.ids = ids;
  a.wts = weights;
  a.logits = (const uint16_t*)logits;
  a.n = n;
  a.k = k;
  a.ids_out = ids;
  a.w_out = weights;
  a.gw = (const uint8_t*)gu_w;
  a.gs = gu_s;
  a.gc = gu_c;
  a.gcb = gu_codebook;
  a.dw = (const uint8_t*)dn_w;
  a.ds = dn_s;
  a.dc = dn_c;
  a.dcb = dn_codebook;
  a.out = (uint16_t*)out;
  a.H = H;
  a.I = I;
  a.status = (uint64_t*)workspace;
  a.sticky = (uint32_t*)((uint8_t*)workspace + RES_STICKY);
  a.hidden = (uint64_t*)((uint8_t*)workspace + RES_HEADER);
  a.spin_limit = recompute_all ? 0u : spin_limit ? spin_limit : (1u << 20);
  a.items = k * (I / GU_UNITS);
  const int blocks = H / block_rows, grid = std::max(a.items, blocks);
  a.dn_first = grid - blocks;
  const hipStream_t s = (hipStream_t)stream;
#define D3_FUSED_ROUTE(KIND, KI, RW)                                                                                   \
  do {                                                                                                                 \
    if (!logits) hipLaunchKernelGGL((resident_fused_kernel<KIND, 2048, KI, RW, 1, false>), dim3(grid), dim3(256), 0, s, a); \
    else if (n <= 64) hipLaunchKernelGGL((resident_fused_kernel<KIND, 2048, KI, RW, 1, true>), dim3(grid), dim3(256), 0, s, a); \
    else if (n <= 128) hipLaunchKernelGGL((resident_fused_kernel<KIND, 2048, KI, RW, 2, true>), dim3(grid), dim3(256), 0, s, a); \
    else hipLaunchKernelGGL((resident_fused_kernel<KIND, 2048, KI, RW, 4, true>), dim3(grid), dim3(256), 0, s, a);      \
  } while (0)
#define D3_FUSED(KIND)                                                                                                 \
  do {                                                                                                                 \
    if (I == 768 && block_rows == 8) D3_FUSED_ROUTE(KIND, 768, 2);                                                     \
    else if (I == 768) D3_FUSED_ROUTE(KIND, 768, 1);                                                                   \
    else if (block_rows == 8) D3_FUSED_ROUTE(KIND, 512, 2);                                                            \
    else D3_FUSED_ROUTE(KIND, 512, 1);                                                                                 \
  } while (0)
  switch (kind) {
    case 0: D3_FUSED(0); break;
    case 1: D3_FUSED(1); break;
    case 4: D3_FUSED(4); break;
    case 6: D3_FUSED(6); break;
    default: return fail(std::string(name) + ": kind 0, 1, 4 or 6");
  }
#undef D3_FUSED
#undef D3_FUSED_ROUTE
  return done(name);
}

int d3_resident_status(void* workspace, uint32_t* status) {
  if (!workspace || !status) return fail("d3_resident_status: null pointer");
  uint8_t* sticky = (uint8_t*)workspace + RES_STICKY;
  hipError_t e = hipMemcpy(status, sticky, 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "d3_resident_status");
  const uint32_t zero = 0;
  e = hipMemcpy(sticky, &zero, 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(e, "d3_resident_status");
  return 0;
}

int d3_decode_codes(int32_t bits, const void* rows, const void* scales, const float* codebook, int32_t R, int32_t K,
                    void* out, void* stream) {
  if (!rows || !scales || !out) return fail("d3_decode_codes: null pointer");
  const bool table = bits == D3_DECODE_TABLE_W4;
  if (table) bits = 4;
  if (bits == 4 && !codebook) return fail("d3_decode_codes: 4 bits need a codebook");
  if ((bits != 4 && bits != 6) || R < 1 || K < 32 || K % 32) return fail("d3_decode_codes: bits 4 or 6, K % 32 == 0");
  const int64_t threads = (int64_t)R * (K / 16);
  const dim3 grid((unsigned)((threads + 255) / 256));
  const hipStream_t s = (hipStream_t)stream;
  const uint8_t *rb = (const uint8_t*)rows, *sb = (const uint8_t*)scales;
  int8_t* o = (int8_t*)out;
  if (table) hipLaunchKernelGGL((decode_codes_kernel<4, true>), grid, dim3(256), 0, s, rb, sb, codebook, R, K, o);
  else if (bits == 4) hipLaunchKernelGGL((decode_codes_kernel<4, false>), grid, dim3(256), 0, s, rb, sb, codebook, R, K, o);
  else hipLaunchKernelGGL((decode_codes_kernel<6, false>), grid, dim3(256), 0, s, rb, sb, codebook, R, K, o);
  return done("d3_decode_codes");
}

}  // extern "C"
