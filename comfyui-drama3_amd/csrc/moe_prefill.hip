// The routed-expert MoE layer for many rows (a prompt's pass, or many decode lines) on A8 banks: the rows' (row,
// expert) pairs grouped by expert and run as grouped MFMA GEMMs, each expert's weights read once for all its rows.
//
// Replaces the reference's resident_prefill (drama3/offload.py:139-149: argsort / bincount().tolist() grouping on the
// host, then grouped_int8 / grouped_fp8 / grouped_codes, kernels.py:365-464,538-587, whose lanes hold 64 weights in
// float registers and loop the group's rows with FMAs). Same layer semantics as the fused decode kernel (the oracle's
// moe_layer): per-row int8 or e4m3 activations, SiLU(gate) * up quantized per (row, expert) pair, routing-weighted sum.
//
// Launches, all stream-ordered and graph-capturable (no host sync; the grouping happens on the device):
//   route      top-k per row (d3_route's kernel), unless the caller hands ids / weights in
//   group      one workgroup: per-expert counts (LDS atomics), offsets, and the pairs in expert order
//   quantize   activations per row, in the format's storage order
//   gate_up    grid (I / 16, E): 16 hidden units of one expert (16 gate + 16 up rows), K split over 4 waves per
//              tile, the weights held in registers while the expert's pairs go by 16 at a time; SiLU(gate) * up
//   quantize   the hidden rows, per pair
//   down       grid (H / 32, E): 32 output rows of one expert against its pairs; the product, scaled by the pair's
//              routing weight, lands in the pair's own row
//   reduce     out[t] = bf16(sum over the row's k pairs, in routing order)
// Results do not depend on the order of pairs within an expert (every output element is its own dot product), so the
// grouping may use atomics.
#include "formats.hpp"
#include "../../include/drama3_moe.h"

#include <string>

namespace d3 {
int fail(const std::string& msg);
int hip_fail(hipError_t err, const char* what);

namespace {

constexpr int MAX_EXPERTS = 1024;

struct PrefillArgs {
  const int64_t* ids;     // [P] pair p = t * k + j -> expert
  const float* weights;   // [P]
  const int* counts;      // [E]
  const int* offsets;     // [E + 1]
  const int* perm;        // [P] sorted position -> pair
  const uint8_t* xq;      // [T, H] storage order
  const float* xs;        // [T]
  float* h;               // [P, I] by sorted position
  const uint8_t* hq;      // [P, I]
  const float* hs;        // [P]
  float* parts;           // [P, H] by pair
  const uint8_t* gu_w;
  const uint16_t* gu_s;
  const uint8_t* dn_w;
  const uint16_t* dn_s;
  int k;
  int inter;              // I
};

// ---------------------------------------------------------------------------------------------------------- group
__global__ void __launch_bounds__(1024) group_kernel(const int64_t* ids, int P, int E, int* counts, int* offsets,
                                                     int* perm) {
  __shared__ int cnt[MAX_EXPERTS], cur[MAX_EXPERTS];
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  // ids outside [0, E) (a caller's error) count as the nearest expert instead of reaching outside the tables
  for (int p = tid; p < P; p += 1024) atomicAdd(&cnt[(int)min<int64_t>(max<int64_t>(ids[p], 0), E - 1)], 1);
  __syncthreads();
  if (tid < 64) {
    // exclusive scan by wave 0: each lane sums a contiguous run of experts, then the runs are scanned
    const int per = (E + 63) / 64, lo = tid * per, hi = min(E, lo + per);
    int run = 0;
    for (int e = lo; e < hi; e++) run += cnt[e];
    int incl = run;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int v = __shfl_up(incl, o);
      if (tid >= o) incl += v;
    }
    int at = incl - run;
    for (int e = lo; e < hi; e++) {
      cur[e] = at;
      offsets[e] = at;
      counts[e] = cnt[e];
      at += cnt[e];
    }
    if (tid == 63) offsets[E] = incl;
  }
  __syncthreads();
  for (int p = tid; p < P; p += 1024) perm[atomicAdd(&cur[(int)min<int64_t>(max<int64_t>(ids[p], 0), E - 1)], 1)] = p;
}

// ------------------------------------------------------------------------------------------------------- quantize
// One wave per row of `width` floats (bf16 with BF16): absmax, then codes in the format's storage order and the
// row's scale.
template <int F, bool BF16>
__global__ void __launch_bounds__(256) quantize_rows_kernel(const void* src, int rows, int width, uint8_t* q,
                                                            float* scale) {
  constexpr float QMAX = act_qmax<F>();
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int chunks = width / 8;
  float amax = 0.0f;
  for (int c = lane; c < chunks; c += 64) {
    float v[8];
    if constexpr (BF16) {
      const i32x4 r = *(const i32x4*)((const uint16_t*)src + (size_t)row * width + 8 * c);
      const uint32_t w4[4] = {(uint32_t)r.x, (uint32_t)r.y, (uint32_t)r.z, (uint32_t)r.w};
#pragma unroll
      for (int i = 0; i < 4; i++) { v[2 * i] = bf16_to_f32(w4[i] & 0xFFFFu); v[2 * i + 1] = bf16_to_f32(w4[i] >> 16); }
    } else {
      const f32x4 a = *(const f32x4*)((const float*)src + (size_t)row * width + 8 * c);
      const f32x4 b = *(const f32x4*)((const float*)src + (size_t)row * width + 8 * c + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, fabsf(v[i]));
  }
  amax = wave_max_f32(amax);
  const float inv = amax > 0.0f ? QMAX / amax : 0.0f;
  for (int c = lane; c < chunks; c += 64) {
    float v[8];
    if constexpr (BF16) {
      const i32x4 r = *(const i32x4*)((const uint16_t*)src + (size_t)row * width + 8 * c);
      const uint32_t w4[4] = {(uint32_t)r.x, (uint32_t)r.y, (uint32_t)r.z, (uint32_t)r.w};
#pragma unroll
      for (int i = 0; i < 4; i++) { v[2 * i] = bf16_to_f32(w4[i] & 0xFFFFu); v[2 * i + 1] = bf16_to_f32(w4[i] >> 16); }
    } else {
      const f32x4 a = *(const f32x4*)((const float*)src + (size_t)row * width + 8 * c);
      const f32x4 b = *(const f32x4*)((const float*)src + (size_t)row * width + 8 * c + 4);
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    store_act8<F>(q + (size_t)row * width + 8 * c, v, inv);
  }
  if (lane == 0) scale[row] = amax / QMAX;
}

// ------------------------------------------------------------------------------------------- grouped MFMA products
// A workgroup computes TILES 16-row tiles of one expert's bank against all of the expert's pairs. Its KS * TILES
// waves split the work: wave w takes tile w / KS and the K-slice w % KS (SW = K / 128 / KS steps of 128 columns), whose
// weight bytes it holds in registers while it walks the pairs 16 at a time; the KS partial products of a tile meet in
// LDS. Per MFMA, lane l reads weight row l % 16 and pair l % 16, lane group l / 16 covers 32 columns of a step.
//   MODE 0 (gate_up): TILES = 2 = 16 gate rows and the matching 16 up rows (hidden units 16 bx ..), epilogue
//                     SiLU(gate) * up into h[sorted position].
//   MODE 1 (down):    TILES 16-row tiles of output rows (TILES * 16 bx ..), epilogue scaled by the pair's hidden scale
//                     and routing weight into parts[pair].
template <int F, int SW> struct Slice {
  Raw<F> raw[SW];
};

// one lane's 32 activation bytes of step `st`
D3_INLINE void load_act(const uint8_t* act, int st, int q, bool valid, i32x4& lo, i32x4& hi) {
  lo = i32x4{0, 0, 0, 0};
  hi = i32x4{0, 0, 0, 0};
  if (valid) {
    lo = *(const i32x4*)(act + 128 * st + 32 * q);
    hi = *(const i32x4*)(act + 128 * st + 32 * q + 16);
  }
}

template <int F, int K, int KS, int TILES, int MODE>
__global__ void __launch_bounds__(64 * KS * TILES) grouped_kernel(PrefillArgs a) {
  constexpr int SW = K / 128 / KS;
  constexpr int SHIFT = unpack_shift(F);
  constexpr int RB = row_bytes(F, K);
  constexpr int H = 2048;
  const int bx = blockIdx.x, e = blockIdx.y;
  const int n = a.counts[e];
  if (n == 0) return;
  const int first = a.offsets[e];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, q = lane >> 4, col = lane & 15;
  const int tile = w / KS, ks = w % KS, st0 = ks * SW;
  // bank rows of this wave's tile
  size_t row0;
  const uint8_t* bank;
  const uint16_t* sbank;
  if constexpr (MODE == 0) {
    row0 = (size_t)e * 2 * a.inter + (tile ? a.inter : 0) + 16 * bx;
    bank = a.gu_w;
    sbank = a.gu_s;
  } else {
    row0 = (size_t)e * H + 16 * (TILES * bx + tile);
    bank = a.dn_w;
    sbank = a.dn_s;
  }
  Slice<F, SW> sl;
  {
    const uint8_t* row = bank + (row0 + col) * RB;
#pragma unroll
    for (int j = 0; j < SW; j++) load_step<F>(sl.raw[j], row, st0 + j, q);
  }
  // scales of the accumulator rows 4q + i: per row (I8, F8) or per (row, step) (W4, W6)
  float rs[4], gsc[SW][4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if constexpr (group_scaled(F)) {
#pragma unroll
      for (int j = 0; j < SW; j++) gsc[j][i] = bf16_to_f32(sbank[(row0 + 4 * q + i) * (K / 128) + st0 + j]);
      rs[i] = 1.0f;
    } else {
      rs[i] = bf16_to_f32(sbank[row0 + 4 * q + i]);
    }
  }
  __shared__ float part[TILES][KS][16][17];
  const uint8_t* acts = MODE == 0 ? a.xq : a.hq;
  for (int c0 = 0; c0 < n; c0 += 16) {
    const bool valid = c0 + col < n;
    const int sp = first + c0 + (valid ? col : 0);
    const uint8_t* act;
    if constexpr (MODE == 0) act = acts + (size_t)(a.perm[sp] / a.k) * K;
    else act = acts + (size_t)sp * K;
    i32x4 lo[SW], hi[SW];
#pragma unroll
    for (int j = 0; j < SW; j++) load_act(act, st0 + j, q, valid, lo[j], hi[j]);
    f32x4 y;
    if constexpr (F == FMT_F8) {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < SW; j++) acc = step_f8(sl.raw[j], lo[j], hi[j], acc);
      y = acc;
    } else if constexpr (F == FMT_I8) {
      i32x4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < SW; j++) acc = step_i8<F>(sl.raw[j], lo[j], hi[j], acc);
#pragma unroll
      for (int i = 0; i < 4; i++) y[i] = (float)acc[i];
    } else {
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < SW; j++) {
        const i32x4 g = step_i8<F>(sl.raw[j], lo[j], hi[j], i32x4{0, 0, 0, 0});
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] += (float)(g[i] >> SHIFT) * gsc[j][i];
      }
      y = acc;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) part[tile][ks][4 * q + i][col] = y[i] * rs[i];
    __syncthreads();
    if constexpr (MODE == 0) {
      // 16 units x 16 pairs, one per thread of the first 256
      if (tid < 256) {
        const int u = tid & 15, j = tid >> 4;
        if (c0 + j < n) {
          float g = 0.0f, up = 0.0f;
#pragma unroll
          for (int k2 = 0; k2 < KS; k2++) {
            g += part[0][k2][u][j];
            up += part[1][k2][u][j];
          }
          const float xs = a.xs[a.perm[first + c0 + j] / a.k];
          g *= xs;
          up *= xs;
          a.h[(size_t)(first + c0 + j) * a.inter + 16 * bx + u] = g / (1.0f + __expf(-g)) * up;
        }
      }
    } else {
      // TILES * 16 rows x 16 pairs
      for (int o = tid; o < TILES * 256; o += 64 * KS * TILES) {
        const int r = o & (16 * TILES - 1), j = o / (16 * TILES);
        if (c0 + j < n) {
          const int t2 = r >> 4, rr = r & 15;
          float v = 0.0f;
#pragma unroll
          for (int k2 = 0; k2 < KS; k2++) v += part[t2][k2][rr][j];
          const int sp2 = first + c0 + j, pair = a.perm[sp2];
          a.parts[(size_t)pair * H + 16 * TILES * bx + r] = v * a.hs[sp2] * a.weights[pair];
        }
      }
    }
    __syncthreads();
  }
}

// out[t, c] = bf16(sum over j < k of parts[t * k + j, c]); two columns per thread
__global__ void __launch_bounds__(256) reduce_kernel(const float* parts, int T, int k, int H, uint16_t* out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)T * (H / 2)) return;
  const int t = (int)(idx / (H / 2)), c = 2 * (int)(idx % (H / 2));
  float s0 = 0.0f, s1 = 0.0f;
  for (int j = 0; j < k; j++) {
    const f32x2 v = *(const f32x2*)(parts + ((size_t)t * k + j) * H + c);
    s0 += v.x;
    s1 += v.y;
  }
  *(uint32_t*)(out + (size_t)t * H + c) = f32_to_bf16(s0) | (f32_to_bf16(s1) << 16);
}

// ------------------------------------------------------------------------------------------------------- host side
struct Layout {
  size_t ids, weights, counts, offsets, perm, xq, xs, h, hq, hs, parts, total;
};
size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }
Layout layout(int64_t T, int64_t k, int64_t H, int64_t I, int64_t E) {
  Layout L;
  const int64_t P = T * k;
  size_t at = 0;
  auto take = [&](size_t bytes) { const size_t o = at; at = align256(at + bytes); return o; };
  L.ids = take(P * 8);
  L.weights = take(P * 4);
  L.counts = take(E * 4);
  L.offsets = take((E + 1) * 4);
  L.perm = take(P * 4);
  L.xq = take(T * H);
  L.xs = take(T * 4);
  L.h = take(P * I * 4);
  L.hq = take(P * I);
  L.hs = take(P * 4);
  L.parts = take(P * H * 4);
  L.total = at;
  return L;
}

// gate_up: K = H = 2048 in 4 slices of 4 steps, 2 tiles (gate, up) -> 8 waves; down: K = I in 2 slices, 2 tiles
template <int F, int H, int I> void launch_products(const PrefillArgs& pa, int E, hipStream_t s) {
  hipLaunchKernelGGL((grouped_kernel<F, H, 4, 2, 0>), dim3(I / 16, E), dim3(512), 0, s, pa);
}
template <int F, int H, int I> void launch_down(const PrefillArgs& pa, int E, hipStream_t s) {
  hipLaunchKernelGGL((grouped_kernel<F, I, (I / 128) % 2 == 0 ? 2 : 1, 2, 1>), dim3(H / 32, E), dim3((I / 128) % 2 == 0 ? 256 : 128), 0, s, pa);
}

template <int F> void launch_quantize(const void* src, bool bf16, int rows, int width, uint8_t* q, float* scale,
                                      hipStream_t s) {
  const dim3 grid((rows + 3) / 4);
  if (bf16) hipLaunchKernelGGL((quantize_rows_kernel<F, true>), grid, dim3(256), 0, s, src, rows, width, q, scale);
  else hipLaunchKernelGGL((quantize_rows_kernel<F, false>), grid, dim3(256), 0, s, src, rows, width, q, scale);
}

template <int F, int H, int I> void run(const PrefillArgs& pa, const d3_moe_a8_prefill_desc& d, const Layout& L,
                                        uint8_t* ws, hipStream_t s) {
  const int P = d.T * d.topk;
  launch_quantize<F>(d.x, true, d.T, H, ws + L.xq, (float*)(ws + L.xs), s);
  launch_products<F, H, I>(pa, d.E, s);
  launch_quantize<F>(ws + L.h, false, P, I, ws + L.hq, (float*)(ws + L.hs), s);
  launch_down<F, H, I>(pa, d.E, s);
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" {

int d3_route(const void* logits, int32_t rows, int32_t n, int32_t k, int64_t* ids, float* weights, void* stream);

int64_t d3_moe_a8_prefill_workspace_bytes(int32_t T, int32_t topk, int32_t H, int32_t I, int32_t E) {
  if (T < 1 || topk < 1 || H < 1 || I < 1 || E < 1) return -1;
  return (int64_t)layout(T, topk, H, I, E).total;
}

int d3_moe_a8_prefill(const d3_moe_a8_prefill_desc* d, void* stream) {
  if (!d) return fail("d3_moe_a8_prefill: null desc");
  if (!d->x || !d->gate_up || !d->gate_up_scale || !d->down || !d->down_scale || !d->out || !d->workspace)
    return fail("d3_moe_a8_prefill: null pointer");
  if (!d->logits && (!d->ids_in || !d->weights_in)) return fail("d3_moe_a8_prefill: logits or ids_in / weights_in");
  if (d->format < D3_FMT_I8 || d->format > D3_FMT_F8) return fail("d3_moe_a8_prefill: format");
  if (d->H != 2048 || (d->I != 768 && d->I != 512)) return fail("d3_moe_a8_prefill: H 2048, I 768 or 512");
  if (d->T < 1 || d->topk < 1 || d->topk > 32 || d->E < d->topk || d->E > MAX_EXPERTS || (d->logits && d->E > 1024))
    return fail("d3_moe_a8_prefill: T >= 1, 1 <= topk <= 32, topk <= E <= 1024");
  const Layout L = layout(d->T, d->topk, d->H, d->I, d->E);
  if (d->workspace_bytes < (int64_t)L.total) return fail("d3_moe_a8_prefill: workspace too small");
  const hipStream_t s = (hipStream_t)stream;
  uint8_t* ws = (uint8_t*)d->workspace;
  const int P = d->T * d->topk;
  int64_t* ids = (int64_t*)(ws + L.ids);
  float* weights = (float*)(ws + L.weights);
  if (d->logits) {
    const int rc = d3_route(d->logits, d->T, d->E, d->topk, ids, weights, stream);
    if (rc) return rc;
  } else {
    hipError_t err = hipMemcpyAsync(ids, d->ids_in, (size_t)P * 8, hipMemcpyDeviceToDevice, s);
    if (err == hipSuccess) err = hipMemcpyAsync(weights, d->weights_in, (size_t)P * 4, hipMemcpyDeviceToDevice, s);
    if (err != hipSuccess) return hip_fail(err, "d3_moe_a8_prefill: copy routing");
  }
  if (d->ids_out && d->logits) {
    hipError_t err = hipMemcpyAsync(d->ids_out, ids, (size_t)P * 8, hipMemcpyDeviceToDevice, s);
    if (err == hipSuccess && d->weights_out)
      err = hipMemcpyAsync(d->weights_out, weights, (size_t)P * 4, hipMemcpyDeviceToDevice, s);
    if (err != hipSuccess) return hip_fail(err, "d3_moe_a8_prefill: copy routing out");
  }
  hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), 0, s, (const int64_t*)ids, P, d->E, (int*)(ws + L.counts),
                     (int*)(ws + L.offsets), (int*)(ws + L.perm));
  PrefillArgs pa;
  pa.ids = ids;
  pa.weights = weights;
  pa.counts = (const int*)(ws + L.counts);
  pa.offsets = (const int*)(ws + L.offsets);
  pa.perm = (const int*)(ws + L.perm);
  pa.xq = ws + L.xq;
  pa.xs = (const float*)(ws + L.xs);
  pa.h = (float*)(ws + L.h);
  pa.hq = ws + L.hq;
  pa.hs = (const float*)(ws + L.hs);
  pa.parts = (float*)(ws + L.parts);
  pa.gu_w = (const uint8_t*)d->gate_up;
  pa.gu_s = (const uint16_t*)d->gate_up_scale;
  pa.dn_w = (const uint8_t*)d->down;
  pa.dn_s = (const uint16_t*)d->down_scale;
  pa.k = d->topk;
  pa.inter = d->I;
  const bool i768 = d->I == 768;
  switch (d->format) {
    case D3_FMT_I8: i768 ? run<FMT_I8, 2048, 768>(pa, *d, L, ws, s) : run<FMT_I8, 2048, 512>(pa, *d, L, ws, s); break;
    case D3_FMT_W4: i768 ? run<FMT_W4, 2048, 768>(pa, *d, L, ws, s) : run<FMT_W4, 2048, 512>(pa, *d, L, ws, s); break;
    case D3_FMT_W6: i768 ? run<FMT_W6, 2048, 768>(pa, *d, L, ws, s) : run<FMT_W6, 2048, 512>(pa, *d, L, ws, s); break;
    default: i768 ? run<FMT_F8, 2048, 768>(pa, *d, L, ws, s) : run<FMT_F8, 2048, 512>(pa, *d, L, ws, s); break;
  }
  const int64_t threads = (int64_t)d->T * (d->H / 2);
  hipLaunchKernelGGL(reduce_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, (const float*)pa.parts,
                     d->T, d->topk, d->H, (uint16_t*)d->out);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "d3_moe_a8_prefill");
}

}  // extern "C"
