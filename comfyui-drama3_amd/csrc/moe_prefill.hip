// The routed-expert MoE layer for many rows (a prompt's pass, or many decode lines) on A8 banks: the rows' (row,
// expert) pairs grouped by expert and run as grouped MFMA GEMMs, each expert's weights read once for all its rows.
//
// Replaces the reference's resident_prefill (drama3/offload.py:139-149: argsort / bincount().tolist() grouping on the
// host, then grouped_int8 / grouped_fp8 / grouped_codes, kernels.py:365-464,538-587, whose lanes hold 64 weights in
// float registers and loop the group's rows with FMAs). Same layer semantics as the fused decode kernel (the oracle's
// moe_layer): per-row int8 or e4m3 activations, SiLU(gate) * up quantized per (row, expert) pair, routing-weighted sum.
//
// Launches, all stream-ordered and graph-capturable (no host sync; the grouping happens on the device):
//   route      a wave per row: its top-k (as d3_route computes it), or the caller's ids / weights, and its
//              activations quantized once, by row, in the format's storage order
//   group      one workgroup: per-expert counts (LDS atomics), offsets, and the pairs in expert order
//   gate_up    grid (I / 16, E): 16 hidden units of one expert (16 gate + 16 up rows), K split over 4 waves per
//              tile, the weights held in registers while the expert's pairs go by 16 at a time, each pair's row of
//              activations read through perm; SiLU(gate) * up
//   quantize   the hidden rows, per pair
//   down       grid (H / 32, E): 32 output rows of one expert against its pairs; the product, scaled by the pair's
//              routing weight, lands in the pair's own row
//   reduce     out[t] = bf16(sum over the row's k pairs, in routing order)
// Results do not depend on the order of pairs within an expert (every output element is its own dot product), so the
// grouping may use atomics.
#include "formats.hpp"
#include "../../include/drama3_moe.h"

#include <algorithm>
#include <string>

namespace d3 {
int fail(const std::string& msg);
int hip_fail(hipError_t err, const char* what);

namespace {

constexpr int MAX_EXPERTS = 1024;
constexpr int UNIT_PAIRS = 128;  // pairs per work unit (see the grouped products)

struct PrefillArgs {
  const int64_t* ids;     // [P] pair p = t * k + j -> expert
  const float* weights;   // [P]
  const int* counts;      // [E]
  const int* offsets;     // [E + 1]
  const int* perm;        // [P] sorted position -> pair
  const uint8_t* xq;      // [T, H] storage order, by row
  const float* xs;        // [T]
  float* h;               // [P, I] by sorted position
  const uint8_t* hq;      // [P, I]
  const float* hs;        // [P] the hidden row's scale times the pair's routing weight
  float* parts;           // [P, H] by pair
  const uint8_t* gu_w;
  const uint16_t* gu_s;
  const uint8_t* dn_w;
  const uint16_t* dn_s;
  const int4* units;      // (expert, first position, pairs <= UNIT_PAIRS, 0): the experts' pairs in runs of at
                          // most UNIT_PAIRS, experts with most pairs first
  const int* meta;        // [0]: units
  int k;
  int inter;              // I
};

// ---------------------------------------------------------------------------------------------------------- group
// Per-expert pair counts (LDS atomics), their offsets, the pairs in expert order, and the work units: each expert's
// pairs in runs of at most UNIT_PAIRS, experts with most pairs first (ties: lower id first), the order the product
// kernels take their work in (long work starts first).
D3_INLINE int wave_exclusive_scan(int v, int lane, int& total) {
  int incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  total = __shfl(incl, 63);
  return incl - v;
}

// (a workgroup of 1024 threads; ids may be in LDS or device memory; inv_lds, if given, gets each pair's sorted
// position)
D3_INLINE void group_pairs(const int64_t* ids, int P, int E, int* counts, int* offsets, int* perm, int4* units,
                           int* meta, int* inv_lds = nullptr) {
  __shared__ int cnt[MAX_EXPERTS], cur[MAX_EXPERTS], by_rank[MAX_EXPERTS], rank_base[MAX_EXPERTS];
  __shared__ int used;
  const int tid = threadIdx.x;
  for (int e = tid; e < E; e += 1024) cnt[e] = 0;
  if (tid == 0) used = 0;
  __syncthreads();
  // ids outside [0, E) (a caller's error) count as the nearest expert instead of reaching outside the tables
  for (int p = tid; p < P; p += 1024) atomicAdd(&cnt[(int)min<int64_t>(max<int64_t>(ids[p], 0), E - 1)], 1);
  __syncthreads();
  if (tid < 64) {
    // exclusive scan of the counts by wave 0, each lane over a contiguous run of experts
    const int per = (E + 63) / 64, lo = tid * per, hi = min(E, lo + per);
    int run = 0;
    for (int e = lo; e < hi; e++) run += cnt[e];
    int total;
    int at = wave_exclusive_scan(run, tid, total);
    for (int e = lo; e < hi; e++) {
      cur[e] = at;
      offsets[e] = at;
      counts[e] = cnt[e];
      at += cnt[e];
    }
    if (tid == 0) offsets[E] = total;
  }
  // each used expert's rank (most pairs first, then lower id): S consecutive lanes per expert, each comparing its
  // count with E2 / S of the others (E2: E rounded up to a power of two), the partial ranks summed across the S lanes
  // (a loop over all E per thread was a serial chain of E LDS reads)
  {
    int e2 = 1;
    while (e2 < E) e2 <<= 1;
    const int S = min(64, min(1024 / e2, e2)), span = e2 / S;
    const int e = tid / S, s = tid % S;
    const int c = e < E ? cnt[e] : 0;
    int rank = 0;
    for (int f = s * span; f < s * span + span; f++)
      if (f < E) rank += cnt[f] > c || (cnt[f] == c && f < e);
    for (int off = S >> 1; off > 0; off >>= 1) rank += __shfl_xor(rank, off);
    if (e < E && s == 0 && c > 0) {
      atomicAdd(&used, 1);
      by_rank[rank] = e;
    }
  }
  __syncthreads();
  const int U = used;
  if (tid < 64) {
    const int per = (U + 63) / 64, lo = tid * per, hi = min(U, lo + per);
    int run = 0;
    for (int r = lo; r < hi; r++) run += (cnt[by_rank[r]] + UNIT_PAIRS - 1) / UNIT_PAIRS;
    int total;
    int at = wave_exclusive_scan(run, tid, total);
    for (int r = lo; r < hi; r++) {
      rank_base[r] = at;
      at += (cnt[by_rank[r]] + UNIT_PAIRS - 1) / UNIT_PAIRS;
    }
    if (tid == 0) meta[0] = total;
  }
  __syncthreads();
  for (int r = tid; r < U; r += 1024) {
    const int e = by_rank[r], c = cnt[e], first = cur[e];
    for (int u = 0; u * UNIT_PAIRS < c; u++)
      units[rank_base[r] + u] = int4{e, first + u * UNIT_PAIRS, min(UNIT_PAIRS, c - u * UNIT_PAIRS), 0};
  }
  __syncthreads();
  for (int p = tid; p < P; p += 1024) {
    const int at = atomicAdd(&cur[(int)min<int64_t>(max<int64_t>(ids[p], 0), E - 1)], 1);
    perm[at] = p;
    if (inv_lds) inv_lds[p] = at;
  }
}

__global__ void __launch_bounds__(1024) group_kernel(const int64_t* ids, int P, int E, int* counts, int* offsets,
                                                     int* perm, int4* units, int* meta) {
  group_pairs(ids, P, E, counts, offsets, perm, units, meta);
}

// One row of x (bf16, H columns; lane l holds columns 512 c + 8 l .. + 7 in xr[c]) quantized per row: codes in the
// format's storage order at q, the row's scale (absmax / QMAX) at scale.
template <int F, int H>
D3_INLINE void quantize_row(const i32x4* xr, int lane, uint8_t* q, float* scale) {
  constexpr float QMAX = act_qmax<F>();
  float v[H / 512][8];
  float amax = 0.0f;
#pragma unroll
  for (int c = 0; c < H / 512; c++) {
    const uint32_t w4[4] = {(uint32_t)xr[c].x, (uint32_t)xr[c].y, (uint32_t)xr[c].z, (uint32_t)xr[c].w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[c][2 * j] = bf16_to_f32(w4[j] & 0xFFFFu);
      v[c][2 * j + 1] = bf16_to_f32(w4[j] >> 16);
      amax = fmaxf(amax, fmaxf(fabsf(v[c][2 * j]), fabsf(v[c][2 * j + 1])));
    }
  }
  amax = wave_max_f32(amax);
  const float inv = amax > 0.0f ? QMAX / amax : 0.0f;
#pragma unroll
  for (int c = 0; c < H / 512; c++) store_act8<F>(q + 512 * c + 8 * lane, v[c], inv);
  if (lane == 0) *scale = amax / QMAX;
}

// ----------------------------------------------------------------------------------------------- route + quantize
// A wave per row: the row's top-k of E <= 64 KPL bf16 logits (kernels.py:39-67 as d3_route's kernel computes it: keys
// by value then lower index, k rounds of a wave max, the softmax's exponentials summed in rank order, bf16-rounded),
// or the caller's ids / weights; then the row's activations quantized once (quantize_row).
template <int F, int H, int KPL>
__global__ void __launch_bounds__(256) route_quant_kernel(const uint16_t* logits, const int64_t* ids_in,
                                                          const float* weights_in, const uint16_t* x, int T, int E,
                                                          int k, int64_t* ids, float* weights, int64_t* ids_out,
                                                          float* weights_out, uint8_t* xq, float* xs) {
  const int lane = threadIdx.x & 63, t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  i32x4 xr[H / 512];
#pragma unroll
  for (int c = 0; c < H / 512; c++) xr[c] = *(const i32x4*)(x + (size_t)t * H + 512 * c + 8 * lane);
  if (logits) {
    uint32_t key[KPL];
#pragma unroll
    for (int j = 0; j < KPL; j++) {
      const int e = lane + 64 * j;
      const uint32_t raw = logits[(size_t)t * E + min(e, E - 1)];  // branch-free: every load in flight at once
      key[j] = e < E ? route_key(raw, e) : 0u;
    }
    int id = 0;  // lane r keeps round r's expert and logit
    float top = 0.0f;
    for (int r = 0; r < k; r++) {
      uint32_t m = key[0];
#pragma unroll
      for (int j = 1; j < KPL; j++) m = max(m, key[j]);
      m = wave_max_u32_v(m);
#pragma unroll
      for (int j = 0; j < KPL; j++) key[j] = key[j] == m ? 0u : key[j];
      if (lane == r) {
        id = route_key_index(m);
        top = route_key_value(m);
      }
    }
    const float top0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(top), 0));
    const float ex = lane < k ? expf(top - top0) : 0.0f;
    float total = 0.0f;
    for (int r = 0; r < k; r++) total += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), r));
    if (lane < k) {
      const float wt = bf16_round(ex / total);
      ids[(size_t)t * k + lane] = id;
      weights[(size_t)t * k + lane] = wt;
      if (ids_out) ids_out[(size_t)t * k + lane] = id;
      if (weights_out) weights_out[(size_t)t * k + lane] = wt;
    }
  } else {
    for (int j = lane; j < k; j += 64) {
      ids[(size_t)t * k + j] = ids_in[(size_t)t * k + j];
      weights[(size_t)t * k + j] = weights_in[(size_t)t * k + j];
    }
  }
  quantize_row<F, H>(xr, lane, xq + (size_t)t * H, xs + t);
}

// ----------------------------------------------------------------------------------------- few rows, one launch
// T <= 16 rows in one workgroup of 16 waves, the steps route and group of the many-row path in one launch: wave t
// routes row t (the fused layer's TopKeys, kernels.py:39-67's rule; or copies the given ids and weights) and
// quantizes it (loaded with the logits), the workgroup groups the pairs (group_pairs).
struct SmallPrepArgs {
  const uint16_t* logits;   // [T, E] bf16, or null with ids_in / weights_in
  const int64_t* ids_in;
  const float* weights_in;
  const uint16_t* x;        // [T, H] bf16
  int T, E, k;
  int64_t* ids;             // [P]
  float* weights;           // [P]
  int64_t* ids_out;         // optional
  float* weights_out;       // optional
  int* counts;
  int* offsets;
  int* perm;
  int4* units;
  int* meta;
  uint8_t* xq;              // [T, H] by row
  float* xs;                // [T]
};

template <int F, int H, int KPL>
__global__ void __launch_bounds__(1024) small_prep_kernel(SmallPrepArgs a) {
  constexpr float QMAX = act_qmax<F>();
  __shared__ int64_t lids[16 * 8];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int T = a.T, E = a.E, k = a.k, P = T * k;
  i32x4 xr[H / 512];
  if (w < T) {
#pragma unroll
    for (int c = 0; c < H / 512; c++) xr[c] = *(const i32x4*)(a.x + (size_t)w * H + 512 * c + 8 * lane);
    if (a.logits) {
      uint32_t lb[KPL];
#pragma unroll
      for (int j = 0; j < KPL; j++) lb[j] = a.logits[(size_t)w * E + min(lane + 64 * j, E - 1)];
      TopKeys<KPL> tk(lb, lane, E);
      tk.rounds(lane, 0, k);
      const float wt = route_weight(tk.mine, lane, k);
      if (lane < k) {
        const int64_t id = route_key_index(tk.mine);
        lids[w * k + lane] = id;
        a.ids[w * k + lane] = id;
        a.weights[w * k + lane] = wt;
        if (a.ids_out) a.ids_out[w * k + lane] = id;
        if (a.weights_out) a.weights_out[w * k + lane] = wt;
      }
    } else if (lane < k) {
      const int64_t id = a.ids_in[w * k + lane];
      lids[w * k + lane] = id;
      a.ids[w * k + lane] = id;
      a.weights[w * k + lane] = a.weights_in[w * k + lane];
    }
  }
  __syncthreads();
  group_pairs(lids, P, E, a.counts, a.offsets, a.perm, a.units, a.meta);
  __syncthreads();
  if (w < T) quantize_row<F, H>(xr, lane, a.xq + (size_t)w * H, a.xs + w);
}

// ------------------------------------------------------------------------------------------------------- quantize
// The hidden rows h [P, WIDTH] float (by sorted position) quantized for the down products, one wave per row, read once
// into registers: absmax, then codes in the format's storage order, and the row's scale times the routing weight of
// its pair (pair_weight[perm[row]]), so that the down products need no other factor.
template <int F, int WIDTH>
__global__ void __launch_bounds__(256) quantize_rows_kernel(const float* src, int rows, uint8_t* q, float* scale,
                                                            const float* pair_weight, const int* perm) {
  constexpr float QMAX = act_qmax<F>();
  constexpr int CHUNKS = WIDTH / 8, CPL = (CHUNKS + 63) / 64;  // 8-value chunks, per lane
  const int lane = threadIdx.x & 63, row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  float v[CPL][8];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const int c = lane + 64 * i;
#pragma unroll
    for (int j = 0; j < 8; j++) v[i][j] = 0.0f;
    if (c < CHUNKS) {
      const f32x4 a = *(const f32x4*)(src + (size_t)row * WIDTH + 8 * c);
      const f32x4 b = *(const f32x4*)(src + (size_t)row * WIDTH + 8 * c + 4);
      v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
      v[i][4] = b.x; v[i][5] = b.y; v[i][6] = b.z; v[i][7] = b.w;
    }
#pragma unroll
    for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[i][j]));
  }
  amax = wave_max_f32(amax);
  const float inv = amax > 0.0f ? QMAX / amax : 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; i++) {
    const int c = lane + 64 * i;
    if (c < CHUNKS) store_act8<F>(q + (size_t)row * WIDTH + 8 * c, v[i], inv);
  }
  if (lane == 0) scale[row] = amax / QMAX * pair_weight[perm[row]];
}

// ------------------------------------------------------------------------------------------- grouped MFMA products
// The grouped products, persistent: a work item is (unit, tile): a run of at most UNIT_PAIRS of one expert's pairs
// against the expert's 16 hidden units (gate_up: its 16 gate and 16 up rows) or 64 output rows (down). Items come
// experts with most pairs first; workgroup b of G takes items b, 2G - 1 - b, 2G + b, 4G - 1 - b, ... (rounds of G
// in alternating direction, so that the workgroups that draw a round's heaviest items draw the next round's
// lightest). Its 4 waves split K into KS
// slices (SW steps of 128 columns each) and 16-row tile pairs: a wave holds its two tiles' bytes of its slice in
// registers and walks the expert's pairs 16 at a time (one MFMA per tile and step; lane l reads weight row l % 16
// and pair l % 16, lane group l / 16 covers 32 columns of a step); the slices' partial products meet in LDS.
//   MODE 0 (gate_up): K = H, 4 slices, tiles = gate and up rows of units 16 it .. 16 it + 15; epilogue SiLU(gate) *
//                     up into h[sorted position].
//   MODE 1 (down):    K = I, 2 slices, 2 tile pairs = output rows 64 it .. 64 it + 63; epilogue scaled by the pair's
//                     hidden scale and routing weight into parts[pair].
template <int F, int H, int I, int MODE> struct Geometry {
  static constexpr int K = MODE == 0 ? H : I;
  static constexpr int KS = MODE == 0 ? 4 : 2;
  static constexpr int TILES = MODE == 0 ? 2 : 4;
  static constexpr int SW = K / 128 / KS;
  static constexpr int PER_EXPERT = MODE == 0 ? I / 16 : H / 64;  // items per expert
  static constexpr int RB = row_bytes(F, K);
};

template <int F, int SW> struct Weights {
  Raw<F> raw[2][SW];
  float rs[2][4];  // I8 / F8: the accumulator rows' scales, per tile
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

template <int F, int H, int I, int MODE>
D3_INLINE size_t tile_row0(const PrefillArgs& a, int e, int it, int tile) {
  if constexpr (MODE == 0) return (size_t)e * 2 * I + (tile ? I : 0) + 16 * it;
  else return (size_t)e * H + 64 * it + 16 * tile;
}

template <int F, int H, int I, int MODE>
D3_INLINE void load_weights(Weights<F, Geometry<F, H, I, MODE>::SW>& wt, const PrefillArgs& a, int e, int it,
                            int tp, int ks, int lane) {
  using G = Geometry<F, H, I, MODE>;
  const int q = lane >> 4;
  const uint8_t* bank = MODE == 0 ? a.gu_w : a.dn_w;
  const uint16_t* sb = MODE == 0 ? a.gu_s : a.dn_s;
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const size_t row0 = tile_row0<F, H, I, MODE>(a, e, it, 2 * tp + t);
    const uint8_t* row = bank + (row0 + (lane & 15)) * G::RB;
#pragma unroll
    for (int j = 0; j < G::SW; j++) load_step<F>(wt.raw[t][j], row, ks * G::SW + j, q);
    if constexpr (!group_scaled(F)) {
#pragma unroll
      for (int i = 0; i < 4; i++) wt.rs[t][i] = bf16_to_f32(sb[row0 + 4 * q + i]);
    }
  }
}

// One item: the unit's pairs 16 at a time against the weights in `wt`. (A prefetch of the next item's weights into a
// second buffer during this one held twice the registers and left two workgroups per CU instead of three; without
// it, FP8 / int8 / W4A8 / W6A8 at 256 rows and Zipf routing ran 168.1 / 167.6 / 127.6 / 160.7 us per layer against
// 171.0 / 169.0 / 131.9 / 166.7.) With row-scaled weights (int8, FP8) the next item's weights go into the same
// registers in the item's last tile, once its products have read them (`next_wt`), and stream during that tile's
// epilogue and barriers: 164.6 / 164.3 us against 167.8 / 167.7. (Group-scaled weights kept two workgroups per CU
// that way: W4A8 128.2 against 125.8.) Activation rows are read without a branch (columns past the unit's pairs
// read its first pair and their products are never stored). colv / colp: per column (pair) of a tile, its epilogue
// scale and (down) its pair index, staged in LDS by wave 0.
constexpr bool late_weights(int F) { return !group_scaled(F); }
template <int F, int H, int I, int MODE>
D3_INLINE void compute_tile(const PrefillArgs& a, const int* __restrict__ perm,
                            const Weights<F, Geometry<F, H, I, MODE>::SW>& wt, int4 unit_n, int4 unit, int it,
                            int c0, const float* gs, float (*part)[Geometry<F, H, I, MODE>::KS][16][17], float* colv,
                            int* colp, int& pr, Weights<F, Geometry<F, H, I, MODE>::SW>* next_wt, int it_n) {
  using G = Geometry<F, H, I, MODE>;
  constexpr int SW = G::SW, KS = G::KS, K = G::K, STEPS = K / 128;
  constexpr int SHIFT = unpack_shift(F);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, q = lane >> 4, col = lane & 15;
  const int ks = w % KS, tp = w / KS;
  const int first = unit.y, n = unit.z;
  const bool valid = c0 + col < n;
  const int sp = first + (valid ? c0 + col : 0);
  // gate_up reads the pair's own row of x (row pr / k, pr = perm[sp], loaded a tile ahead); the next tile's pair
  // (this item's, or the next item's first) is requested before this tile's activations, so it is back by then
  size_t arow = (size_t)sp;
  int pr_next = 0;
  if constexpr (MODE == 0) {
    const bool more = c0 + 16 < n;
    const int nfirst = more ? first : unit_n.y, nn = more ? n : unit_n.z, nc0 = more ? c0 + 16 : 0;
    pr_next = perm[nfirst + min(nc0 + col, nn - 1)];
    arow = (size_t)(pr / a.k);
  }
  const uint8_t* act = (MODE == 0 ? a.xq : a.hq) + arow * K + 32 * q;
  i32x4 lo[SW], hi[SW];
#pragma unroll
  for (int j = 0; j < SW; j++) {
    lo[j] = *(const i32x4*)(act + 128 * (ks * SW + j));
    hi[j] = *(const i32x4*)(act + 128 * (ks * SW + j) + 16);
  }
  if (w == 0 && lane < 16) {
    colv[col] = valid ? (MODE == 0 ? a.xs[arow] : a.hs[sp]) : 0.0f;
    if constexpr (MODE == 1) colp[col] = valid ? a.perm[sp] : 0;
  }
#pragma unroll
  for (int t = 0; t < 2; t++) {
    f32x4 y;
    if constexpr (F == FMT_F8) {
      f32x4 acc;
      i32x8 fa[SW], fb[SW];
#pragma unroll
      for (int j = 0; j < SW; j++) {
        fa[j] = f8_operand(wt.raw[t][j]);
        fb[j] = f8_operand(lo[j], hi[j]);
      }
      acc = mfma_f8_chain<SW>(fa, fb);
#pragma unroll
      for (int i = 0; i < 4; i++) y[i] = acc[i] * wt.rs[t][i];
    } else if constexpr (F == FMT_I8) {
      i32x4 acc = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < SW; j++) acc = step_i8<F>(wt.raw[t][j], lo[j], hi[j], acc);
#pragma unroll
      for (int i = 0; i < 4; i++) y[i] = (float)acc[i] * wt.rs[t][i];
    } else {
      const float* g = gs + (2 * tp + t) * 16 * STEPS;
      f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < SW; j++) {
        const i32x4 d = step_i8<F>(wt.raw[t][j], lo[j], hi[j], i32x4{0, 0, 0, 0});
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] += (float)(d[i] >> SHIFT) * g[(4 * q + i) * STEPS + ks * SW + j];
      }
      y = acc;
    }
#pragma unroll
    for (int i = 0; i < 4; i++) part[2 * tp + t][ks][4 * q + i][col] = y[i];
  }
  if (next_wt) load_weights<F, H, I, MODE>(*next_wt, a, unit_n.x, it_n, tp, ks, lane);
  __syncthreads();
  if constexpr (MODE == 0) {
    // 16 units x 16 pairs, one per thread
    const int u = tid & 15, j = tid >> 4;
    if (c0 + j < n) {
      float gv = 0.0f, uv = 0.0f;
#pragma unroll
      for (int k2 = 0; k2 < KS; k2++) {
        gv += part[0][k2][u][j];
        uv += part[1][k2][u][j];
      }
      const float xs = colv[j];
      gv *= xs;
      uv *= xs;
      a.h[(size_t)(first + c0 + j) * I + 16 * it + u] = gv / (1.0f + __expf(-gv)) * uv;
    }
  } else {
    // 64 rows x 16 pairs, four per thread; hs carries the pair's routing weight
#pragma unroll
    for (int r4 = 0; r4 < 4; r4++) {
      const int o = tid + 256 * r4, r = o & 63, j = o >> 6;
      if (c0 + j < n) {
        float v = 0.0f;
#pragma unroll
        for (int k2 = 0; k2 < KS; k2++) v += part[r >> 4][k2][r & 15][j];
        a.parts[(size_t)colp[j] * H + 64 * it + r] = v * colv[j];
      }
    }
  }
  __syncthreads();
  if constexpr (MODE == 0) pr = pr_next;
}

template <int F, int H, int I, int MODE>
D3_INLINE void compute_item(const PrefillArgs& a, const int* __restrict__ perm,
                            Weights<F, Geometry<F, H, I, MODE>::SW>& wt, int4 unit_n, int4 unit, int it,
                            float* gs, float (*part)[Geometry<F, H, I, MODE>::KS][16][17], float* colv, int* colp,
                            int& pr, bool more, int it_n) {
  using G = Geometry<F, H, I, MODE>;
  constexpr int STEPS = G::K / 128;
  const int tid = threadIdx.x;
  if constexpr (group_scaled(F)) {
    // group scales of the item's rows: gs[tile][row][step]
    const uint16_t* sb = MODE == 0 ? a.gu_s : a.dn_s;
    for (int o = tid; o < G::TILES * 16 * STEPS; o += 256) {
      const int t = o / (16 * STEPS), r = (o / STEPS) % 16, st = o % STEPS;
      gs[o] = bf16_to_f32(sb[(tile_row0<F, H, I, MODE>(a, unit.x, it, t) + r) * STEPS + st]);
    }
    __syncthreads();
  }
  const int last = (unit.z - 1) & ~15;
  if constexpr (late_weights(F)) {
    for (int c0 = 0; c0 < last; c0 += 16)
      compute_tile<F, H, I, MODE>(a, perm, wt, unit_n, unit, it, c0, gs, part, colv, colp, pr, nullptr, 0);
    compute_tile<F, H, I, MODE>(a, perm, wt, unit_n, unit, it, last, gs, part, colv, colp, pr, more ? &wt : nullptr,
                                it_n);
  } else {
    for (int c0 = 0; c0 <= last; c0 += 16)
      compute_tile<F, H, I, MODE>(a, perm, wt, unit_n, unit, it, c0, gs, part, colv, colp, pr, nullptr, 0);
  }
}

// units / meta / perm come as separate read-only kernel arguments so that their (uniform) loads are scalar loads:
// those complete apart from the waves' vector loads.
template <int F, int H, int I, int MODE>
__global__ void __launch_bounds__(256) grouped_kernel(PrefillArgs a, const int4* __restrict__ units,
                                                      const int* __restrict__ meta, const int* __restrict__ perm) {
  using G = Geometry<F, H, I, MODE>;
  __shared__ float part[G::TILES][G::KS][16][17];
  __shared__ float gs[group_scaled(F) ? G::TILES * 16 * (G::K / 128) : 1];
  __shared__ float colv[16];
  __shared__ int colp[16];
  const int n_items = meta[0] * G::PER_EXPERT;
  int i = blockIdx.x;
  if (i >= n_items) return;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, ks = w % G::KS, tp = w / G::KS;
  int4 unit = units[i / G::PER_EXPERT];
  int it = i % G::PER_EXPERT;
  const int g = (int)gridDim.x, b = (int)blockIdx.x;
  int rnd = 0;  // the round of item i
  auto item_of = [&](int r) { return r * g + ((r & 1) ? g - 1 - b : b); };
  Weights<F, G::SW> wt;
  // gate_up: this lane's pair (column lane % 16) of the first tile, ahead of the weights
  int pr = MODE == 0 ? perm[unit.y + min(lane & 15, unit.z - 1)] : 0;
  if (late_weights(F)) load_weights<F, H, I, MODE>(wt, a, unit.x, it, tp, ks, lane);
  while (true) {
    if (!late_weights(F)) load_weights<F, H, I, MODE>(wt, a, unit.x, it, tp, ks, lane);
    // the next item (this one again after the last: the next tile's pair is read from it)
    const int in = item_of(rnd + 1);
    const bool more = in < n_items;
    const int4 unit_n = units[(more ? in : i) / G::PER_EXPERT];
    const int it_n = (more ? in : i) % G::PER_EXPERT;
    compute_item<F, H, I, MODE>(a, perm, wt, unit_n, unit, it, gs, part, colv, colp, pr, more, it_n);
    if (!more) break;
    i = in;
    rnd++;
    unit = unit_n;
    it = it_n;
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
  size_t ids, weights, counts, offsets, perm, units, meta, xq, xs, h, hq, hs, parts, total;
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
  L.units = take((E + P / UNIT_PAIRS + 1) * 16);
  L.meta = take(16);
  L.xq = take(T * H);
  L.xs = take(T * 4);
  L.h = take(P * I * 4);
  L.hq = take(P * I);
  L.hs = take(P * 4);
  L.parts = take(P * H * 4);
  L.total = at;
  return L;
}

// Persistent grids: as many workgroups as the device holds at once (the kernels stop at the item count).
template <int F, int H, int I, int MODE> int resident_grid() {
  static int grid = 0;
  if (grid == 0) {
    int dev = 0, cus = 0, per = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, grouped_kernel<F, H, I, MODE>, 256, 0) != hipSuccess ||
        per < 1)
      return 1024;
    grid = cus * per;
  }
  return grid;
}
template <int F, int H, int I> void launch_products(const PrefillArgs& pa, int max_units, hipStream_t s) {
  const int grid = std::min(resident_grid<F, H, I, 0>(), max_units * (I / 16));
  hipLaunchKernelGGL((grouped_kernel<F, H, I, 0>), dim3(grid), dim3(256), 0, s, pa, pa.units, pa.meta, pa.perm);
}
template <int F, int H, int I> void launch_down(const PrefillArgs& pa, int max_units, hipStream_t s) {
  const int grid = std::min(resident_grid<F, H, I, 1>(), max_units * (H / 64));
  hipLaunchKernelGGL((grouped_kernel<F, H, I, 1>), dim3(grid), dim3(256), 0, s, pa, pa.units, pa.meta, pa.perm);
}

template <int F, int KPL> void launch_small(const SmallPrepArgs& sa, hipStream_t s) {
  hipLaunchKernelGGL((small_prep_kernel<F, 2048, KPL>), dim3(1), dim3(1024), 0, s, sa);
}

template <int F, int KPL> void launch_route_quant(const d3_moe_a8_prefill_desc& d, int64_t* ids, float* weights,
                                                 uint8_t* xq, float* xs, hipStream_t s) {
  hipLaunchKernelGGL((route_quant_kernel<F, 2048, KPL>), dim3((d.T + 3) / 4), dim3(256), 0, s,
                     (const uint16_t*)d.logits, d.ids_in, d.weights_in, (const uint16_t*)d.x, d.T, d.E, d.topk, ids,
                     weights, d.logits ? d.ids_out : nullptr, d.logits ? d.weights_out : nullptr, xq, xs);
}
template <int F> void route_quant(const d3_moe_a8_prefill_desc& d, int64_t* ids, float* weights, uint8_t* xq,
                                  float* xs, hipStream_t s) {
  if (d.E <= 128) launch_route_quant<F, 2>(d, ids, weights, xq, xs, s);
  else if (d.E <= 256) launch_route_quant<F, 4>(d, ids, weights, xq, xs, s);
  else launch_route_quant<F, 16>(d, ids, weights, xq, xs, s);
}

template <int F, int WIDTH> void launch_quantize(const float* src, int rows, uint8_t* q, float* scale,
                                                 const float* pair_weight, const int* perm, hipStream_t s) {
  hipLaunchKernelGGL((quantize_rows_kernel<F, WIDTH>), dim3((rows + 3) / 4), dim3(256), 0, s, src, rows, q, scale,
                     pair_weight, perm);
}

template <int F, int H, int I> void run(const PrefillArgs& pa, const d3_moe_a8_prefill_desc& d, const Layout& L,
                                        uint8_t* ws, hipStream_t s) {
  const int P = d.T * d.topk;
  const int max_units = std::min(d.E, P) + P / UNIT_PAIRS;
  launch_products<F, H, I>(pa, max_units, s);
  launch_quantize<F, I>((const float*)(ws + L.h), P, ws + L.hq, (float*)(ws + L.hs), pa.weights, pa.perm, s);
  launch_down<F, H, I>(pa, max_units, s);
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" {

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
  // up to 16 rows: routing, x's quantization and the grouping in one launch (one workgroup). Measured on a 2048 x
  // 768, 128-expert layer, us per layer against the wide launches (then route, group and quantize): int8 66.6 / 70.8 at 7 rows, 70.2 / 74.0 at 8, 84.2 / 87.1 at 12, 97.2 / 98.6 at 16; W4A8
  // 52.1 / 56.6, 55.5 / 59.8, 64.3 / 67.3, 73.6 / 75.3.
  const bool small = d->T <= 16 && d->topk <= 8 && d->E <= 256;
  if (small) {
    SmallPrepArgs sa;
    sa.logits = (const uint16_t*)d->logits;
    sa.ids_in = d->ids_in;
    sa.weights_in = d->weights_in;
    sa.x = (const uint16_t*)d->x;
    sa.T = d->T;
    sa.E = d->E;
    sa.k = d->topk;
    sa.ids = ids;
    sa.weights = weights;
    sa.ids_out = d->logits ? d->ids_out : nullptr;
    sa.weights_out = d->logits ? d->weights_out : nullptr;
    sa.counts = (int*)(ws + L.counts);
    sa.offsets = (int*)(ws + L.offsets);
    sa.perm = (int*)(ws + L.perm);
    sa.units = (int4*)(ws + L.units);
    sa.meta = (int*)(ws + L.meta);
    sa.xq = ws + L.xq;
    sa.xs = (float*)(ws + L.xs);
    const bool kpl2 = d->E <= 128;
    switch (d->format) {
      case D3_FMT_I8: kpl2 ? launch_small<FMT_I8, 2>(sa, s) : launch_small<FMT_I8, 4>(sa, s); break;
      case D3_FMT_W4: kpl2 ? launch_small<FMT_W4, 2>(sa, s) : launch_small<FMT_W4, 4>(sa, s); break;
      case D3_FMT_W6: kpl2 ? launch_small<FMT_W6, 2>(sa, s) : launch_small<FMT_W6, 4>(sa, s); break;
      default: kpl2 ? launch_small<FMT_F8, 2>(sa, s) : launch_small<FMT_F8, 4>(sa, s); break;
    }
  } else {
    // routing (or the caller's) and x quantized by row, a wave per row
    uint8_t* xq = ws + L.xq;
    float* xs = (float*)(ws + L.xs);
    switch (d->format) {
      case D3_FMT_I8: route_quant<FMT_I8>(*d, ids, weights, xq, xs, s); break;
      case D3_FMT_W4: route_quant<FMT_W4>(*d, ids, weights, xq, xs, s); break;
      case D3_FMT_W6: route_quant<FMT_W6>(*d, ids, weights, xq, xs, s); break;
      default: route_quant<FMT_F8>(*d, ids, weights, xq, xs, s); break;
    }
  }
  if (!small)
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), 0, s, (const int64_t*)ids, P, d->E, (int*)(ws + L.counts),
                       (int*)(ws + L.offsets), (int*)(ws + L.perm), (int4*)(ws + L.units), (int*)(ws + L.meta));
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
  pa.units = (const int4*)(ws + L.units);
  pa.meta = (const int*)(ws + L.meta);
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
