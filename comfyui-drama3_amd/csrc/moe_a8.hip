// The fused routed-expert MoE layer for A8 expert banks (int8, W4, W6 or FP8 weights; int8 or e4m3 activations
// quantized per row): route -> gate_up -> SiLU(gate) * up -> down -> routing-weighted sum, in one launch.
//
// This replaces the reference's chain of launches for one decode row (drama3/offload.py:108-123: rotate, gemv,
// rotate(swiglu), gemv, weighted_sum, after kernels.route at drama3/model.py:116-118) and its row-by-row loop over
// batched lines (drama3/model.py:111-113): M rows share one launch and every expert any of them routes to is read
// once.
//
// Work decomposition. Every workgroup (4 waves) first routes all M rows (top-k of the router logits, softmax over the
// k, bf16-rounded weights: kernels.py:39-67's semantics), builds the sorted union of their experts (U of them) and
// groups it into down chunks of at most 8 experts and 32 (expert, row) pairs. It quantizes the activations into LDS.
// Then it takes its work items (persistent; the dealing is described below):
//   gate_up item (u, tile): gate rows 16 tile .. 16 tile + 15 and the matching up rows of expert u, two 16-row MFMA
//     tiles over K = H (the 4 waves split K); the expert's rows are the MFMA columns. The epilogue applies the scales
//     and SiLU(gate) * up and publishes 16 hidden units per row.
//   down item (chunk c, block b): output rows 8 b .. 8 b + 7 of every expert of the chunk, over K = I. Each wave packs
//     two experts into one 16-row MFMA tile (rows 0-7 and 8-15) with both experts' rows as columns. It loads its
//     weights first, then collects the chunk's hidden rows as they are published, quantizes them into LDS and runs.
//     When the chunk holds every expert (always for M = 1) it writes the weighted sum straight to `out`; otherwise it
//     publishes its partial outputs and the last chunk's item for block b sums them.
// Items are ordered every gate_up item, then the down items chunk by chunk, and gate_up item k and down item k go to
// workgroup k mod gridDim, which takes its items in that order (W4A8 at two rows: gate_up(chunk 0), gate_up(chunk 1),
// down(chunk 0), gate_up(chunk 2), ..., round-robin): every wait is on items of lower index. The grid is at most what
// the device holds at once, so every workgroup is resident and the lowest unfinished item can always run: no wait
// can block forever. Waits are bounded anyway (spin_limit).
// A wait that gives up (a producer that is not resident, because another kernel holds part of the device, or a
// spin_limit hit) does not leave the output wrong: its workgroup computes what it waited for itself, with the same
// code on the same inputs, so the words it uses are the ones the producers would have published, bit for bit. The
// launch's give-up word makes the launch's other waits stop soon and do the same; a sticky bit records that it
// happened (d3_moe_a8_status).
//
// Hand-off: hidden units, each gate_up item's absmax and partial outputs are 64-bit words (value, epoch) written and
// read with device-coherent accesses (common.hpp), with no counter or flag in between: a word that has not landed yet
// is told apart by its epoch and read again. The epoch is the dispatch ID plus a salt from the queue's address
// (launch_epoch), new for every dispatch, so a workspace carries over from launch to launch (and graph replay to
// replay, on any stream) with nothing to clear. Launches that overlap on one workspace race.
#include "formats.hpp"
#include "../../include/drama3_moe.h"

#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

namespace d3 {

// workspace header (32-bit words, 256 bytes apart): the launch give-up word (64-bit: the epoch of the last launch in
// which a wait gave up, and a reason), then the sticky bits d3_moe_a8_status reads (bit 0: a wait gave up and its
// workgroup computed the missing values itself; bit 1: a wait still failed after that, the launch's output is not
// valid)
enum : int { SYNC_STATUS = 0, SYNC_STICKY = 64, SYNC_WORDS = 128 };
constexpr int MAX_M = 16, MAX_K = 8, MAX_E = 256, MAX_PAIRS = MAX_M * MAX_K;
constexpr int CHUNK_EXPERTS = 8, CHUNK_PAIRS = 32;

struct MoeA8Args {
  const uint16_t* x;
  const uint16_t* logits;
  const uint8_t* gu_w;
  const uint16_t* gu_s;
  const uint8_t* dn_w;
  const uint16_t* dn_s;
  uint16_t* out;
  int64_t* ids_out;
  float* weights_out;
  uint64_t* hidden;  // [M * topk, I] tagged
  uint64_t* tmax;    // [M * topk + 1, I / UT] tagged: absmax of each gate_up item's UT (8 or 16) hidden units
  uint64_t* parts;   // [M * topk, H] tagged
  uint64_t* status;  // the launch give-up word
  uint32_t* sticky;  // sticky status bits
  int M, E, topk;
  uint32_t spin_limit;  // 0: every wait gives up at once (the descriptor's recompute_all)
  // the block around the routed experts (one row): the router's weights [E, H] bf16 (logits computed in the launch
  // instead of read), its logits out [E] bf16; the shared expert (one A8 expert of the layer's format and shape) and
  // its gate [H] bf16
  const uint16_t* router;
  uint16_t* logits_out;
  const uint8_t* sh_gu_w;
  const uint16_t* sh_gu_s;
  const uint8_t* sh_dn_w;
  const uint16_t* sh_dn_s;
  const uint16_t* sh_gate;
  uint64_t* logitw;   // [E] tagged logits (router)
  uint64_t* sharedw;  // [H] tagged: the shared expert's gated output, bf16-rounded
  int dn_first;       // one-row schedule: workgroups dn_first .. dn_first + H / 8 - 1 take the down blocks
};

// LDS carve-up (bytes), shared by host (launch size) and device.
struct Lds {
  int xq, sx, rt_id, rt_w, emask, ulist, ucount, utok, upair, chunk_first, misc, red, hq, hs, lparts, slot_pair,
      pair_slot, slot_first, fparts, gfirst, gpair, total;
  __host__ __device__ Lds(int M, int topk, int H, int I) {
    int o = 0;
    auto take = [&](int bytes) { int at = o; o += (bytes + 15) & ~15; return at; };
    const int pairs = M * topk;
    const int pmax = pairs < CHUNK_PAIRS ? pairs : CHUNK_PAIRS;
    xq = take(M * H);
    sx = take(MAX_M * 4);
    rt_id = take(MAX_M * MAX_K * 4);
    rt_w = take(MAX_M * MAX_K * 4);
    emask = take(MAX_E * 4);
    ulist = take(MAX_E * 4);
    ucount = take(MAX_E * 4);
    utok = take(MAX_PAIRS * MAX_M);
    upair = take(MAX_PAIRS * MAX_M);
    chunk_first = take((MAX_PAIRS + 1) * 4);
    misc = take(64);
    red = take(2 * 2 * 4 * 256 * 4);
    hq = take(pmax * I);
    hs = take(pmax * 4);
    lparts = take(pmax * 8 * 4);
    slot_pair = take(pmax * 4);
    pair_slot = take(MAX_PAIRS * 4);
    slot_first = take((CHUNK_EXPERTS + 1) * 4);
    fparts = take(pairs * 8 * 4);  // every pair's 8 partial outputs of a block (chunks exceed one at 9 experts)
    gfirst = take((MAX_PAIRS + 1) * 4);
    gpair = take(MAX_PAIRS * 4);
    total = o;
  }
};

// Workgroup flags in LDS (misc[2 ..]): a wave that gave up a wait sets one; the workgroup reads it after its next
// barrier and then computes what was missing itself (see down_compute).
enum : int { FLAG_HIDDEN = 0, FLAG_SHARED = 1, FLAG_PARTS = 2, FLAG_SH_HIDDEN = 3, N_FLAGS = 4 };
// polls allowed when reading back words the workgroup has just published itself (current at the first read that goes
// past the caches)
constexpr uint32_t RECOVER_LIMIT = 1u << 16;

// What a workgroup knows after its prologue.
struct Ctx {
  const MoeA8Args* a;
  uint8_t* xq;
  float* sx;
  int* rt_id;
  float* rt_w;
  int* ulist;
  int* ucount;
  uint8_t* utok;
  uint8_t* upair;
  int* chunk_first;
  int* misc;
  uint32_t* emask;  // [MAX_E] the union's build: rows per expert, then (union position << 16 | rows)
  float* red;
  uint8_t* hq;
  float* hs;
  float* lparts;
  int* slot_pair;
  int* pair_slot;
  int* slot_first;
  float* fparts;
  // the general schedule's slots, numbered over the whole union once per launch: union expert u's pairs hold slots
  // gfirst[u] .. gfirst[u + 1] - 1, slot s holds pair gpair[s] (and pair_slot maps back)
  int* gfirst;
  int* gpair;
  int* flags;  // [N_FLAGS] see FLAG_*
  int U, nch, n_dn;
  uint32_t epoch;
};

D3_INLINE void note_recovery(const MoeA8Args& a, uint32_t bit) {
  __hip_atomic_fetch_or(a.sticky, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The recovery paths are calls, not inlined, taking plain values only: their registers then do not count against the
// kernels' fast paths (inlined, the fused kernels lost a workgroup per CU or spilled on their fast paths), and the
// kernel's context stays in registers (a reference to it would put it in scratch memory, read back on the fast path).
#define RECOVERY_FN __device__ __noinline__

// the launch's dynamic LDS (every kernel here has one array, carved up by Lds)
extern __shared__ __attribute__((aligned(16))) uint8_t d3_lds[];

// a workgroup's view of its LDS and the launch (the flags are cleared by make_ctx only)
D3_INLINE Ctx view_ctx(const MoeA8Args& a, int H, int I, uint32_t epoch) {
  uint8_t* lds = d3_lds;
  const Lds L(a.M, a.topk, H, I);
  Ctx cx;
  cx.a = &a;
  cx.xq = lds + L.xq;
  cx.sx = (float*)(lds + L.sx);
  cx.rt_id = (int*)(lds + L.rt_id);
  cx.rt_w = (float*)(lds + L.rt_w);
  cx.ulist = (int*)(lds + L.ulist);
  cx.ucount = (int*)(lds + L.ucount);
  cx.utok = lds + L.utok;
  cx.upair = lds + L.upair;
  cx.chunk_first = (int*)(lds + L.chunk_first);
  cx.misc = (int*)(lds + L.misc);
  cx.emask = (uint32_t*)(lds + L.emask);
  cx.red = (float*)(lds + L.red);
  cx.hq = lds + L.hq;
  cx.hs = (float*)(lds + L.hs);
  cx.lparts = (float*)(lds + L.lparts);
  cx.slot_pair = (int*)(lds + L.slot_pair);
  cx.pair_slot = (int*)(lds + L.pair_slot);
  cx.slot_first = (int*)(lds + L.slot_first);
  cx.gfirst = (int*)(lds + L.gfirst);
  cx.gpair = (int*)(lds + L.gpair);
  cx.fparts = (float*)(lds + L.fparts);
  cx.flags = cx.misc + 2;
  cx.epoch = epoch;
  return cx;
}

D3_INLINE Ctx make_ctx(const MoeA8Args& a, int H, int I) {
  Ctx cx = view_ctx(a, H, I, launch_epoch());
  if (threadIdx.x < N_FLAGS) cx.flags[threadIdx.x] = 0;
  return cx;
}

// The launch's arguments where the kernel received them (its kernarg segment: the one argument, at offset 0), for the
// recovery calls, which take this pointer as a parameter: then nothing of the kernel's own context has to go through
// memory to reach them. Only inside a kernel: a called function's ABI does not carry the kernarg segment pointer.
D3_INLINE const MoeA8Args* kernel_args() { return (const MoeA8Args*)__builtin_amdgcn_kernarg_segment_ptr(); }

// The context of a recovery call: as make_ctx, with the union's size and chunk count the workgroup left in LDS
D3_INLINE Ctx recovery_ctx(const MoeA8Args* args, int H, int I, uint32_t epoch) {
  Ctx cx = view_ctx(*args, H, I, epoch);
  cx.U = cx.misc[0];
  cx.nch = cx.misc[1];
  cx.n_dn = cx.nch * (H / 8);
  return cx;
}

// gate_up item: hidden units UT tile .. UT tile + UT - 1 (UT = 8 NSUB) of expert u, i.e. NSUB 16-row MFMA tiles
// (sub-tile s: gate rows UT tile + 8 s .. + 7 as rows 0-7, the matching up rows as rows 8-15)
// (`between` runs once the item's weight rows are on their way, before it reads the slot tables or x; `after` once its
// products are done, before its reduction)
template <int F, int H, int I, int NSUB = 2, typename Between, typename After>
D3_INLINE void gate_up_item(const Ctx& cx, int u, int tile, int parity, int e, int nu, Between between,
                                After after, const uint8_t* gu_w, const uint16_t* gu_s) {
  static_assert(NSUB == 1 || NSUB == 2, "8 or 16 hidden units per item");
  constexpr int UT = 8 * NSUB, T = I / UT;  // hidden units per item, items per expert
  constexpr int SPW = H / 512;  // steps per wave
  constexpr int RB = row_bytes(F, H);
  constexpr int SHIFT = unpack_shift(F);
  const MoeA8Args& a = *cx.a;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, q = lane >> 4, col = lane & 15;
  const int ra = lane & 15;
  auto row_of = [&](int sub, int r) {
    return (size_t)e * (2 * I) + (r < 8 ? UT * tile + 8 * sub + r : I + UT * tile + 8 * sub + r - 8);
  };
  Raw<F> raw[NSUB][SPW];
#pragma unroll
  for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
    for (int s = 0; s < SPW; s++) load_step<F>(raw[sub][s], gu_w + row_of(sub, ra) * RB, w * SPW + s, q);
  float sc[NSUB][SPW][4];
  if constexpr (group_scaled(F)) {
#pragma unroll
    for (int sub = 0; sub < NSUB; sub++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int s = 0; s < SPW; s++) sc[sub][s][i] = bf16_to_f32(gu_s[row_of(sub, 4 * q + i) * (H / 128) + w * SPW + s]);
  }
  // row scales for the epilogue (wave 0, unit j = lane & 15), fetched with the rows
  float gs = 1.0f, us = 1.0f;
  if constexpr (!group_scaled(F)) {
    if (w == 0) {
      gs = bf16_to_f32(gu_s[(size_t)e * (2 * I) + UT * tile + (lane & (UT - 1))]);
      us = bf16_to_f32(gu_s[(size_t)e * (2 * I) + I + UT * tile + (lane & (UT - 1))]);
    }
  }
  between();
  const bool active = col < nu;
  const uint8_t* xp = cx.xq + (size_t)(active ? cx.utok[u * MAX_M + col] : 0) * H;
  float* rd = cx.red + parity * 2048;
#pragma unroll
  for (int sub = 0; sub < NSUB; sub++) {
    i32x4 iacc = {0, 0, 0, 0};
    f32x4 facc = {0.0f, 0.0f, 0.0f, 0.0f};
    i32x8 fa[SPW], fb[SPW];
#pragma unroll
    for (int s = 0; s < SPW; s++) {
      i32x4 xlo = {0, 0, 0, 0}, xhi = {0, 0, 0, 0};
      if (active) {
        const uint8_t* p = xp + 128 * (w * SPW + s) + 32 * q;
        xlo = *(const i32x4*)p;
        xhi = *(const i32x4*)(p + 16);
      }
      if constexpr (F == FMT_I8) {
        iacc = step_i8<F>(raw[sub][s], xlo, xhi, iacc);
      } else if constexpr (F == FMT_F8) {
        fa[s] = f8_operand(raw[sub][s]);
        fb[s] = f8_operand(xlo, xhi);
      } else {
        const i32x4 g = step_i8<F>(raw[sub][s], xlo, xhi, i32x4{0, 0, 0, 0});
#pragma unroll
        for (int i = 0; i < 4; i++) facc[i] += (float)(g[i] >> SHIFT) * sc[sub][s][i];
      }
    }
    if constexpr (F == FMT_F8) facc = mfma_f8_chain<SPW>(fa, fb);
#pragma unroll
    for (int i = 0; i < 4; i++)
      rd[sub * 1024 + w * 256 + (4 * q + i) * 16 + col] = F == FMT_I8 ? __int_as_float(iacc[i]) : facc[i];
  }
  after();
  __syncthreads();
  if (w == 0) {
    for (int idx = lane; idx < 16 * nu; idx += 64) {
      // lanes 16 n + j, j < UT: unit j of the item for its n-th row (with UT = 8, lanes j >= 8 publish nothing)
      const int n = idx >> 4, j = idx & 15, sub = (j >> 3) & (NSUB - 1), jj = j & 7;
      const bool unit = j < UT;
      const float* rs = rd + sub * 1024;
      float g, up;
      if constexpr (F == FMT_I8) {
        int gi = 0, ui = 0;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
          gi += __float_as_int(rs[ww * 256 + jj * 16 + n]);
          ui += __float_as_int(rs[ww * 256 + (8 + jj) * 16 + n]);
        }
        g = (float)gi;
        up = (float)ui;
      } else {
        g = 0.0f;
        up = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
          g += rs[ww * 256 + jj * 16 + n];
          up += rs[ww * 256 + (8 + jj) * 16 + n];
        }
      }
      if constexpr (!group_scaled(F)) {
        g *= gs;
        up *= us;
      }
      const float s = cx.sx[cx.utok[u * MAX_M + n]];
      g *= s;
      up *= s;
      const float h = g / (1.0f + __expf(-g)) * up;
      const int p = cx.upair[u * MAX_M + n];
      if (unit) put_tagged(a.hidden + (size_t)p * I + UT * tile + j, h, cx.epoch);
      // absmax of the row's UT units: lanes 16n .. 16n + 15 (quad swaps, half-row and row mirrors)
      float m = unit ? fabsf(h) : 0.0f;
      m = fmaxf(m, __int_as_float(dpp_i32(__float_as_int(m), 0xB1)));
      m = fmaxf(m, __int_as_float(dpp_i32(__float_as_int(m), 0x4E)));
      m = fmaxf(m, __int_as_float(dpp_i32(__float_as_int(m), 0x141)));
      m = fmaxf(m, __int_as_float(dpp_i32(__float_as_int(m), 0x140)));
      if (j == 0) put_tagged(a.tmax + (size_t)p * T + tile, m, cx.epoch);
    }
  }
}

// Every gate_up item of chunk c's experts, computed and published by this workgroup: the recovery of a down item whose
// wait for them gave up.
template <int F, int H, int I, int NSUB>
D3_INLINE void recompute_gate_up(const Ctx& cx, int c) {
  constexpr int T = I / (8 * NSUB);
  const MoeA8Args& a = *cx.a;
  int parity = 0;
#pragma unroll 1
  for (int u = cx.chunk_first[c]; u < cx.chunk_first[c + 1]; u++) {
#pragma unroll 1
    for (int tile = 0; tile < T; tile++) {
      gate_up_item<F, H, I, NSUB>(cx, u, tile, parity, cx.ulist[u], cx.ucount[u], [] {}, [] {}, a.gu_w, a.gu_s);
      parity ^= 1;
    }
  }
}


// A down item's weight rows (this lane's: local expert 2w + (row / 8), output row 8 hb + row % 8) and the scales of
// its accumulator rows, held in registers from their loads to the item's products.
template <int F, int I>
struct DownRows {
  static constexpr int STEPS = I / 128;
  Raw<F> raw[STEPS];
  // scales as loaded (bf16 pairs, converted where the products use them, so that nothing waits for the loads
  // before then): W4 / W6 the 4 rows' group scales, row-major [4][STEPS]; I8 / F8 the 4 row scales
  uint32_t sw[group_scaled(F) ? 2 * STEPS : 2];
  D3_INLINE float scale(int i, int s) const {  // group scale of row i, step s (W4 / W6)
    const int k = i * STEPS + s;
    return bf16_to_f32((k & 1) ? sw[k >> 1] >> 16 : sw[k >> 1] & 0xFFFFu);
  }
  D3_INLINE float row_scale(int i) const {  // I8 / F8
    return bf16_to_f32((i & 1) ? sw[i >> 1] >> 16 : sw[i >> 1] & 0xFFFFu);
  }
};

// issue the loads of down item (c, hb): output rows 8 hb .. 8 hb + 7 of the experts of chunk c
template <int F, int H, int I>
D3_INLINE void down_load(const Ctx& cx, int c, int hb, DownRows<F, I>& d) {
  constexpr int STEPS = I / 128;
  constexpr int RB = row_bytes(F, I);
  const MoeA8Args& a = *cx.a;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, q = lane >> 4;
  const int u0 = cx.chunk_first[c], ne = cx.chunk_first[c + 1] - u0;
  const int ra = lane & 15;
  const int lj_a = 2 * w + (ra >> 3);
#pragma unroll
  for (int s = 0; s < STEPS; s++) d.raw[s] = Raw<F>{};
  if (lj_a < ne) {
    const int e = cx.ulist[u0 + lj_a];
    const uint8_t* wp = a.dn_w + ((size_t)e * H + 8 * hb + (ra & 7)) * RB;
#pragma unroll
    for (int s = 0; s < STEPS; s++) load_step<F>(d.raw[s], wp, s, q);
  }
  // scales of this lane's accumulator rows 4q + i: local expert 2w + q / 2, output row 8 hb + 4 (q % 2) + i (the 4
  // rows' scales are contiguous: 8 bytes, or 4 * STEPS * 2 bytes of group scales, aligned to their size's 8 / 16)
  const int lj_c = 2 * w + (q >> 1);
  const int e_c = cx.ulist[u0 + min(lj_c, ne - 1)];
  const uint16_t* sp = a.dn_s + ((size_t)e_c * H + 8 * hb + 4 * (q & 1)) * (group_scaled(F) ? STEPS : 1);
  if constexpr (group_scaled(F)) {
    static_assert(STEPS % 2 == 0, "whole 16-byte groups of scales");
#pragma unroll
    for (int k = 0; k < STEPS / 2; k++) {
      const i32x4 v = *(const i32x4*)(sp + 8 * k);
      d.sw[4 * k] = (uint32_t)v.x;
      d.sw[4 * k + 1] = (uint32_t)v.y;
      d.sw[4 * k + 2] = (uint32_t)v.z;
      d.sw[4 * k + 3] = (uint32_t)v.w;
    }
  } else {
    const i32x2 v = *(const i32x2*)sp;
    d.sw[0] = (uint32_t)v.x;
    d.sw[1] = (uint32_t)v.y;
  }
}

// The gather of down item (c, hb): the chunk's pairs' hidden rows, quantized into LDS slots (hq, hs). Returns whether
// this wave gave up waiting for words not yet published (wave-uniform).
// The pairs' hidden rows are gathered two at a time per wave (a pair per half-wave: the tiles' maxima and the values
// in one round trip). Each wave gathers its own two experts' pairs, or with SPREAD the chunk's pairs go round the
// workgroup's 8 half-waves (one round trip for up to 8 pairs, where a wave whose experts hold 3 or more needed two).
// Without GLOBAL the gather is issued once the wave's weight rows have arrived (its loads complete in order, so
// anything issued earlier would be read early and come back no sooner); with GLOBAL it goes out behind them at once.
// The words carry their epoch, so a gather that finds every word current needs nothing else. Otherwise the stale words
// are read again, coherently, until they are current. (Not a counter of finished items first: every waiting wave would
// poll the same few words, and by the time a first gather is back the late items are mostly published.)
template <int F, int H, int I, int NSUB, bool GLOBAL, bool SPREAD>
D3_INLINE bool down_gather(const Ctx& cx, int c, uint32_t limit) {
  constexpr float QMAX = act_qmax<F>();
  const MoeA8Args& a = *cx.a;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int u0 = cx.chunk_first[c], ne = cx.chunk_first[c + 1] - u0;
  const int* slot_first = GLOBAL ? cx.gfirst + u0 : cx.slot_first;
  const int gb = GLOBAL ? cx.gfirst[u0] : 0;      // the chunk's first slot in the launch-wide numbering
  const int* slot_pair = GLOBAL ? cx.gpair + gb : cx.slot_pair;
  // slot_first[lj] - gb: the chunk's slots count from 0 (its LDS rows)
  const int P = slot_first[ne] - gb;
  constexpr int T = I / (8 * NSUB);     // gate_up items per expert
  constexpr int HPL = I / 32;           // hidden words per lane of a half-wave
  static_assert(I % 32 == 0, "whole words per lane");
  constexpr int TPH = (T + 31) / 32;    // tile maxima per lane of a half-wave
  const int la = 2 * w, lb = 2 * w + 1;
  const bool has_b = lb < ne;
  const bool gathers = SPREAD || la < ne;
  const int s0 = SPREAD || !gathers ? 0 : slot_first[la] - gb;
  const int s1 = SPREAD ? P : !gathers ? 0 : slot_first[has_b ? lb + 1 : la + 1] - gb;
  bool gave = false;
  if (gathers) {
    if (!GLOBAL) settle();
    const int half = lane >> 5, hl = lane & 31;
    for (int sp = SPREAD ? 2 * w : s0; sp < s1; sp += SPREAD ? 8 : 2) {
      const int slot = sp + half;
      const bool on = slot < s1;
      const int p = slot_pair[on ? slot : s0];
      // lane hl reads words hl + 32 j: every load covers 256 contiguous bytes of the half-wave's row
      const uint64_t* hrow = a.hidden + (size_t)p * I + hl;
      // every lane loads (addresses clamped to a pair and an item of the unit), without a branch per load; lanes
      // without a word of their own then hold a current word of value 0
      const uint64_t* trow = a.tmax + (size_t)p * T;
      const uint64_t cur = (uint64_t)cx.epoch << 32;
      uint64_t mw[TPH], vw[HPL];
#pragma unroll
      for (int k = 0; k < TPH; k++) mw[k] = get_tagged_cached(trow + min(hl + 32 * k, T - 1));
#pragma unroll
      for (int j = 0; j < HPL; j++) vw[j] = get_tagged_cached(hrow + 32 * j);
#pragma unroll
      for (int k = 0; k < TPH; k++)
        if (!on || hl + 32 * k >= T) mw[k] = cur;
#pragma unroll
      for (int j = 0; j < HPL; j++)
        if (!on) vw[j] = cur;
      // words not yet current: read again, coherently. The check ORs the words' tag differences and compares once
      // (a compare and a mask step per word made a serial chain of some 30 dependent steps)
      uint32_t stale = 0;
#pragma unroll
      for (int k = 0; k < TPH; k++) stale |= tag_diff(mw[k], cx.epoch);
#pragma unroll
      for (int j = 0; j < HPL; j++) stale |= tag_diff(vw[j], cx.epoch);
      if (limit == 0) {
        gave = true;  // recompute_all: as if the producers never came
      } else if (!__all(stale == 0u)) {
        // While waiting, only the item maxima are read again (TPH words a lane; an item stores its maximum after its
        // hidden words): re-reading every stale hidden word each round cost as much memory traffic, over the down
        // blocks, as their weight rows. Once the maxima are current, the hidden words still stale are read again.
        uint32_t polls = 0;
        while (true) {
          uint32_t stale_m = 0;
#pragma unroll
          for (int k = 0; k < TPH; k++) {
            if (!tag_is(mw[k], cx.epoch)) mw[k] = get_tagged(trow + min(hl + 32 * k, T - 1));
            stale_m |= tag_diff(mw[k], cx.epoch);
          }
          if (__all(stale_m == 0u)) {
            stale = 0;
#pragma unroll
            for (int j = 0; j < HPL; j++) {
              if (!tag_is(vw[j], cx.epoch)) vw[j] = get_tagged(hrow + 32 * j);
              stale |= tag_diff(vw[j], cx.epoch);
            }
            if (__all(stale == 0u)) break;
          }
          if (!keep_polling(polls, a.status, limit, cx.epoch, limit == RECOVER_LIMIT)) {
            gave = true;
            break;
          }
        }
      }
      // the pair's absmax over its tiles' maxima: a half-wave reduction (rows 0-1 or 2-3 of the wave)
      float m = 0.0f;
#pragma unroll
      for (int k = 0; k < TPH; k++) m = fmaxf(m, tagged_value(mw[k]));
      m = fmaxf(m, __int_as_float(dpp_i32(__float_as_int(m), 0xB1)));
      m = fmaxf(m, __int_as_float(dpp_i32(__float_as_int(m), 0x4E)));
      m = fmaxf(m, __int_as_float(dpp_i32(__float_as_int(m), 0x141)));
      m = fmaxf(m, __int_as_float(dpp_i32(__float_as_int(m), 0x140)));
      const float m0 = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 0)),
                             __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 16)));
      const float m1 = fmaxf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 32)),
                             __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 48)));
      const float amax = half ? m1 : m0;
      const float inv = amax > 0.0f ? QMAX / amax : 0.0f;
      if (on) {
        uint8_t* hrow_q = cx.hq + (size_t)slot * I;
#pragma unroll
        for (int j = 0; j < HPL; j++) hrow_q[act8_pos<F>(hl + 32 * j)] = (uint8_t)act8_byte<F>(tagged_value(vw[j]), inv);
        if (hl == 0) cx.hs[slot] = amax / QMAX;
      }
    }
  }
  return gave;
}

// The products of down item (c, hb) against the gathered slots: each wave's two experts' 8 output rows, times the
// slots' scales, into lparts [slot, 8].
template <int F, int H, int I, bool GLOBAL>
D3_INLINE void down_products(const Ctx& cx, int c, const DownRows<F, I>& d) {
  constexpr int STEPS = I / 128;
  constexpr int SHIFT = unpack_shift(F);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, q = lane >> 4, col = lane & 15;
  const int u0 = cx.chunk_first[c], ne = cx.chunk_first[c + 1] - u0;
  const int* slot_first = GLOBAL ? cx.gfirst + u0 : cx.slot_first;
  const int gb = GLOBAL ? cx.gfirst[u0] : 0;
  const int la = 2 * w, lb = 2 * w + 1;
  const bool has_b = lb < ne;
  if (la < ne) {
    const int na = slot_first[la + 1] - slot_first[la];
    const int nb = has_b ? slot_first[lb + 1] - slot_first[lb] : 0;
    const bool one_pass = na + nb <= 16;
    const bool rows_b = q >= 2;
    for (int pass = 0; pass < (one_pass ? 1 : 2); pass++) {
      // columns: pass 0 = a's pairs (then b's, in one pass); pass 1 = b's pairs
      int slot = -1;
      if (pass == 0) {
        if (col < na) slot = slot_first[la] - gb + col;
        else if (one_pass && col < na + nb) slot = slot_first[lb] - gb + col - na;
      } else if (col < nb) {
        slot = slot_first[lb] - gb + col;
      }
      const uint8_t* xp = cx.hq + (size_t)(slot >= 0 ? slot : 0) * I;
      i32x4 iacc = {0, 0, 0, 0};
      f32x4 facc = {0.0f, 0.0f, 0.0f, 0.0f};
      i32x8 fa[STEPS], fb[STEPS];
#pragma unroll
      for (int s = 0; s < STEPS; s++) {
        i32x4 xlo = {0, 0, 0, 0}, xhi = {0, 0, 0, 0};
        if (slot >= 0) {
          xlo = *(const i32x4*)(xp + 128 * s + 32 * q);
          xhi = *(const i32x4*)(xp + 128 * s + 32 * q + 16);
        }
        if constexpr (F == FMT_I8) {
          iacc = step_i8<F>(d.raw[s], xlo, xhi, iacc);
        } else if constexpr (F == FMT_F8) {
          fa[s] = f8_operand(d.raw[s]);
          fb[s] = f8_operand(xlo, xhi);
        } else {
          const i32x4 g = step_i8<F>(d.raw[s], xlo, xhi, i32x4{0, 0, 0, 0});
#pragma unroll
          for (int i = 0; i < 4; i++) facc[i] += (float)(g[i] >> SHIFT) * d.scale(i, s);
        }
      }
      if constexpr (F == FMT_F8) facc = mfma_f8_chain<STEPS>(fa, fb);
      // this lane's accumulator rows belong to expert a (q < 2) or b (q >= 2); keep the products of matching columns
      const bool valid = slot >= 0 && (one_pass ? (rows_b ? col >= na : col < na) : (pass == 0 ? !rows_b : rows_b));
      if (valid) {
        const float hsc = cx.hs[slot];
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int r = 4 * (q & 1) + i;
          float y;
          if constexpr (F == FMT_I8) y = (float)iacc[i] * d.row_scale(i);
          else if constexpr (F == FMT_F8) y = facc[i] * d.row_scale(i);
          else y = facc[i];
          cx.lparts[slot * 8 + r] = y * hsc;
        }
      }
    }
  }
}

// Down item (c, hb) up to its partial outputs (lparts) once its loads are out: the slot tables, the gather, the
// products. GLOBAL: the slots come from the launch-wide tables (general schedule) and the gather goes out behind the
// weight rows at once; otherwise thread 0 numbers the chunk's slots first and the gather waits for the weight rows
// (one row: see one_row_layer). Returns false when a wave's wait gave up (the same in every thread).
// RECOVERY: the item run again after such a give-up, computing everything it depends on itself: every gate_up item of
// the chunk first (the same code on the same inputs, publishing the words the items would have published), its rows
// loaded again, then the gather reads its own words back.
template <int F, int H, int I, int NSUB, bool GLOBAL, bool SPREAD, bool RECOVERY>
D3_INLINE bool down_compute(const Ctx& cx, int c, int hb, DownRows<F, I>& d) {
  const int tid = threadIdx.x;
  if (RECOVERY) {
    recompute_gate_up<F, H, I, NSUB>(cx, c);
    down_load<F, H, I>(cx, c, hb, d);
    __syncthreads();  // the recomputed words are stored (the barrier waits for them) before anyone reads them back
  }
  if (!GLOBAL) {
    if (tid == 0) {
      const int u0 = cx.chunk_first[c], ne = cx.chunk_first[c + 1] - u0;
      int slot = 0;
      for (int lj = 0; lj < ne; lj++) {
        const int uu = u0 + lj;
        cx.slot_first[lj] = slot;
        for (int n = 0; n < cx.ucount[uu]; n++) {
          const int p = cx.upair[uu * MAX_M + n];
          cx.slot_pair[slot] = p;
          cx.pair_slot[p] = slot;
          slot++;
        }
      }
      cx.slot_first[ne] = slot;
    }
    __syncthreads();
  }
  const bool gave = down_gather<F, H, I, NSUB, GLOBAL, SPREAD>(cx, c, RECOVERY ? RECOVER_LIMIT : cx.a->spin_limit);
  if (gave && (tid & 63) == 0) {
    if (RECOVERY) note_recovery(*cx.a, 2u);
    else cx.flags[FLAG_HIDDEN] = 1;
  }
  // the slots are in LDS before the products read them: this wave's own, or with SPREAD every wave's
  if (SPREAD) __syncthreads();
  else settle();
  if (RECOVERY || (SPREAD ? cx.flags[FLAG_HIDDEN] == 0 : !gave)) down_products<F, H, I, GLOBAL>(cx, c, d);
  __syncthreads();
  return RECOVERY || cx.flags[FLAG_HIDDEN] == 0;
}

template <int F, int H, int I, int NSUB, bool RECOVERY>
D3_INLINE bool shared_down_block(const Ctx& cx, int b, const i32x4* xraw);

// the rest of down item (c, hb) once its loads are out: down_compute, then the weighted sum (one chunk: straight to
// `out`, plus the shared expert's term in the block) or the partial outputs (MULTI: several chunks, the last chunk's
// item sums them). Returns false when a wait gave up (the same in every thread); the caller then runs the item again
// with RECOVERY, which computes everything the item depends on itself: the chunk's gate_up items, the shared expert's
// block of output rows, the other chunks' partial outputs of this block.
template <int F, int H, int I, int NSUB, bool GLOBAL, bool SPREAD, bool MULTI, bool RECOVERY>
D3_INLINE bool down_finish(const Ctx& cx, int c, int hb, DownRows<F, I>& d) {
  const MoeA8Args& a = *cx.a;
  const int tid = threadIdx.x;
  const int M = a.M, K8 = a.topk;
  const uint32_t limit = RECOVERY ? RECOVER_LIMIT : a.spin_limit;
  if (!down_compute<F, H, I, NSUB, GLOBAL, SPREAD, RECOVERY>(cx, c, hb, d)) return false;
  if (!MULTI || cx.nch == 1) {
    // every row's experts are in this chunk
    if (RECOVERY && a.sh_dn_w) {
      // the shared expert's block of 64 output rows holding these 8, computed here
      const int lane = tid & 63;
      i32x4 xraw[H / 512];
#pragma unroll
      for (int k = 0; k < H / 512; k++) xraw[k] = *(const i32x4*)(a.x + 512 * k + 8 * lane);
      shared_down_block<F, H, I, NSUB, true>(cx, hb >> 3, xraw);
      __syncthreads();
    }
    for (int idx = tid; idx < M * 8; idx += 256) {
      const int t = idx >> 3, r = idx & 7;
      float acc = 0.0f;
      for (int j = 0; j < K8; j++) acc = fmaf(cx.lparts[cx.pair_slot[t * K8 + j] * 8 + r], cx.rt_w[t * MAX_K + j], acc);
      if (a.sh_dn_w) {
        // the shared expert's gated output of this row (one row): the block's sum of two bf16 tensors
        const uint64_t* src = a.sharedw + 8 * hb + r;
        uint64_t word = RECOVERY ? get_tagged(src) : limit == 0 ? 0 : get_tagged_cached(src);
        uint32_t polls = 0;
        while (!tag_is(word, cx.epoch) && keep_polling(polls, a.status, limit, cx.epoch, limit == RECOVER_LIMIT)) word = get_tagged(src);
        if (!tag_is(word, cx.epoch)) {
          if (RECOVERY) note_recovery(a, 2u);
          else cx.flags[FLAG_SHARED] = 1;
        }
        acc = bf16_round(acc) + tagged_value(word);
      }
      a.out[(size_t)t * H + 8 * hb + r] = (uint16_t)f32_to_bf16(acc);
    }
    if (!RECOVERY && a.sh_dn_w) {
      __syncthreads();
      if (cx.flags[FLAG_SHARED] != 0) return false;
    }
    return true;
  }
  {
    const int u0 = cx.chunk_first[c], ne = cx.chunk_first[c + 1] - u0;
    const int* slot_first = GLOBAL ? cx.gfirst + u0 : cx.slot_first;
    const int gb = GLOBAL ? cx.gfirst[u0] : 0;
    const int* slot_pair = GLOBAL ? cx.gpair + gb : cx.slot_pair;
    const int P = slot_first[ne] - gb;
    for (int idx = tid; idx < P * 8; idx += 256) {
      const int slot = idx >> 3, r = idx & 7;
      put_tagged(a.parts + (size_t)slot_pair[slot] * H + 8 * hb + r, cx.lparts[slot * 8 + r], cx.epoch);
    }
  }
  if (c != cx.nch - 1) return true;
  if (RECOVERY) {
    // the other chunks' items of this block, computed here
    __syncthreads();  // lparts and the slot tables are rewritten by the next chunk
#pragma unroll 1
    for (int c2 = 0; c2 < cx.nch - 1; c2++) {
      down_compute<F, H, I, NSUB, GLOBAL, SPREAD, true>(cx, c2, hb, d);
      const int v0 = cx.chunk_first[c2], nv = cx.chunk_first[c2 + 1] - v0;
      const int* sf2 = GLOBAL ? cx.gfirst + v0 : cx.slot_first;
      const int gb2 = GLOBAL ? cx.gfirst[v0] : 0;
      const int* sp2 = GLOBAL ? cx.gpair + gb2 : cx.slot_pair;
      for (int idx = tid; idx < (sf2[nv] - gb2) * 8; idx += 256) {
        const int slot = idx >> 3, r = idx & 7;
        put_tagged(a.parts + (size_t)sp2[slot] * H + 8 * hb + r, cx.lparts[slot * 8 + r], cx.epoch);
      }
      __syncthreads();  // stored before they are read back; lparts and the slot tables are rewritten next
    }
  }
  // the last chunk's item gathers every pair's partial outputs of this block
  for (int idx = tid; idx < M * K8 * 8; idx += 256) {
    const int p = idx >> 3, r = idx & 7;
    const uint64_t* src = a.parts + (size_t)p * H + 8 * hb + r;
    uint64_t word = RECOVERY ? get_tagged(src) : limit == 0 ? 0 : get_tagged_cached(src);
    uint32_t polls = 0;
    while (!tag_is(word, cx.epoch) && keep_polling(polls, a.status, limit, cx.epoch, limit == RECOVER_LIMIT)) word = get_tagged(src);
    if (!tag_is(word, cx.epoch)) {
      if (RECOVERY) note_recovery(a, 2u);
      else cx.flags[FLAG_PARTS] = 1;
    }
    cx.fparts[idx] = tagged_value(word);
  }
  __syncthreads();
  if (!RECOVERY && cx.flags[FLAG_PARTS] != 0) return false;
  for (int idx = tid; idx < M * 8; idx += 256) {
    const int t = idx >> 3, r = idx & 7;
    float acc = 0.0f;
    for (int j = 0; j < K8; j++) acc = fmaf(cx.fparts[(t * K8 + j) * 8 + r], cx.rt_w[t * MAX_K + j], acc);
    a.out[(size_t)t * H + 8 * hb + r] = (uint16_t)f32_to_bf16(acc);
  }
  return true;
}

// After a recovery: the workgroup's flags cleared once every wave has read them (the caller's barriers since), and
// the event recorded in the sticky bits
D3_INLINE void end_recovery(const Ctx& cx) {
  __syncthreads();
  if (threadIdx.x < N_FLAGS) cx.flags[threadIdx.x] = 0;
}

// Down item (c, hb) run again with RECOVERY after a wait gave up (a call: see RECOVERY_FN).
template <int F, int H, int I, int NSUB, bool GLOBAL, bool SPREAD, bool MULTI>
RECOVERY_FN void recover_down(const MoeA8Args* args, uint32_t epoch, int c, int hb) {
  const Ctx cx = recovery_ctx(args, H, I, epoch);
  if (threadIdx.x == 0) note_recovery(*cx.a, 1u);
  DownRows<F, I> d;
  down_finish<F, H, I, NSUB, GLOBAL, SPREAD, MULTI, true>(cx, c, hb, d);
  end_recovery(cx);
}

// down item (c, hb) of the general schedule (GLOBAL as for down_finish)
template <int F, int H, int I, bool GLOBAL>
D3_INLINE void down_item(const Ctx& cx, int c, int hb) {
  __syncthreads();  // the previous item's readers of the slot tables and partial outputs are done
  DownRows<F, I> d;
  down_load<F, H, I>(cx, c, hb, d);
  if (!down_finish<F, H, I, 2, GLOBAL, true, true, false>(cx, c, hb, d))
    recover_down<F, H, I, 2, GLOBAL, true, true>(kernel_args(), cx.epoch, c, hb);
}

// The router's logit e for one row, as bf16 bits: bf16(x . router[e]) with float sums (model.py:115), x as every wave
// holds it (lane l: columns 512 k + 8 l .. + 7 of chunk k); the same in every lane.
// bf16(x . v) with float sums in the block's order: lane l takes columns 512 k + 8 l .. + 7, then a wave sum
template <int H>
D3_INLINE float row_dot(const uint16_t* v, const i32x4* xraw, int lane) {
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < H / 512; k++) {
    const i32x4 wv = *(const i32x4*)(v + 512 * k + 8 * lane);
    const uint32_t xs[4] = {(uint32_t)xraw[k].x, (uint32_t)xraw[k].y, (uint32_t)xraw[k].z, (uint32_t)xraw[k].w};
    const uint32_t ws[4] = {(uint32_t)wv.x, (uint32_t)wv.y, (uint32_t)wv.z, (uint32_t)wv.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      acc = fmaf(bf16_to_f32(xs[j] & 0xFFFFu), bf16_to_f32(ws[j] & 0xFFFFu), acc);
      acc = fmaf(bf16_to_f32(xs[j] >> 16), bf16_to_f32(ws[j] >> 16), acc);
    }
  }
  return wave_sum_f32(acc);
}

template <int H>
D3_INLINE uint32_t router_dot(const MoeA8Args& a, int e, const i32x4* xraw, int lane) {
  return f32_to_bf16(row_dot<H>(a.router + (size_t)e * H, xraw, lane));
}

// the shared expert's gate weight of a row: bf16(sigmoid(bf16(x . gate))), as model.py:123's bf16 ops round it
template <int H>
D3_INLINE float shared_gate_weight(const uint16_t* gate, const i32x4* xraw, int lane) {
  const float g = bf16_round(row_dot<H>(gate, xraw, lane));
  return bf16_round(1.0f / (1.0f + expf(-g)));
}

// router_dot published as a tagged word (its bf16 bits) for every routing wave
template <int H>
D3_INLINE void router_logit(const MoeA8Args& a, uint32_t epoch, int e, const i32x4* xraw, int lane) {
  const uint32_t bits = router_dot<H>(a, e, xraw, lane);
  if (lane == 0) {
    put_tagged(a.logitw + e, __uint_as_float(bits), epoch);
    if (a.logits_out) a.logits_out[e] = (uint16_t)bits;
  }
}

// The router's logits as bf16 bits for experts lane + 64 j, once every one is published (reads of words not yet
// landed are repeated, bounded by spin_limit). When the wait gives up, the wave computes the logits still missing
// itself (router_dot: the value their workgroups would have published).
template <int H, int KPL>
D3_INLINE void gather_logits(const MoeA8Args& a, uint32_t epoch, int lane, uint32_t* lb, const i32x4* xraw) {
  uint64_t wv[KPL];
#pragma unroll
  for (int j = 0; j < KPL; j++) wv[j] = get_tagged_cached(a.logitw + min(lane + 64 * j, a.E - 1));
  bool fresh = a.spin_limit != 0;  // recompute_all: as if no logit had come
#pragma unroll
  for (int j = 0; j < KPL; j++) fresh = fresh && tag_is(wv[j], epoch);
  if (!__all(fresh)) {
    uint32_t polls = 0;
    bool ok = false;
    while (!ok && a.spin_limit != 0) {
      ok = true;
#pragma unroll
      for (int j = 0; j < KPL; j++) {
        if (!tag_is(wv[j], epoch)) wv[j] = get_tagged(a.logitw + min(lane + 64 * j, a.E - 1));
        ok = ok && tag_is(wv[j], epoch);
      }
      ok = __all(ok);
      if (!ok && !keep_polling(polls, a.status, a.spin_limit, epoch)) break;
    }
    if (!ok) {
      if (lane == 0) note_recovery(a, 1u);
#pragma unroll
      for (int j = 0; j < KPL; j++) {
        uint64_t missing = __ballot((a.spin_limit == 0 || !tag_is(wv[j], epoch)) && lane + 64 * j < a.E);
        while (missing != 0u) {
          const int l = __builtin_ctzll(missing);
          missing &= missing - 1u;
          const uint32_t bits = router_dot<H>(a, l + 64 * j, xraw, lane);
          if (lane == l) wv[j] = bits;
        }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < KPL; j++) lb[j] = (uint32_t)wv[j] & 0xFFFFu;
}

// x (bf16, as every wave holds it) quantized per row into LDS (xq, sx[0]): wave w stores chunk w (H = 2048), the
// columns its MFMA steps read
template <int F, int H>
D3_INLINE void quantize_x_lds(const Ctx& cx, const i32x4* xraw) {
  constexpr float QMAX = act_qmax<F>();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  float v[H / 512][8];
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < H / 512; k++) {
    const uint32_t wv[4] = {(uint32_t)xraw[k].x, (uint32_t)xraw[k].y, (uint32_t)xraw[k].z, (uint32_t)xraw[k].w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[k][2 * j] = bf16_to_f32(wv[j] & 0xFFFFu);
      v[k][2 * j + 1] = bf16_to_f32(wv[j] >> 16);
      amax = fmaxf(amax, fmaxf(fabsf(v[k][2 * j]), fabsf(v[k][2 * j + 1])));
    }
  }
  amax = wave_max_f32(amax);
  const float inv = amax > 0.0f ? QMAX / amax : 0.0f;
#pragma unroll
  for (int k = 0; k < H / 512; k++)
    if (k == w) store_act8<F>(cx.xq + 512 * k + 8 * lane, v[k], inv);
  if (lane == 0) cx.sx[0] = amax / QMAX;
}

// The shared expert's hidden row (pair topk) and its items' maxima, lane l holding words l + 64 j (each load covers
// 512 contiguous bytes); words not yet published are read again, coherently, until they carry the launch's epoch
// (polling the expert's counter first, as every waiting wave of these blocks would, cost 2-2.5 us per block). Returns
// whether the wave gave up.
template <int I, int T, int TPW, int HPW>
D3_INLINE bool shared_gather(const Ctx& cx, uint32_t limit, uint64_t* mw, uint64_t* vw, bool cached) {
  const MoeA8Args& a = *cx.a;
  const int lane = threadIdx.x & 63;
  const uint64_t* hrow = a.hidden + (size_t)a.topk * I;
  const uint64_t* trow = a.tmax + (size_t)a.topk * T;
#pragma unroll
  for (int k = 0; k < TPW; k++)
    mw[k] = cached ? get_tagged_cached(trow + min(lane + 64 * k, T - 1)) : get_tagged(trow + min(lane + 64 * k, T - 1));
#pragma unroll
  for (int j = 0; j < HPW; j++) vw[j] = cached ? get_tagged_cached(hrow + lane + 64 * j) : get_tagged(hrow + lane + 64 * j);
  bool fresh = true;
#pragma unroll
  for (int k = 0; k < TPW; k++) fresh = fresh && tag_is(mw[k], cx.epoch);
#pragma unroll
  for (int j = 0; j < HPW; j++) fresh = fresh && tag_is(vw[j], cx.epoch);
  if (limit == 0) return true;  // recompute_all
  if (__all(fresh)) return false;
  uint32_t polls = 0;
  while (true) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < TPW; k++) {
      if (!tag_is(mw[k], cx.epoch)) mw[k] = get_tagged(trow + min(lane + 64 * k, T - 1));
      ok = ok && tag_is(mw[k], cx.epoch);
    }
#pragma unroll
    for (int j = 0; j < HPW; j++) {
      if (!tag_is(vw[j], cx.epoch)) vw[j] = get_tagged(hrow + lane + 64 * j);
      ok = ok && tag_is(vw[j], cx.epoch);
    }
    if (__all(ok)) return false;
    if (!keep_polling(polls, a.status, limit, cx.epoch, limit == RECOVER_LIMIT)) return true;
  }
}

// A block of 64 output rows of the shared expert for one row (wave w: rows 64 b + 16 w .. + 15, one 16-row MFMA tile
// against the shared hidden row as column 0): its gated output bf16(bf16(sigmoid(bf16(x . gate))) * bf16(y)), as
// model.py:123 rounds it, published as tagged words for the routed down blocks to add. Every wave of the workgroup
// calls it. Returns false when a wave's wait for the shared hidden row gave up (the same in every thread); RECOVERY
// then runs it again computing the shared expert's gate_up items first (as recompute_gate_up does for the routed
// experts).
template <int F, int H, int I, int NSUB, bool RECOVERY>
D3_INLINE bool shared_down_block(const Ctx& cx, int b, const i32x4* xraw) {
  constexpr int STEPS = I / 128;
  constexpr int RB = row_bytes(F, I);
  constexpr int SHIFT = unpack_shift(F);
  constexpr float QMAX = act_qmax<F>();
  constexpr int T = I / (8 * NSUB);
  constexpr int TPW = (T + 63) / 64;  // item maxima per lane
  constexpr int HPW = I / 64;
  const MoeA8Args& a = *cx.a;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, q = lane >> 4, col = lane & 15;
  const int K8 = a.topk;
  const int r0 = 64 * b + 16 * w;
  if (RECOVERY) {
    if (tid == 0) {
      cx.utok[K8 * MAX_M] = 0;
      cx.upair[K8 * MAX_M] = (uint8_t)K8;
    }
    quantize_x_lds<F, H>(cx, xraw);
    __syncthreads();
#pragma unroll 1
    for (int tile = 0; tile < T; tile++)
      gate_up_item<F, H, I, NSUB>(cx, K8, tile, tile & 1, 0, 1, [] {}, [] {}, a.sh_gu_w, a.sh_gu_s);
    __syncthreads();  // the recomputed words are stored before anyone reads them back
  }
  Raw<F> raw[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; s++) load_step<F>(raw[s], a.sh_dn_w + (size_t)(r0 + (lane & 15)) * RB, s, q);
  // scales of accumulator rows r0 + 4q + i, as loaded (see DownRows)
  uint32_t sw[group_scaled(F) ? 2 * STEPS : 2];
  const uint16_t* sp = a.sh_dn_s + (size_t)(r0 + 4 * q) * (group_scaled(F) ? STEPS : 1);
  if constexpr (group_scaled(F)) {
#pragma unroll
    for (int k = 0; k < STEPS / 2; k++) {
      const i32x4 v = *(const i32x4*)(sp + 8 * k);
      sw[4 * k] = (uint32_t)v.x;
      sw[4 * k + 1] = (uint32_t)v.y;
      sw[4 * k + 2] = (uint32_t)v.z;
      sw[4 * k + 3] = (uint32_t)v.w;
    }
  } else {
    const i32x2 v = *(const i32x2*)sp;
    sw[0] = (uint32_t)v.x;
    sw[1] = (uint32_t)v.y;
  }
  auto half = [&](int k) { return bf16_to_f32((k & 1) ? sw[k >> 1] >> 16 : sw[k >> 1] & 0xFFFFu); };
  // the gate: x . shared_gate (model.py:123), then its sigmoid, each rounded to bf16 as the block's ops round them
  const float gw = shared_gate_weight<H>(a.sh_gate, xraw, lane);
  // the shared hidden row, gathered once this wave's rows have landed
  settle();
  uint64_t mw[TPW], vw[HPW];
  const bool gave = shared_gather<I, T, TPW, HPW>(cx, RECOVERY ? RECOVER_LIMIT : a.spin_limit, mw, vw, !RECOVERY);
  if (RECOVERY) {
    if (gave && lane == 0) note_recovery(a, 2u);
  } else {
    if (gave && lane == 0) cx.flags[FLAG_SH_HIDDEN] = 1;
    __syncthreads();
    if (cx.flags[FLAG_SH_HIDDEN] != 0) return false;
  }
  float tm = 0.0f;
#pragma unroll
  for (int k = 0; k < TPW; k++) tm = fmaxf(tm, tagged_value(mw[k]));
  const float amax = wave_max_f32(tm);
  const float inv = amax > 0.0f ? QMAX / amax : 0.0f;
  uint8_t* hq = cx.hq + (size_t)w * I;  // this wave's own copy of the quantized row
#pragma unroll
  for (int j = 0; j < HPW; j++) hq[act8_pos<F>(lane + 64 * j)] = (uint8_t)act8_byte<F>(tagged_value(vw[j]), inv);
  lds_settle();
  // rows r0 + 4q + i against the row (column 0)
  i32x4 iacc = {0, 0, 0, 0};
  f32x4 facc = {0.0f, 0.0f, 0.0f, 0.0f};
  i32x8 fa[STEPS], fb[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; s++) {
    i32x4 xlo = {0, 0, 0, 0}, xhi = {0, 0, 0, 0};
    if (col == 0) {
      xlo = *(const i32x4*)(hq + 128 * s + 32 * q);
      xhi = *(const i32x4*)(hq + 128 * s + 32 * q + 16);
    }
    if constexpr (F == FMT_I8) {
      iacc = step_i8<F>(raw[s], xlo, xhi, iacc);
    } else if constexpr (F == FMT_F8) {
      fa[s] = f8_operand(raw[s]);
      fb[s] = f8_operand(xlo, xhi);
    } else {
      const i32x4 g = step_i8<F>(raw[s], xlo, xhi, i32x4{0, 0, 0, 0});
#pragma unroll
      for (int i = 0; i < 4; i++) facc[i] += (float)(g[i] >> SHIFT) * half(i * STEPS + s);
    }
  }
  if constexpr (F == FMT_F8) facc = mfma_f8_chain<STEPS>(fa, fb);
  if (col == 0) {
    const float hs = amax / QMAX;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float y;
      if constexpr (F == FMT_I8) y = (float)iacc[i] * half(i);
      else if constexpr (F == FMT_F8) y = facc[i] * half(i);
      else y = facc[i];
      put_tagged(a.sharedw + r0 + 4 * q + i, bf16_round(gw * bf16_round(y * hs)), cx.epoch);
    }
  }
  return true;
}

// shared_down_block run again with RECOVERY after a wait gave up (a call: see RECOVERY_FN)
template <int F, int H, int I, int NSUB>
RECOVERY_FN void recover_shared(const MoeA8Args* args, uint32_t epoch, int b) {
  const Ctx cx = recovery_ctx(args, H, I, epoch);
  const MoeA8Args& a = *cx.a;
  if (threadIdx.x == 0) note_recovery(a, 1u);
  const int lane = threadIdx.x & 63;
  i32x4 xraw[H / 512];
#pragma unroll
  for (int k = 0; k < H / 512; k++) xraw[k] = *(const i32x4*)(a.x + 512 * k + 8 * lane);
  shared_down_block<F, H, I, NSUB, true>(cx, b, xraw);
  end_recovery(cx);
}

// One row (M = 1) with a workgroup for each gate_up tile: workgroup i < k T computes gate_up tile i % T of the expert
// at routing rank i / T and, for i < H / 8, down block i, so the down rows are requested only once the workgroup's
// gate_up rows have arrived and the gate_up rows, which the hand-off waits for, are not queued behind them.
// Every wave routes the row itself and its gate_up rows go out after the rounds that name their expert (no workgroup
// barrier before them); the remaining rounds, the softmax, the x slice its MFMA steps read (H = 2048: wave w reads x
// chunk w) and the slot tables are written while they are in flight. Every wave writes the same values, so nothing
// waits for another wave until the gate_up reduction.
// The block around the experts: with a router, workgroups 0 .. E-1 first compute one logit each and every routing
// wave gathers them; with a shared expert, workgroups k T .. k T + T - 1 compute its gate_up tiles (hidden row k)
// and the next H / 64 its output in blocks of 64 rows, which the down blocks add to the routed sum.
template <int F, int H, int I, int NSUB, int KPL>
D3_INLINE void one_row_layer(Ctx& cx, int i) {
  static_assert(H == 2048, "wave w's K slice is x chunk w");
  constexpr int T = I / (8 * NSUB), NHB = H / 8;  // gate_up items per expert, down blocks
  const MoeA8Args& a = *cx.a;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int E = a.E, K8 = a.topk;
  const int routed = K8 * T;
  const bool is_shared = i >= routed;
  // given logits go out first: routing waits for them, and a wave's loads complete in order
  uint32_t lb[KPL];
#pragma unroll
  for (int j = 0; j < KPL; j++) lb[j] = 0u;
  if (!a.router && !is_shared) {
#pragma unroll
    for (int j = 0; j < KPL; j++) lb[j] = a.logits[min(lane + 64 * j, E - 1)];
  }
  i32x4 xraw[H / 512];
#pragma unroll
  for (int k = 0; k < H / 512; k++) xraw[k] = *(const i32x4*)(a.x + 512 * k + 8 * lane);
  if (a.router && i < E && w == 0) router_logit<H>(a, cx.epoch, i, xraw, lane);
  if (i >= routed + T) {
    __syncthreads();  // the LDS flags are cleared (make_ctx) before any wave sets one
    if (!shared_down_block<F, H, I, NSUB, false>(cx, i - routed - T, xraw))
      recover_shared<F, H, I, NSUB>(kernel_args(), cx.epoch, i - routed - T);
    return;
  }
  const int u = is_shared ? K8 : i / T, tile = is_shared ? i - routed : i % T;
  const int hb = i - a.dn_first;
  const bool has_down = hb >= 0 && hb < NHB && !is_shared;
  if (a.router && !is_shared) gather_logits<H, KPL>(a, cx.epoch, lane, lb, xraw);
  TopKeys<KPL> tk(lb, lane, E);
  if (!is_shared) tk.rounds(lane, 0, u + 1);
  const int e = is_shared ? 0 : route_key_index((uint32_t)__builtin_amdgcn_readlane((int)tk.mine, u));
  cx.U = K8;
  cx.nch = 1;
  cx.n_dn = NHB;
  DownRows<F, I> d;
  gate_up_item<F, H, I, NSUB>(
      cx, u, tile, 0, e, 1,
      [&]() {
        if (has_down) {
          tk.rounds(lane, u + 1, K8);
          const float wt = route_weight(tk.mine, lane, K8);
          if (lane < K8) {
            const int id = route_key_index(tk.mine);
            cx.rt_id[lane] = id;
            cx.rt_w[lane] = wt;
            cx.ulist[lane] = id;
            cx.ucount[lane] = 1;
            cx.utok[lane * MAX_M] = 0;
            cx.upair[lane * MAX_M] = (uint8_t)lane;
            if (hb == 0 && w == 0) {
              if (a.ids_out) a.ids_out[lane] = id;
              if (a.weights_out) a.weights_out[lane] = wt;
            }
          }
          if (lane == 0) {
            cx.chunk_first[0] = 0;
            cx.chunk_first[1] = K8;
            cx.misc[0] = K8;
            cx.misc[1] = 1;
          }
        }
        quantize_x_lds<F, H>(cx, xraw);
        if (lane == 0) {
          cx.utok[u * MAX_M] = 0;
          cx.upair[u * MAX_M] = (uint8_t)u;
        }
        lds_settle();
      },
      [&]() {
        if (has_down) down_load<F, H, I>(cx, 0, hb, d);
      },
      is_shared ? a.sh_gu_w : a.gu_w, is_shared ? a.sh_gu_s : a.gu_s);
  if (has_down && !down_finish<F, H, I, NSUB, false, false, false, false>(cx, 0, hb, d))
    recover_down<F, H, I, NSUB, false, false, false>(kernel_args(), cx.epoch, 0, hb);
}

// The one-row schedule as its own kernel: k I / UT + I / UT + H / 64 workgroups (UT = 8 NSUB hidden units per
// gate_up item). Compiled for three workgroups per CU (168 registers a lane), which the 8-unit items need (768 of them
// at k 8, I 768) and the 16-unit ones keep for latency. The recovery calls (recover_down, recover_shared) keep the
// recovery's own registers out of the fast path, but the call convention still costs it: with the calls the int8
// kernel spills some 80 registers a lane (149 without them), one-row int8 14.42 -> 14.71 us. Inlined instead, the
// recovery spilled more (FP8 one row 14.4 -> 20.5 us).
// (int8 with 16-unit items, the block's schedule, at two workgroups per CU instead: its 464 workgroups fit either way,
// and then nothing spills; block int8 25.4 -> 22.0 us. FP8 / W4A8 / W6A8 measured 21.2 / 16.7 / 19.5 us at three
// and 22.1 / 17.1 / 19.3 at two.)
constexpr int one_row_blocks_per_cu(int F, int NSUB) { return NSUB == 2 && F == FMT_I8 ? 2 : 3; }
template <int F, int H, int I, int NSUB>
__global__ void __launch_bounds__(256, one_row_blocks_per_cu(F, NSUB)) moe_a8_one_row_kernel(MoeA8Args a) {
  Ctx cx = make_ctx(a, H, I);
  if (a.E <= 128) one_row_layer<F, H, I, NSUB, 2>(cx, (int)blockIdx.x);
  else one_row_layer<F, H, I, NSUB, 4>(cx, (int)blockIdx.x);
}

// The general schedule, persistent: compiled for WPC workgroups per CU, the grid being as many as fit. Two per CU
// (the registers of 256 a lane hold a down item's gathered rows without spills): with the items dealt by kind
// (BALANCED, see the item loops at the end) two beat three at every row count measured (int8 2 rows 24.1 / 27.9 us
// per layer, 3 rows 32.4 / 36.0, 6 rows 57.6 / 64.5, 16 rows 143 / 164). (Round-robin, int8, two / three per CU: 2 rows 25.4 / 29.4,
// 3 rows 40.8 / 39.5, 4 rows 45.8 / 49.4, 5 rows 58.6 / 61.9.)
template <int F, int H, int I, int WPC, bool BALANCED>
__global__ void __launch_bounds__(256, WPC) moe_a8_kernel(MoeA8Args a) {
  constexpr int T = I / 16;
  constexpr int NHB = H / 8;
  constexpr float QMAX = act_qmax<F>();
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int M = a.M, E = a.E, K8 = a.topk;
  Ctx cx = make_ctx(a, H, I);
  // the down items' schedule (see the item loop): launch-wide slots and lag 2 for the 4- and 6-bit formats
  constexpr bool EARLY = F == FMT_W4 || F == FMT_W6;
  constexpr int LAG = EARLY ? 2 : 1;

  // ---- per row: routed by wave t % 4 and its activations quantized by wave (t + 1) % 4, so that with one row the
  // two loads and what follows them overlap; each wave issues its loads before using any of them
  for (int i = 0; 4 * i < M; i++) {
    const int tr = 4 * i + w, tq = 4 * i + ((w + 3) & 3);
    const bool do_route = tr < M, do_quant = tq < M;
    const uint16_t* lg = a.logits + (size_t)(do_route ? tr : 0) * E;
    const uint16_t* xr = a.x + (size_t)(do_quant ? tq : 0) * H;
    uint32_t lb[4];
#pragma unroll
    for (int j = 0; j < 4; j++) lb[j] = do_route && lane + 64 * j < E ? lg[lane + 64 * j] : 0u;
    i32x4 xraw[H / 512];
#pragma unroll
    for (int k = 0; k < H / 512; k++) xraw[k] = do_quant ? *(const i32x4*)(xr + 512 * k + 8 * lane) : i32x4{0, 0, 0, 0};
    if (do_route) {
      const uint32_t mine = E <= 128 ? top_keys<2>(lb, lane, E, K8) : top_keys<4>(lb, lane, E, K8);
      // softmax over the k, the exponentials in parallel and their sum in rank order (kernels.py:57-61)
      const float top0 = route_key_value((uint32_t)__builtin_amdgcn_readlane((int)mine, 0));
      const float ex = lane < K8 ? expf(route_key_value(mine) - top0) : 0.0f;
      float total = 0.0f;
#pragma unroll
      for (int r = 0; r < MAX_K; r++)
        if (r < K8) total += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), r));
      if (lane < K8) {
        const int id = route_key_index(mine);
        cx.rt_id[tr * MAX_K + lane] = id;
        cx.rt_w[tr * MAX_K + lane] = bf16_round(ex / total);
        if (M == 1) {
          // one row: its experts in routing order are the union, one pair each, all in one down chunk
          cx.ulist[lane] = id;
          cx.ucount[lane] = 1;
          cx.utok[lane * MAX_M] = 0;
          cx.upair[lane * MAX_M] = (uint8_t)lane;
          if constexpr (EARLY) {
            cx.gfirst[lane] = lane;
            cx.gpair[lane] = lane;
            cx.pair_slot[lane] = lane;
          }
        }
      }
      if (M == 1 && lane == 0) {
        if constexpr (EARLY) cx.gfirst[K8] = K8;
        cx.chunk_first[0] = 0;
        cx.chunk_first[1] = K8;
        cx.misc[0] = K8;
        cx.misc[1] = 1;
      }
    }
    if (do_quant) {
      float v[H / 512][8];
      float amax = 0.0f;
#pragma unroll
      for (int k = 0; k < H / 512; k++) {
        const uint32_t wv[4] = {(uint32_t)xraw[k].x, (uint32_t)xraw[k].y, (uint32_t)xraw[k].z, (uint32_t)xraw[k].w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          v[k][2 * i] = bf16_to_f32(wv[i] & 0xFFFFu);
          v[k][2 * i + 1] = bf16_to_f32(wv[i] >> 16);
          amax = fmaxf(amax, fmaxf(fabsf(v[k][2 * i]), fabsf(v[k][2 * i + 1])));
        }
      }
      amax = wave_max_f32(amax);
      const float inv = amax > 0.0f ? QMAX / amax : 0.0f;
#pragma unroll
      for (int k = 0; k < H / 512; k++) store_act8<F>(cx.xq + (size_t)tq * H + 512 * k + 8 * lane, v[k], inv);
      if (lane == 0) cx.sx[tq] = amax / QMAX;
    }
  }
  __syncthreads();

  // ---- union of the rows' experts, ascending, built by wave 0: lane l owns experts l, l + 64, l + 128, l + 192.
  // Each expert's mask of rows comes from LDS atomics, one per (row, rank) pair; the experts are compacted by a
  // ballot; each pair then finds its place among its expert's rows (rows ascending) from the expert's word.
  if (M > 1 && w == 0) {
    const int npairs = M * K8;
#pragma unroll
    for (int k = 0; k < 4; k++) cx.emask[lane + 64 * k] = 0u;
    lds_settle();
    for (int p = lane; p < npairs; p += 64) {
      const int t = p / K8;
      atomicOr(&cx.emask[cx.rt_id[t * MAX_K + p - t * K8]], 1u << t);
    }
    lds_settle();
    uint32_t m[4];
#pragma unroll
    for (int k = 0; k < 4; k++) m[k] = lane + 64 * k < E ? cx.emask[lane + 64 * k] : 0u;
    // and, for the 4- and 6-bit formats, the launch-wide slots: union expert pos holds slots gfirst[pos] .. + its
    // pair count - 1 (a scan of the counts over the lanes)
    int base = 0, sbase = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int e = lane + 64 * k;
      const uint64_t ball = __ballot(m[k] != 0u);
      const int pos = base + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(ball >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)ball, 0u));
      const int cnt = __popc(m[k]);
      int incl = cnt;
      if constexpr (EARLY) {
#pragma unroll
        for (int dd = 1; dd < 64; dd <<= 1) {
          const int v = __shfl_up(incl, dd);
          if (lane >= dd) incl += v;
        }
      }
      const int g0 = sbase + incl - cnt;
      if (m[k] != 0u) {
        cx.ulist[pos] = e;
        cx.ucount[pos] = cnt;
        if constexpr (EARLY) cx.gfirst[pos] = g0;
        cx.emask[e] = (uint32_t)pos << 16 | m[k];  // rows < 16: the mask fits the low half
      }
      base += __popcll(ball);
      if constexpr (EARLY) sbase += __shfl(incl, 63);
    }
    if (EARLY && lane == 0) cx.gfirst[base] = sbase;
    lds_settle();
    for (int p = lane; p < npairs; p += 64) {
      const int t = p / K8;
      const uint32_t word = cx.emask[cx.rt_id[t * MAX_K + p - t * K8]];
      const int pos = (int)(word >> 16), n = __popc(word & 0xFFFFu & ((1u << t) - 1u));
      cx.utok[pos * MAX_M + n] = (uint8_t)t;
      cx.upair[pos * MAX_M + n] = (uint8_t)p;
      if constexpr (EARLY) {
        cx.gpair[cx.gfirst[pos] + n] = p;
        cx.pair_slot[p] = cx.gfirst[pos] + n;
      }
    }
    // down chunks: consecutive experts, at most CHUNK_EXPERTS of them and CHUNK_PAIRS pairs; with M * topk <= 32
    // pairs that is simply 8 experts each
    if (M * K8 <= CHUNK_PAIRS) {
      const int nch = (base + CHUNK_EXPERTS - 1) / CHUNK_EXPERTS;
      for (int c = lane; c <= nch; c += 64) cx.chunk_first[c] = min(c * CHUNK_EXPERTS, base);
      if (lane == 0) cx.misc[1] = nch;
    } else if (lane == 0) {
      int nch = 0, ne = 0, np = 0;
      cx.chunk_first[0] = 0;
      for (int u = 0; u < base; u++) {
        const int n = cx.ucount[u];
        if (ne == CHUNK_EXPERTS || np + n > CHUNK_PAIRS) {
          cx.chunk_first[++nch] = u;
          ne = 0;
          np = 0;
        }
        ne++;
        np += n;
      }
      cx.chunk_first[++nch] = base;
      cx.misc[1] = nch;
    }
    if (lane == 0) cx.misc[0] = base;
  }
  if (blockIdx.x == 0) {
    for (int i = tid; i < M * K8; i += 256) {
      if (a.ids_out) a.ids_out[i] = cx.rt_id[(i / K8) * MAX_K + i % K8];
      if (a.weights_out) a.weights_out[i] = cx.rt_w[(i / K8) * MAX_K + i % K8];
    }
  }
  if (M > 1) __syncthreads();
  const int U = cx.misc[0];
  cx.U = U;
  cx.nch = cx.misc[1];
  cx.n_dn = cx.nch * NHB;
  const int n_items = U * T + cx.n_dn;
  // When the down items of a chunk start. With the 8-bit formats the gate_up streams are the long part, and the
  // chunk's down items follow the next chunk's gate_up items (lag 1), each numbering its slots first (thread 0), so
  // that their gathers come once most words are published: gathers issued earlier compete with the streams. With
  // the 4- and 6-bit formats the down items are the tail: they follow two chunks' gate_up items (lag 2) and gather
  // behind their weight rows at once, from slots numbered once per launch. Measured, us per layer at 2 / 3 / 4 / 5
  // rows: W4A8 21.6 / 30.9 / 38.9 / 48.4 with the 8-bit choice, 21.5 / 30.2 / 36.4 / 48.1 with this one; W6A8 at 4
  // rows 45.9 / 43.5; int8 25.2 / 38.8 / 44.6 / 55.8 against 26.3 / 40.3 / 45.3 / 56.7 with the 4-bit choice.
  // (EARLY and LAG are set at the top of the kernel.)
  int parity = 0;
  if constexpr (BALANCED) {
    // Every gate_up item first, then the down items chunk by chunk; gate_up item k and down item k go to workgroup
    // k mod G, so that every workgroup holds as many down items as any other, and each workgroup takes its gate_up
    // items, then its down items (every wait is on items of lower index). Measured, us per layer, the round-robin
    // schedule below / this, two workgroups per CU:
    //   3 rows: int8 41.1 / 32.4, W4A8 31.7 / 25.9, FP8 40.1 / 32.2, W6A8 41.5 / 31.9 (three per CU: 36.0, 31.1,
    //           34.2, 34.2);
    //   4 rows: int8 43.7 / 40.4, W4A8 33.5 / 30.4, FP8 42.9 / 39.6, W6A8 42.4 / 38.3;
    //   5 rows: int8 53.4 / 49.8, W4A8 44.7 / 39.0, FP8 52.8 / 48.9, W6A8 53.3 / 46.9;
    //   2 rows: int8 24.8 / 24.1, FP8 24.5 / 23.9, W6A8 24.5 / 24.5, but W4A8 20.4 / 21.3 (it keeps the round-robin);
    //   rows the layer runs fused only when asked (moe_layer with fused=True, d3_moe_a8_noalloc): int8 6 rows
    //           73.4 / 57.6, 8 rows 88.3 / 69.6, 16 rows 185 / 143; W4A8 6 rows 61.0 / 44.5, 16 rows 149 / 116.
    // (Round-robin over this same order: 2 rows int8 29.8, 3 rows 41.3. Dealt as here but with each chunk's down
    // items after the next one or two chunks' gate_up items, as below: 4 rows int8 42.3, W4A8 32.6.)
    const int G = (int)gridDim.x;
    for (int k = blockIdx.x; k < U * T; k += G) {
      const int u = k / T;  // units are numbered chunk by chunk
      gate_up_item<F, H, I>(cx, u, k % T, parity, cx.ulist[u], cx.ucount[u], [] {}, [] {}, a.gu_w, a.gu_s);
      parity ^= 1;
    }
    for (int k = blockIdx.x; k < cx.n_dn; k += G) down_item<F, H, I, EARLY>(cx, k / NHB, k % NHB);
    return;
  }
  for (int item = blockIdx.x; item < n_items; item += gridDim.x) {
    // segments: gate_up(chunk c), then down(chunk c - LAG)
    int base = 0;
    for (int c = 0; c < cx.nch + LAG; c++) {
      if (c < cx.nch) {
        const int u0 = cx.chunk_first[c], ne = cx.chunk_first[c + 1] - u0;
        if (item < base + ne * T) {
          const int u = u0 + (item - base) / T;
          gate_up_item<F, H, I>(cx, u, (item - base) % T, parity, cx.ulist[u], cx.ucount[u], [] {}, [] {}, a.gu_w,
                                a.gu_s);
          parity ^= 1;
          break;
        }
        base += ne * T;
      }
      if (c >= LAG) {
        if (item < base + NHB) {
          down_item<F, H, I, EARLY>(cx, c - LAG, item - base);
          break;
        }
        base += NHB;
      }
    }
  }
}

}  // namespace d3

// =====================================================================================================================
// Host side
namespace d3 {

thread_local std::string g_error;
int fail(const std::string& msg) {
  g_error = msg;
  return D3_EINVAL;
}
int hip_fail(hipError_t err, const char* what) {
  g_error = std::string(what) + ": " + hipGetErrorString(err);
  return (int)err;
}

// the header, then (pairs + 1 for the shared expert) hidden rows and tile maxima, the pairs' partial outputs, and for
// the block's router and shared expert MAX_E logit words and H output words
__host__ __device__ constexpr int64_t moe_a8_workspace_bytes(int M, int topk, int H, int I) {
  return SYNC_WORDS * 4 + ((int64_t)M * topk + 1) * I * 8 + ((int64_t)M * topk + 1) * (I / 8) * 8 +
         (int64_t)M * topk * H * 8 + (int64_t)(MAX_E + H) * 8;
}

// ---- The entry that allocates nothing (d3_moe_a8_noalloc) -----------------------------------------------------------
// Its workspace is this file-scope array, one copy per GPU, sized for the largest layer the fused kernels take: 16
// rows, top-8, H 2048, I 768 (3.0 MB). In host code `scratch` names a host-side stand-in, not device memory: the
// device address comes from hipGetSymbolAddress, once per device (scratch_on), and only that address is used.
constexpr int64_t SCRATCH_BYTES = moe_a8_workspace_bytes(MAX_M, MAX_K, 2048, 768);
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

// zeroes n bytes (a multiple of 16) at p: the workspace's words must start with tag 0, which no epoch equals
// The block for several rows around the routed layer (model.py:107-124): the router's logits of M rows (self.gate(flat),
// model.py:115), a wave per (row, expert), with router_dot's arithmetic, so each row's logits equal the one-row block's
template <int H>
__global__ void __launch_bounds__(256) router_logits_kernel(const uint16_t* x, const uint16_t* router, int M, int E,
                                                            uint16_t* logits) {
  const int lane = threadIdx.x & 63, g = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (g >= M * E) return;
  const int t = g / E, e = g - t * E;
  i32x4 xraw[H / 512];
#pragma unroll
  for (int k = 0; k < H / 512; k++) xraw[k] = *(const i32x4*)(x + (size_t)t * H + 512 * k + 8 * lane);
  const uint32_t bits = f32_to_bf16(row_dot<H>(router + (size_t)e * H, xraw, lane));
  if (lane == 0) logits[g] = (uint16_t)bits;
}

// out[t] = routed[t] + bf16(gw_t * shared[t]) rounded to bf16 (model.py:123: the shared expert's output scaled by
// bf16(sigmoid(bf16(x . gate))), added to the routed output, each a bf16 tensor), as the one-row block's down blocks
// combine them. A workgroup per row: wave 0 computes the row's gate weight.
template <int H>
__global__ void __launch_bounds__(256) block_combine_kernel(const uint16_t* x, const uint16_t* gate,
                                                            const uint16_t* routed, const uint16_t* shared,
                                                            uint16_t* out) {
  __shared__ float gw;
  const int t = blockIdx.x, lane = threadIdx.x & 63;
  if (threadIdx.x < 64) {
    i32x4 xraw[H / 512];
#pragma unroll
    for (int k = 0; k < H / 512; k++) xraw[k] = *(const i32x4*)(x + (size_t)t * H + 512 * k + 8 * lane);
    const float w = shared_gate_weight<H>(gate, xraw, lane);
    if (lane == 0) gw = w;
  }
  __syncthreads();
  for (int h = threadIdx.x; h < H; h += 256) {
    const size_t i = (size_t)t * H + h;
    const float y = bf16_to_f32(routed[i]) + bf16_round(gw * bf16_to_f32(shared[i]));
    out[i] = (uint16_t)f32_to_bf16(y);
  }
}

__global__ void __launch_bounds__(256) fill_zero_kernel(uint4* p, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (int64_t)gridDim.x * 256)
    p[i] = uint4{0u, 0u, 0u, 0u};
}

constexpr int MAX_DEVICES = 64;

// The current device's copy of `scratch`: its address from hipGetSymbolAddress (checked), looked up once per device
// with that device current. With `clear`, the first call on the device also zeroes it by a fill kernel on `stream` (a
// kernel, so that no memset node is recorded) unless `stream` is capturing a graph: the array is zero when the library
// loads, and a clear recorded into a graph would run on every replay. Returns nullptr and sets the error on failure.
void* scratch_on(hipStream_t stream, bool clear, int* err) {
  static std::mutex mu;
  static void* ptrs[MAX_DEVICES] = {};
  static bool cleared[MAX_DEVICES] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) { *err = hip_fail(e, "hipGetDevice"); return nullptr; }
  if (dev < 0 || dev >= MAX_DEVICES) { *err = fail("d3_moe_a8_noalloc: device index beyond 64"); return nullptr; }
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) { *err = hip_fail(e, "d3_moe_a8_noalloc: hipGetSymbolAddress"); return nullptr; }
    ptrs[dev] = p;
  }
  if (clear && !cleared[dev]) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &capture);
    if (e != hipSuccess) { *err = hip_fail(e, "d3_moe_a8_noalloc: hipStreamIsCapturing"); return nullptr; }
    if (capture == hipStreamCaptureStatusNone) {
      hipLaunchKernelGGL(fill_zero_kernel, dim3(768), dim3(256), 0, stream, (uint4*)ptrs[dev], SCRATCH_BYTES / 16);
      e = hipGetLastError();
      if (e != hipSuccess) { *err = hip_fail(e, "d3_moe_a8_noalloc: clearing the workspace"); return nullptr; }
    }
    cleared[dev] = true;
  }
  return ptrs[dev];
}

using KernelFn = void (*)(MoeA8Args);

template <int F, int H, int I> KernelFn kernel_of(int unit, int M) {
  if (unit == 8) return moe_a8_one_row_kernel<F, H, I, 1>;
  if (unit == 16) return moe_a8_one_row_kernel<F, H, I, 2>;
  // two workgroups per CU, items dealt by kind (BALANCED), except W4A8 at two rows (round-robin)
  if (M == 2 && F == FMT_W4) return moe_a8_kernel<F, H, I, 2, false>;
  return moe_a8_kernel<F, H, I, 2, true>;
}

// the fused layer's kernel for a format, shape and row count: the general schedule (unit 0) or the one-row schedule
// with gate_up items of `unit` (8 or 16) hidden units
KernelFn pick_kernel(int fmt, int H, int I, int M, int unit = 0) {
#define D3_CASE(F, HH, II) \
  if (fmt == F && H == HH && I == II) return kernel_of<F, HH, II>(unit, M);
#define D3_SHAPES(F) D3_CASE(F, 2048, 768) D3_CASE(F, 2048, 512)
  D3_SHAPES(FMT_I8) D3_SHAPES(FMT_W4) D3_SHAPES(FMT_W6) D3_SHAPES(FMT_F8)
#undef D3_SHAPES
#undef D3_CASE
  return nullptr;
}

// workgroups the device holds at once for a kernel and LDS size (cached per device)
int resident_capacity(KernelFn fn, int lds_bytes, int* err) {
  static std::mutex mu;
  static std::map<std::tuple<int, void*, int>, int> cache;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) { *err = hip_fail(e, "hipGetDevice"); return 0; }
  std::lock_guard<std::mutex> lock(mu);
  auto key = std::make_tuple(dev, (void*)fn, lds_bytes);
  auto it = cache.find(key);
  if (it != cache.end()) return it->second;
  int per_cu = 0, cus = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, (const void*)fn, 256, lds_bytes);
  if (e != hipSuccess) { *err = hip_fail(e, "hipOccupancyMaxActiveBlocksPerMultiprocessor"); return 0; }
  e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) { *err = hip_fail(e, "hipDeviceGetAttribute"); return 0; }
  int cap = per_cu * cus;
  cache[key] = cap;
  return cap;
}

int launch_moe_a8(const d3_moe_a8_desc* d, hipStream_t stream) {
  if (!d) return fail("d3_moe_a8: null descriptor");
  if (d->M < 1 || d->M > MAX_M) return fail("d3_moe_a8: M must be 1..16");
  if (d->topk < 1 || d->topk > MAX_K) return fail("d3_moe_a8: topk must be 1..8");
  if (d->E < d->topk || d->E > MAX_E) return fail("d3_moe_a8: E must be topk..256");
  KernelFn fn = pick_kernel(d->format, d->H, d->I, d->M);
  if (!fn) return fail("d3_moe_a8: no kernel for this format and shape (H 2048; I 512 or 768)");
  if (!d->x || !(d->logits || d->router) || !d->gate_up || !d->gate_up_scale || !d->down || !d->down_scale || !d->out ||
      !d->workspace)
    return fail("d3_moe_a8: null pointer");
  if (((uintptr_t)d->gate_up_scale | (uintptr_t)d->down_scale) & 15u)
    return fail("d3_moe_a8: scale tensors must be 16-byte aligned");
  const bool shared = d->shared_gate_up != nullptr;
  if (shared && (!d->shared_gate_up_scale || !d->shared_down || !d->shared_down_scale || !d->shared_gate))
    return fail("d3_moe_a8: the shared expert needs gate_up, down, their scales and its gate");
  if (shared && (((uintptr_t)d->shared_gate_up_scale | (uintptr_t)d->shared_down_scale) & 15u))
    return fail("d3_moe_a8: scale tensors must be 16-byte aligned");
  const int64_t need = moe_a8_workspace_bytes(d->M, d->topk, d->H, d->I);
  if (d->workspace_bytes < need) return fail("d3_moe_a8: workspace too small");
  const Lds L(d->M, d->topk, d->H, d->I);
  int err = 0;
  const int cap = resident_capacity(fn, L.total, &err);
  if (err) return err;
  if (cap < 1) return fail("d3_moe_a8: the kernel does not fit on a compute unit");
  const int umax = d->M * d->topk < d->E ? d->M * d->topk : d->E;
  // chunks hold up to 8 experts and 32 pairs; a chunk per expert bounds their count
  const int nch = umax;
  const int items = umax * (d->I / 16) + nch * (d->H / 8);
  int grid = items < cap ? items : cap;
  // one row: a workgroup per gate_up item, the first H / 8 of them also taking a down block (one_row_layer), when the
  // device holds them all at once. Items of 8 hidden units first: k I / 8 workgroups (768 at k 8, I 768) put the
  // same gate_up bytes on every CU, where 16-unit items (384) put two on half the CUs, which then finish last.
  if (d->item_units != 0 && d->item_units != 8 && d->item_units != 16)
    return fail("d3_moe_a8: item_units must be 0, 8 or 16");
  KernelFn fn1 = nullptr;
  int tiles = 0, unit_used = 0;
  for (int unit = 8; d->grid <= 0 && d->M == 1 && unit <= 16 && !fn1; unit += 8) {
    if (d->item_units != 0 && unit != d->item_units) continue;
    const int t = d->topk * (d->I / unit) + (shared ? d->I / unit + d->H / 64 : 0);
    if (d->topk * (d->I / unit) < d->H / 8 || (d->router && t < d->E)) continue;
    KernelFn f = pick_kernel(d->format, d->H, d->I, d->M, unit);
    const int cap1 = resident_capacity(f, L.total, &err);
    if (err) return err;
    if (t <= cap1) {
      fn1 = f;
      tiles = t;
      unit_used = unit;
    }
  }
  const bool one_row = fn1 != nullptr;
  if (d->grid > 0) grid = d->grid < grid ? d->grid : grid;
  else if (one_row) grid = tiles;
  if ((d->router || shared) && !one_row)
    return fail("d3_moe_a8: the router and the shared expert run in the one-row schedule (M = 1, grid 0)");
  if (d->item_units != 0 && !one_row)
    return fail("d3_moe_a8: item_units applies to the one-row schedule (M = 1, grid 0), whose workgroups must all fit "
                "on the device at once");

  MoeA8Args a;
  a.x = (const uint16_t*)d->x;
  a.logits = (const uint16_t*)d->logits;
  a.gu_w = (const uint8_t*)d->gate_up;
  a.gu_s = (const uint16_t*)d->gate_up_scale;
  a.dn_w = (const uint8_t*)d->down;
  a.dn_s = (const uint16_t*)d->down_scale;
  a.out = (uint16_t*)d->out;
  a.ids_out = d->ids_out;
  a.weights_out = d->weights_out;
  uint8_t* ws = (uint8_t*)d->workspace;
  a.status = (uint64_t*)(ws + SYNC_STATUS * 4);
  a.sticky = (uint32_t*)ws + SYNC_STICKY;
  const size_t pairs = (size_t)d->M * d->topk;
  a.hidden = (uint64_t*)(ws + SYNC_WORDS * 4);
  a.tmax = a.hidden + (pairs + 1) * d->I;
  a.parts = a.tmax + (pairs + 1) * (d->I / 8);
  a.logitw = a.parts + pairs * d->H;
  a.sharedw = a.logitw + MAX_E;
  a.M = d->M;
  a.E = d->E;
  a.topk = d->topk;
  // 0 inside the kernel: every wait gives up at once (recompute_all)
  a.spin_limit = d->recompute_all ? 0u : d->spin_limit ? d->spin_limit : (1u << 20);
  a.router = (const uint16_t*)d->router;
  a.logits_out = (uint16_t*)d->logits_out;
  a.sh_gu_w = (const uint8_t*)d->shared_gate_up;
  a.sh_gu_s = (const uint16_t*)d->shared_gate_up_scale;
  a.sh_dn_w = (const uint8_t*)d->shared_down;
  a.sh_dn_s = (const uint16_t*)d->shared_down_scale;
  a.sh_gate = (const uint16_t*)d->shared_gate;
  // Which of the routed gate_up workgroups also take the down blocks: those routed at ranks 0-2 land their gate_up rows
  // first, and their down rows then compete with the later ranks' gate_up rows, which the hand-off waits for; from
  // workgroup 256 on (ranks 2.7-5.3 with 8-unit items) they go out once most gate_up rows are in. The shorter streams
  // of the 4- and 6-bit formats favour the first workgroups (late down rows become the tail). Measured, us per layer,
  // first down workgroup 0 / 256 with 8-unit items: int8 15.5 / 14.5, FP8 15.6 / 14.5, W6A8 13.9 / 13.8, W4A8 11.6 /
  // 12.2; 0 / 128 with 16-unit items (block with a shared expert): int8 20.0 / 19.5, FP8 19.9 / 19.4, W6A8 18.6 /
  // 19.6, W4A8 16.8 / 17.5.
  a.dn_first = 0;
  if (one_row) {
    const int late = d->topk * (d->I / unit_used) - d->H / 8;  // the last workgroups that can take them all
    const bool big = d->format == FMT_I8 || d->format == FMT_F8;
    if (unit_used == 8 && d->format != FMT_W4) a.dn_first = late < 256 ? late : 256;
    if (unit_used == 16 && big) a.dn_first = late < 128 ? late : 128;
  }
  hipLaunchKernelGGL(one_row ? fn1 : fn, dim3(grid), dim3(256), L.total, stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "d3_moe_a8 launch");
  return 0;
}

}  // namespace d3

extern "C" {

const char* d3_last_error(void) { return d3::g_error.c_str(); }
int d3_version(void) { return 1; }

int d3_router_logits(const void* x, const void* router, int32_t M, int32_t H, int32_t E, void* logits, void* stream) {
  if (!x || !router || !logits) return d3::fail("d3_router_logits: null pointer");
  if (H != 2048) return d3::fail("d3_router_logits: H = 2048");
  if (M < 0 || E < 1 || E > d3::MAX_E) return d3::fail("d3_router_logits: M >= 0, 1 <= E <= 256");
  if (M == 0) return 0;
  hipLaunchKernelGGL(d3::router_logits_kernel<2048>, dim3((M * E + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                     (const uint16_t*)x, (const uint16_t*)router, M, E, (uint16_t*)logits);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : d3::hip_fail(e, "d3_router_logits launch");
}

int d3_block_combine(const void* x, const void* gate, const void* routed, const void* shared, int32_t M, int32_t H,
                     void* out, void* stream) {
  if (!x || !gate || !routed || !shared || !out) return d3::fail("d3_block_combine: null pointer");
  if (H != 2048) return d3::fail("d3_block_combine: H = 2048");
  if (M < 0) return d3::fail("d3_block_combine: M >= 0");
  if (M == 0) return 0;
  hipLaunchKernelGGL(d3::block_combine_kernel<2048>, dim3(M), dim3(256), 0, (hipStream_t)stream, (const uint16_t*)x,
                     (const uint16_t*)gate, (const uint16_t*)routed, (const uint16_t*)shared, (uint16_t*)out);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : d3::hip_fail(e, "d3_block_combine launch");
}

int64_t d3_moe_a8_workspace_bytes(int32_t M, int32_t topk, int32_t H, int32_t I) {
  return d3::moe_a8_workspace_bytes(M, topk, H, I);
}

int d3_moe_a8(const d3_moe_a8_desc* desc, void* stream) { return d3::launch_moe_a8(desc, (hipStream_t)stream); }

int d3_moe_a8_noalloc(const d3_moe_a8_desc* desc, void* stream) {
  if (!desc) return d3::fail("d3_moe_a8_noalloc: null descriptor");
  const int64_t need = d3::moe_a8_workspace_bytes(desc->M, desc->topk, desc->H, desc->I);
  if (desc->M < 1 || desc->topk < 1 || desc->H < 1 || desc->I < 1 || need > d3::SCRATCH_BYTES)
    return d3::fail("d3_moe_a8_noalloc: the layer needs " + std::to_string(need) + " bytes of workspace, more than the " +
                    std::to_string(d3::SCRATCH_BYTES) + " of the static one (at most 16 rows, top-8, H 2048, I 768)");
  int err = 0;
  void* ws = d3::scratch_on((hipStream_t)stream, true, &err);
  if (!ws) return err;
  d3_moe_a8_desc d = *desc;
  d.workspace = ws;
  d.workspace_bytes = d3::SCRATCH_BYTES;
  return d3::launch_moe_a8(&d, (hipStream_t)stream);
}

int d3_moe_a8_status(void* workspace, uint32_t* status) {
  if (!workspace || !status) return d3::fail("d3_moe_a8_status: null pointer");
  uint8_t* sticky = (uint8_t*)workspace + d3::SYNC_STICKY * 4;
  hipError_t e = hipMemcpy(status, sticky, 4, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return d3::hip_fail(e, "d3_moe_a8_status");
  const uint32_t zero = 0;
  e = hipMemcpy(sticky, &zero, 4, hipMemcpyHostToDevice);
  if (e != hipSuccess) return d3::hip_fail(e, "d3_moe_a8_status");
  return 0;
}

int d3_moe_a8_noalloc_status(uint32_t* status) {
  if (!status) return d3::fail("d3_moe_a8_noalloc_status: null pointer");
  int err = 0;
  void* ws = d3::scratch_on(nullptr, false, &err);
  if (!ws) return err;
  return d3_moe_a8_status(ws, status);
}

}  // extern "C"
