// Device helpers shared by every kernel of the routed-expert path: bfloat16 and float8 conversions, wave64
// reductions over DPP, and the MFMA step types. gfx950 (CDNA4) only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef int i32x2 __attribute__((ext_vector_type(2)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define D3_INLINE __device__ __forceinline__

// ---------------------------------------------------------------------------------------------------------------
// bfloat16 <-> float. The narrowing rounds to nearest, ties to even, as a cast does (kernels.py:33-37 rounds the same
// way); NaN stays NaN.
D3_INLINE float bf16_to_f32(uint32_t b) { return __uint_as_float(b << 16); }
D3_INLINE uint32_t f32_to_bf16(float v) {
  uint32_t b = __float_as_uint(v);
  if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (b >> 16) | 0x40u;
  return (b + 0x7FFFu + ((b >> 16) & 1u)) >> 16;
}
D3_INLINE float bf16_round(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// float8 e4m3fn -> float through the hardware converter (OCP e4m3fn on gfx950: 0x7F / 0xFF are NaN). `word` holds
// four codes; HI picks bytes 2-3 instead of 0-1.
template <bool HI> D3_INLINE f32x2 fp8x2_to_f32(uint32_t word) { return __builtin_amdgcn_cvt_pk_f32_fp8((int)word, HI); }

// float -> float8 e4m3fn, to nearest and ties to even, saturating at +-448. Written from the format's definition
// (1 sign, 4 exponent bits biased by 7, 3 mantissa bits, no infinities): the value is rounded on the e4m3 grid of its
// binade (step 2^(e-3), or 2^-9 below 2^-6), which rintf does exactly after scaling by a power of two.
D3_INLINE uint32_t f32_to_fp8(float v) {
  uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
  float a = fabsf(v);
  if (!(a == a)) return sign | 0x7Fu;   // NaN
  if (a >= 464.0f) return sign | 0x7Eu; // saturate (448 is the largest finite; 464 is the midpoint to 512)
  int e = (int)((__float_as_uint(a) >> 23) & 0xFFu) - 127;  // a's binade
  if (e < -6) e = -6;                                        // subnormal range shares 2^-6's step
  float inv_step = __uint_as_float((uint32_t)(3 - e + 127) << 23);  // 2^(3-e)
  float m = rintf(a * inv_step);  // exact scaling by a power of two, then round half to even
  // m in [8, 16] for normals (16 means a carry into the next binade), [0, 8] for subnormals
  uint32_t code;
  if (m >= 16.0f) { e += 1; m = 8.0f; }
  if (m < 8.0f) {
    code = (uint32_t)m;  // subnormal (e == -6): exponent field 0
  } else {
    code = ((uint32_t)(e + 7) << 3) | ((uint32_t)m - 8u);
  }
  if (code > 0x7Eu) code = 0x7Eu;
  return sign | code;
}

// two floats -> two float8 e4m3fn codes (byte 0: a, byte 1: b) through the hardware converter, to nearest and ties to
// even; for |v| < 464 (the kernels feed it |v| <= 448) it agrees with f32_to_fp8 bit for bit.
D3_INLINE uint32_t f32x2_to_fp8x2(float a, float b) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false) & 0xFFFFu;
}
// four floats -> four codes, byte i from value i (the second pair goes to the high half-word)
D3_INLINE uint32_t f32x4_to_fp8x4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// ---------------------------------------------------------------------------------------------------------------
// Wave64 reductions. DPP within each row of 16 lanes (quad swaps, half-row and row mirrors), then the four row results
// read into scalars. Every lane gets the result; the order of combination is fixed, so float sums are deterministic.
D3_INLINE int dpp_i32(int v, int ctrl) {
  switch (ctrl) {
    case 0xB1: return __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    case 0x4E: return __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    case 0x141: return __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
    default: return __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
  }
}

D3_INLINE uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)dpp_i32((int)v, 0xB1));   // quad_perm [1,0,3,2]
  v = max(v, (uint32_t)dpp_i32((int)v, 0x4E));   // quad_perm [2,3,0,1]
  v = max(v, (uint32_t)dpp_i32((int)v, 0x141));  // row_half_mirror
  v = max(v, (uint32_t)dpp_i32((int)v, 0x140));  // row_mirror
  uint32_t a = __builtin_amdgcn_readlane((int)v, 0), b = __builtin_amdgcn_readlane((int)v, 16);
  uint32_t c = __builtin_amdgcn_readlane((int)v, 32), d = __builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}

// the same maximum left in every lane's register (rows of 16 by DPP, then the row pairs and halves exchanged with
// permlane16 / permlane32 swaps): no scalar round trip, so a chain of reductions stays on the vector unit
D3_INLINE uint32_t wave_max_u32_v(uint32_t v) {
  v = max(v, (uint32_t)dpp_i32((int)v, 0xB1));
  v = max(v, (uint32_t)dpp_i32((int)v, 0x4E));
  v = max(v, (uint32_t)dpp_i32((int)v, 0x141));
  v = max(v, (uint32_t)dpp_i32((int)v, 0x140));
  const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  v = max((uint32_t)r16[0], (uint32_t)r16[1]);
  const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  return max((uint32_t)r32[0], (uint32_t)r32[1]);
}

D3_INLINE float wave_max_f32(float v) {
  v = fmaxf(v, __int_as_float(dpp_i32(__float_as_int(v), 0xB1)));
  v = fmaxf(v, __int_as_float(dpp_i32(__float_as_int(v), 0x4E)));
  v = fmaxf(v, __int_as_float(dpp_i32(__float_as_int(v), 0x141)));
  v = fmaxf(v, __int_as_float(dpp_i32(__float_as_int(v), 0x140)));
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

D3_INLINE float wave_sum_f32(float v) {
  v += __int_as_float(dpp_i32(__float_as_int(v), 0xB1));
  v += __int_as_float(dpp_i32(__float_as_int(v), 0x4E));
  v += __int_as_float(dpp_i32(__float_as_int(v), 0x141));
  v += __int_as_float(dpp_i32(__float_as_int(v), 0x140));
  float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (a + b) + (c + d);
}

D3_INLINE int wave_sum_i32(int v) {
  v += dpp_i32(v, 0xB1);
  v += dpp_i32(v, 0x4E);
  v += dpp_i32(v, 0x141);
  v += dpp_i32(v, 0x140);
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
         __builtin_amdgcn_readlane(v, 48);
}

// ---------------------------------------------------------------------------------------------------------------
// Device-scope hand-off between workgroups of one launch (the fused layer's hidden rows and partial outputs).
// Each exchanged float travels as one 64-bit word, its bits and the launch's epoch, written and read with relaxed
// device-scope atomics. The compiler issues those as device-coherent (sc1) accesses, which go past the per-XCD L2s, so
// no L2-wide writeback or invalidate (what an agent-scope release / acquire fence costs) is needed, and a word carries
// its own validity: a consumer polls the words it needs until all show the current epoch, with no flag or counter in
// between. Polls are bounded (keep_polling): past the bound the consumer computes what it waited for itself, so a
// hand-off that never comes (a producer that is not resident) can never hang the device.
D3_INLINE void put_tagged(uint64_t* p, float v, uint32_t epoch) {
  __hip_atomic_store(p, (uint64_t)__float_as_uint(v) | ((uint64_t)epoch << 32), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
D3_INLINE uint64_t get_tagged(const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
// A first read that may be served by this XCD's caches: one workgroup's miss brings the line in for the others. A
// stale line (read before the producer's store landed) shows an old epoch, and the word is then read with get_tagged.
D3_INLINE uint64_t get_tagged_cached(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
D3_INLINE bool tag_is(uint64_t word, uint32_t epoch) { return (uint32_t)(word >> 32) == epoch; }
// the bits in which a word's tag differs from `epoch`: OR them over many words and test once
D3_INLINE uint32_t tag_diff(uint64_t word, uint32_t epoch) { return (uint32_t)(word >> 32) ^ epoch; }
D3_INLINE float tagged_value(uint64_t word) { return __uint_as_float((uint32_t)word); }

// The launch's epoch, the tag of every word it publishes: the dispatch's ID (the HSA queue's packet index of this
// launch, the same for every workgroup and larger for every later dispatch on the queue, graph replays included; LLVM's
// intrinsic, which clang does not expose as a builtin) plus a salt from the queue's address (a kernel argument the
// hardware preloads). Two queues count their dispatches independently; with the salt, a launch on one queue does not
// take the words another queue's launch left behind for its own, so a workspace may move between streams (a graph
// replayed on a stream other than the one it was captured on included). Never 0, the tag of a zeroed workspace.
extern "C" __device__ uint64_t d3_dispatch_id() __asm("llvm.amdgcn.dispatch.id");
D3_INLINE uint32_t launch_epoch() {
  const uint64_t q = (uint64_t)__builtin_amdgcn_queue_ptr();
  const uint32_t salt = (uint32_t)((q >> 6) ^ (q >> 32)) * 0x9E3779B1u;
  const uint32_t e = (uint32_t)d3_dispatch_id() + 1u + salt;
  return e == 0u ? 1u : e;
}
D3_INLINE uint64_t signal_load64(const uint64_t* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// every memory access of this wave so far has completed (its LDS writes are visible to its own lanes)
D3_INLINE void settle() { __builtin_amdgcn_s_waitcnt(0); }
// this wave's LDS accesses (and scalar loads) have completed; its vector loads may still be in flight
// (s_waitcnt lgkmcnt(0) with vmcnt and expcnt left at their maxima: 0xC07F in the gfx9 encoding)
D3_INLINE void lds_settle() { __builtin_amdgcn_s_waitcnt(0xC07F); }

D3_INLINE uint32_t signal_add_ret(uint32_t* counter, uint32_t v) {
  return __hip_atomic_fetch_add(counter, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
D3_INLINE uint32_t signal_load(const uint32_t* counter) {
  return __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
D3_INLINE void signal_store(uint32_t* counter, uint32_t v) {
  __hip_atomic_store(counter, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A launch's give-up word: (epoch << 32) | reason, stored by the first wait of that launch that stops waiting. Every
// other wait of the same launch then stops soon too (the waiting workgroups compute what they waited for themselves);
// the word of an earlier launch carries another epoch and stops nothing.
D3_INLINE bool launch_gave_up(const uint64_t* status, uint32_t epoch) {
  return (uint32_t)(signal_load64(status) >> 32) == epoch;
}
D3_INLINE void give_up(uint64_t* status, uint32_t epoch) {
  __hip_atomic_store(status, ((uint64_t)epoch << 32) | 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// one more poll allowed? Past `limit` polls it records the launch's give-up; every 32 polls it also checks whether
// another wait of the launch gave up (unless `alone`: a recovery's read-back of its own words, which must not stop
// for that).
D3_INLINE bool keep_polling(uint32_t& polls, uint64_t* status, uint32_t limit, uint32_t epoch, bool alone = false) {
  if (!alone && (polls & 31u) == 31u && launch_gave_up(status, epoch)) return false;
  if (++polls > limit) {
    give_up(status, epoch);
    return false;
  }
  __builtin_amdgcn_s_sleep(1);
  return true;
}

// ---------------------------------------------------------------------------------------------------------------
// Routing keys: a bf16 logit and its expert index as one 32-bit integer whose order is "larger logit first, then lower
// index" (the order route_experts ranks by, kernels.py:50-55); -0 ranks as +0. Top-k is then k rounds of a wave max.
D3_INLINE uint32_t route_key(uint32_t logit_bits, int index) {
  uint32_t b = logit_bits == 0x8000u ? 0u : logit_bits;
  const uint32_t ord = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
  return (ord << 16) | (0xFFFFu - (uint32_t)index);
}
D3_INLINE int route_key_index(uint32_t key) { return (int)(0xFFFFu - (key & 0xFFFFu)); }
D3_INLINE float route_key_value(uint32_t key) {
  const uint32_t ord = key >> 16;
  return bf16_to_f32((ord & 0x8000u) ? (ord & 0x7FFFu) : (~ord & 0xFFFFu));
}

// Top-k of a row's router logits (bf16 bits lb[j] for experts lane + 64 j, KPL of them per lane), one round at a time:
// round r takes the wave-wide max over each lane's largest remaining key and lane r keeps it, so after k rounds lanes
// 0 .. k-1 hold the k largest keys, descending, ties to the lower index (kernels.py:50-55).
template <int KPL>
struct TopKeys {
  uint32_t key[KPL], lm, mine;
  D3_INLINE TopKeys(const uint32_t* lb, int lane, int E) : lm(0u), mine(0u) {
#pragma unroll
    for (int j = 0; j < KPL; j++) {
      key[j] = lane + 64 * j < E ? route_key(lb[j], lane + 64 * j) : 0u;
      lm = max(lm, key[j]);
    }
  }
  // rounds from .. to - 1 (to <= 8)
  D3_INLINE void rounds(int lane, int from, int to) {
#pragma unroll
    for (int r = 0; r < 8; r++) {
      if (r >= from && r < to) {
        const uint32_t m = wave_max_u32_v(lm);
        mine = lane == r ? m : mine;
        lm = 0u;
#pragma unroll
        for (int j = 0; j < KPL; j++) {
          key[j] = key[j] == m ? 0u : key[j];
          lm = max(lm, key[j]);
        }
      }
    }
  }
};
template <int KPL>
D3_INLINE uint32_t top_keys(const uint32_t* lb, int lane, int E, int k) {
  TopKeys<KPL> t(lb, lane, E);
  t.rounds(lane, 0, k);
  return t.mine;
}

// The softmax over a row's k routed logits (lanes 0 .. k-1 hold the keys, descending): this lane's weight, the
// exponentials in parallel and their sum in rank order (kernels.py:57-61), bf16-rounded.
D3_INLINE float route_weight(uint32_t mine, int lane, int k) {
  const float top0 = route_key_value((uint32_t)__builtin_amdgcn_readlane((int)mine, 0));
  const float ex = lane < k ? expf(route_key_value(mine) - top0) : 0.0f;
  float total = 0.0f;
#pragma unroll
  for (int r = 0; r < 8; r++)
    if (r < k) total += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ex), r));
  return bf16_round(ex / total);
}
