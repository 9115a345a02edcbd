// The host-offload option's two device-side steps, behind kernels.py's resolve / await_cpu (reference semantics:
// drama3/kernels.py:78-220; wrappers kernels.py:617-633).
//
// resolve_kernel: one decode row's experts of one layer through the slot cache, on the device. Semantics: each routed
// expert's use count decays by half every `half_life` passes and gains one; an expert with a slot keeps it; a missed
// one is read from the bank by the GEMVs (filling a slot on the way), or, with `cpu`, part of the missed ones go to
// the CPU (their number set by `share`, the most used staying on the GPU), and of those the most used ones (count >=
// `admit`) reserve a slot for the host's copy while the step's and the layer's budgets last. Each expert that gets a
// slot takes, in routing order, the free slot with the lowest index, else the slot whose owner has the lowest decayed
// count (ties to the lower slot), never one this layer used nor one being copied in.
//
// Design (gfx950, one workgroup of 256 threads):
//   * wave 0 does the per-expert bookkeeping with a lane per routed expert (k <= 32): counts, the route of each
//     expert, and its rank among the experts of a route by a lane-parallel count over (count, index) keys; the CPU /
//     GPU split, the reservations and the read counters come from ballots and population counts;
//   * taking a slot only takes that slot out of the candidates (its new owner is an expert of this layer), so the
//     slots the experts get are the n smallest (decayed count, slot) keys among the candidates, handed out in routing
//     order. All four waves select them: each thread keeps the smallest key of its own slots above the last one
//     picked from them, a workgroup minimum picks the next key, and only the thread that owned it looks again;
//   * wave 0 then writes the table, owners and pending flags, lane by lane.
//
// await_cpu_kernel: a decode layer's bounded wait for the experts it left to the CPU. One wave: a ballot over the plan
// tells whether any expert is the CPU's; lane 0 then polls the host's flag (pinned host memory, system-scope loads)
// until it reaches the layer's step or `timeout_us` passes (s_memrealtime, a 100 MHz counter); the wave copies the
// host's bf16 result, four values a lane at a time, or writes zeros and sets took_over for a late host (the GEMVs then
// run those experts themselves).
#include "common.hpp"
#include "../../include/drama3_moe.h"

#include <string>

namespace d3 {
int fail(const std::string& msg);
int hip_fail(hipError_t err, const char* what);

namespace {

constexpr int MAX_ROW_EXPERTS = 32;
constexpr int RESOLVE_THREADS = 256;
// how a routed expert is served (plan code = route, RESERVE reported as the CPU's code 2)
enum Route : int { CACHED = 0, FILL = 1, ON_CPU = 2, RESERVE = 3 };
constexpr uint64_t NO_KEY = ~0ull;

// a non-negative float's order as an unsigned integer, with -1 (a free slot) below every count
D3_INLINE uint32_t count_order(float v) { return v < 0.0f ? 0u : __float_as_uint(v) + 1u; }

// The decayed use count of `key` at step `now` (the form every step of the cache uses, so comparisons agree)
D3_INLINE float decayed(const float* score, const int* at, int key, int now, float log2_decay) {
  return score[key] * exp2f(log2_decay * (float)(now - at[key]));
}

// A slot's eviction key: (count order << 32) | slot, smaller first; NO_KEY when the slot may not be taken (being
// copied in, or its owner used by this layer)
D3_INLINE uint64_t slot_key(int s, const int* owner, const int* pending, const float* score, const int* at, int now,
                            float log2_decay) {
  const int key = owner[s];
  if (key < 0) return (uint64_t)(uint32_t)s;  // free: count order 0
  if (pending[s] || at[key] == now) return NO_KEY;
  return ((uint64_t)count_order(decayed(score, at, key, now, log2_decay)) << 32) | (uint32_t)s;
}

// Within a wave: how many lanes of `subset` rank above this lane's `order` (larger first; orders are distinct)
D3_INLINE int rank_among(uint64_t subset, uint64_t order) {
  int above = 0;
  while (subset) {
    const int j = __builtin_ctzll(subset);
    subset &= subset - 1;
    const uint64_t other = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(order >> 32), j) << 32) |
                           (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)order, j);
    above += other > order;
  }
  return above;
}

D3_INLINE uint64_t wave_min_u64(uint64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const uint64_t w = ((uint64_t)(uint32_t)__shfl_xor((int)(v >> 32), o) << 32) | (uint32_t)__shfl_xor((int)(uint32_t)v, o);
    v = w < v ? w : v;
  }
  return v;
}

__global__ void __launch_bounds__(RESOLVE_THREADS) resolve_kernel(
    const int64_t* ids, int k, int layer, int layers, int experts, int* table, int* owner, float* score, int* at,
    int* pending, int count, int* clock, int* budget, int* plan, int* reads, int* step, const float* share,
    float log2_decay, int cpu, float admit) {
  __shared__ int now_s, wanted_s;
  __shared__ uint64_t best_s[RESOLVE_THREADS / 64];
  __shared__ int picked_s[MAX_ROW_EXPERTS];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int base = layer * experts;
  int key = -1, route = CACHED, slot_now = -1;
  uint64_t needs = 0;
  // ---- the row's experts, a lane each (wave 0)
  if (w == 0) {
    int tick = 0;
    if (lane == 0) {
      tick = clock[0] + (layer == 0);
      if (layer == 0) clock[0] = tick;
      step[0] = tick * layers + layer;
    }
    const int now = __builtin_amdgcn_readfirstlane(tick) * layers + layer;
    const bool mine = lane < k;
    float uses = 0.0f;
    if (mine) {
      key = base + (int)ids[lane];
      const float kept = at[key] < 0 ? 0.0f : decayed(score, at, key, now, log2_decay);
      uses = kept + 1.0f;
      score[key] = uses;
      at[key] = now;
      slot_now = table[key];
    }
    // rank order: larger count first, then the lower routing position
    const uint64_t order = mine ? ((uint64_t)__float_as_uint(uses) << 32) | (uint32_t)(63 - lane) : 0ull;
    if (!cpu) {
      route = slot_now >= 0 ? CACHED : FILL;
    } else {
      // missed experts not being copied in are split; those being copied in stay with the CPU
      const uint64_t split = __ballot(mine && slot_now == -1);
      const float misses = (float)__popcll(split), s = share[0];
      const int on_gpu = (int)__fadd_rn(__fmul_rn(misses, s), __fmul_rn(0.5f, __fsub_rn(1.0f, s)));
      const int r = rank_among(split, order);
      route = slot_now >= 0 ? CACHED : slot_now != -1 ? ON_CPU : r < on_gpu ? FILL : uses >= admit ? RESERVE : ON_CPU;
      // the reservations the budgets allow, to the most used first
      const uint64_t want = __ballot(mine && route == RESERVE);
      const int allowed = min(budget[0], budget[1]);
      if (route == RESERVE && rank_among(want, order) >= allowed) route = ON_CPU;
      const int granted = __popcll(__ballot(mine && route == RESERVE));
      if (lane == 0) budget[0] -= granted;
    }
    const int hits = __popcll(__ballot(mine && route == CACHED));
    const int fills = __popcll(__ballot(mine && route == FILL));
    if (lane == 0) {
      reads[0] += hits;
      reads[1] += fills;
      reads[2] += k - hits - fills;
    }
    needs = __ballot(mine && (route == FILL || route == RESERVE));
    if (lane == 0) {
      now_s = now;
      wanted_s = __popcll(needs);
    }
  }
  __syncthreads();
  // ---- the n best slots (all waves), n = experts that need one
  const int n = wanted_s, now = now_s;
  if (n > 0) {
    // this thread's slots are tid, tid + 256, ...; its candidate is the smallest key above `floor`
    uint64_t floor = 0, mine_key = NO_KEY;
    bool first = true;
    auto look = [&]() {
      uint64_t best = NO_KEY;
      for (int s = tid; s < count; s += RESOLVE_THREADS) {
        const uint64_t kk = slot_key(s, owner, pending, score, at, now, log2_decay);
        if ((first || kk > floor) && kk < best) best = kk;
      }
      mine_key = best;
      first = false;
    };
    look();
    for (int j = 0; j < n; j++) {
      const uint64_t wmin = wave_min_u64(mine_key);
      if (lane == 0) best_s[w] = wmin;
      __syncthreads();
      uint64_t pick = best_s[0];
#pragma unroll
      for (int q = 1; q < RESOLVE_THREADS / 64; q++) pick = best_s[q] < pick ? best_s[q] : pick;
      if (tid == 0) picked_s[j] = pick == NO_KEY ? -1 : (int)(uint32_t)pick;
      if (pick != NO_KEY && mine_key == pick) {  // its owner looks for its next candidate
        floor = pick;
        look();
      }
      __syncthreads();  // best_s is rewritten by the next round
    }
  }
  // ---- hand the picks out in routing order and write the plan (wave 0)
  if (w == 0 && lane < k) {
    int slot = slot_now >= 0 ? slot_now : -1;
    if ((needs >> lane) & 1ull) {
      const int j = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(needs >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)needs, 0u));
      const int s = picked_s[j];
      if (s >= 0) {
        const int old = owner[s];
        if (old >= 0) table[old] = -1;
        owner[s] = key;
        if (route == FILL) {
          table[key] = s;
        } else {
          table[key] = -2 - s;
          pending[s] = 1;
        }
        slot = s;
      }
    }
    plan[2 * lane] = slot;
    plan[2 * lane + 1] = route == RESERVE ? ON_CPU : route;
  }
}

__global__ void __launch_bounds__(64) await_cpu_kernel(const int* plan, int k, const int* flag, const int* step,
                                                       const uint16_t* result, int64_t timeout_ticks, float* out,
                                                       int* took_over, int H) {
  const int lane = threadIdx.x;
  // the CPU's experts: plan code 2 (k <= 64 at this wave's width; more are folded in per lane)
  bool cpu_expert = false;
  for (int e = lane; e < k; e += 64) cpu_expert = cpu_expert || plan[2 * e + 1] == ON_CPU;
  const bool waits = __ballot(cpu_expert) != 0ull;
  int arrived = 0;
  if (waits && lane == 0) {
    const int expected = step[0];
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    while (!(arrived = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == expected) &&
           (int64_t)(__builtin_amdgcn_s_memrealtime() - t0) <= timeout_ticks)
      __builtin_amdgcn_s_sleep(2);
    __atomic_thread_fence(__ATOMIC_ACQUIRE);  // the host wrote the result before the flag
    took_over[0] = !arrived;
  } else if (lane == 0) {
    took_over[0] = 0;
  }
  arrived = __builtin_amdgcn_readfirstlane(arrived);
  for (int i = 4 * lane; i < H; i += 256) {
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (arrived) {
#pragma unroll
      for (int j = 0; j < 4; j++)
        if (i + j < H) v[j] = bf16_to_f32(__hip_atomic_load(result + i + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM));
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
      if (i + j < H) out[i + j] = v[j];
  }
}

}  // namespace
}  // namespace d3

using namespace d3;

extern "C" {

int d3_resolve(const int64_t* ids, int32_t k, int32_t layer, int32_t layers, int32_t experts, int32_t* table,
               int32_t* owner, float* score, int32_t* at, int32_t* pending, int32_t count, int32_t* clock,
               int32_t* budget, int32_t* plan, int32_t* reads, int32_t* step, const float* share, double half_life,
               int32_t cpu, double admit, void* stream) {
  if (!ids || !table || !owner || !score || !at || !pending || !clock || !budget || !plan || !reads || !step || !share)
    return fail("d3_resolve: null pointer");
  if (k < 1 || k > MAX_ROW_EXPERTS || layer < 0 || layer >= layers || experts < 1 || count < 1 || half_life <= 0)
    return fail("d3_resolve: 1 <= k <= 32, 0 <= layer < layers, count >= 1, half_life > 0");
  const float log2_decay = -1.0f / ((float)half_life * (float)layers);
  hipLaunchKernelGGL(resolve_kernel, dim3(1), dim3(RESOLVE_THREADS), 0, (hipStream_t)stream, ids, k, layer, layers,
                     experts, table, owner, score, at, pending, count, clock, budget, plan, reads, step, share,
                     log2_decay, cpu, (float)admit);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "d3_resolve");
}

int d3_await_cpu(const int32_t* plan, int32_t k, const int32_t* flag, const int32_t* step, const void* result,
                 int32_t timeout_us, float* out, int32_t* took_over, int32_t H, void* stream) {
  if (!plan || !flag || !step || !result || !out || !took_over) return fail("d3_await_cpu: null pointer");
  if (k < 1 || H < 1 || timeout_us < 0) return fail("d3_await_cpu: k, H >= 1, timeout_us >= 0");
  const int64_t ticks = (int64_t)timeout_us * 100;  // s_memrealtime runs at 100 MHz
  hipLaunchKernelGGL(await_cpu_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, (const int*)plan, k,
                     (const int*)flag, (const int*)step, (const uint16_t*)result, ticks, out, (int*)took_over, H);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "d3_await_cpu");
}

}  // extern "C"
