// The host-offload option's two device-side steps, behind kernels.py's resolve / await_cpu (kernels.py:617-633):
//
//   resolve_kernel    the slot cache's lookup and eviction for one decode row's experts of one layer, on the device so
//                     a decode step never waits on the host (kernels.py:78-191). Every expert keeps a use count that
//                     halves every `half_life` passes; a cached expert keeps its slot, a missed one takes the slot of
//                     the cached expert with the lowest decayed count (a free slot first), never one this layer used nor
//                     one being copied in. With `cpu`, the missed experts are split between the GPU (fill while
//                     reading, plan code 1) and the CPU (code 2), the most used of the CPU's reserving a slot for the
//                     host's copy (table entry -2 - slot, `pending`) while the step's and the layer's budgets last.
//   await_cpu_kernel  a decode layer's bounded wait for the experts it left to the CPU: one lane polls the host flag
//                     (pinned host memory) until it reaches the layer's step or `timeout_us` passes, then the block
//                     copies the host's bf16 result; a late host yields zeros and took_over, after which the GEMVs run
//                     those experts themselves (kernels.py:193-220).
//
// One workgroup of 1024 threads (16 waves of 64) for resolve: the per-expert bookkeeping is a few dozen values, the
// eviction scan walks every slot once per filled expert with a workgroup-wide (value, index) minimum through DPP and
// LDS. The wait's clock is s_memrealtime (a constant 100 MHz counter).
#include "common.hpp"
#include "../../include/drama3_moe.h"

#include <string>

namespace d3 {
int fail(const std::string& msg);
int hip_fail(hipError_t err, const char* what);

namespace {

constexpr int MAX_ROW_EXPERTS = 32;
constexpr float NEVER = 3.0e38f;  // a slot that may not be taken
constexpr int NO_INDEX = 0x7FFFFFFF;

// (value, index) minimum of a wave, ties to the lower index
D3_INLINE void wave_argmin(float& v, int& i) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(v, o);
    const int oi = __shfl_xor(i, o);
    if (ov < v || (ov == v && oi < i)) {
      v = ov;
      i = oi;
    }
  }
}

__global__ void __launch_bounds__(1024) resolve_kernel(const int64_t* ids, int k, int layer, int layers, int experts,
                                                       int* table, int* owner, float* score, int* at, int* pending,
                                                       int count, int* clock, int* budget, int* plan, int* reads,
                                                       int* step, const float* share, float log2_decay, int cpu,
                                                       float admit) {
  __shared__ int slot_of[MAX_ROW_EXPERTS], fill[MAX_ROW_EXPERTS];
  __shared__ float uses[MAX_ROW_EXPERTS];
  __shared__ float best_v[16];
  __shared__ int best_i[16];
  __shared__ int now_s;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int base = layer * experts;
  if (tid == 0) {
    if (layer == 0) clock[0] += 1;
    const int now = clock[0] * layers + layer;
    now_s = now;
    step[0] = now;
  }
  __syncthreads();
  const int now = now_s;
  if (tid < k) {
    const int key = base + (int)ids[tid];
    const float kept = at[key] < 0 ? 0.0f : score[key] * exp2f(log2_decay * (float)(now - at[key]));
    score[key] = kept + 1.0f;
    uses[tid] = kept + 1.0f;
    at[key] = now;
    const int slot = table[key];
    slot_of[tid] = slot >= 0 ? slot : -1;
    // 0 cached, 1 GPU fills, 2 CPU, 3 CPU reserving a slot, 4 missed and not yet split
    fill[tid] = slot >= 0 ? 0 : !cpu ? 1 : slot == -1 ? 4 : 2;
  }
  __syncthreads();
  if (tid == 0) {
    // the split of the missed experts that finishes first: the GPU takes the `gpu` most used
    int ahead[MAX_ROW_EXPERTS], misses = 0;
    for (int e = 0; e < k; e++) {
      ahead[e] = 0;
      for (int o = 0; o < k; o++)
        if (fill[e] == 4 && fill[o] == 4 && (uses[o] > uses[e] || (uses[o] == uses[e] && o < e))) ahead[e]++;
      misses += fill[e] == 4;
    }
    const int gpu = (int)((float)misses * share[0] + 0.5f * (1.0f - share[0]));
    for (int e = 0; e < k; e++)
      if (fill[e] == 4) fill[e] = ahead[e] < gpu ? 1 : uses[e] >= admit ? 3 : 2;
    // the `allowed` most used of the CPU's keep their reservation
    const int allowed = min(budget[0], budget[1]);
    int granted = 0;
    for (int e = 0; e < k; e++) {
      if (fill[e] != 3) continue;
      int before = 0;
      for (int o = 0; o < k; o++)
        if (fill[o] == 3 && (uses[o] > uses[e] || (uses[o] == uses[e] && o < e))) before++;
      if (before < allowed) granted++;
      else fill[e] = 5;
    }
    budget[0] -= granted;
    int counted[3] = {0, 0, 0};
    for (int e = 0; e < k; e++) {
      if (fill[e] == 5) fill[e] = 2;
      counted[fill[e] == 0 ? 0 : fill[e] == 1 ? 1 : 2]++;
    }
    reads[0] += counted[0];
    reads[1] += counted[1];
    reads[2] += counted[2];
  }
  __syncthreads();
  for (int e = 0; e < k; e++) {
    if (fill[e] != 1 && fill[e] != 3) continue;
    float v = NEVER;
    int i = NO_INDEX;
    for (int s = tid; s < count; s += 1024) {
      const int key = owner[s];
      const float sv = key < 0 ? -1.0f
                       : pending[s] || at[key] == now ? NEVER
                                                      : score[key] * exp2f(log2_decay * (float)(now - at[key]));
      if (sv < v) {  // slots ascend per thread, so the first minimum is the lowest index
        v = sv;
        i = s;
      }
    }
    wave_argmin(v, i);
    if (lane == 0) {
      best_v[w] = v;
      best_i[w] = i;
    }
    __syncthreads();
    if (w == 0) {
      v = lane < 16 ? best_v[lane] : NEVER;
      i = lane < 16 ? best_i[lane] : NO_INDEX;
      wave_argmin(v, i);
      // every slot this layer's or pending: the expert goes without one (the GEMVs read it from the bank unfilled)
      if (lane == 0 && v < NEVER) {
        const int key = base + (int)ids[e];
        const int old = owner[i];
        if (old >= 0) table[old] = -1;
        owner[i] = key;
        if (fill[e] == 1) {
          table[key] = i;
        } else {
          table[key] = -2 - i;
          pending[i] = 1;
        }
        slot_of[e] = i;
      }
    }
    __syncthreads();
  }
  if (tid < k) {
    plan[2 * tid] = slot_of[tid];
    plan[2 * tid + 1] = fill[tid] == 3 ? 2 : fill[tid];
  }
}

__global__ void __launch_bounds__(256) await_cpu_kernel(const int* plan, int k, const int* flag, const int* step,
                                                        const uint16_t* result, int64_t timeout_ticks, float* out,
                                                        int* took_over, int H) {
  __shared__ int ready_s;
  if (threadIdx.x == 0) {
    int wanted = 0;
    for (int e = 0; e < k; e++) wanted |= plan[2 * e + 1] == 2;
    int ready = 0;
    if (wanted) {
      const int expected = step[0];
      const uint64_t start = __builtin_amdgcn_s_memrealtime();
      while (true) {
        if (__hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) == expected) {
          ready = 1;
          break;
        }
        if ((int64_t)(__builtin_amdgcn_s_memrealtime() - start) > timeout_ticks) break;
        __builtin_amdgcn_s_sleep(2);
      }
      // the host wrote its result before the flag: see it
      __atomic_thread_fence(__ATOMIC_ACQUIRE);
    }
    ready_s = ready;
    took_over[0] = wanted && !ready;
  }
  __syncthreads();
  const int ready = ready_s;
  for (int i = threadIdx.x; i < H; i += 256) {
    const uint32_t b = ready ? (uint32_t)__hip_atomic_load(result + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) : 0u;
    out[i] = ready ? bf16_to_f32(b) : 0.0f;
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
  hipLaunchKernelGGL(resolve_kernel, dim3(1), dim3(1024), 0, (hipStream_t)stream, ids, k, layer, layers, experts, table,
                     owner, score, at, pending, count, clock, budget, plan, reads, step, share, log2_decay, cpu,
                     (float)admit);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "d3_resolve");
}

int d3_await_cpu(const int32_t* plan, int32_t k, const int32_t* flag, const int32_t* step, const void* result,
                 int32_t timeout_us, float* out, int32_t* took_over, int32_t H, void* stream) {
  if (!plan || !flag || !step || !result || !out || !took_over) return fail("d3_await_cpu: null pointer");
  if (k < 1 || H < 1 || timeout_us < 0) return fail("d3_await_cpu: k, H >= 1, timeout_us >= 0");
  const int64_t ticks = (int64_t)timeout_us * 100;  // s_memrealtime runs at 100 MHz
  hipLaunchKernelGGL(await_cpu_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, (const int*)plan, k,
                     (const int*)flag, (const int*)step, (const uint16_t*)result, ticks, out, (int*)took_over, H);
  const hipError_t err = hipGetLastError();
  return err == hipSuccess ? 0 : hip_fail(err, "d3_await_cpu");
}

}  // extern "C"
