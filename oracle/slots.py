"""Oracle for the host-offload option's device steps (test infrastructure only): the slot cache's resolve and the
bounded wait for the host's experts, restated from drama3/kernels.py:78-220 in numpy (float32 where the kernel
computes in float32).

Pinned by tests/test_oracle_slots.py through invariants the cache must keep whatever its arithmetic: table and owner
agree; cached experts keep their slots; a victim is never an expert this layer used nor one being copied in; the
victim is the brute-force minimum of the decayed use counts (free slots first, ties to the lower slot); the CPU /
GPU split and the reservations follow their stated counts on hand-built cases.
"""
import numpy as np

NEVER = np.float32(3.0e38)


def new_state(layers, experts, slots, budget=(0, 0)):
    """Empty cache state: table [L * E] (slot, -1, or -2 - slot while pending), owner [slots] (key or -1), score and
    at per key, pending per slot, the pass clock, the step's / layer's reservation budgets, read counters, the step."""
    return {"table": np.full(layers * experts, -1, np.int32), "owner": np.full(slots, -1, np.int32),
            "score": np.zeros(layers * experts, np.float32), "at": np.full(layers * experts, -1, np.int32),
            "pending": np.zeros(slots, np.int32), "clock": np.zeros(1, np.int32),
            "budget": np.array(budget, np.int32), "reads": np.zeros(3, np.int32), "step": np.zeros(1, np.int32)}


def decayed(score, at, now, log2_decay):
    return np.float32(score * np.exp2(np.float32(log2_decay * np.float32(now - at))))


def resolve_ref(ids, layer, layers, experts, half_life, cpu, admit, st, share):
    """kernels.py:78-191 resolve_experts on state `st` (updated in place): plan [k, 2] int32 = (slot, code), code 0
    cached, 1 the GPU reads the bank and fills the slot, 2 the CPU runs it (slot reserved for the host's copy, or
    -1)."""
    ids = [int(e) for e in ids]
    k = len(ids)
    base = layer * experts
    log2_decay = np.float32(-1.0) / np.float32(np.float32(half_life) * np.float32(layers))
    if layer == 0:
        st["clock"][0] += 1
    now = int(st["clock"][0]) * layers + layer
    st["step"][0] = now
    uses, slot_of, fill = [], [], []
    for e in range(k):
        key = base + ids[e]
        kept = np.float32(0) if st["at"][key] < 0 else decayed(st["score"][key], st["at"][key], now, log2_decay)
        st["score"][key] = np.float32(kept + np.float32(1))
        uses.append(np.float32(kept + np.float32(1)))
        st["at"][key] = now
        slot = int(st["table"][key])
        slot_of.append(slot if slot >= 0 else -1)
        fill.append(0 if slot >= 0 else 1 if not cpu else 4 if slot == -1 else 2)

    def rank(e, cat):
        return sum(1 for o in range(k) if fill[o] == cat and (uses[o] > uses[e] or (uses[o] == uses[e] and o < e)))

    misses = sum(1 for f in fill if f == 4)
    s = np.float32(share)
    gpu = int(np.float32(np.float32(misses) * s + np.float32(0.5) * (np.float32(1) - s)))
    ahead = [rank(e, 4) if fill[e] == 4 else 0 for e in range(k)]
    for e in range(k):
        if fill[e] == 4:
            fill[e] = 1 if ahead[e] < gpu else 3 if uses[e] >= np.float32(admit) else 2
    allowed = min(int(st["budget"][0]), int(st["budget"][1]))
    before = [rank(e, 3) if fill[e] == 3 else 0 for e in range(k)]
    for e in range(k):
        if fill[e] == 3:
            if before[e] < allowed:
                st["budget"][0] -= 1
            else:
                fill[e] = 2
    for e in range(k):
        st["reads"][0 if fill[e] == 0 else 1 if fill[e] == 1 else 2] += 1
    for e in range(k):
        if fill[e] not in (1, 3):
            continue
        best, index = NEVER, None
        for i in range(len(st["owner"])):
            key = int(st["owner"][i])
            if key < 0:
                v = np.float32(-1)
            elif st["pending"][i] or st["at"][key] == now:
                v = NEVER
            else:
                v = decayed(st["score"][key], st["at"][key], now, log2_decay)
            if v < best:
                best, index = v, i
        if index is None:
            continue
        key = base + ids[e]
        old = int(st["owner"][index])
        if old >= 0:
            st["table"][old] = -1
        st["owner"][index] = key
        if fill[e] == 1:
            st["table"][key] = index
        else:
            st["table"][key] = -2 - index
            st["pending"][index] = 1
        slot_of[e] = index
    return np.array([[slot_of[e], 2 if fill[e] == 3 else fill[e]] for e in range(k)], np.int32)


def await_ref(plan, flag, step, result_bits, ready_in_time=True):
    """kernels.py:193-220 await_cpu: (out float32 [1, H], took_over). Without CPU experts in the plan nothing is
    awaited (zeros, took_over 0); with them, the host's bf16 result if its flag reached the step in time, else zeros
    and took_over 1."""
    wanted = bool(np.any(np.asarray(plan).reshape(-1, 2)[:, 1] == 2))
    ready = wanted and int(flag) == int(step) and ready_in_time
    H = np.asarray(result_bits).shape[-1]
    if ready:
        out = (np.asarray(result_bits, np.uint32).reshape(1, H) << 16).view(np.float32)
    else:
        out = np.zeros((1, H), np.float32)
    return out, int(wanted and not ready)
