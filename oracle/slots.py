"""Oracle for the host-offload option (test infrastructure only): the slot cache's resolve and the bounded wait for
the host's experts, restated from drama3/kernels.py:78-220 in numpy (float32 where the kernel computes in float32);
and the cache's host-side lookups and prompt passes (drama3/offload.py:454-552, 660-732), restated one expert at a
time as the reference runs them. The use counts decay by the resolve kernel's formula on both sides
(count * 2^(log2_decay * (now - at)), log2_decay = -1 / (half_life * layers) in float32), so that the host's and the
device's views of a count agree bit for bit.

The resolve and the wait are pinned by tests/test_oracle_slots.py through invariants the cache must keep whatever its
arithmetic: table and owner agree; cached experts keep their slots; a victim is never an expert this layer used nor
one being copied in; the victim is the brute-force minimum of the decayed use counts (free slots first, ties to the
lower slot); the CPU / GPU split and the reservations follow their stated counts on hand-built cases. The host-side
rules are pinned there too: hand-built passes with known outcomes, the same invariants, and the claims checked
against a brute-force minimum over the slots.
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


# ---- the host-side lookups and prompt passes, one expert at a time (drama3/offload.py:454-552, 660-732)
def _log2_decay(half_life, layers):
    return np.float32(-1.0) / np.float32(np.float32(half_life) * np.float32(layers))


def host_now(st, layer, layers):
    """A host pass's step for `layer` (offload.py:666-670): the first layer starts a new pass."""
    if layer == 0:
        st["clock"][0] += 1
    return int(st["clock"][0]) * layers + layer


def host_use_ref(st, layer, layers, experts, half_life, n_experts):
    """offload.py:685-692 use: every expert of the list counts a use at this step; {expert: slot} of the cached ones."""
    now = host_now(st, layer, layers)
    d = _log2_decay(half_life, layers)
    for e in experts:
        key = layer * n_experts + int(e)
        kept = np.float32(0) if st["at"][key] < 0 else decayed(st["score"][key], st["at"][key], now, d)
        st["score"][key] = np.float32(kept + np.float32(1))
        st["at"][key] = now
    return {int(e): int(st["table"][layer * n_experts + int(e)]) for e in experts
            if st["table"][layer * n_experts + int(e)] >= 0}


def host_room_ref(st, layer, layers):
    """offload.py:717-720 room: slots not holding an expert `layer` used in this pass."""
    now = int(st["clock"][0]) * layers + layer
    return sum(1 for key in st["owner"] if key < 0 or st["at"][key] != now)


def host_claim_ref(st, layer, layers, expert, half_life, n_experts):
    """offload.py:694-715 claim + assign: the slot of the least used cached expert, a free slot first (value -1), the
    lowest slot among equals, never a slot holding an expert `layer` used in this pass; its old expert leaves the
    table."""
    now = int(st["clock"][0]) * layers + layer
    d = _log2_decay(half_life, layers)
    best, index = np.float32(np.inf), None
    for s, key in enumerate(st["owner"]):
        if key < 0:
            v = np.float32(-1)
        elif st["at"][key] == now:
            continue
        else:
            v = decayed(st["score"][key], st["at"][key], now, d)
        if v < best:
            best, index = v, s
    assert index is not None, "no slot left for this layer"
    key = layer * n_experts + int(expert)
    old = int(st["owner"][index])
    if old >= 0:
        st["table"][old] = -1
    st["owner"][index] = key
    st["table"][key] = index
    return index


def host_decode_ref(st, layer, layers, experts, half_life, n_experts):
    """offload.py:721-732 slots: a decode row's experts looked up; each missed one, in routing order, claims a slot;
    reads += (hits, misses, 0). Returns the slots in routing order."""
    cached = host_use_ref(st, layer, layers, experts, half_life, n_experts)
    out = [cached[int(e)] if int(e) in cached else host_claim_ref(st, layer, layers, e, half_life, n_experts)
           for e in experts]
    st["reads"][0] += len(cached)
    st["reads"][1] += len(experts) - len(cached)
    return out


def _by_rows(experts, counts):
    """The experts, most rows first, the lower expert first among equals (a stable sort, offload.py:478)."""
    return sorted(experts, key=lambda e: -counts[e])


def prompt_fill_ref(st, layer, layers, counts, half_life):
    """offload.py:468-484, the kernels' prompt pass: the used experts counted; the uncached ones, most rows first, fill
    the free slots in ascending order, up to count // layers of them. Returns ({expert: slot} of cached and filled,
    filled experts, the rest of the uncached ones most rows first)."""
    n_experts = len(counts)
    used = [e for e in range(n_experts) if counts[e]]
    slots_of = host_use_ref(st, layer, layers, used, half_life, n_experts)
    rest = _by_rows([e for e in used if e not in slots_of], counts)
    free = [s for s, key in enumerate(st["owner"]) if key < 0]
    fills = rest[:min(len(st["owner"]) // layers, len(free))]
    for e, s in zip(fills, free):
        key = layer * n_experts + e
        st["owner"][s] = key
        st["table"][key] = s
        slots_of[e] = s
    return slots_of, fills, rest[len(fills):]


def prompt_keep_ref(st, layer, layers, counts, half_life):
    """offload.py:528-545, the prompt pass without kernels: the used experts counted; the uncached ones with most rows,
    up to min(count // layers, room) of them, claim slots in ascending expert order (the others are read from host
    memory). Returns {expert: slot} of cached and kept experts."""
    n_experts = len(counts)
    used = [e for e in range(n_experts) if counts[e]]
    cached = host_use_ref(st, layer, layers, used, half_life, n_experts)
    share = min(len(st["owner"]) // layers, host_room_ref(st, layer, layers))
    keep = set(_by_rows([e for e in used if e not in cached], counts)[:share])
    out = dict(cached)
    for e in used:
        if e in keep:
            out[e] = host_claim_ref(st, layer, layers, e, half_life, n_experts)
    return out


def split_ref(experts, counts, expert_bytes, cpu_scale, gpu_scale, cpu_expert_us, cpu_row_us, bytes_per_us):
    """offload.py:514-526: each expert (most rows first) goes to the CPU if the CPU, with it, would be done no later
    than the GPU with it read over PCIe; (CPU experts, the CPU's and the GPU's modelled us, unscaled)."""
    transfer = gpu_scale * expert_bytes / bytes_per_us
    on_cpu, cpu_us, gpu_us = [], 0.0, 0.0
    for e in experts:
        cost = cpu_scale * (cpu_expert_us + cpu_row_us * counts[e])
        if cpu_us + cost <= gpu_us + transfer:
            on_cpu.append(e)
            cpu_us += cost
        else:
            gpu_us += transfer
    return on_cpu, cpu_us / cpu_scale, gpu_us / gpu_scale
