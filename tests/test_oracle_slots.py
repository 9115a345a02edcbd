"""Pins of oracle/slots.py (the slot cache's resolve and the wait for the host, drama3/kernels.py:78-220) through the
invariants a decayed-LFU slot cache must keep and hand-built cases of its CPU / GPU split. CPU only."""
import numpy as np
import pytest

from oracle import slots


def check_consistent(st):
    for s, key in enumerate(st["owner"]):
        if key >= 0:
            assert st["table"][key] in (s, -2 - s)
    for key, t in enumerate(st["table"]):
        if t >= 0:
            assert st["owner"][t] == key and not st["pending"][t]
        elif t <= -2:
            assert st["owner"][-2 - t] == key and st["pending"][-2 - t]


@pytest.mark.parametrize("cpu", [0, 1])
def test_random_trace_keeps_invariants_and_evicts_the_least_used(cpu):
    rng = np.random.default_rng(cpu)
    L, E, S, k = 3, 16, 6, 4
    st = slots.new_state(L, E, S, budget=(2, 1))
    half_life = 2.0
    log2_decay = np.float32(-1.0) / np.float32(np.float32(half_life) * np.float32(L))
    for step in range(12):
        for layer in range(L):
            st["budget"][0] = 2  # the step's reservations
            ids = rng.choice(E, k, replace=False)
            before = {key: dict(table=int(st["table"][key])) for key in range(L * E)}
            owner_before = st["owner"].copy()
            pending_before = st["pending"].copy()
            plan = slots.resolve_ref(ids, layer, L, E, half_life, cpu, 3.0, st, 0.5)
            now = int(st["step"][0])
            assert now == int(st["clock"][0]) * L + layer
            check_consistent(st)
            for e, (slot, code) in enumerate(plan):
                key = layer * E + int(ids[e])
                if before[key]["table"] >= 0:  # cached: keeps its slot
                    assert code == 0 and slot == before[key]["table"]
                assert st["at"][key] == now
            # victims: slots whose owner changed were free, or held an expert neither used now nor pending
            for s in range(S):
                if owner_before[s] != st["owner"][s] and owner_before[s] >= 0:
                    assert not pending_before[s]
                    assert st["table"][owner_before[s]] == -1
            # brute force: every slot taken from an earlier owner was a minimum of the decayed counts among the
            # candidates at that time (free slots count -1); checked for the first fill of the call
            fills = [(e, int(s)) for e, (s, c) in enumerate(plan) if c in (1, 2) and s >= 0
                     and before[layer * E + int(ids[e])]["table"] < 0]
            if fills:
                _, s0 = fills[0]
                vals = []
                for s in range(S):
                    key = owner_before[s]
                    if key < 0:
                        vals.append(-1.0)
                    elif pending_before[s] or (st["at"][key] == now and st["owner"][s] == key):
                        vals.append(np.inf)
                    else:
                        vals.append(float(slots.decayed(st["score"][key], st["at"][key], now, log2_decay)))
                assert vals[s0] == min(vals) and s0 == int(np.argmin(vals))
            # settle the host's copies: pending slots become cached (SlotPool.settle)
            for s in range(S):
                if st["pending"][s]:
                    st["pending"][s] = 0
                    st["table"][st["owner"][s]] = s


def test_split_between_gpu_and_cpu():
    """Four missed experts, share 0.5: the GPU takes the int(4 * 0.5 + 0.25) = 2 most used; of the CPU's, the ones used
    admit times or more reserve a slot while the budget lasts (here 1), the rest get none."""
    L, E, S = 1, 8, 8
    st = slots.new_state(L, E, S, budget=(1, 4))
    st["score"][:4] = [5.0, 4.0, 3.0, 2.5]
    st["at"][:4] = 0
    st["clock"][0] = 0  # this call makes the pass 1, step 1: one step of decay
    plan = slots.resolve_ref([3, 2, 1, 0], 0, L, E, 1e9, 1, 2.0, st, 0.5)
    codes = {int(e): tuple(p) for e, p in zip([3, 2, 1, 0], plan)}
    assert codes[0][1] == 1 and codes[1][1] == 1          # the two most used: GPU fills
    assert codes[2][1] == 2 and codes[2][0] >= 0          # next: CPU, reserves (uses 4 >= admit, budget 1)
    assert codes[3] == (-1, 2)                           # budget spent: CPU without a slot
    assert st["budget"][0] == 0 and list(st["reads"]) == [0, 2, 2]
    assert st["table"][2] == -2 - codes[2][0] and st["pending"][codes[2][0]] == 1


def test_await_ref():
    plan_cpu = np.array([[0, 0], [-1, 2]])
    plan_gpu = np.array([[0, 0], [1, 1]])
    res = np.array([0x3F80, 0xC000], np.uint16)  # 1.0, -2.0
    out, took = slots.await_ref(plan_cpu, 7, 7, res)
    assert list(out[0]) == [1.0, -2.0] and took == 0
    out, took = slots.await_ref(plan_cpu, 6, 7, res)
    assert np.all(out == 0) and took == 1
    out, took = slots.await_ref(plan_gpu, 6, 7, res)
    assert np.all(out == 0) and took == 0


def test_slots_taken_are_the_smallest_keys_in_routing_order():
    """Taking a slot takes only that slot out of the candidates (its new owner is an expert of this layer), so the
    slots a call hands out are the n smallest (decayed count, slot) keys among the slots that may be taken, free
    slots first, in the order of the experts that need one. The device kernel selects them that way; here the
    oracle's sequential scans are checked against it on random traces."""
    rng = np.random.default_rng(11)
    for trial in range(200):
        L, E = int(rng.integers(1, 5)), int(rng.integers(8, 64))
        k = int(rng.integers(1, min(9, E)))
        st = slots.new_state(L, E, int(rng.integers(1, 3 * E)), budget=(int(rng.integers(0, 4)), 2))
        cpu, share = int(rng.integers(0, 2)), float(rng.choice([0.0, 0.5]))
        for _ in range(6):
            for layer in range(L):
                ids = rng.choice(E, k, replace=False)
                now = (int(st["clock"][0]) + (layer == 0)) * L + layer
                log2_decay = np.float32(-1.0) / np.float32(np.float32(3.0) * np.float32(L))
                routed = {layer * E + int(e) for e in ids}
                keys = []
                for s, key in enumerate(st["owner"]):
                    if key < 0:
                        keys.append((-1.0, s))
                    elif not st["pending"][s] and int(key) not in routed:
                        keys.append((float(slots.decayed(st["score"][key], st["at"][key], now, log2_decay)), s))
                before = st["owner"].copy()
                plan = slots.resolve_ref(ids, layer, L, E, 3.0, cpu, 2.5, st, share)
                # slots handed out by this call: each expert's slot that it did not already own, in routing order
                taken = [int(plan[e, 0]) for e in range(k) if plan[e, 0] >= 0 and before[plan[e, 0]] != layer * E + int(ids[e])]
                assert taken == [s for _, s in sorted(keys)[:len(taken)]]
            for s in np.nonzero(st["pending"])[0]:
                st["pending"][s] = 0
                st["table"][st["owner"][s]] = s


# ---- the host-side rules (host_*_ref, prompt_*_ref, split_ref)
def test_host_claims_evict_the_least_used_worked_by_hand():
    """8 slots, one layer of 12 experts: pass 1 uses 0-7 (free slots 0-7 in order); passes 2 and 3 use 0-6 again, so
    expert 7 is the least used; pass 4's miss (9) takes its slot 7, and expert 7 leaves the table."""
    st = slots.new_state(1, 12, 8)
    assert slots.host_decode_ref(st, 0, 1, list(range(8)), 128, 12) == list(range(8))
    for _ in range(2):
        assert slots.host_decode_ref(st, 0, 1, list(range(7)), 128, 12) == list(range(7))
    assert slots.host_decode_ref(st, 0, 1, [9], 128, 12) == [7]
    assert st["table"][7] == -1 and st["table"][9] == 7 and st["owner"][7] == 9
    assert list(st["reads"]) == [14, 9, 0] and st["clock"][0] == 4


def test_host_claim_is_the_brute_force_minimum():
    rng = np.random.default_rng(3)
    for _ in range(100):
        L, E, S = 2, 12, int(rng.integers(4, 20))
        st = slots.new_state(L, E, S)
        for _ in range(int(rng.integers(1, 6))):
            for layer in range(L):
                slots.host_use_ref(st, layer, L, list(rng.choice(E, 3, replace=False)), 2.0, E)
        layer = int(rng.integers(0, L))
        now = int(st["clock"][0]) * L + layer
        d = np.float32(-1.0) / np.float32(np.float32(2.0) * np.float32(L))
        vals = [(-1.0 if k < 0 else np.inf if st["at"][k] == now else float(slots.decayed(st["score"][k], st["at"][k],
                                                                                          now, d)), s)
                for s, k in enumerate(st["owner"])]
        if min(vals)[0] == np.inf:
            continue
        want = min(vals)[1]
        assert slots.host_claim_ref(st, layer, L, 11, 2.0, E) == want


def test_prompt_fill_worked_by_hand():
    """8 slots, 2 layers (share 4): rows 1, 5, 2, 5, 0, 3; the four uncached experts with most rows (1, 3, 5, 2; ties to
    the lower expert) fill the free slots 0-3 in that order, and expert 0 is the rest."""
    st = slots.new_state(2, 6, 8)
    got, fills, rest = slots.prompt_fill_ref(st, 0, 2, [1, 5, 2, 5, 0, 3], 128)
    assert got == {1: 0, 3: 1, 5: 2, 2: 3} and fills == [1, 3, 5, 2] and rest == [0]


def test_prompt_keep_never_takes_a_slot_the_layer_reads():
    """4 slots, 2 layers (share 2): layer 0's experts 0 and 1 cached in slots 0 and 1, slots 2 and 3 free. A pass using
    0, 1 (cached) and 2, 3, 4 (rows 3, 9, 9): room is 2 (slots 0 and 1 are read), so the two with most rows, 3 and 4,
    claim the free slots 2 and 3 in ascending expert order; 2 is read from host memory."""
    st = slots.new_state(2, 6, 4)
    slots.host_decode_ref(st, 0, 2, [0, 1], 128, 6)
    got = slots.prompt_keep_ref(st, 0, 2, [1, 1, 3, 9, 9, 0], 128)
    assert got == {0: 0, 1: 1, 3: 2, 4: 3}


def test_split_worked_by_hand():
    """PCIe 100 us per expert; the CPU 60 + 13 per row: costs 190, 99, 73, 73 for rows 10, 3, 1, 1. e0 goes to the GPU
    (190 > 0 + 100), e1 to the CPU (99 <= 100 + 100), e2 to the CPU (172 <= 200), e3 to the GPU (245 > 200)."""
    counts = {0: 10, 1: 3, 2: 1, 3: 1}
    assert slots.split_ref([0, 1, 2, 3], counts, 1_200_000, 1.0, 1.0, 60, 13, 12e3) == ([1, 2], 172.0, 200.0)
    # a CPU twice as slow as modelled: only e1 (198 <= 200); the modelled times come back unscaled
    assert slots.split_ref([0, 1, 2, 3], counts, 1_200_000, 2.0, 1.0, 60, 13, 12e3) == ([1], 99.0, 300.0)
