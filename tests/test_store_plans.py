"""The expert store's host-side slot choices against the oracle's one-expert-at-a-time restatement of the reference
(oracle/slots.py host_*_ref / prompt_*_ref / split_ref), on random traces, on the CPU.

offload.SlotPool makes a pass's choices in batches on the device (one sort of the pool per batch, masked scatters);
the oracle claims one expert at a time as the reference's SlotPool does. After every call the slots handed out, the
kernels' fill flags and the whole cache state must agree: table, owner, at, clock and read counters exactly, use
counts within float32 rounding (rtol 2e-6: the two sides' exp2 may differ in the last place, so after each call the
pool continues from the oracle's counts). Slot contents are checked against the banks after every copy."""
import numpy as np
import pytest
import torch

from drama3 import offload
from oracle import slots as ref

HALF_LIFE = offload.HALF_LIFE


def small_banks(layers, E, rows=(3, 2), cols=(8, 4)):
    out = []
    for layer in range(layers):
        banks = []
        for b in range(2):
            q = (torch.arange(E * rows[b] * cols[b], dtype=torch.int32).view(E * rows[b], cols[b])
                 + 100000 * (2 * layer + b))
            s = torch.arange(E * rows[b], dtype=torch.float32) + 1000.0 * layer + 0.5 * b
            banks.append(offload.HostBank(E, {"_qdata": q, "scale": s}, False))
        out.append(tuple(banks))
    return out


def new_pool(L, E, count):
    banks = small_banks(L, E)
    pool = offload.SlotPool(banks, 0, "cpu")
    if count != pool.count:   # a budget of `count` experts
        pool = offload.SlotPool(banks, count * pool.expert_bytes, "cpu")
    assert pool.count == count
    return pool, banks


def check_state(pool, st):
    for name in ("table", "owner", "at", "clock", "reads", "pending"):
        assert np.array_equal(getattr(pool, name).numpy(), st[name]), name
    assert np.allclose(pool.score.numpy(), st["score"], rtol=2e-6, atol=0)
    pool.score.copy_(torch.from_numpy(st["score"]))


def check_contents(pool, banks, layer, expert_slots):
    for e, s in expert_slots.items():
        for i, bank in enumerate(banks[layer]):
            want = bank.take(bank.fields, e, e + 1)
            for name, got in pool.slot_fields(i, s).items():
                assert torch.equal(got, want[name]), (layer, e, s, name)


def fill_in(pool, banks, layer, expert_slots):
    """What the pass's reader does with the slots it was given to fill (the grouped kernels as they read a filled
    expert, prefill_host before its products): copy the experts in."""
    for e, s in expert_slots.items():
        pool.write([s], [bank.take(bank.fields, e, e + 1) for bank in banks[layer]])
    check_contents(pool, banks, layer, expert_slots)


def random_counts(rng, E, rows):
    counts = np.zeros(E, np.int64)
    hot = rng.choice(E, int(rng.integers(1, E + 1)), replace=False)
    counts[hot] = rng.integers(1, rows + 1, hot.shape[0])
    return counts


@pytest.mark.parametrize("seed", range(8))
def test_random_traces_match_the_oracle(seed):
    rng = np.random.default_rng(seed)
    L, E = int(rng.integers(1, 4)), int(rng.integers(6, 24))
    count = int(rng.integers(8, max(9, L * E)))
    pool, banks = new_pool(L, E, count)
    st = ref.new_state(L, E, count)
    for _ in range(10):
        for layer in range(L):
            op = rng.integers(0, 3)
            if op == 0:   # a decode row through the host lookup
                k = int(rng.integers(1, min(8, E) + 1))
                ids = [int(e) for e in rng.choice(E, k, replace=False)]
                want = ref.host_decode_ref(st, layer, L, ids, HALF_LIFE, E)
                got = pool.slots(layer, ids, banks[layer]).tolist()
                assert got == want
                check_contents(pool, banks, layer, dict(zip(ids, got)))
            elif op == 1:  # a prompt pass through the kernels: the fills
                counts = random_counts(rng, E, 5)
                want_slots, want_fills, want_rest = ref.prompt_fill_ref(st, layer, L, counts, HALF_LIFE)
                slot, fill, order, uncached = pool.prompt_fills(layer, torch.from_numpy(counts))
                assert {e: s for e, s in enumerate(slot.tolist()) if s >= 0} == want_slots
                assert [e for e, f in enumerate(fill.tolist()) if f] == sorted(want_fills)
                rest = [e for e, r in zip(order.tolist(), (uncached & ~fill)[order].tolist()) if r]
                assert rest == want_rest
                fill_in(pool, banks, layer, {e: s for e, (s, f) in enumerate(zip(slot.tolist(), fill.tolist())) if f})
            else:          # a prompt pass without kernels: the claimed experts
                counts = random_counts(rng, E, 5)
                want = ref.prompt_keep_ref(st, layer, L, counts, HALF_LIFE)
                slot, keep = pool.prompt_keep(layer, torch.from_numpy(counts))
                assert {e: s for e, s in enumerate(slot.tolist()) if s >= 0} == want
                fill_in(pool, banks, layer, {e: s for e, (s, k) in enumerate(zip(slot.tolist(), keep.tolist())) if k})
            check_state(pool, st)
            table, owner = pool.table.tolist(), pool.owner.tolist()
            for s, key in enumerate(owner):
                assert key < 0 or table[key] == s


@pytest.mark.parametrize("seed", range(4))
def test_claims_and_room_match_the_oracle(seed):
    """use, then single claims until the layer has no room: each claim equals the oracle's scan, room counts down."""
    rng = np.random.default_rng(100 + seed)
    L, E = 2, 10
    pool, banks = new_pool(L, E, 9)
    st = ref.new_state(L, E, 9)
    for _ in range(4):
        for layer in range(L):
            used = [int(e) for e in rng.choice(E, int(rng.integers(1, 6)), replace=False)]
            assert pool.use(layer, used) == ref.host_use_ref(st, layer, L, used, HALF_LIFE, E)
            check_state(pool, st)
            for e in rng.permutation([e for e in range(E) if e not in used])[:3]:
                assert pool.room(layer) == ref.host_room_ref(st, layer, L)
                if pool.room(layer) == 0:
                    with pytest.raises(RuntimeError, match="every slot"):
                        pool.claim(layer, int(e))
                    break
                assert pool.claim(layer, int(e)) == ref.host_claim_ref(st, layer, L, int(e), HALF_LIFE, E)
                check_state(pool, st)


def test_prompt_fills_hand_built():
    """Worked by hand: 8 slots, 2 layers (a layer's share of the cache: 4). Layer 0 uses experts 0-5 with rows
    1, 5, 2, 5, 0, 3: nothing is cached, the four with most rows (1 and 3 with 5, then 5 with 3, then 2 with 2; ties
    to the lower expert) fill slots 0-3 in that order; expert 0 is left for host memory."""
    pool, _ = new_pool(2, 6, 8)
    slot, fill, order, uncached = pool.prompt_fills(0, torch.tensor([1, 5, 2, 5, 0, 3]))
    assert slot.tolist() == [-1, 0, 3, 1, -1, 2]
    assert fill.tolist() == [False, True, True, True, False, True]
    assert order.tolist()[:5] == [1, 3, 5, 2, 0] and uncached.tolist() == [True, True, True, True, False, True]
    # the next pass over layer 0 finds them cached (no fills); the clock moved to pass 2
    slot, fill, _, _ = pool.prompt_fills(0, torch.tensor([0, 1, 1, 0, 0, 1]))
    assert slot.tolist() == [-1, 0, 3, -1, -1, 2] and not fill.any() and pool.clock.item() == 2


@pytest.mark.parametrize("seed", range(4))
def test_split_matches_the_oracle(seed):
    rng = np.random.default_rng(200 + seed)
    store = offload.ExpertStore(0, False)
    for _ in range(50):
        n = int(rng.integers(0, 30))
        experts = [int(e) for e in rng.permutation(64)[:n]]
        counts = {e: int(rng.integers(1, 40)) for e in experts}
        store.cpu_scale, store.gpu_scale = float(rng.uniform(0.3, 3)), float(rng.uniform(0.3, 3))
        nbytes = int(rng.integers(1, 10)) * 1_000_000
        want = ref.split_ref(experts, counts, nbytes, store.cpu_scale, store.gpu_scale, offload.CPU_EXPERT_US,
                             offload.CPU_ROW_US, offload.PCIE_BYTES_PER_US)
        got = store.split(experts, counts, nbytes)
        assert got[0] == want[0] and got[1] == pytest.approx(want[1]) and got[2] == pytest.approx(want[2])


def test_reserved_copies_land_between_steps_on_the_host_device():
    """The decode phase's reservations (as after_layer leaves them) are copied into their slots when the phase ends,
    and mapped; pending marks clear. On the CPU there is no copy stream: the pool still maps them (settle)."""
    pool, banks = new_pool(2, 6, 8)
    pool.device_state()                    # a decode phase starts
    pool.owner[3], pool.table[1 * 6 + 4], pool.pending[3] = 10, -2 - 3, 1   # as resolve leaves a reservation
    pool.reserved.append((1, 4, 3))
    if not torch.cuda.is_available():
        pool._copies.submit = lambda writes, pairs: (writes(), pool._copies.batches.append((_Done(), pairs)))
    pool.host()
    assert pool.table[10].item() == 3 and pool.pending[3].item() == 0 and pool.reserved == []
    check_contents(pool, banks, 1, {4: 3})


class _Done:
    def query(self):
        return True
