"""drama3.offload and drama3.kernels on the CPU: the reference's public names and signatures (tests/golden/
reference_api.json, read from drama3/offload.py and drama3/kernels.py by make_api_list.py), the helper functions
against the oracle and closed forms, the slot pool's host-side lookups, the prompt split's cost model, and an
ExpertStore's host path (host-lookup decode, prefill_host) against the oracle's resident layer.

Bars: signatures and constants equal; dequantize_fp8 within one float32 rounding of the float64 product; dense bf16
paths (the reference's own CPU arithmetic) within rel-L2 2e-2 of the oracle; float32 paths within 1e-5."""
import ast
import inspect
import json
import pathlib

import numpy as np
import pytest
import torch
import torch.nn as nn

from drama3 import kernels, offload
from oracle import numerics
from oracle import reference as ref

API = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_api.json").read_text())
MODULES = {"offload": offload, "kernels": kernels}


def _params(fn):
    out = []
    for p in inspect.signature(fn).parameters.values():
        default = None if p.default is inspect.Parameter.empty else p.default
        out.append([p.name, p.kind.name, default])
    return out


def _same(mine, theirs):
    """Parameter lists equal: names and kinds; defaults compared as values."""
    assert [p[:2] for p in mine] == [p[:2] for p in theirs]
    for (name, _, d_mine), (_, _, d_ref) in zip(mine, theirs):
        assert (d_ref is None and d_mine is None) or d_mine == ast.literal_eval(d_ref), name


@pytest.mark.parametrize("module", sorted(MODULES))
def test_reference_surface(module):
    api, mod = API[module], MODULES[module]
    for name, value in api["constants"].items():
        assert hasattr(mod, name), name
        assert getattr(mod, name) == pytest.approx(value), name
    for name, params in api["functions"].items():
        assert callable(getattr(mod, name, None)), name
        _same(_params(getattr(mod, name)), params)
    for name, cls in api["classes"].items():
        mine = getattr(mod, name, None)
        assert inspect.isclass(mine), name
        for base in cls["bases"]:
            want = nn.Module if base == "nn.Module" else getattr(mod, base)
            assert issubclass(mine, want), (name, base)
        for method, params in cls["methods"].items():
            assert callable(getattr(mine, method, None)), f"{name}.{method}"
            _same(_params(getattr(mine, method)), params)


def test_store_instance_attributes():
    """The attributes the reference's loader.py / generate.py / model.py read off a store."""
    store = offload.ExpertStore(123, False)
    for name in ("banks", "cache", "cache_bytes", "pin", "sync_free", "cpu_side", "cpu_experts", "rotation"):
        assert hasattr(store, name), name
    assert store.cache_bytes == 123 and store.pin is False and store.sync_free is False and store.cache is None


# ------------------------------------------------------------------------------------------------ the helpers
def test_fp8_experts_raise_off_gfx950():
    mod = offload.FP8Experts(2, 256, 128, device="cpu", dtype=torch.bfloat16)
    assert mod.sync_free(torch.device("cpu")) is False
    with pytest.raises(RuntimeError, match="gfx950"):
        mod(torch.zeros((1, 256), dtype=torch.bfloat16), torch.zeros((1, 1), dtype=torch.long),
            torch.ones((1, 1), dtype=torch.bfloat16))


def test_host_embedding():
    emb = nn.Embedding(50, 8)
    host = offload.HostEmbedding(emb)
    ids = torch.tensor([[3, 7, 3], [0, 49, 12]])
    assert torch.equal(host(ids), emb(ids))
    assert host(ids, torch.bfloat16).dtype == torch.bfloat16


def test_hadamard_against_the_oracle():
    for size in (4, 16, 256):
        h = offload.hadamard(size).double().numpy()
        np.testing.assert_allclose(h, numerics.hadamard(size), atol=1e-7)
        np.testing.assert_allclose(h @ h, np.eye(size), atol=1e-6)   # symmetric and orthogonal: its own inverse
    with pytest.raises(ValueError):
        offload.hadamard(8)


def test_dequantize_fp8_against_the_oracle():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((2, 256, 384)).astype(np.float32)
    bank = ref.quantize_fp8_block(w)     # scale grid [4, 3]: a transposed grid would not broadcast
    got = offload.dequantize_fp8(torch.from_numpy(bank["weight"]).view(torch.float8_e4m3fn),
                                 torch.from_numpy(bank["scale"]), torch.float32).double().numpy()
    want = ref.fp8_rows(bank["weight"], bank["scale"])
    np.testing.assert_allclose(got, want, rtol=2.0 ** -24, atol=0)


def test_gather_experts_picks_whole_experts():
    E, rows = 5, 4
    fields = {"_qdata": torch.arange(E * rows * 3).view(E * rows, 3), "scale": torch.arange(E * rows).float()}
    ids = torch.tensor([3, 0, 3])
    got = offload.gather_experts(fields, ids, E)
    for name, t in fields.items():
        want = torch.cat([t[e * rows:(e + 1) * rows] for e in ids.tolist()])
        assert torch.equal(got[name], want)
    dense = torch.randn(E * rows, 6)
    assert torch.equal(offload.gather_experts(dense, ids, E), torch.cat([dense[e * rows:(e + 1) * rows] for e in ids]))


def test_experts_decode_against_float64():
    rng = np.random.default_rng(1)
    k, H, I = 3, 64, 32
    x = rng.standard_normal((1, H))
    gu = rng.standard_normal((k * 2 * I, H)) * 0.1
    dn = rng.standard_normal((k * H, I)) * 0.1
    w = rng.dirichlet(np.ones(k))
    want = np.zeros(H)
    for e in range(k):
        y = gu[e * 2 * I:(e + 1) * 2 * I] @ x[0]
        want += w[e] * (dn[e * H:(e + 1) * H] @ (ref.silu(y[:I]) * y[I:]))
    t = {n: torch.from_numpy(v).float() for n, v in (("x", x), ("gu", gu), ("dn", dn), ("w", w))}
    got = offload.experts_decode(t["x"], t["gu"], t["dn"], t["w"])
    assert got.shape == (1, H)
    np.testing.assert_allclose(got[0].double().numpy(), want, rtol=1e-5, atol=1e-5)


def int8_layer(rng, E, H, I):
    gu = rng.standard_normal((E, 2 * I, H)).astype(np.float32) * 0.05
    dn = rng.standard_normal((E, H, I)).astype(np.float32) * 0.05
    return ref.quantize_int8_convrot(gu), ref.quantize_int8_convrot(dn)


def test_experts_on_cpu_against_the_oracle():
    """The int8 CPU path (torch's int8-weight matmul, bf16 activations) for runs of rows per expert."""
    rng = np.random.default_rng(2)
    E, H, I = 4, 256, 256
    gu, dn = int8_layer(rng, E, H, I)
    banks = tuple(offload.QuantHostBank.from_fields(E, "int8", {n: torch.from_numpy(v) for n, v in b.items()}, False)
                  for b in (gu, dn))
    experts, counts = [2, 0, 3], [2, 1, 3]
    x = numerics.bf16_round(rng.standard_normal((sum(counts), H)).astype(np.float32))
    x_rot = numerics.bf16_round(ref.rotate_ref(x.astype(np.float64)).astype(np.float32))
    got = offload.experts_on_cpu(banks, experts, counts, torch.from_numpy(x_rot).to(torch.bfloat16),
                                 offload.hadamard(256)).numpy()
    want = np.zeros_like(got, dtype=np.float64)
    row = 0
    for e, n in zip(experts, counts):
        wg, wd = ref.expert_rows("int8", gu, e, 2 * I, None), ref.expert_rows("int8", dn, e, H, None)
        for _ in range(n):
            y = wg @ x_rot[row]
            want[row] = wd @ ref.rotate_ref((ref.silu(y[:I]) * y[I:])[None])[0]
            row += 1
    assert np.linalg.norm(got - want) <= 2e-2 * np.linalg.norm(want)


def test_split_follows_the_cost_model():
    """The greedy split, worked by hand: PCIe 100 us per expert; the CPU 60 + 13 per row, scaled."""
    store = offload.ExpertStore(0, False)
    counts = {0: 10, 1: 3, 2: 1, 3: 1}
    bytes_100us = int(100 * offload.PCIE_BYTES_PER_US)
    # costs 190, 99, 73, 73: e0 to the GPU (190 > 100), e1 (99 <= 100 + 100), e2 (172 <= 200), e3 to the GPU (245 > 200)
    assert store.split([0, 1, 2, 3], counts, bytes_100us) == ([1, 2], 172.0, 200.0)
    store.cpu_scale = 2.0   # a slower CPU than modelled: e1 (198 <= 200) only; modelled times come back unscaled
    assert store.split([0, 1, 2, 3], counts, bytes_100us) == ([1], 99.0, 300.0)
    store.cpu_scale, store.gpu_scale = 1.0, 0.5   # a faster bus, 50 us an expert: e1 only (99 <= 50 + 50)
    on_cpu, cpu_us, gpu_us = store.split([0, 1, 2, 3], counts, bytes_100us)
    assert on_cpu == [1] and cpu_us == 99.0 and gpu_us == 300.0


# ------------------------------------------------------------------------------------------- the slot pool, host side
def small_banks(layers, E, rows=4, cols=8):
    out = []
    for layer in range(layers):
        banks = []
        for b in range(2):
            q = torch.arange(E * rows * cols, dtype=torch.int32).view(E * rows, cols) + 1000 * (2 * layer + b)
            banks.append(offload.HostBank(E, {"_qdata": q, "scale": torch.arange(E * rows).float() + layer}, False))
        out.append(tuple(banks))
    return out


def test_slot_pool_lookups():
    layers, E = 2, 6
    banks = small_banks(layers, E)
    pool = offload.SlotPool(banks, 0, "cpu")   # a budget of nothing still gives 8 slots
    assert pool.count == 8 and pool.free_slots() == list(range(8))
    # a pass over layer 0: nothing cached, the misses take the free slots in order, each filled from its expert
    placed = pool.slots(0, [4, 1], banks[0]).tolist()
    assert placed == [0, 1] and pool.reads.tolist() == [0, 2, 0]
    for slot, e in zip(placed, [4, 1]):
        for i, bank in enumerate(banks[0]):
            for name, t in pool.slot_fields(i, slot).items():
                assert torch.equal(t, bank.take(bank.fields, e, e + 1)[name])
    gathered = pool.gather(0, torch.tensor(placed))
    assert torch.equal(gathered["_qdata"], torch.cat([banks[0][0].take(banks[0][0].fields, e, e + 1)["_qdata"]
                                                      for e in (4, 1)]))
    assert pool.use(1, [0, 1, 2, 3, 4, 5]) == {}   # the same pass (only layer 0 starts one): nothing of layer 1 cached
    for e in range(6):
        pool.insert(1, e, [b.take(b.fields, e, e + 1) for b in banks[1]])
    # 8 slots: layer 0's two experts and layer 1's six; the pool is full and layer 1 used all of its own
    assert pool.free_slots() == [] and pool.room(1) == 2 and pool.room(0) == 6
    # a new pass: layer 0 uses expert 4 twice more; a claim for layer 0 must not evict expert 4 (used in this pass)
    for _ in range(2):
        assert pool.use(0, [4]) == {4: 0}
    slot = pool.claim(0, 2)
    assert slot != 0
    table, owner = pool.table.tolist(), pool.owner.tolist()
    assert table[0 * E + 2] == slot and owner[slot] == 2 and owner[0] == 4
    # every owner maps back to its slot; every cached key's slot names it
    for s, key in enumerate(owner):
        assert key < 0 or table[key] == s
    for key, s in enumerate(table):
        assert s < 0 or owner[s] == key


def test_slot_pool_evicts_the_least_used():
    layers, E = 1, 12
    banks = small_banks(layers, E)
    pool = offload.SlotPool(banks, 0, "cpu")
    # fill all 8 slots in pass 1, then use experts 0..6 again in pass 2 and 3: expert 7 is the least used
    pool.slots(0, list(range(8)), banks[0])
    for _ in range(2):
        pool.slots(0, list(range(7)), banks[0])
    pool.slots(0, [9], banks[0])   # pass 4: a miss evicts expert 7
    table = pool.table.tolist()
    assert table[7] == -1 and table[9] >= 0 and all(table[e] >= 0 for e in range(7))
    assert pool.reads.tolist() == [14, 9, 0]


def test_reservation_budget_changes_only_in_a_decode_phase():
    banks = small_banks(2, 6)
    pool = offload.SlotPool(banks, 0, "cpu")
    start = pool.reserve
    pool.promote()   # no decode phase: nothing to copy, the budget stays
    assert pool.reserve == start and pool.budget.tolist() == [start, max(1, -(-2 * start // 2))]
    pool.use(0, [1])
    assert pool.reserve == start


# ------------------------------------------------------------------------------------------- the store's host path
def store_on_cpu(kind, layers, E, H, I, seed, slots_bytes=0):
    rng = np.random.default_rng(seed)
    store, np_banks = offload.ExpertStore(0, False), []
    for _ in range(layers):
        gu = rng.standard_normal((E, 2 * I, H)).astype(np.float32) * 0.05
        dn = rng.standard_normal((E, H, I)).astype(np.float32) * 0.05
        if kind == "int8":
            b = (ref.quantize_int8_convrot(gu), ref.quantize_int8_convrot(dn))
        else:
            b = (ref.quantize_fp8_block(gu), ref.quantize_fp8_block(dn))
        np_banks.append(b)
        store.add_fields(kind, *({n: torch.from_numpy(v) for n, v in f.items()} for f in b), E)
    store.cache = offload.SlotPool(store.banks, slots_bytes, "cpu")
    store.codebooks = [(None, None)] * layers
    return store, np_banks


@pytest.mark.parametrize("kind", ["int8", "fp8"])
def test_store_host_path_against_the_oracle(kind):
    """sync_free off (the paths without kernels): decode rows through the host lookup and dense bf16 products,
    prompts through prefill_host, with 8 slots for 2 x 6 experts (hits, evictions and straight host reads)."""
    layers, E, H, I, k = 2, 6, 256, 256, 2
    store, np_banks = store_on_cpu(kind, layers, E, H, I, 3)
    rng = np.random.default_rng(4)
    for step in range(3):
        for layer in range(layers):
            x = numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
            ids = rng.choice(E, k, replace=False)
            w = numerics.bf16_round(rng.dirichlet(np.ones(k)).astype(np.float32))
            got = store.forward(layer, torch.from_numpy(x).view(torch.bfloat16), torch.from_numpy(ids)[None],
                                torch.from_numpy(w)[None].to(torch.bfloat16))
            assert got.shape == (1, H) and got.dtype == torch.bfloat16
            want = numerics.bf16_bits_to_f32(ref.resident_decode_ref(x, ids, w, np_banks[layer], (2 * I, H), kind,
                                                                     (None, None)))
            err = np.linalg.norm(got.float().numpy() - want)
            assert err <= 2e-2 * np.linalg.norm(want), (step, layer)
    T = 10
    for layer in range(layers):
        x = numerics.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
        idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
        w = numerics.bf16_round(rng.dirichlet(np.ones(k), T).astype(np.float32))
        got = store.forward(layer, torch.from_numpy(x).view(torch.bfloat16), torch.from_numpy(idx),
                            torch.from_numpy(w).to(torch.bfloat16))
        want = numerics.bf16_bits_to_f32(ref.resident_prefill_ref(x, idx, w, np_banks[layer], (2 * I, H), kind,
                                                                  (None, None)))
        assert got.shape == (T, H)
        assert np.linalg.norm(got.float().numpy() - want) <= 2e-2 * np.linalg.norm(want), layer
    table, owner = store.cache.table.tolist(), store.cache.owner.tolist()
    for s, key in enumerate(owner):
        assert key < 0 or table[key] == s


def test_store_rejects_mixed_layers():
    store, _ = store_on_cpu("int8", 1, 4, 256, 256, 5)
    with pytest.raises(ValueError, match="same format"):
        rng = np.random.default_rng(0)
        b = ref.quantize_fp8_block(rng.standard_normal((4, 512, 256)).astype(np.float32))
        fields = {n: torch.from_numpy(v) for n, v in b.items()}
        store.add_fields("fp8", fields, dict(fields), 4)
