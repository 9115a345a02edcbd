"""offload.ExpertStore end to end on the GPU, through the reference's own entry points (add / session / forward /
after_layer / between_steps, OffloadedExperts), and a converted file loaded by drama3/loader.py.

- Resident session (every bank fits): forward's decode and prefill against the oracle's resident_decode_ref /
  resident_prefill_ref, within one bf16 step plus 1e-5 of the row's largest value.
- Slot session (a cache smaller than the banks; banks in pinned host memory, kernels.resolve, the GEMVs' fill while
  reading): every expert's bytes are the same whether read from a slot or from host memory, so decode rows are
  bit-identical to resident_decode_unfused over the same banks, and prompts to resident_prefill.
- With the CPU side (int8, a small cache) the CPU's experts run in bf16 on the host as the reference's do, so the bar
  is that path's float tolerance: rel-L2 2e-2 against the resident decode / prefill.
- A file written in the converted layout and loaded onto the device (loader.load_experts -> ExpertTable.place)
  decodes and prefills as the oracle does from the same banks, and as a store holding the same file."""
import numpy as np
import pytest
import torch

from drama3 import loader, offload
from oracle import numerics
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
H, I, E, K = 2048, 768, 16, 8


def make_layers(kind, layers, seed):
    """Per layer: ((gate_up fields, down fields) as numpy, (codebooks)) in the reference's layouts."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(layers):
        gu = rng.standard_normal((E, 2 * I, H)).astype(np.float32) * 0.02
        dn = rng.standard_normal((E, H, I)).astype(np.float32) * 0.02
        if kind == "int8":
            out.append(((ref.quantize_int8_convrot(gu), ref.quantize_int8_convrot(dn)), (None, None)))
        elif kind == "fp8":
            out.append(((ref.quantize_fp8_block(gu), ref.quantize_fp8_block(dn)), (None, None)))
        else:
            (a, ca), (b, cb) = ref.quantize_codes(gu, int(kind[1])), ref.quantize_codes(dn, int(kind[1]))
            out.append(((a, b), (ca, cb)))
    return out


def tensors(fields):
    return {n: torch.from_numpy(np.ascontiguousarray(v)) for n, v in fields.items()}


def cb_tensor(c, device="cpu"):
    return None if c is None else torch.from_numpy(c).to(device)


def make_store(kind, layers, cache_experts, pin=True):
    store = offload.ExpertStore(0, pin)
    for banks, cbs in layers:
        store.add_fields(kind, tensors(banks[0]), tensors(banks[1]), E, tuple(cb_tensor(c) for c in cbs))
    expert_bytes = store.bank_bytes // (len(layers) * E)
    store.cache_bytes = cache_experts * expert_bytes
    return store


def on_device(layers):
    return ([tuple({n: t.to(DEV) for n, t in tensors(b).items()} for b in banks) for banks, _ in layers],
            [tuple(cb_tensor(c, DEV) for c in cbs) for _, cbs in layers])


def bf16(a):
    return torch.from_numpy(numerics.f32_to_bf16_bits(np.asarray(a, np.float32))).view(torch.bfloat16).to(DEV)


def bits(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def assert_bf16_close(got_bits, expect_bits):
    a = numerics.bf16_bits_to_f32(np.asarray(got_bits)).astype(np.float64)
    b = numerics.bf16_bits_to_f32(np.asarray(expect_bits)).astype(np.float64)
    assert np.all(np.isfinite(a))
    bound = 2.0 ** -7 * np.abs(b) + 1e-5 * np.abs(b).max()
    assert np.all(np.abs(a - b) <= bound), np.abs(a - b).max()


def decode_row(rng):
    x = numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    ids = rng.choice(E, K, replace=False)
    w = numerics.bf16_round(rng.dirichlet(np.ones(K)).astype(np.float32))
    return x, ids, w


def prompt(rng, T, k):
    x = numerics.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    w = numerics.bf16_round(rng.dirichlet(np.ones(k), T).astype(np.float32))
    return x, idx, w


def dev_bf16_bits(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV).view(torch.bfloat16)


# --------------------------------------------------------------------------------------------- resident session
@pytest.mark.parametrize("kind", ["int8", "fp8", "w4", "w6"])
def test_resident_session_against_the_oracle(kind):
    layers = make_layers(kind, 2, 11)
    store = make_store(kind, layers, 0)
    store.cache_bytes = 0            # as much as is free: every bank fits
    modules = [offload.OffloadedExperts(store, layer) for layer in range(len(layers))]
    rng = np.random.default_rng(12)
    with store.session(DEV, [], False, 64):
        assert store.resident is not None and store.sync_free and modules[0].sync_free(DEV)
        for layer, ((banks, cbs), mod) in enumerate(zip(layers, modules)):
            x, ids, w = decode_row(rng)
            got = mod(dev_bf16_bits(x), torch.from_numpy(ids)[None].to(DEV), bf16(w)[None])
            assert got.shape == (1, H) and got.dtype == torch.bfloat16
            assert_bf16_close(bits(got), ref.resident_decode_ref(x, ids, w, banks, (2 * I, H), kind, cbs))
            x, idx, w = prompt(rng, 12, 4)
            got = mod(dev_bf16_bits(x), torch.from_numpy(idx).to(DEV), bf16(w))
            assert got.shape == (12, H) and got.dtype == torch.bfloat16
            assert_bf16_close(bits(got), ref.resident_prefill_ref(x, idx, w, banks, (2 * I, H), kind, cbs))
    assert store.cache is None and store.resident is None and not store.sync_free and not modules[0].sync_free(DEV)


# ------------------------------------------------------------------------------------------------- slot session
@pytest.mark.parametrize("kind", ["int8", "w4", "fp8"])
def test_slot_decode_equals_resident_decode(kind):
    layers, steps = make_layers(kind, 3, 1), 4
    store = make_store(kind, layers, 40)   # 40 slots for 48 experts: hits and evictions
    resident, rcbs = on_device(layers)
    rng = np.random.default_rng(2)
    with store.session(DEV, [], False, 0):
        assert store.resident is None and store.sync_free and store.cache.count == 40 and store.cpu_side is None
        for step in range(steps):
            for layer in range(len(layers)):
                x, ids, w = decode_row(rng)
                xd, idd, wd = dev_bf16_bits(x), torch.from_numpy(ids).to(DEV), bf16(w)
                got = store.forward(layer, xd, idd[None], wd[None])
                want = offload.resident_decode_unfused(xd, idd, wd, resident[layer], (2 * I, H), kind, rcbs[layer])
                assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (step, layer)
        torch.cuda.synchronize()
        hits, fills, cpu = store.cache.reads.tolist()
        assert cpu == 0 and hits + fills == steps * len(layers) * K and fills > 0 and hits > 0
        table, owner = store.cache.table.cpu().numpy(), store.cache.owner.cpu().numpy()
        for s, key in enumerate(owner):
            assert key < 0 or table[key] == s


@pytest.mark.parametrize("kind", ["int8", "w4", "fp8"])
def test_slot_prefill_equals_resident_prefill(kind):
    """A prompt's pass through the slot cache (cached experts from their slots, the most used misses filling free
    slots, the rest read from host memory) gives the resident prefill's bits, pass after pass."""
    layers = make_layers(kind, 2, 5)
    store = make_store(kind, layers, 12)
    resident, rcbs = on_device(layers)
    rng = np.random.default_rng(6)
    with store.session(DEV, [], False, 0, cpu_experts=False):
        for rep in range(2):
            for layer in range(len(layers)):
                x, idx, w = prompt(rng, 24, 4)
                xd, idxd, wd = dev_bf16_bits(x), torch.from_numpy(idx).to(DEV), bf16(w)
                got = store.forward(layer, xd, idxd, wd)
                want = offload.resident_prefill(xd, idxd, wd, resident[layer], (2 * I, H), kind, rcbs[layer], E)
                assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (rep, layer)
        owner = store.cache.owner.cpu().numpy()
        assert (owner >= 0).sum() > 0   # the passes filled slots


@pytest.mark.parametrize("kind", ["int8", "fp8", "w4", "w6"])
def test_slot_prefill_hot_experts_fill_once(kind):
    """Experts with many rows (100 and 70 rows: four and three 32-row passes of the grouped products) that are not
    cached: the first pass of each reads it from host memory and copies it into its slot, the later passes read the
    slot once the first passes are done (fills_first). The output equals the resident prefill's bits, the filled slots
    hold the experts' bytes, and the next pass finds them cached."""
    layers = make_layers(kind, 2, 9)
    store = make_store(kind, layers, 12)
    resident, rcbs = on_device(layers)
    rng = np.random.default_rng(10)
    T, k, hot = 100, 4, (5, 11)
    with store.session(DEV, [], False, 0, cpu_experts=False):
        for rep in range(2):
            x, idx, w = prompt(rng, T, k)
            others = [e for e in range(E) if e not in hot]
            for t in range(T):   # expert 5 in every row, expert 11 in 70 of them
                fixed = [hot[0]] + ([hot[1]] if t < 70 else [])
                idx[t] = fixed + list(rng.choice(others, k - len(fixed), replace=False))
            xd, idxd, wd = dev_bf16_bits(x), torch.from_numpy(idx).to(DEV), bf16(w)
            got = store.forward(0, xd, idxd, wd)
            want = offload.resident_prefill(xd, idxd, wd, resident[0], (2 * I, H), kind, rcbs[0], E)
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), rep
            table = store.cache.table.cpu().numpy()
            for e in hot:
                s = int(table[e])
                assert s >= 0, (rep, e)   # layer 0's key of expert e: its slot
                for i, bank in enumerate(store.banks[0]):
                    want_fields = bank.take(bank.fields, e, e + 1)
                    for name, t in store.cache.slot_fields(i, s).items():
                        assert torch.equal(t.cpu(), want_fields[name]), (rep, e, name)


@pytest.mark.parametrize("kind", ["int8", "w4"])
def test_slot_prefill_captured_in_a_graph(kind):
    """Without the CPU side a prompt's pass through the slot cache waits on nothing on the host (the pass's plan, fills
    and groups are made on the device), so it can be captured in a HIP graph: both layers' passes captured once and
    replayed five times with new rows and routing copied in between, each output equal to the resident prefill's bits
    while the cache fills across replays."""
    layers = make_layers(kind, 2, 15)
    store = make_store(kind, layers, 10)
    resident, rcbs = on_device(layers)
    rng = np.random.default_rng(16)
    T, k = 20, 4
    with store.session(DEV, [], False, 0, cpu_experts=False):
        x, idx, w = prompt(rng, T, k)
        xs, idxs, ws = dev_bf16_bits(x), torch.from_numpy(idx).to(DEV), bf16(w)
        stream = torch.cuda.Stream(DEV)
        stream.wait_stream(torch.cuda.current_stream(DEV))
        with torch.cuda.stream(stream):
            for layer in range(2):   # eager first: kernels' constants, allocator pools
                store.forward(layer, xs, idxs, ws)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                outs = [store.forward(layer, xs, idxs, ws) for layer in range(2)]
        torch.cuda.synchronize()
        for rep in range(5):
            x, idx, w = prompt(rng, T, k)
            xs.copy_(dev_bf16_bits(x))
            idxs.copy_(torch.from_numpy(idx).to(DEV))
            ws.copy_(bf16(w))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for layer in range(2):
                want = offload.resident_prefill(xs, idxs, ws, resident[layer], (2 * I, H), kind, rcbs[layer], E)
                assert torch.equal(outs[layer].view(torch.int16), want.view(torch.int16)), (rep, layer)
        torch.cuda.synchronize()
        table, owner = store.cache.table.cpu().numpy(), store.cache.owner.cpu().numpy()
        assert (owner >= 0).sum() > 0 and int(store.cache.clock) == 6   # one eager pass, five replayed
        for s, key in enumerate(owner):
            assert key < 0 or table[key] == s


def test_cpu_side_decode():
    """int8 with the CPU side: the missed experts the GPU leaves to the CPU come back through the host mailbox (or, if
    the host is late, the GPU runs them itself); the slots the CPU's experts reserved are copied in between steps."""
    layers, steps = make_layers("int8", 2, 3), 4
    store = make_store("int8", layers, 8)
    resident, _ = on_device(layers)
    rng = np.random.default_rng(4)
    with store.session(DEV, [], True, 0, cpu_experts=True):
        assert store.cpu_experts and store.cpu_side is not None
        for step in range(steps):
            for layer in range(len(layers)):
                x, ids, w = decode_row(rng)
                xd, idd, wd = dev_bf16_bits(x), torch.from_numpy(ids).to(DEV), bf16(w)
                got = store.forward(layer, xd, idd[None], wd[None])
                store.after_layer(layer)
                torch.cuda.synchronize()
                want = offload.resident_decode(xd, idd, wd, resident[layer], (2 * I, H), "int8", (None, None)).float()
                assert torch.linalg.norm(got.float() - want) <= 2e-2 * torch.linalg.norm(want), (step, layer)
            store.between_steps()
        assert int(store.cache.reads[2]) > 0
        store.cache.settle()
        torch.cuda.synchronize()
        table, owner, pending = (t.cpu().numpy() for t in (store.cache.table, store.cache.owner, store.cache.pending))
        assert not pending.any()
        for s, key in enumerate(owner):
            assert key < 0 or table[key] == s


def test_cpu_split_prefill():
    """int8 prompt with the CPU split: experts with few rows run on the CPU beside the grouped kernels; the result
    is the resident prefill's within the CPU path's tolerance, and the split's measured scale moved."""
    layers = make_layers("int8", 2, 7)
    store = make_store("int8", layers, 8)
    resident, _ = on_device(layers)
    rng = np.random.default_rng(8)
    with store.session(DEV, [], False, 0, cpu_experts=True):
        assert store.cpu_experts
        for layer in range(len(layers)):
            x, idx, w = prompt(rng, 16, 4)
            xd, idxd, wd = dev_bf16_bits(x), torch.from_numpy(idx).to(DEV), bf16(w)
            got = store.forward(layer, xd, idxd, wd).float()
            want = offload.resident_prefill(xd, idxd, wd, resident[layer], (2 * I, H), "int8", (None, None), E).float()
            assert torch.linalg.norm(got - want) <= 2e-2 * torch.linalg.norm(want), layer
    assert store.cpu_scale != 1.0


# ------------------------------------------------------------------------------------------------ a loaded file
@pytest.mark.parametrize("kind", ["int8", "fp8", "w4", "w6"])
def test_loaded_file(tmp_path, kind):
    layers = make_layers(kind, 2, 21)
    path = tmp_path / f"{kind}.safetensors"
    loader.write_experts(path, kind, {l: (tuple(tensors(b) for b in banks), tuple(cb_tensor(c) for c in cbs))
                                      for l, (banks, cbs) in enumerate(layers)}, {"num_experts": E})
    table = offload.ExpertTable(DEV)
    for layer, (k, banks, cbs) in loader.load_experts(path, device="cuda:0").items():
        assert k == kind and all(t.device == DEV for b in banks for t in b.values())
        table.place(layer, k, banks[0], banks[1], cbs)
    assert table.bytes == sum(v.nbytes for banks, _ in layers for b in banks for v in b.values())
    store = offload.ExpertStore(0, True)
    for layer, (k, banks, cbs) in loader.load_experts(path).items():
        store.add_fields(k, banks[0], banks[1], E, cbs)
    rng = np.random.default_rng(22)
    with store.session(DEV, [], False, 16):
        assert store.resident is not None
        for layer, (banks, cbs) in enumerate(layers):
            x, ids, w = decode_row(rng)
            xd, idd, wd = dev_bf16_bits(x), torch.from_numpy(ids).to(DEV), bf16(w)
            got = table.decode(layer, xd, idd, wd, E)
            assert_bf16_close(bits(got), ref.resident_decode_ref(x, ids, w, banks, (2 * I, H), kind, cbs))
            assert torch.equal(store.forward(layer, xd, idd[None], wd[None]).view(torch.int16), got.view(torch.int16))
            x, idx, w = prompt(rng, 10, 4)
            xd, idxd, wd = dev_bf16_bits(x), torch.from_numpy(idx).to(DEV), bf16(w)
            got = table.prefill(layer, xd, idxd, wd, E)
            assert_bf16_close(bits(got), ref.resident_prefill_ref(x, idx, w, banks, (2 * I, H), kind, cbs))
            assert torch.equal(store.forward(layer, xd, idxd, wd).view(torch.int16), got.view(torch.int16))
