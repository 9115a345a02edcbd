"""The host-offload option end to end (offload.HostExperts: banks in pinned host memory, a SlotPool in HBM,
kernels.resolve, the GEMVs' fill-while-reading, the CPU side's handshake through kernels.await_cpu) against the
HBM-resident decode of the same banks.

Without the CPU side every expert's bytes are the same whether read from a slot or from host memory, so the outputs
must be bit-identical to the resident decode through the same kernels (resident_decode_unfused); the two-launch
resident decode agrees within float tolerance (torch's silu for FP8 where the fused kernel uses expf). With it, the CPU's experts run in bf16 on the host (as the reference's
do), so the bar is the float tolerance of the reference's own CPU path: rel-L2 2e-2."""
import numpy as np
import pytest
import torch

from drama3 import offload
from oracle import numerics
from oracle import reference as ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
H, I, E, K = 2048, 768, 16, 8


def make_layers(kind, layers, seed):
    rng = np.random.default_rng(seed)
    out, cbs = [], []
    for _ in range(layers):
        gu = rng.standard_normal((E, 2 * I, H)).astype(np.float32) * 0.02
        dn = rng.standard_normal((E, H, I)).astype(np.float32) * 0.02
        if kind == "int8":
            banks, cb = (ref.quantize_int8_convrot(gu), ref.quantize_int8_convrot(dn)), (None, None)
        elif kind == "fp8":
            banks, cb = (ref.quantize_fp8_block(gu), ref.quantize_fp8_block(dn)), (None, None)
        else:
            (a, ca), (b, cb2) = ref.quantize_codes(gu, int(kind[1])), ref.quantize_codes(dn, int(kind[1]))
            banks, cb = (a, b), (ca, cb2)
        out.append(tuple({n: torch.from_numpy(v) for n, v in b.items()} for b in banks))
        cbs.append(tuple(None if c is None else torch.from_numpy(c) for c in cb))
    return out, cbs


@pytest.mark.parametrize("kind", ["int8", "w4", "fp8"])
def test_slot_path_equals_resident_decode(kind):
    layers, steps = 3, 4
    host_layers, cbs = make_layers(kind, layers, 1)
    he = offload.HostExperts(kind, host_layers, E, 40, DEV, codebooks=cbs)  # 40 of 48 experts: hits and evictions
    resident = [tuple({n: t.to(DEV) for n, t in b.items()} for b in banks) for banks in host_layers]
    rcbs = [tuple(None if c is None else c.to(DEV) for c in cb) for cb in cbs]
    rng = np.random.default_rng(2)
    for step in range(steps):
        for layer in range(layers):
            x = torch.from_numpy(numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32)))
            x = x.view(torch.bfloat16).to(DEV)
            ids = torch.from_numpy(rng.choice(E, K, replace=False)).to(DEV)
            w = torch.from_numpy(rng.dirichlet(np.ones(K)).astype(np.float32)).to(DEV).to(torch.bfloat16)
            got = he.decode(layer, x, ids, w)
            want = offload.resident_decode_unfused(x, ids, w, resident[layer], (2 * I, H), kind, rcbs[layer])
            assert torch.equal(got, want), (step, layer)
            fused = offload.resident_decode(x, ids, w, resident[layer], (2 * I, H), kind, rcbs[layer])
            assert torch.linalg.norm(fused.float() - want.float()) <= 1e-2 * torch.linalg.norm(want.float())
    torch.cuda.synchronize()
    hits, fills, cpu = he.cache.reads.tolist()
    assert cpu == 0 and hits + fills == steps * layers * K and fills > 0 and hits > 0
    # table and owner agree
    table, owner = he.cache.table.cpu().numpy(), he.cache.owner.cpu().numpy()
    for s, key in enumerate(owner):
        if key >= 0:
            assert table[key] == s


def test_cpu_side_handshake():
    """int8 with the CPU side: the missed experts the GPU leaves to the CPU come back through the host flag (or, if
    the host is late, the GPU runs them itself); the output matches the resident decode within the CPU path's float
    tolerance, and the slots the CPU's experts reserved are copied in between steps."""
    layers, steps = 2, 4
    host_layers, cbs = make_layers("int8", layers, 3)
    he = offload.HostExperts("int8", host_layers, E, 8, DEV, cpu_side=True)
    resident = [tuple({n: t.to(DEV) for n, t in b.items()} for b in banks) for banks in host_layers]
    rng = np.random.default_rng(4)
    cpu_seen = 0
    for step in range(steps):
        for layer in range(layers):
            x = torch.from_numpy(numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32)))
            x = x.view(torch.bfloat16).to(DEV)
            ids = torch.from_numpy(rng.choice(E, K, replace=False)).to(DEV)
            w = torch.from_numpy(rng.dirichlet(np.ones(K)).astype(np.float32)).to(DEV).to(torch.bfloat16)
            got = he.decode(layer, x, ids, w)
            he.after_layer(layer)
            torch.cuda.synchronize()
            want = offload.resident_decode(x, ids, w, resident[layer], (2 * I, H), "int8", (None, None)).float()
            assert torch.linalg.norm(got.float() - want) <= 2e-2 * torch.linalg.norm(want), (step, layer)
        he.between_steps()
        cpu_seen = int(he.cache.reads[2])
    assert cpu_seen > 0
    he.cache.settle()
    torch.cuda.synchronize()
    table, owner, pending = (t.cpu().numpy() for t in (he.cache.table, he.cache.owner, he.cache.pending))
    assert not pending.any()
    for s, key in enumerate(owner):
        if key >= 0:
            assert table[key] == s
