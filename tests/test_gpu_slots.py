"""GPU parity of the slot cache's resolve and the bounded wait for the host (kernels.resolve / kernels.await_cpu ->
d3_resolve / d3_await_cpu) with the oracle (oracle/slots.py): plans and the whole cache state equal after every call
(decayed counts within float32 rounding), the wait's three outcomes exact."""
import numpy as np
import pytest
import torch

from drama3 import kernels
from oracle import slots

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def to_dev(st):
    return {n: torch.from_numpy(v.copy()).to(DEV) for n, v in st.items()}


def compare(dst, st):
    for n, v in st.items():
        got = dst[n].cpu().numpy()
        if n == "score":
            assert np.allclose(got, v, rtol=2e-6, atol=0), n
        else:
            assert np.array_equal(got, v), n


@pytest.mark.parametrize("cpu,share,slots_n", [(0, 0.0, 6), (1, 0.5, 6), (1, 0.3, 40), (0, 0.0, 1500)])
def test_resolve_trace_matches_oracle(cpu, share, slots_n):
    rng = np.random.default_rng(7 + cpu + slots_n)
    L, E, k = 4, 64, 8
    st = slots.new_state(L, E, slots_n, budget=(3, 2))
    dst = to_dev(st)
    share_t = torch.tensor([share], dtype=torch.float32, device=DEV)
    for step in range(6):
        st["budget"][0] = 3
        dst["budget"][0] = 3
        for layer in range(L):
            ids = rng.choice(E, k, replace=False)
            want = slots.resolve_ref(ids, layer, L, E, 3.0, cpu, 2.5, st, share)
            got = kernels.resolve(torch.from_numpy(ids).to(DEV), layer, L, E, 3.0, cpu, 2.5, dst["table"],
                                  dst["owner"], dst["score"], dst["at"], dst["pending"], dst["clock"], dst["budget"],
                                  dst["reads"], dst["step"], share_t)
            assert np.array_equal(got.cpu().numpy(), want), (step, layer)
            compare(dst, st)
        # the host's copies land between steps
        for s in np.nonzero(st["pending"])[0]:
            st["pending"][s] = 0
            st["table"][st["owner"][s]] = s
        dst = to_dev(st)


def test_await_cpu_outcomes():
    H = 2048
    res_np = (np.arange(H, dtype=np.uint32) % 1000 + 0x3C00).astype(np.uint16)
    result = torch.from_numpy(res_np).pin_memory()
    flag = torch.zeros(1, dtype=torch.int32).pin_memory()
    step = torch.tensor([5], dtype=torch.int32, device=DEV)
    took = torch.zeros(1, dtype=torch.int32, device=DEV)
    plan_cpu = torch.tensor([[0, 0], [-1, 2], [3, 1]], dtype=torch.int32, device=DEV)
    plan_gpu = torch.tensor([[0, 0], [3, 1]], dtype=torch.int32, device=DEV)
    # the host is on time: its flag already holds the step
    flag[0] = 5
    out = kernels.await_cpu(plan_cpu, flag, step, result, 100000, took)
    want, want_took = slots.await_ref(plan_cpu.cpu().numpy(), 5, 5, res_np)
    assert np.array_equal(out.cpu().numpy(), want) and took.item() == want_took == 0
    # the host is late: the wait ends after its bound (200 us) with zeros and took_over
    flag[0] = 4
    out = kernels.await_cpu(plan_cpu, flag, step, result, 200, took)
    want, want_took = slots.await_ref(plan_cpu.cpu().numpy(), 4, 5, res_np)
    assert np.array_equal(out.cpu().numpy(), want) and took.item() == want_took == 1
    # no CPU experts: nothing awaited
    out = kernels.await_cpu(plan_gpu, flag, step, result, 200, took)
    assert torch.all(out == 0) and took.item() == 0
