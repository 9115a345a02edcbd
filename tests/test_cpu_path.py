"""The CPU baseline path (oracle/cpu_path.py, the reference's dequant-then-matmul restated) against a float64
computation of the same dequantized experts, and its many-rows form against its one-row form. CPU only."""
import numpy as np
import pytest
import torch

from drama3 import formats
from oracle import a8, cpu_path
from oracle.numerics import bf16_bits_to_f32

H, I, E, K = 256, 128, 6, 3


def banks(fmt, seed):
    gen = torch.Generator().manual_seed(seed)
    gu = formats.quantize(torch.randn((E, 2 * I, H), generator=gen) * 0.05, fmt)
    dn = formats.quantize(torch.randn((E, H, I), generator=gen) * 0.05, fmt)
    return (gu.weight, gu.scale), (dn.weight, dn.scale)


def deq(bank, fmt, rows, cols, e):
    w, s = bank
    packed = w[e * rows:(e + 1) * rows].numpy()
    sb = s[e * rows:(e + 1) * rows].contiguous().view(torch.int16).numpy().view(np.uint16)
    return a8.dequantize(packed, sb, fmt)


@pytest.mark.parametrize("fmt", [0, 1, 2, 3])
def test_layer_matches_float64_of_the_same_experts(fmt):
    gate_up, down = banks(fmt, fmt)
    gen = torch.Generator().manual_seed(10 + fmt)
    x = torch.randn((1, H), generator=gen).to(torch.bfloat16)
    ids = torch.tensor([4, 1, 5])
    w = torch.tensor([0.5, 0.3, 0.2]).to(torch.bfloat16)
    got = cpu_path.layer(x, ids, w, gate_up, down, fmt, H, I).numpy()
    xf = bf16_bits_to_f32(x.view(torch.int16).numpy().view(np.uint16))[0].astype(np.float64)
    want = np.zeros(H)
    for e, we in zip(ids.tolist(), w.float().tolist()):
        y = deq(gate_up, fmt, 2 * I, H, e) @ xf
        h = y[:I] / (1 + np.exp(-y[:I])) * y[I:]
        want += we * (deq(down, fmt, H, I, e) @ h)
    # bf16 weights, activations and hidden: a few bf16 steps
    assert np.linalg.norm(got - want) <= 2e-2 * np.linalg.norm(want)


@pytest.mark.parametrize("fmt", [0, 3])
def test_grouped_layer_equals_row_by_row(fmt):
    gate_up, down = banks(fmt, 20 + fmt)
    gen = torch.Generator().manual_seed(30)
    x = torch.randn((5, H), generator=gen).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=gen)[:K] for _ in range(5)])
    w = torch.rand((5, K), generator=gen).to(torch.bfloat16)
    got = cpu_path.grouped_layer(x, ids, w, gate_up, down, fmt, H, I)
    for t in range(5):
        one = cpu_path.layer(x[t:t + 1], ids[t], w[t], gate_up, down, fmt, H, I)
        assert torch.allclose(got[t], one, rtol=1e-5, atol=1e-6)
