"""Pins the oracle's numerics (oracle/numerics.py) against torch's casts and closed forms."""
import numpy as np
import pytest
import torch

from oracle import numerics


def test_bf16_rounding_matches_torch_cast():
    rng = np.random.default_rng(0)
    # float32 inputs (the scale is float64; what overflows float32 becomes inf and is dropped below)
    with np.errstate(over="ignore"):
        v = (rng.standard_normal(200_000) * 10.0 ** rng.integers(-30, 30, 200_000)).astype(np.float32)
    # exact ties: the lower 16 bits 0x8000, both parities of the kept bit
    ties = (rng.integers(0, 2**16, 4096, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    ties = ties[np.isfinite(ties)]
    v = np.concatenate([v, ties, np.float32([0.0, -0.0, 1.0, -1.0, 3.4e38, -3.4e38, 1e-40])])
    assert v.dtype == np.float32
    v = v[np.isfinite(v)]
    ours = numerics.f32_to_bf16_bits(v)
    theirs = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    back = numerics.bf16_bits_to_f32(ours)
    assert np.array_equal(back, torch.from_numpy(v).to(torch.bfloat16).float().numpy())


def test_e4m3_decode_matches_torch_for_every_code():
    codes = np.arange(256, dtype=np.uint8)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    ours = numerics.e4m3_decode(codes)
    finite = np.isfinite(theirs)
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    assert np.array_equal(ours[finite], theirs[finite])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6


def test_e4m3_encode_matches_torch_cast_in_range():
    rng = np.random.default_rng(1)
    v = (rng.standard_normal(300_000) * np.exp(rng.uniform(-14, 6, 300_000))).astype(np.float32)
    v = np.clip(v, -463.9, 463.9)
    # every representable value and every midpoint between neighbours (ties to even)
    table = numerics.E4M3[:127].astype(np.float64)
    mids = ((table[1:] + table[:-1]) / 2).astype(np.float32)
    v = np.concatenate([v, numerics.E4M3[:127], -numerics.E4M3[:127], mids, -mids])
    ours = numerics.e4m3_encode(v)
    theirs = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    zero = (ours & 0x7F) == 0
    # torch keeps the sign of a value that rounds to zero as the encoder does
    assert np.array_equal(ours[~zero], theirs[~zero])
    assert np.array_equal(ours[zero] & 0x7F, theirs[zero] & 0x7F)


def test_e4m3_encode_saturates():
    assert numerics.e4m3_encode(np.float32([464.0, 1e6, -500.0])).tolist() == [0x7E, 0x7E, 0xFE]


def test_hadamard_closed_form():
    h = numerics.hadamard(256)
    assert np.allclose(h, h.T)
    assert np.allclose(h @ h, np.eye(256), atol=1e-12)
    assert np.all(np.abs(np.abs(h) - 1 / 16) < 1e-15)
    # the first row of kron^4(h4) is the kron of h4's first rows
    r = np.array([1, 1, 1, -1.0])
    expect = np.kron(np.kron(np.kron(r, r), r), r) / 16
    assert np.allclose(h[0], expect)


def butterfly_rotate(row):
    """rotate_rows' in-place network (drama3/kernels.py:245-257): strides 1, 4, 16, 64 of the 4-point butterfly
    (a+b+c-d, a+b-c+d, a-b+c+d, -a+b+c+d) on each 256-column group, then / 16."""
    row = np.array(row, dtype=np.float64)
    K = row.shape[0]
    stride = 1
    while stride < 256:
        for t in range(K // 4):
            within, low = t & 63, (t & 63) % stride
            high = within // stride
            i = (t >> 6) * 256 + high * stride * 4 + low
            a, b, c, d = row[i], row[i + stride], row[i + 2 * stride], row[i + 3 * stride]
            row[i], row[i + stride], row[i + 2 * stride], row[i + 3 * stride] = a + b + c - d, a + b - c + d, a - b + c + d, -a + b + c + d
        stride *= 4
    return row / 16


def test_butterfly_network_equals_dense_hadamard():
    """Two statements of ConvRot in the reference agree: the kernel's butterflies and offload.hadamard's kron."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal(768)
    dense = (x.reshape(3, 256) @ numerics.hadamard(256)).reshape(-1)
    assert np.allclose(butterfly_rotate(x), dense, atol=1e-12)
