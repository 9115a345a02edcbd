"""Pins the A8 oracle (oracle/a8.py): packing round trips, its quantizers against the product's independent torch
quantizers (drama3/formats.py), exact dot products against brute force, routing against brute force and the
reference's torch fallback (drama3/model.py:120-121), and the layer against an unquantized float64 layer."""
import numpy as np
import pytest
import torch

from drama3 import formats
from oracle import a8, numerics
from oracle.numerics import bf16_bits_to_f32, e4m3_decode, f32_to_bf16_bits

FMTS = [a8.FMT_I8, a8.FMT_W4, a8.FMT_W6, a8.FMT_F8]


@pytest.mark.parametrize("fmt,lo,hi", [(a8.FMT_W4, -8, 7), (a8.FMT_W6, -32, 31)])
def test_pack_round_trip(fmt, lo, hi):
    rng = np.random.default_rng(3)
    q = rng.integers(lo, hi + 1, size=(7, 512))
    packed = a8.pack_w4(q) if fmt == a8.FMT_W4 else a8.pack_w6(q)
    assert packed.shape == (7, a8.row_bytes(fmt, 512))
    assert np.array_equal(a8.codes(packed, fmt), q)
    # every byte pattern is a valid packing: bytes -> codes -> bytes is the identity
    raw = rng.integers(0, 256, size=(5, a8.row_bytes(fmt, 256)), dtype=np.uint8)
    back = a8.pack_w4(a8.codes(raw, fmt)) if fmt == a8.FMT_W4 else a8.pack_w6(a8.codes(raw, fmt))
    assert np.array_equal(back, raw)


def test_w4_nibble_order():
    # byte b: column 2b in the low nibble, 2b + 1 in the high one; two's complement
    packed = np.array([[0x71, 0x8F]], dtype=np.uint8)
    assert a8.unpack_w4(packed).tolist() == [[1, 7, -1, -8]]


def test_w6_unit_layout():
    # q_12 = -1 (all six bits set) spreads over the top bits of bytes 0, 4 and 8; q_0 = 5 sits in byte 0's low bits
    q = np.zeros((1, 16), dtype=np.int64)
    q[0, 0], q[0, 12] = 5, -1
    b = a8.pack_w6(q)[0]
    assert b[0] == (5 | 0xC0) and b[4] == 0xC0 and b[8] == 0xC0
    assert all(b[i] == 0 for i in range(12) if i not in (0, 4, 8))


def test_w6_le3_layout_and_conversion():
    """The "4 per 3 bytes, little-endian, low bits first" W6 layout: values 1, -1, 5, -32 are the 24-bit word
    1 | 63 << 6 | 5 << 12 | 32 << 18; converting it to the A8 W6 layout and back keeps every code, for every byte
    pattern of the A8 layout."""
    q = torch.tensor([[1, -1, 5, -32]])
    word = 1 | 63 << 6 | 5 << 12 | 32 << 18
    assert formats.pack_w6_le3(q).tolist() == [[word & 0xFF, (word >> 8) & 0xFF, word >> 16]]
    rng = np.random.default_rng(6)
    codes = torch.from_numpy(rng.integers(-32, 32, size=(5, 256)))
    le3 = formats.pack_w6_le3(codes)
    assert torch.equal(formats.unpack_w6_le3(le3).long(), codes)
    a8_rows = formats.w6_from_le3(le3)
    assert np.array_equal(a8.codes(a8_rows.numpy(), a8.FMT_W6), codes.numpy())
    raw = torch.from_numpy(rng.integers(0, 256, size=(4, 192), dtype=np.uint8))
    assert torch.equal(formats.w6_from_le3(formats.w6_to_le3(raw)), raw)


@pytest.mark.parametrize("fmt", FMTS)
def test_oracle_quantizer_matches_product_quantizer(fmt):
    """Two independent implementations of each format (numpy here, torch in drama3/formats.py) agree bit for bit."""
    torch.manual_seed(4)
    w = torch.randn(3, 48, 256) * 0.02
    w[0, 0] = 0.0  # an all-zero row
    bank = formats.quantize(w, fmt)
    packed, sbits = a8.quantize_weights(w.reshape(-1, 256).numpy(), fmt)
    assert np.array_equal(bank.weight.numpy(), packed)
    assert np.array_equal(bank.scale.view(torch.int16).numpy().view(np.uint16), sbits)
    assert np.array_equal(formats.codes(bank).numpy(), a8.codes(packed, fmt).view(np.int8))


@pytest.mark.parametrize("fmt", FMTS)
def test_quantization_error_is_bounded(fmt):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    packed, sbits = a8.quantize_weights(w, fmt)
    back = a8.dequantize(packed, sbits, fmt)
    s = bf16_bits_to_f32(sbits).astype(np.float64)
    if fmt == a8.FMT_F8:
        # e4m3 keeps 3 mantissa bits: relative error <= 2^-4 for normals, absolute <= 2^-10 s in the subnormal range
        err = np.abs(back - w)
        assert np.all(err <= np.maximum(np.abs(w) * 2.0 ** -4, s[:, None] * 2.0 ** -10) * 1.0001)
    else:
        step = s[:, None] if fmt == a8.FMT_I8 else np.repeat(s, 128, axis=1)
        assert np.all(np.abs(back - w) <= step / 2 * 1.0001 + 1e-12)


@pytest.mark.parametrize("fmt", FMTS)
def test_group_dots_brute_force(fmt):
    rng = np.random.default_rng(6)
    K = 256
    if fmt == a8.FMT_F8:
        packed = rng.integers(0, 256, size=(3, K), dtype=np.uint8)
        packed[(packed & 0x7F) == 0x7F] = 0x38  # no NaN codes
        act = rng.integers(0, 256, size=(2, K), dtype=np.uint8)
        act[(act & 0x7F) == 0x7F] = 0x30
    else:
        packed = rng.integers(0, 256, size=(3, a8.row_bytes(fmt, K)), dtype=np.uint8)
        act = rng.integers(-127, 128, size=(2, K)).astype(np.int8)
    got = a8.group_dots(packed, fmt, act)
    w = a8.codes(packed, fmt)
    for r in range(3):
        for g in range(K // 128):
            for c in range(2):
                s = 0
                for k in range(128 * g, 128 * g + 128):
                    if fmt == a8.FMT_F8:
                        s += float(e4m3_decode(w[r, k])) * float(e4m3_decode(act[c, k]))
                    else:
                        s += int(w[r, k]) * int(act[c, k])
                assert got[r, g, c] == s


def test_route_brute_force_with_ties():
    # ties break to the lower index; -0 ties with +0
    vals = np.float32([[0.5, 2.0, 2.0, -1.0, 0.0, -0.0, 2.0, 1.5]])
    bits = f32_to_bf16_bits(vals)
    ids, w = a8.route(bits, 4)
    assert ids.tolist() == [[1, 2, 6, 7]]
    ex = np.exp(np.float64([2.0, 2.0, 2.0, 1.5]) - 2.0)
    assert np.allclose(w[0], ex / ex.sum(), rtol=2 ** -8)
    ids, _ = a8.route(f32_to_bf16_bits(np.float32([[0.0, -0.0, -0.0, 0.0, -1.0]])), 3)
    assert ids.tolist() == [[0, 1, 2]]


def test_route_matches_reference_torch_fallback():
    """model.py:120-121: softmax over all experts, top-k, renormalize, cast to bf16 - the same weights up to bf16
    rounding and the same selected logits (bf16 logits tie often; the kernel then takes the lower index, torch.topk
    either one)."""
    rng = np.random.default_rng(7)
    logits = torch.from_numpy(rng.standard_normal((6, 128)).astype(np.float32)).to(torch.bfloat16)
    ids, w = a8.route(logits.view(torch.int16).numpy().view(np.uint16), 8)
    tw, ti = torch.softmax(logits.float(), dim=-1).topk(8, dim=-1)
    tw = (tw / tw.sum(dim=-1, keepdim=True)).to(torch.bfloat16).float()
    lv = logits.float().numpy()
    assert np.array_equal(np.take_along_axis(lv, ids, 1), np.take_along_axis(lv, ti.numpy(), 1))
    assert np.allclose(w, tw.numpy(), rtol=2 ** -7, atol=0)


def test_quantize_act_properties():
    rng = np.random.default_rng(8)
    x = rng.standard_normal((4, 2048)).astype(np.float32)
    q, s = a8.quantize_act(x, a8.FMT_I8)
    assert np.abs(q).max() == 127
    for m in range(4):
        assert np.abs(q[m, np.argmax(np.abs(x[m]))]) == 127
        assert np.all(np.abs(q[m] * np.float64(s[m]) - x[m]) <= s[m] / 2 * 1.0001)
    q8, s8 = a8.quantize_act(x, a8.FMT_F8)
    assert np.nanmax(np.abs(e4m3_decode(q8))) == 448.0
    z, sz = a8.quantize_act(np.zeros((1, 256), dtype=np.float32), a8.FMT_I8)
    assert not z.any() and sz[0] == 0


@pytest.mark.parametrize("fmt", FMTS)
def test_layer_close_to_unquantized_layer(fmt):
    """The A8 layer stays within quantization error of the same layer in float64 with float activations."""
    rng = np.random.default_rng(9)
    E, H, I, k, M = 8, 256, 128, 4, 3
    gu = (rng.standard_normal((E, 2 * I, H)) * 0.05).astype(np.float32)
    dn = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    x = f32_to_bf16_bits(rng.standard_normal((M, H)).astype(np.float32))
    logits = f32_to_bf16_bits(rng.standard_normal((M, E)).astype(np.float32))
    banks = {"gate_up": [a8.quantize_weights(gu[e], fmt) for e in range(E)],
             "down": [a8.quantize_weights(dn[e], fmt) for e in range(E)]}
    out, ids, w, _ = a8.moe_layer(x, logits, (2 * I, H), (H, I), fmt, k, lambda b, e: banks[b][e])
    xf = bf16_bits_to_f32(x).astype(np.float64)
    ref = np.zeros((M, H))
    for m in range(M):
        for j in range(k):
            e = ids[m, j]
            y = gu[e].astype(np.float64) @ xf[m]
            h = y[:I] / (1 + np.exp(-y[:I])) * y[I:]
            ref[m] += w[m, j] * (dn[e].astype(np.float64) @ h)
    got = bf16_bits_to_f32(out).astype(np.float64)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    # measured: I8 0.020, W4 0.237 (uniform 4-bit on Gaussian weights), W6 0.054, F8 0.070
    assert rel < {a8.FMT_I8: 0.03, a8.FMT_W4: 0.30, a8.FMT_W6: 0.08, a8.FMT_F8: 0.10}[fmt]


def test_layer_gate_up_order_matters():
    """A planted swap of gate and up changes the result well beyond rounding, so the fused kernel's tests would
    catch that mistake."""
    rng = np.random.default_rng(10)
    E, H, I, k = 4, 256, 128, 2
    gu = (rng.standard_normal((E, 2 * I, H)) * 0.05).astype(np.float32)
    dn = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    x = f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    logits = f32_to_bf16_bits(rng.standard_normal((1, E)).astype(np.float32))
    swapped = np.concatenate([gu[:, I:], gu[:, :I]], axis=1)
    fetch = lambda w: (lambda b, e: a8.quantize_weights(w[e] if b == "gate_up" else dn[e], a8.FMT_I8))
    out, *_ = a8.moe_layer(x, logits, (2 * I, H), (H, I), a8.FMT_I8, k, fetch(gu))
    bad, *_ = a8.moe_layer(x, logits, (2 * I, H), (H, I), a8.FMT_I8, k, fetch(swapped))
    a, b = bf16_bits_to_f32(out), bf16_bits_to_f32(bad)
    assert np.linalg.norm(a - b) / np.linalg.norm(a) > 0.3


# ------------------------------------------------------------------------------------------------------------ block
def _bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)


def _bits_of(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_router_logits_against_torch_bf16_linear():
    """a8.router_logits is model.py:115's bf16 linear: torch's CPU bf16 linear gives the same bits on nearly every
    logit (its float32 sums in another order may cross a rounding boundary) and stays within one bf16 step; with the
    router's rows transposed (a planted index mistake) it does not."""
    rng = np.random.default_rng(3)
    x = numerics.f32_to_bf16_bits(rng.standard_normal((16, 2048)).astype(np.float32))
    r = numerics.f32_to_bf16_bits((rng.standard_normal((128, 2048)) * 0.02).astype(np.float32))
    got = numerics.bf16_bits_to_f32(a8.router_logits(x, r)).astype(np.float64)
    lib = torch.nn.functional.linear(_bf16(x), _bf16(r)).float().numpy().astype(np.float64)
    assert np.all(np.abs(got - lib) <= 2.0 ** -7 * np.abs(lib) + 1e-6)
    assert (got == lib).mean() >= 0.98
    planted = numerics.bf16_bits_to_f32(a8.router_logits(x, r.reshape(2048, 128).T.copy().reshape(128, 2048)))
    assert (planted.astype(np.float64) == lib).mean() < 0.1


def test_block_combine_against_torch_bf16_ops():
    """a8.block_combine is model.py:123 evaluated by torch on bf16 tensors: out + sigmoid(gate(x)) * shared(x). Same
    bits on nearly every element; taking the sigmoid of the gate before its bf16 rounding (a planted mistake) or
    skipping the product's rounding changes many more."""
    rng = np.random.default_rng(4)
    M, H = 64, 2048
    x = numerics.f32_to_bf16_bits(rng.standard_normal((M, H)).astype(np.float32))
    g = numerics.f32_to_bf16_bits((rng.standard_normal(H) * 0.05).astype(np.float32))
    routed = numerics.f32_to_bf16_bits((rng.standard_normal((M, H)) * 0.1).astype(np.float32))
    shared = numerics.f32_to_bf16_bits((rng.standard_normal((M, H)) * 0.1).astype(np.float32))
    got = a8.block_combine(routed, shared, x, g)
    gate = torch.nn.functional.linear(_bf16(x), _bf16(g)[None, :])                  # [M, 1] bf16
    lib = _bits_of(_bf16(routed) + torch.sigmoid(gate) * _bf16(shared))
    same = (got == lib).mean()
    assert same >= 0.99, same
    gv, lv = numerics.bf16_bits_to_f32(got), numerics.bf16_bits_to_f32(lib)
    assert np.all(np.abs(gv - lv) <= 2.0 ** -7 * np.abs(lv) + 1e-6)
    # planted: the sigmoid of the unrounded float gate, the product unrounded
    xf = numerics.bf16_bits_to_f32(x).astype(np.float64)
    gf = numerics.bf16_bits_to_f32(g).astype(np.float64)
    gw = (1.0 / (1.0 + np.exp(-(xf @ gf)))).astype(np.float32)
    wrong = numerics.f32_to_bf16_bits((numerics.bf16_bits_to_f32(routed) +
                                       gw[:, None] * numerics.bf16_bits_to_f32(shared)).astype(np.float32))
    assert (wrong == lib).mean() < same - 0.05


@pytest.mark.parametrize("fmt", FMTS)
def test_layer_equals_dense_math_on_its_own_operands(fmt):
    """The oracle layer against the same layer written as dense float64 algebra on its own quantized operands: each
    weight row decoded on its own (a8.codes, then times the bf16 scale of its row or its 128-column group, written
    here from the format's definition), the activations dequantized, plain matrix products, SiLU(gate) * up, the hidden
    rows quantized again, the routing-weighted sum. This path shares no arithmetic with the oracle's grouped integer
    sums, so a misplaced scale group, a dropped activation scale or a wrong hidden quantization fails it; the two agree
    to rounding: the same bf16 bits on at least 99% of the outputs, within one bf16 step on all. A planted mistake, the group scales shifted by one group (a row scale
    format: each row's scale taken from the next row), moves the result far beyond the bar."""
    rng = np.random.default_rng(19)
    E, H, I, k, M = 8, 512, 256, 4, 3
    gu = (rng.standard_normal((E, 2 * I, H)) * 0.05).astype(np.float32)
    dn = (rng.standard_normal((E, H, I)) * 0.05).astype(np.float32)
    x = f32_to_bf16_bits(rng.standard_normal((M, H)).astype(np.float32))
    logits = f32_to_bf16_bits(rng.standard_normal((M, E)).astype(np.float32))
    banks = {"gate_up": [a8.quantize_weights(gu[e], fmt) for e in range(E)],
             "down": [a8.quantize_weights(dn[e], fmt) for e in range(E)]}
    out, ids, w, _ = a8.moe_layer(x, logits, (2 * I, H), (H, I), fmt, k, lambda b, e: banks[b][e])

    def dense(packed, scale_bits, shift=0):
        rows, cols = packed.shape[0], (packed.shape[1] if fmt in (a8.FMT_I8, a8.FMT_F8) else
                                       packed.shape[1] * (2 if fmt == a8.FMT_W4 else 4) // (1 if fmt == a8.FMT_W4 else 3))
        if fmt == a8.FMT_F8:
            v = e4m3_decode(packed).astype(np.float64)
        elif fmt == a8.FMT_I8:
            v = packed.view(np.int8).astype(np.float64)
        else:
            v = a8.codes(packed, fmt).astype(np.float64)
        s = bf16_bits_to_f32(scale_bits).astype(np.float64).reshape(rows, -1)
        s = np.roll(s, shift, axis=1 if s.shape[1] > 1 else 0)
        return v * np.repeat(s, cols // s.shape[1], axis=1)

    def layer(shift):
        xq, xs = a8.quantize_act(bf16_bits_to_f32(x), fmt)
        xd = (e4m3_decode(xq) if fmt == a8.FMT_F8 else xq).astype(np.float64) * xs.astype(np.float64)[:, None]
        res = np.zeros((M, H))
        for m in range(M):
            for j in range(k):
                e = ids[m, j]
                y = dense(*banks["gate_up"][e], shift) @ xd[m]
                h = (y[:I] / (1.0 + np.exp(-y[:I])) * y[I:]).astype(np.float32)
                hq, hs = a8.quantize_act(h[None], fmt)
                hd = (e4m3_decode(hq) if fmt == a8.FMT_F8 else hq).astype(np.float64)[0] * np.float64(hs[0])
                res[m] += np.float64(w[m, j]) * (dense(*banks["down"][e], shift) @ hd)
        return res

    got = bf16_bits_to_f32(out).astype(np.float64)
    ref = bf16_bits_to_f32(f32_to_bf16_bits(layer(0).astype(np.float32))).astype(np.float64)   # the output's rounding
    assert (got == ref).mean() >= 0.99, (got == ref).mean()
    assert np.all(np.abs(got - ref) <= 2.0 ** -8 * np.abs(ref))
    planted = layer(1)
    assert np.linalg.norm(got - planted) > 0.05 * np.linalg.norm(planted)
