"""Pins of oracle/reference.py (the reference's kernels restated) against closed forms, brute force, a library
(torch's e4m3fn cast) and hand-built cases whose answers are fixed by the reference's definitions
(drama3/kernels.py:25-587, drama3/offload.py:108-176). CPU only."""
import numpy as np
import pytest
import torch

from oracle import numerics
from oracle import reference as ref


# ---------------------------------------------------------------------------------------------------------- e4m3
def test_e4m3_ref_matches_ocp_e4m3fn_and_reads_nan_codes_as_480():
    codes = np.arange(256, dtype=np.uint8)
    got = ref.e4m3_ref(codes)
    lib = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy().astype(np.float64)
    finite = (codes & 0x7F) != 0x7F
    assert np.array_equal(got[finite], lib[finite])
    assert got[0x7F] == 480.0 and got[0xFF] == -480.0
    # subnormals: 2^-6 * m / 8
    assert np.array_equal(got[1:8], 2.0 ** -6 * np.arange(1, 8) / 8)


# --------------------------------------------------------------------------------------------------------- route
def _bits(values):
    return numerics.f32_to_bf16_bits(np.asarray(values, np.float32))


def test_route_ref_sorted_descending_ties_to_lower_index():
    rng = np.random.default_rng(0)
    for n, k in ((8, 3), (64, 8), (128, 8), (256, 8), (40, 32)):
        v = rng.integers(-4, 4, size=(5, n)).astype(np.float32) * 0.5  # many ties
        ids, w = ref.route_ref(_bits(v), k)
        for r in range(5):
            expect = sorted(range(n), key=lambda i: (-v[r, i], i))[:k]
            assert list(ids[r]) == expect
            top = v[r, expect].astype(np.float64)
            closed = np.exp(top - top[0]) / np.exp(top - top[0]).sum()
            # float32 arithmetic then bf16 rounding: within one bf16 step of the exact value
            assert np.all(np.abs(w[r] - closed) <= 2.0 ** -8 * closed + 1e-7)
            assert np.array_equal(numerics.bf16_round(w[r]), w[r])


def test_route_ref_single_winner_and_uniform():
    ids, w = ref.route_ref(_bits([[0, 0, 5, 0]]), 1)
    assert ids[0, 0] == 2 and w[0, 0] == 1.0
    ids, w = ref.route_ref(_bits([[1, 1, 1, 1]]), 4)
    assert list(ids[0]) == [0, 1, 2, 3] and np.all(w == 0.25)


def test_weighted_sum_ref():
    parts = np.array([[1.0, 2.0, -3.0], [0.5, 0.25, 1.0]], np.float32)
    out = ref.weighted_sum_ref(parts, np.array([0.5, 2.0], np.float32))
    assert np.array_equal(numerics.bf16_bits_to_f32(out)[0], np.array([1.5, 1.5, 0.5], np.float32))


# -------------------------------------------------------------------------------------------------------- rotate
def _butterfly(row):
    """The stride-1/4/16/64 butterfly of kernels.py:241-255 with its four sign patterns, / 16."""
    row = np.array(row, np.float64)
    K = row.shape[0]
    stride = 1
    while stride < 256:
        for t in range(K // 4):
            within, low, high = t & 63, (t & 63) % stride, (t & 63) // stride
            i = (t >> 6) * 256 + high * stride * 4 + low
            a, b, c, d = row[i], row[i + stride], row[i + 2 * stride], row[i + 3 * stride]
            row[i], row[i + stride], row[i + 2 * stride], row[i + 3 * stride] = (
                a + b + c - d, a + b - c + d, a - b + c + d, -a + b + c + d)
        stride *= 4
    return row * 0.0625


def test_rotate_ref_equals_the_butterfly_network_and_is_an_involution():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 512))
    got = ref.rotate_ref(x)
    for r in range(3):
        assert np.allclose(got[r], _butterfly(x[r]), rtol=0, atol=1e-12)
    assert np.allclose(ref.rotate_ref(got), x, atol=1e-12)  # H symmetric and orthogonal
    g, u = rng.standard_normal((2, 256)), rng.standard_normal((2, 256))
    assert np.allclose(ref.rotate_ref(np.concatenate([g, u], 1), swiglu=True),
                       ref.rotate_ref(g / (1 + np.exp(-g)) * u), atol=1e-12)


def test_rotate_ref_unit_vector_is_a_hadamard_row():
    x = np.zeros((1, 256))
    x[0, 3] = 1.0
    row = ref.rotate_ref(x)[0]
    assert np.allclose(np.abs(row), 1 / 16)
    # row 3 of h4 kron ... has -1 where the low digit is 0 (h4 row 3 = [-1, 1, 1, 1]) and no other digit is 3
    assert row[0] < 0 and row[1] > 0


# -------------------------------------------------------------------------------------------------- code decoding
def _decode_formula(code, sbyte, bits, codebook):
    s = np.float32(ref.e4m3_ref(sbyte))
    v = np.float32(code - 32) if bits == 6 else np.float32(codebook[code])
    return int(np.clip(np.rint(np.float32(v * s)), -127, 127))


@pytest.mark.parametrize("bits", [4, 6])
def test_decode_codes_ref_exhaustive_codes_and_scales(bits):
    codebook = ref.default_codebook()
    ncodes = 1 << bits
    K = 16 * 256  # one 16-column group per scale byte
    codes = np.tile(np.arange(ncodes), 256 * 16 // ncodes + 1)[:K]
    rows = []
    for shift in range(ncodes // 16 if ncodes > 16 else 1):
        rows.append(np.roll(codes, 16 * shift))
    code = np.stack(rows).astype(np.uint32)
    scale = np.tile(np.arange(256, dtype=np.uint8), (code.shape[0], 1))
    got = ref.decode_codes_ref(ref.pack_codes(code, bits), scale, bits, codebook)
    for r in range(code.shape[0]):
        for c in range(K):
            assert got[r, c] == _decode_formula(int(code[r, c]), int(scale[r, c // 16]), bits, codebook)


def test_decode_codes_ref_layout_planted_bytes():
    """Byte b of the nibble plane holds columns 2b (low) and 2b + 1 (high); at 6 bits, high-plane byte i (after the K/2
    nibble bytes) holds columns 4i .. 4i + 3, two bits each from bit 0 (kernels.py:466-483 reads a little-endian u32
    per 16 columns at K/2 + 4v, column j at bits 2j)."""
    K = 64
    one = np.uint8(0x38)  # e4m3 1.0
    scale = np.full((1, K // 16), one, np.uint8)
    q = np.zeros((1, K * 6 // 8), np.uint8)
    q[0, 5] = 0x21  # columns 10 (code 1) and 11 (code 2)
    q[0, K // 2 + 5] = 0b01_00_00_10  # columns 20 (high 2) and 23 (high 1)
    got = ref.decode_codes_ref(q, scale, 6)[0].astype(int)
    expect = np.full(K, -32)
    expect[10], expect[11] = 1 - 32, 2 - 32
    expect[20], expect[23] = 32 - 32, 16 - 32
    assert np.array_equal(got, expect)
    cb = np.arange(16, dtype=np.float32) - 8
    q4 = np.zeros((1, K // 2), np.uint8)
    q4[0, 3] = 0xF0  # column 7 -> code 15
    got4 = ref.decode_codes_ref(q4, scale, 4, cb)[0].astype(int)
    expect4 = np.full(K, -8)
    expect4[7] = 7
    assert np.array_equal(got4, expect4)


# ------------------------------------------------------------------------------------------------- decode GEMVs
def _int8_bank(rng, E, N, K):
    return {"_qdata": rng.integers(-127, 128, size=(E * N, K), dtype=np.int8),
            "scale": rng.uniform(0.001, 0.01, size=E * N).astype(np.float32)}


def test_gemv_int8_ref_plan_semantics():
    rng = np.random.default_rng(2)
    E, N, K, slots = 6, 32, 256, 3
    host = _int8_bank(rng, E, N, K)
    slot = {"_qdata": np.zeros((slots * N, K), np.int8), "scale": np.zeros(slots * N, np.float32)}
    slot["_qdata"][N:2 * N] = host["_qdata"][4 * N:5 * N]  # expert 4 cached in slot 1
    slot["scale"][N:2 * N] = host["scale"][4 * N:5 * N]
    x = rng.standard_normal((1, K)).astype(np.float32)
    ids = np.array([4, 2, 5, 0])
    plan = np.array([[1, 0], [2, 1], [-1, 1], [0, 2]])  # cached, miss filling slot 2, miss without slot, CPU's
    out = ref.gemv_int8_ref(x, ids, plan, False, False, slot, host, N)

    def direct(e):
        w = host["_qdata"][e * N:(e + 1) * N].astype(np.float64) * host["scale"][e * N:(e + 1) * N, None]
        return w @ x[0].astype(np.float64)
    assert np.allclose(out[0], direct(4)) and np.allclose(out[1], direct(2)) and np.allclose(out[2], direct(5))
    assert np.all(out[3] == 0)
    assert np.array_equal(slot["_qdata"][2 * N:3 * N], host["_qdata"][2 * N:3 * N])
    assert np.array_equal(slot["scale"][2 * N:3 * N], host["scale"][2 * N:3 * N])
    late = ref.gemv_int8_ref(x, ids, plan, True, True, slot, host, N)
    assert np.all(late[:3] == 0) and np.allclose(late[3], direct(0))
    assert np.all(ref.gemv_int8_ref(x, ids, plan, False, True, slot, host, N) == 0)


def test_gemv_fp8_ref_block_scales():
    rng = np.random.default_rng(3)
    E, N, K = 2, 256, 256
    w = rng.integers(0, 256, size=(E * N, K)).astype(np.uint8)
    w[(w & 0x7F) == 0x7F] = 0
    s = rng.uniform(0.5, 2, size=(E * N // 128, K // 128)).astype(np.float32)
    x = rng.standard_normal((2, K)).astype(np.float32)
    ids, plan = np.array([1, 0]), np.array([[1, 0], [0, 0]])
    bank = {"weight": w, "scale": s}
    out = ref.gemv_fp8_ref(x, ids, plan, bank, bank, N)
    vals = torch.from_numpy(w).view(torch.float8_e4m3fn).double().numpy()
    for e, xe in ((1, x[0]), (0, x[1])):
        blocks = np.repeat(np.repeat(s[e * 2:(e + 1) * 2], 128, 0), 128, 1)
        expect = (vals[e * N:(e + 1) * N] * blocks) @ xe.astype(np.float64)
        assert np.allclose(out[ids.tolist().index(e)], expect, rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("bits", [4, 6])
def test_grouped_ref_matches_gemv_refs_row_by_row(bits):
    rng = np.random.default_rng(4)
    E, N, K = 4, 32, 256
    w = rng.standard_normal((E, N, K)) * 0.02
    fields, cb = ref.quantize_codes(w, bits)
    x = rng.standard_normal((5, K)).astype(np.float32)
    groups = np.array([[3, 3, 0, 0, 2], [1, 1, 0, 2, 3]])
    out = ref.grouped_ref(f"w{bits}", x, groups, fields, fields, cb, N)
    for t, e in ((0, 3), (1, 3), (2, 1), (3, 1), (4, 1)):
        one = ref.gemv_codes_ref(x[t:t + 1], np.array([e]), np.array([[e, 0]]), fields, fields, cb, bits, N)
        assert np.allclose(out[t], one[0], rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------------------------------- quantizers
@pytest.mark.parametrize("kind,bound", [("int8", 0.02), ("fp8", 0.05), ("w4", 0.15), ("w6", 0.04)])
def test_quantizers_round_trip(kind, bound):
    rng = np.random.default_rng(5)
    w = rng.standard_normal((2, 128, 512)) * 0.02
    if kind == "int8":
        fields, cb = ref.quantize_int8_convrot(w), None
    elif kind == "fp8":
        fields, cb = ref.quantize_fp8_block(w), None
    else:
        fields, cb = ref.quantize_codes(w, int(kind[1]))
    deq = ref.dequantize_bank(kind, fields, cb)
    target = w.reshape(256, 512) if kind == "fp8" else ref.convrot(w).reshape(256, 512)
    err = np.linalg.norm(deq - target) / np.linalg.norm(target)
    assert err < bound, err


# --------------------------------------------------------------------------------------------------------- layer
def _layer_banks(kind, rng, E=4, H=256, I=256):
    gu = rng.standard_normal((E, 2 * I, H)) * 0.05
    dn = rng.standard_normal((E, H, I)) * 0.05
    if kind == "int8":
        banks, cbs = (ref.quantize_int8_convrot(gu), ref.quantize_int8_convrot(dn)), (None, None)
    elif kind == "fp8":
        banks, cbs = (ref.quantize_fp8_block(gu), ref.quantize_fp8_block(dn)), (None, None)
    else:
        (a, ca), (b, cb) = ref.quantize_codes(gu, int(kind[1])), ref.quantize_codes(dn, int(kind[1]))
        banks, cbs = (a, b), (ca, cb)
    return gu, dn, banks, cbs


@pytest.mark.parametrize("kind,bound", [("int8", 0.03), ("fp8", 0.06), ("w4", 0.25), ("w6", 0.06)])
def test_resident_decode_ref_against_unquantized_layer(kind, bound):
    rng = np.random.default_rng(6)
    gu, dn, banks, cbs = _layer_banks(kind, rng)
    I = dn.shape[2]
    x = numerics.f32_to_bf16_bits(rng.standard_normal((1, 256)).astype(np.float32))
    ids, w = np.array([2, 0, 3]), np.array([0.5, 0.3, 0.2], np.float32)
    got = numerics.bf16_bits_to_f32(ref.resident_decode_ref(x, ids, w, banks, (2 * I, 256), kind, cbs))[0]
    xf = numerics.bf16_bits_to_f32(x)[0].astype(np.float64)
    exact = np.zeros(256)
    for e, we in zip(ids, w):
        y = gu[e] @ xf
        exact += we * (dn[e] @ (y[:I] / (1 + np.exp(-y[:I])) * y[I:]))
    err = np.linalg.norm(got - exact) / np.linalg.norm(exact)
    assert err < bound, err
    # a planted mistake in the oracle (gate and up swapped) must not pass the same bound
    swapped = np.zeros(256)
    for e, we in zip(ids, w):
        y = gu[e] @ xf
        swapped += we * (dn[e] @ (y[I:] / (1 + np.exp(-y[I:])) * y[:I]))
    assert np.linalg.norm(got - swapped) / np.linalg.norm(swapped) > 3 * bound


def test_resident_prefill_ref_equals_decode_per_row():
    rng = np.random.default_rng(7)
    _, _, banks, cbs = _layer_banks("int8", rng)
    x = numerics.f32_to_bf16_bits(rng.standard_normal((3, 256)).astype(np.float32))
    idx = np.array([[0, 1], [3, 0], [2, 2]])
    w = np.array([[0.75, 0.25], [0.5, 0.5], [0.6, 0.4]], np.float32)
    got = ref.resident_prefill_ref(x, idx, w, banks, (512, 256), "int8", cbs)
    for t in range(3):
        one = ref.resident_decode_ref(x[t:t + 1], idx[t], w[t], banks, (512, 256), "int8", cbs)
        a, b = numerics.bf16_bits_to_f32(got[t]), numerics.bf16_bits_to_f32(one[0])
        assert np.all(np.abs(a - b) <= 2.0 ** -7 * np.abs(b) + 1e-6)


# ---------------------------------------------------------- FP8 rows (one e4m3 weight, a bf16 scale per output row)
def _fp8_rows_case(N=96, K=512, seed=0):
    rng = np.random.default_rng(seed)
    x = numerics.f32_to_bf16_bits(rng.standard_normal((2, K)).astype(np.float32))
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    codes, sbits = ref.quantize_fp8_rows(w)
    return x, w, codes, sbits


def test_fp8_rows_dequant_matches_torch_bit_for_bit():
    """The dequantized bf16 matrix equals torch's: float8 decode, float32 product with the scale, bf16 cast."""
    _, _, codes, sbits = _fp8_rows_case()
    got = ref.fp8_rows_dequant(codes, sbits)
    wt = torch.from_numpy(codes).view(torch.float8_e4m3fn).float()
    st = torch.from_numpy(sbits.view(np.int16)).view(torch.bfloat16).float()
    want = (wt * st[:, None]).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, want)
    # the scale is absmax / 448 rounded to bf16: every row's largest code sits at the top of the e4m3 range
    assert np.all(np.abs(ref.e4m3_ref(codes)).max(axis=1) >= 416.0)


def test_fp8_rows_linear_against_torch_and_unquantized():
    """Within one bf16 step of torch's bf16 linear on the CPU (float32 sums in another order), within the format's
    error of the unquantized float64 product; rows scaled by their neighbours' scales fail that bar."""
    x, w, codes, sbits = _fp8_rows_case()
    got = numerics.bf16_bits_to_f32(ref.fp8_rows_linear_ref(x, codes, sbits)).astype(np.float64)
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16)
    wd = torch.from_numpy(ref.fp8_rows_dequant(codes, sbits)).to(torch.bfloat16)
    lib = torch.nn.functional.linear(xt, wd).float().numpy().astype(np.float64)
    assert np.all(np.abs(got - lib) <= 2.0 ** -7 * np.abs(lib) + 1e-6)
    exact = numerics.bf16_bits_to_f32(x).astype(np.float64) @ w.astype(np.float64).T
    rel = np.linalg.norm(got - exact) / np.linalg.norm(exact)
    assert rel < 0.05, rel
    # a planted mistake: each row scaled by its neighbour's scale
    planted = numerics.bf16_bits_to_f32(ref.fp8_rows_linear_ref(x, codes, np.roll(sbits, 1))).astype(np.float64)
    assert np.linalg.norm(planted - exact) / np.linalg.norm(exact) > 2 * rel
