"""Parity of the reference-format kernels (kernels.py surface -> libdrama3_moe.so) and the layer entry points of
offload.py with the oracle (oracle/reference.py) on the same seeded inputs.

Bars: routing ids exact and weights within one bf16 step; decoded int8-grid codes bit-exact; float32 GEMV / grouped
outputs within 3e-5 of each output's sum of |w x| (float32 sums in another order than the oracle's float64);
bf16 layer outputs within one bf16 step plus 1e-5 of the row's largest value. FP8 codes 0x7F / 0xFF are left out of
the inputs: the hardware e4m3fn decode reads them as NaN where the reference reads +-480."""
import numpy as np
import pytest
import torch

from drama3 import _lib, kernels, offload
from oracle import numerics
from oracle import reference as ref
from tests.planes_np import split_i8_np

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def pinned(a):
    return torch.from_numpy(np.ascontiguousarray(a)).pin_memory()


def fields_on(fields, where=dev):
    return {n: where(v) for n, v in fields.items()}


def assert_dot_close(got, expect, abs_sum, tol=3e-5):
    got = got.detach().cpu().numpy().astype(np.float64)
    bound = tol * abs_sum + 1e-30
    err = np.abs(got - expect)
    assert np.all(err <= bound), (err / bound).max()


def assert_bf16_close(got_bits, expect_bits):
    a = numerics.bf16_bits_to_f32(np.asarray(got_bits)).astype(np.float64)
    b = numerics.bf16_bits_to_f32(np.asarray(expect_bits)).astype(np.float64)
    assert np.all(np.isfinite(a))
    bound = 2.0 ** -7 * np.abs(b) + 1e-5 * np.abs(b).max()
    assert np.all(np.abs(a - b) <= bound), np.abs(a - b).max()


def bits_of(t):
    return t.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def no_nan_fp8(rng, shape):
    w = rng.integers(0, 256, size=shape).astype(np.uint8)
    w[(w & 0x7F) == 0x7F] = 0x7E
    return w


# ---------------------------------------------------------------------------------------------------------- route
@pytest.mark.parametrize("n,k,rows", [(128, 8, 1), (256, 8, 1), (1024, 32, 3), (64, 1, 5)])
def test_route(n, k, rows):
    rng = np.random.default_rng(n + k)
    v = (rng.integers(-6, 6, size=(rows, n)) * 0.37).astype(np.float32)  # ties on purpose
    bits = numerics.f32_to_bf16_bits(v)
    ids, w = kernels.route(dev(bits).view(torch.bfloat16), k)
    rid, rw = ref.route_ref(bits, k)
    assert np.array_equal(ids.cpu().numpy(), rid)
    got = w.cpu().numpy()
    assert np.all(np.abs(got - rw) <= 2.0 ** -8 * rw + 1e-7)


def test_weighted_sum():
    rng = np.random.default_rng(1)
    parts = rng.standard_normal((8, 2048)).astype(np.float32)
    w = rng.uniform(0, 1, 8).astype(np.float32)
    out = kernels.weighted_sum(dev(parts), dev(w))
    assert out.shape == (1, 2048) and out.dtype == torch.bfloat16
    assert_bf16_close(bits_of(out), ref.weighted_sum_ref(parts, w))


# --------------------------------------------------------------------------------------------------------- rotate
@pytest.mark.parametrize("mode,rows,K", [("f32", 3, 2048), ("bf16", 1, 2048), ("bf16", 2, 768), ("swiglu", 8, 768),
                                         ("swiglu", 8, 512)])
def test_rotate(mode, rows, K):
    rng = np.random.default_rng(K + rows)
    always = torch.ones(1, dtype=torch.int32, device=DEV)
    if mode == "swiglu":
        x = rng.standard_normal((rows, 2 * K)).astype(np.float32)
        got = kernels.rotate(dev(x), always, swiglu=True)
        expect = ref.rotate_ref(x, swiglu=True)
    elif mode == "bf16":
        bits = numerics.f32_to_bf16_bits(rng.standard_normal((rows, K)).astype(np.float32))
        got = kernels.rotate(dev(bits).view(torch.bfloat16), always)
        expect = ref.rotate_ref(numerics.bf16_bits_to_f32(bits))
    else:
        x = rng.standard_normal((rows, K)).astype(np.float32)
        got = kernels.rotate(dev(x), always)
        expect = ref.rotate_ref(x)
    err = np.abs(got.cpu().numpy() - expect).max() / np.abs(expect).max()
    assert err < 2e-6, err


def test_rotate_only_if_zero_writes_nothing():
    x = torch.randn(2, 512, device=DEV)
    out = torch.full((2, 512), 7.0, device=DEV)
    never = torch.zeros(1, dtype=torch.int32, device=DEV)
    _lib.check(_lib.lib().d3_rotate(x.data_ptr(), 0, 2, 512, out.data_ptr(), never.data_ptr(),
                                    _lib.stream_of(DEV)), "d3_rotate")
    assert torch.all(out == 7.0)


def split3_np(v):
    """hi, mid, lo float32 arrays: bf16(v), bf16(v - hi), bf16(v - hi - mid) with float32 differences."""
    v = np.asarray(v, np.float32)
    hi = numerics.bf16_bits_to_f32(numerics.f32_to_bf16_bits(v))
    r = (v - hi).astype(np.float32)
    mid = numerics.bf16_bits_to_f32(numerics.f32_to_bf16_bits(r))
    lo = numerics.bf16_bits_to_f32(numerics.f32_to_bf16_bits((r - mid).astype(np.float32)))
    return hi, mid, lo


def planes_np(planes, P, K):
    return [planes[t].float().cpu().numpy().reshape(P, K) for t in range(3)]


def test_prep_planes_one_plane_holds_bf16_rows():
    """n_planes 1: the gathered bf16 rows themselves, bit for bit."""
    rng = np.random.default_rng(12)
    T, k, K = 19, 4, 2048
    bits = numerics.f32_to_bf16_bits(rng.standard_normal((T, K)).astype(np.float32))
    order = rng.permutation(T * k)
    planes = kernels.prep_planes(dev(bits).view(torch.bfloat16), False, dev(order.astype(np.int64)), k, n_planes=1)
    assert planes.shape == (1, T * k * K)
    assert np.array_equal(planes.view(torch.int16).cpu().numpy().reshape(T * k, K).view(np.uint16), bits[order // k])
    with pytest.raises(RuntimeError, match="1 for bf16 rows"):
        kernels.prep_planes(dev(bits).view(torch.bfloat16), True, n_planes=1)


@pytest.mark.parametrize("mode, rotate", [("f32", False), ("bf16", True), ("bf16", False), ("swiglu", True),
                                          ("swiglu", False)])
def test_prep_planes(mode, rotate):
    """d3_prep_planes: the gathered (row order[p] // k), SwiGLU'd and rotated rows as the oracle's rotate_ref gives
    them (within 2e-6 of the largest, the float32 transform's reordering), split into planes bit for bit as numpy
    splits the kernel's own float32 rows (d3_rotate's, the same transform), and hi + mid + lo within 2^-24 |x|."""
    rng = np.random.default_rng(len(mode) + rotate)
    T, k, K = 37, 3, 768
    order = rng.permutation(T * k)
    if mode == "swiglu":
        x = rng.standard_normal((T * k, 2 * K)).astype(np.float32)
        planes = kernels.prep_planes(dev(x), rotate, swiglu=True)
        rows = x
        want = ref.rotate_ref(x, swiglu=True) if rotate else None
        if not rotate:
            g, u = x[:, :K].astype(np.float64), x[:, K:].astype(np.float64)
            want = g / (1 + np.exp(-g)) * u
        dev_rows = kernels.rotate(dev(x), torch.ones(1, dtype=torch.int32, device=DEV), swiglu=True) if rotate \
            else None
        P = T * k
    else:
        if mode == "bf16":
            bits = numerics.f32_to_bf16_bits(rng.standard_normal((T, K)).astype(np.float32))
            xd, x = dev(bits).view(torch.bfloat16), numerics.bf16_bits_to_f32(bits)
        else:
            x = rng.standard_normal((T, K)).astype(np.float32)
            xd = dev(x)
        planes = kernels.prep_planes(xd, rotate, dev(order.astype(np.int64)), k)
        rows = x[order // k]
        want = ref.rotate_ref(rows) if rotate else rows
        dev_rows = kernels.rotate(dev(rows.astype(np.float32)), torch.ones(1, dtype=torch.int32, device=DEV)) \
            if rotate else None
        P = T * k
    hi, mid, lo = planes_np(planes, P, K)
    total = hi.astype(np.float64) + mid + lo
    assert np.abs(total - want).max() <= 2e-6 * np.abs(want).max()
    if dev_rows is not None or mode != "swiglu":
        exact = dev_rows.cpu().numpy() if dev_rows is not None else want.astype(np.float32)
        h, m, l = split3_np(exact)
        assert np.array_equal(hi, h) and np.array_equal(mid, m) and np.array_equal(lo, l)
        assert np.all(np.abs(total - exact) <= 2.0 ** -24 * np.abs(exact))


@pytest.mark.parametrize("mode, rotate", [("f32", False), ("bf16", True), ("f32", True), ("swiglu", True),
                                          ("swiglu", False)])
def test_prep_planes_i8(mode, rotate):
    """d3_prep_planes_i8: the rows prep_planes gathers, SwiGLUs and rotates, as three int8 planes and a power-of-two
    scale S. Pinned by what the split must satisfy whatever its arithmetic: every plane value in [-127, 127], S the
    smallest power of two with max |v| <= 127 S, and S (a0 + a1 / 254 + a2 / 254^2) within (0.5 / 254^2 + 2^-24) S,
    so 1.25e-7 max |v|, of each value (float64); the planes also equal a numpy split of the kernel's own float32 rows
    (d3_rotate's transform)."""
    rng = np.random.default_rng(60 + len(mode) + rotate)
    T, k, K = 29, 3, 768 if mode != "f32" else 2048
    order = rng.permutation(T * k)
    if mode == "swiglu":
        x = rng.standard_normal((T * k, 2 * K)).astype(np.float32)
        planes, scales = kernels.prep_planes_i8(dev(x), rotate, swiglu=True)
        if rotate:
            rows = kernels.rotate(dev(x), torch.ones(1, dtype=torch.int32, device=DEV), swiglu=True).cpu().numpy()
        else:
            g, u = x[:, :K].astype(np.float64), x[:, K:].astype(np.float64)
            rows = g / (1 + np.exp(-g)) * u
    else:
        if mode == "bf16":
            bits = numerics.f32_to_bf16_bits(rng.standard_normal((T, K)).astype(np.float32))
            xd, x = dev(bits).view(torch.bfloat16), numerics.bf16_bits_to_f32(bits)
        else:
            x = (rng.standard_normal((T, K)) * np.exp(rng.uniform(-20, 20, (T, 1)))).astype(np.float32)
            xd = dev(x)
        planes, scales = kernels.prep_planes_i8(xd, rotate, dev(order.astype(np.int64)), k)
        rows = x[order // k]
        if rotate:
            rows = kernels.rotate(dev(rows.astype(np.float32)), torch.ones(1, dtype=torch.int32, device=DEV)).cpu().numpy()
    P = T * k
    a = [planes[t].cpu().numpy().reshape(P, K).astype(np.float64) for t in range(3)]
    S = scales.cpu().numpy().astype(np.float64)
    assert all(np.abs(p).max() <= 127 for p in a)
    m = np.abs(rows).max(axis=1)
    exact = mode != "swiglu" or rotate   # rows as the kernel computes them (else numpy's exp against the kernel's)
    assert np.all(np.log2(S) == np.round(np.log2(S)))
    if exact:
        assert np.all(m <= 127 * S) and np.all(m > 63.5 * S)
    held = S[:, None] * (a[0] + (a[1] + a[2] / 254) / 254)
    if exact:
        assert np.all(np.abs(held - rows) <= (0.5 / 254 ** 2 + 2.0 ** -24) * S[:, None])
    assert np.all(np.abs(held - rows) <= (1.25e-7 if exact else 2e-6) * m[:, None])
    if exact:
        want = split_i8_np(rows)
        for t in range(3):
            assert np.array_equal(a[t], want[t]), t
        assert np.array_equal(S, want[3])


def test_prep_planes_i8_special_rows():
    """A row of integers times a power of two lies in a0 alone (so one-hot rows are exact); an all-zero row gets
    S = 0 and a row holding inf or NaN S = NaN, with zero planes; the other rows are unaffected."""
    K = 256
    x = np.zeros((5, K), np.float32)
    x[0] = np.arange(K) % 255 - 127            # integers up to 127: S = 1
    x[1, 7] = 3.0                              # one-hot times 3: S = 2^-5, a0 = 96
    x[2, 3], x[2, 9] = np.inf, 1.0
    x[3, 5] = np.nan
    planes, scales = kernels.prep_planes_i8(dev(x), False)
    a = [planes[t].cpu().numpy().reshape(5, K) for t in range(3)]
    S = scales.cpu().numpy()
    assert S[0] == 1.0 and np.array_equal(a[0][0], x[0]) and not a[1][0].any() and not a[2][0].any()
    assert S[1] == 2.0 ** -5 and a[0][1, 7] == 96 and np.count_nonzero(a[0][1]) == 1 and not a[1][1].any()
    assert np.isnan(S[2]) and np.isnan(S[3]) and S[4] == 0.0
    for r in (2, 3, 4):
        assert not any(p[r].any() for p in a), r


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("wdtype", [torch.bfloat16, torch.float32])
def test_combine_rows(dtype, wdtype):
    """d3_combine_rows against numpy: sum over j of w[t, j] * rows[inverse[t k + j]] (float64 sum, then the output
    dtype), within float32 rounding of the sum of |terms| before the output's own rounding; pairs with inverse -1 left
    out."""
    rng = np.random.default_rng(3)
    T, k, H = 29, 8, 2048
    rows = rng.standard_normal((T * k, H)).astype(np.float32)
    inverse = rng.permutation(T * k).astype(np.int32)
    inverse[5] = -1
    w = rng.dirichlet(np.ones(k), T).astype(np.float32)
    wt = torch.from_numpy(w).to(DEV, wdtype)
    wv = wt.float().cpu().numpy().astype(np.float64)
    got = kernels.combine_rows(dev(rows), dev(inverse), wt, dtype).float().cpu().numpy()
    terms = np.zeros((T, k, H))
    for t in range(T):
        for j in range(k):
            at = inverse[t * k + j]
            if at >= 0:
                terms[t, j] = wv[t, j] * rows[at]
    want = terms.sum(1)
    bound = 1e-6 * np.abs(terms).sum(1) + (0 if dtype == torch.float32 else
                                          (2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11) * np.abs(want))
    assert np.all(np.abs(got - want) <= bound + 1e-30)


# ----------------------------------------------------------------------------------------------------- decode
@pytest.mark.parametrize("bits", [4, 6])
def test_decode_codes_bit_exact_exhaustive(bits):
    """Every (code, scale byte) pair, and random rows, decode to the oracle's int8 grid bit for bit."""
    codebook = ref.default_codebook()
    ncodes = 1 << bits
    K = 16 * 256
    codes = np.tile(np.arange(ncodes), K // ncodes + 1)[:K]
    code = np.stack([np.roll(codes, 16 * s) for s in range(max(1, ncodes // 16))]).astype(np.uint32)
    scale = np.tile(np.arange(256, dtype=np.uint8), (code.shape[0], 1))
    q = ref.pack_codes(code, bits)
    got = kernels.decode_codes(dev(q), dev(scale), dev(codebook), bits).cpu().numpy()
    expect = ref.decode_codes_ref(q, scale, bits, codebook)
    finite = np.repeat((scale & 0x7F) != 0x7F, 16, axis=1)
    assert np.array_equal(got[finite], expect[finite])
    rng = np.random.default_rng(bits)
    qr = rng.integers(0, 256, size=(64, 2048 * bits // 8)).astype(np.uint8)
    sr = no_nan_fp8(rng, (64, 2048 // 16))
    got = kernels.decode_codes(dev(qr), dev(sr), dev(codebook), bits).cpu().numpy()
    assert np.array_equal(got, ref.decode_codes_ref(qr, sr, bits, codebook))


def test_decode_table_w4_bit_exact_exhaustive():
    """The resident kernels' 4-bit decode (a table per e4m3 scale byte, byte permutes) against the oracle: every
    (code, scale byte) pair in every position of a 16-code group, NaN scale bytes included (they decode as the
    per-value path decodes them), and random rows."""
    codebook = ref.default_codebook()
    K = 16 * 256
    # row s: group g holds codes (g + s + j) % 16 at its position j, so every code meets every position and scale byte
    code = np.array([[(g + s + j) % 16 for g in range(256) for j in range(16)] for s in range(16)], dtype=np.uint32)
    scale = np.tile(np.arange(256, dtype=np.uint8), (16, 1))
    q = ref.pack_codes(code, 4)
    got = kernels.decode_codes(dev(q), dev(scale), dev(codebook), 4, table=True).cpu().numpy()
    per_value = kernels.decode_codes(dev(q), dev(scale), dev(codebook), 4).cpu().numpy()
    assert np.array_equal(got, per_value)
    finite = np.repeat((scale & 0x7F) != 0x7F, 16, axis=1)
    assert np.array_equal(got[finite], ref.decode_codes_ref(q, scale, 4, codebook)[finite])
    rng = np.random.default_rng(40)
    qr = rng.integers(0, 256, size=(64, 1024)).astype(np.uint8)
    sr = no_nan_fp8(rng, (64, 2048 // 16))
    got = kernels.decode_codes(dev(qr), dev(sr), dev(codebook), 4, table=True).cpu().numpy()
    assert np.array_equal(got, ref.decode_codes_ref(qr, sr, 4, codebook))


# ------------------------------------------------------------------------------------------------------ GEMVs
def int8_bank(rng, E, N, K):
    return {"_qdata": rng.integers(-127, 128, size=(E * N, K), dtype=np.int8),
            "scale": rng.uniform(1e-3, 1e-2, size=E * N).astype(np.float32)}


def abs_sum_int8(bank, ids, x, N):
    out = []
    for j, e in enumerate(ids):
        w = np.abs(bank["_qdata"][e * N:(e + 1) * N].astype(np.float64)) * bank["scale"][e * N:(e + 1) * N, None]
        out.append(w @ np.abs(x[0 if x.shape[0] == 1 else j]))
    return np.stack(out)


@pytest.mark.parametrize("N,K,x_rows", [(1536, 2048, 1), (2048, 768, 8), (1024, 2048, 1), (2048, 512, 8)])
def test_gemv_int8_resident(N, K, x_rows):
    rng = np.random.default_rng(N + K)
    E = 8
    bank = int8_bank(rng, E, N, K)
    ids = np.array([5, 1, 7, 0, 2, 6, 3, 4])
    plan = np.stack([ids, np.zeros_like(ids)], 1).astype(np.int32)
    x = rng.standard_normal((x_rows, K)).astype(np.float32)
    took = torch.zeros(1, dtype=torch.int32, device=DEV)
    f = fields_on(bank)
    got = kernels.gemv_int8(dev(x), dev(ids), dev(plan), took, False, f, f, N)
    expect = ref.gemv_int8_ref(x, ids, plan, False, False, bank, bank, N)
    assert_dot_close(got, expect, abs_sum_int8(bank, ids, x, N))


@pytest.mark.parametrize("host_where", ["device", "pinned"])
def test_gemv_int8_slot_plan(host_where):
    """Cached, filling, slot-less and CPU experts in one launch; then the late launch for the CPU's expert."""
    rng = np.random.default_rng(3)
    E, N, K, slots = 6, 256, 512, 4
    host = int8_bank(rng, E, N, K)
    slot = {"_qdata": np.zeros((slots * N, K), np.int8), "scale": np.zeros(slots * N, np.float32)}
    slot["_qdata"][N:2 * N] = host["_qdata"][4 * N:5 * N]
    slot["scale"][N:2 * N] = host["scale"][4 * N:5 * N]
    ids = np.array([4, 2, 5, 0])
    plan = np.array([[1, 0], [2, 1], [-1, 1], [0, 2]], np.int32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    hf = fields_on(host, dev if host_where == "device" else pinned)
    sf = fields_on(slot)
    for late, took in ((False, 0), (True, 0), (True, 1)):
        slot_np = {n: v.copy() for n, v in slot.items()}
        sf = fields_on(slot_np)
        took_t = torch.full((1,), took, dtype=torch.int32, device=DEV)
        got = kernels.gemv_int8(dev(x), dev(ids), dev(plan), took_t, late, sf, hf, N)
        expect = ref.gemv_int8_ref(x, ids, plan, bool(took), late, slot_np, host, N)
        assert_dot_close(got, expect, abs_sum_int8(host, ids, x, N) + 1e-12)
        for n in slot_np:
            assert np.array_equal(sf[n].cpu().numpy(), slot_np[n]), n


def fp8_bank(rng, E, N, K):
    return {"weight": no_nan_fp8(rng, (E * N, K)),
            "scale": rng.uniform(1e-4, 1e-3, size=(E * N // 128, K // 128)).astype(np.float32)}


def abs_sum_fp8(bank, ids, x, N):
    vals = np.abs(ref.fp8_rows(bank["weight"], bank["scale"]))
    return np.stack([vals[e * N:(e + 1) * N] @ np.abs(x[0 if x.shape[0] == 1 else j]) for j, e in enumerate(ids)])


@pytest.mark.parametrize("N,K,x_rows", [(1536, 2048, 1), (2048, 768, 8)])
def test_gemv_fp8(N, K, x_rows):
    rng = np.random.default_rng(N)
    E = 8
    bank = fp8_bank(rng, E, N, K)
    ids = np.array([3, 0, 6, 1, 7, 2, 5, 4])
    plan = np.stack([ids, np.zeros_like(ids)], 1).astype(np.int32)
    x = rng.standard_normal((x_rows, K)).astype(np.float32)
    f = fields_on(bank)
    got = kernels.gemv_fp8(dev(x), dev(ids), dev(plan), f, f, N)
    expect = ref.gemv_fp8_ref(x, ids, plan, bank, bank, N)
    assert_dot_close(got, expect, abs_sum_fp8(bank, ids, x, N))


def test_gemv_fp8_fill():
    rng = np.random.default_rng(9)
    E, N, K, slots = 4, 256, 512, 3
    host = fp8_bank(rng, E, N, K)
    slot = {"weight": np.zeros((slots * N, K), np.uint8), "scale": np.zeros((slots * N // 128, K // 128), np.float32)}
    ids = np.array([3, 1])
    plan = np.array([[2, 1], [-1, 1]], np.int32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    sf, hf = fields_on(slot), fields_on(host, pinned)
    got = kernels.gemv_fp8(dev(x), dev(ids), dev(plan), sf, hf, N)
    expect = ref.gemv_fp8_ref(x, ids, plan, slot, host, N)
    assert_dot_close(got, expect, abs_sum_fp8(host, ids, x, N))
    for n in slot:
        assert np.array_equal(sf[n].cpu().numpy(), slot[n]), n


def codes_bank(rng, E, N, K, bits):
    return {"_qdata": rng.integers(0, 256, size=(E * N, K * bits // 8)).astype(np.uint8),
            "scale": rng.integers(0x20, 0x40, size=(E * N, K // 16)).astype(np.uint8),
            "s_channel": rng.uniform(1e-4, 1e-3, size=E * N).astype(np.float32)}


def abs_sum_codes(bank, ids, x, N, bits, codebook):
    q = np.abs(ref.decode_codes_ref(bank["_qdata"], bank["scale"], bits, codebook).astype(np.float64))
    q *= bank["s_channel"][:, None]
    return np.stack([q[e * N:(e + 1) * N] @ np.abs(x[0 if x.shape[0] == 1 else j]) for j, e in enumerate(ids)])


@pytest.mark.parametrize("bits", [4, 6])
@pytest.mark.parametrize("N,K,x_rows", [(1536, 2048, 1), (2048, 768, 8)])
def test_gemv_codes(bits, N, K, x_rows):
    rng = np.random.default_rng(bits * N)
    E = 8
    bank = codes_bank(rng, E, N, K, bits)
    cb = ref.default_codebook()
    ids = np.array([2, 7, 0, 5, 1, 3, 6, 4])
    plan = np.stack([ids, np.zeros_like(ids)], 1).astype(np.int32)
    x = rng.standard_normal((x_rows, K)).astype(np.float32)
    f = fields_on(bank)
    got = kernels.gemv_codes(dev(x), dev(ids), dev(plan), f, f, dev(cb) if bits == 4 else None, bits, N)
    expect = ref.gemv_codes_ref(x, ids, plan, bank, bank, cb, bits, N)
    assert_dot_close(got, expect, abs_sum_codes(bank, ids, x, N, bits, cb))


@pytest.mark.parametrize("bits", [4, 6])
def test_gemv_codes_fill(bits):
    rng = np.random.default_rng(20 + bits)
    E, N, K, slots = 4, 128, 512, 2
    host = codes_bank(rng, E, N, K, bits)
    slot = {n: np.zeros((slots * N, *v.shape[1:]), v.dtype) for n, v in host.items()}
    cb = ref.default_codebook()
    ids = np.array([3, 2])
    plan = np.array([[1, 1], [-1, 1]], np.int32)
    x = rng.standard_normal((1, K)).astype(np.float32)
    sf, hf = fields_on(slot), fields_on(host, pinned)
    got = kernels.gemv_codes(dev(x), dev(ids), dev(plan), sf, hf, dev(cb) if bits == 4 else None, bits, N)
    expect = ref.gemv_codes_ref(x, ids, plan, slot, host, cb, bits, N)
    assert_dot_close(got, expect, abs_sum_codes(host, ids, x, N, bits, cb))
    for n in slot:
        assert np.array_equal(sf[n].cpu().numpy(), slot[n]), n


# --------------------------------------------------------------------------------------------------- grouped
def _bank(kind, rng, E, N, K):
    if kind == "int8":
        return int8_bank(rng, E, N, K)
    if kind == "fp8":
        return fp8_bank(rng, E, N, K)
    return codes_bank(rng, E, N, K, int(kind[1]))


def _check_grouped(kind, rng, E, N, K, slots, groups, T, matrix):
    host = _bank(kind, rng, E, N, K)
    slot = {n: np.zeros(((slots * v.shape[0]) // E, *v.shape[1:]), v.dtype) for n, v in host.items()}
    for n, v in host.items():  # expert 2 cached in slot 0
        r = v.shape[0] // E
        slot[n][0:r] = v[2 * r:3 * r]
    cb = ref.default_codebook()
    x = rng.standard_normal((T, K)).astype(np.float32)
    sf, hf = fields_on(slot), fields_on(host)
    out = kernels._grouped({"int8": 0, "fp8": 1, "w4": 4, "w6": 6}[kind], dev(x), dev(groups), sf, hf,
                           dev(cb) if kind == "w4" else None, N, "weight" if kind == "fp8" else "_qdata", matrix)
    expect = ref.grouped_ref(kind, x, groups, slot, host, cb, N)
    if kind == "int8":
        absw = np.abs(host["_qdata"].astype(np.float64)) * host["scale"][:, None]
    elif kind == "fp8":
        absw = np.abs(ref.fp8_rows(host["weight"], host["scale"]))
    else:
        absw = np.abs(ref.decode_codes_ref(host["_qdata"], host["scale"], int(kind[1]), cb).astype(np.float64))
        absw *= host["s_channel"][:, None]
    got = out.cpu().numpy().astype(np.float64)
    for e, _, _, first, rows in groups:
        t = slice(first, first + rows)
        bound = 3e-5 * (np.abs(x[t]) @ absw[e * N:(e + 1) * N].T) + 1e-30
        assert np.all(np.abs(got[t] - expect[t]) <= bound), (kind, e)
    # the filled slots hold their experts' fields, the others are untouched
    want = {n: v.copy() for n, v in slot.items()}
    for e, s, f, _, rows in groups:
        if f:
            for n, v in host.items():
                r = v.shape[0] // E
                want[n][s * r:(s + 1) * r] = v[e * r:(e + 1) * r]
    for n in slot:
        assert np.array_equal(sf[n].cpu().numpy(), want[n]), n


@pytest.mark.parametrize("matrix", [False, True], ids=["valu", "mfma"])
@pytest.mark.parametrize("kind", ["int8", "fp8", "w4", "w6"])
def test_grouped(kind, matrix):
    """Small groups: cached, filling a slot, slot-less, empty, a slot-less one after it."""
    rng = np.random.default_rng(len(kind) + 40)
    # (expert, slot, fill, first, rows): cached, filling slot 2, slot-less, empty, cached again with fill 0
    groups = np.array([[2, 0, 0, 0, 5], [4, 2, 1, 5, 7], [1, -1, 0, 12, 3], [5, 1, 0, 15, 0], [0, -1, 0, 15, 9]],
                      np.int32)
    _check_grouped(kind, rng, 6, 256, 768, 3, groups, 24, matrix)


@pytest.mark.parametrize("N", [128, 256])
@pytest.mark.parametrize("kind", ["int8", "fp8", "w4", "w6"])
def test_grouped_mfma_many_rows(kind, N):
    """The matrix-core path over groups of 0 to 300 rows (several passes over the rows, a fill read on the first pass
    only, ragged last tiles) at K 2048, the prompt's gate_up width; N 128 runs one 16-row tile per wave, N 256 four."""
    rng = np.random.default_rng(len(kind) + 90)
    rows = [300, 1, 17, 129, 0, 64]
    first = np.concatenate([[0], np.cumsum(rows)[:-1]])
    groups = np.array([[2, 0, 0, first[0], rows[0]], [4, 2, 1, first[1], rows[1]], [3, 1, 1, first[2], rows[2]],
                       [1, -1, 0, first[3], rows[3]], [5, -1, 0, first[4], rows[4]], [0, 3, 1, first[5], rows[5]]],
                      np.int32)
    _check_grouped(kind, rng, 6, N, 2048, 4, groups, int(sum(rows)), True)

@pytest.mark.parametrize("kind", ["int8", "fp8", "w4", "w6"])
def test_grouped_rows_through_order(kind):
    """Pair p reading x's row order[p] // k through the products' `order` gives, bit for bit, what the same products
    give over a gathered copy of the rows (a row's planes and scale depend on that row alone); with the plan from
    the grouping's own launch."""
    rng = np.random.default_rng(70 + len(kind))
    E, N, K, T, k = 6, 256, 768, 40, 3
    hf = fields_on(_bank(kind, rng, E, N, K))   # groups (e, e, ..): every expert read from "slot" e
    idx = rng.integers(0, E, (T, k))
    order, inverse, groups, work = kernels.expert_groups(dev(idx.astype(np.int64)), E, plan=True)
    x = dev(rng.standard_normal((T, K)).astype(np.float32))
    cb = dev(ref.default_codebook()) if kind == "w4" else None
    P = T * k
    if kind == "fp8":
        x = x.to(torch.bfloat16)
        got = kernels.grouped_fp8_planes(x.view(1, -1), P, K, groups, work, hf, hf, N, order=order, k=k)
        want = kernels.grouped_fp8_planes(x[order // k].view(1, -1), P, K, groups, work, hf, hf, N)
    else:
        planes, scales = kernels.prep_planes_i8(x, True)
        got = kernels.grouped_i8(kind, planes, scales, P, K, groups, work, hf, hf, cb, N, order=order, k=k)
        planes, scales = kernels.prep_planes_i8(x[order // k], True)
        want = kernels.grouped_i8(kind, planes, scales, P, K, groups, work, hf, hf, cb, N)
    assert torch.equal(got, want)


@pytest.mark.parametrize("K", [256, 512, 1536])
@pytest.mark.parametrize("kind", ["int8", "w4", "w6"])
def test_grouped_i8_widths(kind, K):
    """The int8 cores at bank widths the layer does not use: N = 192 (one row tile per wave for int8 too) and the
    other supported K, against the oracle at the grouped bar."""
    rng = np.random.default_rng(len(kind) + K)
    groups = np.array([[2, 0, 0, 0, 21], [4, 2, 1, 21, 7], [1, -1, 0, 28, 40], [0, -1, 0, 68, 3]], np.int32)
    _check_grouped(kind, rng, 6, 192, K, 3, groups, 71, True)


# ---------------------------------------------------------------------------------------------- the layer
H, I, E = 2048, 768, 8


@pytest.mark.parametrize("kind, matrix, scales",
                         [(k, m, "all") for k in ("int8", "fp8", "w4", "w6") for m in (False, True)]
                         + [("w4", True, "small"), ("w6", True, "small")])
def test_grouped_decodes_exactly(kind, matrix, scales):
    """One-hot activation rows (x = [I; I], K = 256 rows per expert) make each output one weight: out[t, n] = the
    dequantized weight of row n at column t, a single product rounded once to float32, so it must equal the oracle's
    weights (the int8 grid times the row or channel scale, e4m3 times the block scale) bit for bit. Pins the decode
    (every code and scale byte the banks hold) through the grouped products, whatever the summation order. "small":
    the codes' scale bytes all within +-127 / 32, where no value reaches the clamp (a checkpoint's usual scales)."""
    rng = np.random.default_rng(len(kind) + 7)
    E, N, K = 2, 128, 256
    host = _bank(kind, rng, E, N, K)
    if kind in ("w4", "w6"):   # every finite e4m3 scale byte, tiny (all codes to 0) to huge (all clamped to +-127)
        finite = np.array([b for b in range(256) if b & 0x7F != 0x7F], np.uint8)
        if scales == "small":
            finite = finite[np.abs(numerics.e4m3_decode(finite)) <= 127 / 32]
        host["scale"] = rng.choice(finite, size=host["scale"].shape)
    x = np.concatenate([np.eye(K, dtype=np.float32)] * E)
    groups = np.array([[e, -1, 0, e * K, K] for e in range(E)], np.int32)
    cb = ref.default_codebook()
    sf = fields_on({n: np.zeros_like(v) for n, v in host.items()})
    out = kernels._grouped({"int8": 0, "fp8": 1, "w4": 4, "w6": 6}[kind], dev(x), dev(groups), sf, fields_on(host),
                           dev(cb) if kind == "w4" else None, N, "weight" if kind == "fp8" else "_qdata", matrix)
    got = out.cpu().numpy()
    if kind == "int8":
        w = host["_qdata"].astype(np.float32) * host["scale"].reshape(-1, 1)
    elif kind == "fp8":
        w = ref.fp8_rows(host["weight"], host["scale"]).astype(np.float32)
    else:
        w = ref.decode_codes_ref(host["_qdata"], host["scale"], int(kind[1]), cb).astype(np.float32)
        w = w * host["s_channel"].reshape(-1, 1).astype(np.float32)
    for e in range(E):
        want = w[e * N:(e + 1) * N].T
        assert np.array_equal(got[e * K:(e + 1) * K], want), (kind, e, int((got[e * K:(e + 1) * K] != want).sum()))


def layer_banks(kind, seed):
    rng = np.random.default_rng(seed)
    gu = rng.standard_normal((E, 2 * I, H)).astype(np.float32) * 0.02
    dn = rng.standard_normal((E, H, I)).astype(np.float32) * 0.02
    if kind == "int8":
        return (ref.quantize_int8_convrot(gu), ref.quantize_int8_convrot(dn)), (None, None)
    if kind == "fp8":
        return (ref.quantize_fp8_block(gu), ref.quantize_fp8_block(dn)), (None, None)
    (a, ca), (b, cb) = ref.quantize_codes(gu, int(kind[1])), ref.quantize_codes(dn, int(kind[1]))
    return (a, b), (ca, cb)


@pytest.fixture(scope="module", params=["int8", "fp8", "w4", "w6"])
def layer(request):
    banks, cbs = layer_banks(request.param, 70 + len(request.param))
    dbanks = [fields_on(b) for b in banks]
    dcbs = tuple(None if c is None else dev(c) for c in cbs)
    return request.param, banks, cbs, dbanks, dcbs


def test_resident_decode(layer):
    kind, banks, cbs, dbanks, dcbs = layer
    rng = np.random.default_rng(5)
    x = numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    ids = np.array([6, 2, 0, 7])
    w = numerics.bf16_round(np.array([0.4, 0.3, 0.2, 0.1], np.float32))
    got = offload.resident_decode(dev(x).view(torch.bfloat16), dev(ids), dev(w), dbanks, (2 * I, H), kind, dcbs)
    assert got.shape == (1, H) and got.dtype == torch.bfloat16
    assert_bf16_close(bits_of(got), ref.resident_decode_ref(x, ids, w, banks, (2 * I, H), kind, cbs))



@pytest.mark.parametrize("n,k,ties", [(E, 4, False), (E, 1, False), (E, 8, False), (E, 4, True), (256, 6, False),
                                      (200, 8, True)])
def test_resident_decode_routed(layer, n, k, ties):
    """Routing inside the gate_up launch: ids and weights equal kernels.route's and the oracle's route_ref, and the
    output equals route + resident_decode bitwise. With n > E the banks are padded to n experts (zeros) and the logits
    past the first E sit far below the rest, so the E real experts are the ones routed to while the launch ranks all
    n."""
    kind, banks, cbs, dbanks, dcbs = layer
    if n > E:
        dbanks = [{name: torch.cat([t, t.new_zeros((t.shape[0] // E * (n - E), *t.shape[1:]))]) for name, t in b.items()}
                  for b in dbanks]
    rng = np.random.default_rng(13 + n + k)
    x = numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    lf = rng.integers(-2, 3, n).astype(np.float32) if ties else rng.standard_normal(n).astype(np.float32)
    lf[E:] = -30.0
    logits = numerics.f32_to_bf16_bits(lf)
    xd, lg = dev(x).view(torch.bfloat16), dev(logits).view(torch.bfloat16)
    out, ids, w = offload.routed_decode(xd, lg, k, dbanks, (2 * I, H), kind, dcbs)
    rid, rw = kernels.route(lg.view(1, n), k)
    assert torch.equal(ids, rid) and torch.equal(w, rw)
    want_ids, want_w = ref.route_ref(logits, k)
    assert ids.cpu().numpy()[0].tolist() == np.asarray(want_ids).reshape(-1).tolist()
    # the device's expf against numpy's exp: within one bf16 step, as for route itself
    np.testing.assert_allclose(w.cpu().numpy()[0], np.asarray(want_w, np.float32).reshape(-1), rtol=2.0**-7, atol=0)
    want = offload.resident_decode(xd, rid[0], rw[0], dbanks, (2 * I, H), kind, dcbs)
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert_bf16_close(bits_of(out), ref.resident_decode_ref(x, ids.cpu().numpy()[0], w.cpu().numpy()[0], banks,
                                                            (2 * I, H), kind, cbs))

def test_resident_decode_routed_rejects_logits_past_the_banks(layer):
    """More logits than the banks hold experts: a routed id could index past them, so the call is refused."""
    kind, banks, cbs, dbanks, dcbs = layer
    x = torch.zeros((1, H), dtype=torch.bfloat16, device=DEV)
    lg = torch.zeros((E + 8,), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="logits for banks of"):
        offload.routed_decode(x, lg, 4, dbanks, (2 * I, H), kind, dcbs)


def test_resident_prefill(layer):
    kind, banks, cbs, dbanks, dcbs = layer
    rng = np.random.default_rng(6)
    T, k = 12, 4
    x = numerics.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)])
    w = numerics.bf16_round(rng.dirichlet(np.ones(k), T).astype(np.float32))
    got = offload.resident_prefill(dev(x).view(torch.bfloat16), dev(idx), dev(w).to(torch.bfloat16), dbanks,
                                   (2 * I, H), kind, dcbs, E)
    assert got.shape == (T, H) and got.dtype == torch.bfloat16
    assert_bf16_close(bits_of(got), ref.resident_prefill_ref(x, idx, w, banks, (2 * I, H), kind, cbs))


@pytest.mark.parametrize("T", [0, 1, 2])
def test_resident_prefill_few_rows(layer, T):
    """The prompt path at its edges: no rows (an empty [0, H] result, nothing launched past the grouping), and one or
    two rows (every group a single partial tile) against the oracle."""
    kind, banks, cbs, dbanks, dcbs = layer
    rng = np.random.default_rng(40 + T)
    k = 4
    x = numerics.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]) if T else np.zeros((0, k), np.int64)
    w = numerics.bf16_round(rng.dirichlet(np.ones(k), T).astype(np.float32)) if T else np.zeros((0, k), np.float32)
    got = offload.resident_prefill(dev(x).view(torch.bfloat16), dev(idx.astype(np.int64)), dev(w).to(torch.bfloat16),
                                   dbanks, (2 * I, H), kind, dcbs, E)
    assert got.shape == (T, H) and got.dtype == torch.bfloat16
    if T:
        assert_bf16_close(bits_of(got), ref.resident_prefill_ref(x, idx, w, banks, (2 * I, H), kind, cbs))


def test_resident_prefill_graph_replays(layer):
    """The prompt path captured in a HIP graph (grouping with its plan, planes, products, weighted sum; no host sync,
    no memset) gives the eager result bit for bit on every replay, with new rows and routing copied in between."""
    kind, banks, cbs, dbanks, dcbs = layer
    rng = np.random.default_rng(23)
    T, k = 40, 4
    inputs = [(numerics.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32)),
               np.stack([rng.choice(E, k, replace=False) for _ in range(T)]),
               numerics.bf16_round(rng.dirichlet(np.ones(k), T).astype(np.float32))) for _ in range(3)]
    x_buf = dev(inputs[0][0]).view(torch.bfloat16).clone()
    idx_buf = dev(inputs[0][1]).clone()
    w_buf = dev(inputs[0][2]).to(torch.bfloat16)
    run = lambda: offload.resident_prefill(x_buf, idx_buf, w_buf, dbanks, (2 * I, H), kind, dcbs, E)  # noqa: E731
    run()   # constants exist before capture
    stream = torch.cuda.Stream(DEV)
    stream.wait_stream(torch.cuda.current_stream(DEV))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            out = run()
    torch.cuda.current_stream(DEV).wait_stream(stream)
    for x, idx, w in inputs:
        x_buf.copy_(dev(x).view(torch.bfloat16))
        idx_buf.copy_(dev(idx))
        w_buf.copy_(dev(w).to(torch.bfloat16))
        g.replay()
        torch.cuda.synchronize()
        eager = run()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16))


def zipf_topk(rng, T, E, k, s=1.1):
    """[T, k] expert ids: per row a draw of k distinct experts without replacement from Zipf(s) over a random ranking of
    the experts (Gumbel-top-k over log p(rank), p(rank) ~ rank^-s), the prompt routing of the 256-row workload."""
    logp = np.empty(E)
    logp[rng.permutation(E)] = -s * np.log(np.arange(1, E + 1))
    g = logp - np.log(-np.log(rng.uniform(1e-12, 1 - 1e-7, (T, E))))
    return np.argsort(-g, axis=1, kind="stable")[:, :k]


@pytest.mark.parametrize("kind", ["int8", "fp8", "w4", "w6"])
def test_resident_prefill_256_rows_zipf(kind):
    """The prompt workload: 256 rows, top-8 of Zipf(1.1) routing, the layer's shape (H 2048, I 768) over 32 experts
    (random fields of each format: the oracle's dequantization of 64 experts per format would take minutes), so the
    hottest experts take well over 64 rows (several passes of the grouped products) and the coldest one or two.
    Against the oracle's resident layer, at the bf16 bar of the other layer tests."""
    rng = np.random.default_rng(300 + len(kind))
    E, T, k = 32, 256, 8
    banks = (_bank(kind, rng, E, 2 * I, H), _bank(kind, rng, E, H, I))
    cb = ref.default_codebook()
    cbs = (cb, cb) if kind == "w4" else (None, None)
    idx = zipf_topk(rng, T, E, k)
    counts = np.bincount(idx.reshape(-1), minlength=E)
    assert counts.max() > 128 and (counts > 0).sum() >= 24
    w = numerics.bf16_round(rng.dirichlet(np.ones(k), T).astype(np.float32))
    x = numerics.f32_to_bf16_bits(rng.standard_normal((T, H)).astype(np.float32))
    dbanks = [fields_on(b) for b in banks]
    dcbs = tuple(None if c is None else dev(c) for c in cbs)
    got = offload.resident_prefill(dev(x).view(torch.bfloat16), dev(idx.astype(np.int64)), dev(w).to(torch.bfloat16),
                                   dbanks, (2 * I, H), kind, dcbs, E)
    assert_bf16_close(bits_of(got), ref.resident_prefill_ref(x, idx, w, banks, (2 * I, H), kind, cbs))


def test_expert_groups_without_host_sync():
    idx = torch.tensor([[3, 1], [1, 0], [3, 3]], device=DEV)
    order, inverse, groups = offload.expert_groups(idx, 5)
    g = groups.cpu().numpy()
    assert g[:, 4].tolist() == [1, 2, 0, 3, 0] and g[:, 3].tolist() == [0, 1, 3, 3, 6]
    assert idx.reshape(-1)[order].cpu().tolist() == [0, 1, 1, 3, 3, 3]
    assert sorted(order.cpu().tolist()) == list(range(6)) and inverse[order].cpu().tolist() == list(range(6))


def check_plan(work, groups, P, rows=32):
    """work [2 + 2 cap] holds the plan of groups [g, 5] over P rows: every group with rows cut into passes (g, m0),
    m0 = 0, 32, ..; work[0] passes, the work[1] first passes (m0 = 0) listed first, each part by tiles (1 to 2 of
    16 rows), most first."""
    tiles = lambda n: (min(n, rows) + 15) // 16  # noqa: E731
    passes = [(g, m0) for g, (_, _, _, f, r) in enumerate(groups) if r > 0 and f >= 0 and f + r <= P
              for m0 in range(0, r, rows)]
    firsts = sorted(p for p in passes if p[1] == 0)
    n, nf = int(work[0]), int(work[1])
    assert n == len(passes) and nf == len(firsts)
    got = [(int(work[2 + 2 * i]), int(work[3 + 2 * i])) for i in range(n)]
    assert sorted(got[:nf]) == firsts and sorted(got[nf:]) == sorted(p for p in passes if p[1])
    for part in (got[:nf], got[nf:]):
        t = [tiles(groups[g][4] - m0) for g, m0 in part]
        assert t == sorted(t, reverse=True)


@pytest.mark.parametrize("E, T, k, zipf", [(128, 256, 8, True), (256, 2048, 8, True), (1024, 300, 4, False),
                                           (7, 1, 1, False), (64, 0, 8, False)])
def test_expert_groups_kernel(E, T, k, zipf):
    """The counting sort against numpy's stable argsort: the same groups, each group holding the same pairs (in any
    order), order and inverse each other's inverse; ids outside [0, E) after every group with inverse -1."""
    rng = np.random.default_rng(E + T)
    if zipf:
        p = np.arange(1, E + 1) ** -1.1
        idx = np.stack([rng.choice(E, k, replace=False, p=p / p.sum()) for _ in range(T)]).reshape(T, k)
    else:
        idx = rng.integers(0, E, (T, k))
    order, inverse, groups = offload.expert_groups(dev(idx.astype(np.int64)), E)
    order, inverse, g = order.cpu().numpy(), inverse.cpu().numpy(), groups.cpu().numpy()
    flat = idx.reshape(-1)
    counts = np.bincount(flat, minlength=E)
    assert g[:, 0].tolist() == list(range(E)) and g[:, 1].tolist() == list(range(E)) and not g[:, 2].any()
    assert g[:, 4].tolist() == counts.tolist() and g[:, 3].tolist() == (np.cumsum(counts) - counts).tolist()
    want = np.argsort(flat, kind="stable")
    for e in range(E):
        f, r = g[e, 3], g[e, 4]
        assert sorted(order[f:f + r].tolist()) == want[f:f + r].tolist(), e
    assert np.array_equal(inverse[order], np.arange(flat.shape[0]))
    # the plan from the same launch: what d3_grouped_plan makes of these groups, and the plan's own rule
    o2, i2, g2, work = kernels.expert_groups(dev(idx.astype(np.int64)), E, plan=True)
    assert np.array_equal(g2.cpu().numpy(), g)
    check_plan(work.cpu().numpy(), g, flat.shape[0])
    check_plan(kernels.grouped_plan(g2, flat.shape[0]).cpu().numpy(), g, flat.shape[0])
    if T:   # out-of-range ids: placed last, inverse -1
        bad = idx.copy()
        bad[0, 0], bad[-1, -1] = -3, E + 5
        order, inverse, groups = offload.expert_groups(dev(bad.astype(np.int64)), E)
        order, inverse, g = order.cpu().numpy(), inverse.cpu().numpy(), groups.cpu().numpy()
        n = flat.shape[0]
        assert sorted(order.tolist()) == list(range(n)) and g[:, 4].sum() == n - (2 if n > 1 else 1)
        assert inverse[0] == -1 and inverse[n - 1] == -1 and set(order[g[:, 4].sum():].tolist()) == {0, n - 1}


@pytest.mark.parametrize("T, dtype", [(1, torch.bfloat16), (37, torch.float32), (256, torch.bfloat16)])
def test_expert_groups_prep_i8(T, dtype):
    """The grouping and the token rows' int8 planes in one launch: the same groups, pairs, plan and planes (bit for
    bit) as d3_expert_groups and d3_prep_planes_i8 give separately."""
    rng = np.random.default_rng(T)
    E, k, K = 128, 8, 2048
    idx = dev(np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64))
    x = dev(rng.standard_normal((T, K)).astype(np.float32)).to(dtype)
    order, inverse, groups, work, planes, scales = kernels.expert_groups_prep_i8(idx, E, x, True)
    o2, i2, g2, w2 = kernels.expert_groups(idx, E, plan=True)
    g = groups.cpu().numpy()
    assert np.array_equal(g, g2.cpu().numpy())
    check_plan(work.cpu().numpy(), g, T * k)
    o, o2 = order.cpu().numpy(), o2.cpu().numpy()
    for e in range(E):
        f, r = g[e, 3], g[e, 4]
        assert sorted(o[f:f + r].tolist()) == sorted(o2[f:f + r].tolist()), e
    assert np.array_equal(inverse.cpu().numpy()[o], np.arange(T * k))
    p2, s2 = kernels.prep_planes_i8(x, True)
    assert torch.equal(planes, p2) and torch.equal(scales.view(torch.int32), s2.view(torch.int32))


def test_fp8_experts_module():
    banks, _ = layer_banks("fp8", 90)
    mod = offload.FP8Experts(E, H, I, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        for name, b in zip(("gate_up", "down"), banks):
            rows = b["weight"].shape[0] // E
            getattr(mod, f"{name}_weight").copy_(dev(b["weight"]).view(E, rows, -1).view(torch.float8_e4m3fn))
            getattr(mod, f"{name}_scale").copy_(dev(b["scale"]).view(E, rows // 128, -1))
    rng = np.random.default_rng(8)
    x = numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    idx = np.array([[1, 4, 6]])
    w = numerics.bf16_round(np.array([[0.5, 0.3, 0.2]], np.float32))
    got = mod(dev(x).view(torch.bfloat16), dev(idx), dev(w).to(torch.bfloat16))
    assert_bf16_close(bits_of(got), ref.resident_decode_ref(x, idx[0], w[0], banks, (2 * I, H), "fp8", (None, None)))


def test_resident_decode_graph_replays(layer):
    """A decode layer captured in a HIP graph gives the eager result on every replay, with new inputs in place."""
    kind, banks, cbs, dbanks, dcbs = layer
    rng = np.random.default_rng(11)
    xs = [numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32)) for _ in range(3)]
    ids_all = [rng.choice(E, 4, replace=False) for _ in range(3)]
    w = dev(numerics.bf16_round(np.full(4, 0.25, np.float32)))
    x_buf = dev(xs[0]).view(torch.bfloat16).clone()
    ids_buf = dev(ids_all[0]).clone()
    offload.resident_decode(x_buf, ids_buf, w, dbanks, (2 * I, H), kind, dcbs)  # constants exist before capture
    stream = torch.cuda.Stream(DEV)
    stream.wait_stream(torch.cuda.current_stream(DEV))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            out = offload.resident_decode(x_buf, ids_buf, w, dbanks, (2 * I, H), kind, dcbs)
    torch.cuda.current_stream(DEV).wait_stream(stream)
    for x, ids in zip(xs, ids_all):
        x_buf.copy_(dev(x).view(torch.bfloat16))
        ids_buf.copy_(dev(ids))
        g.replay()
        torch.cuda.synchronize()
        eager = offload.resident_decode(x_buf, ids_buf, w, dbanks, (2 * I, H), kind, dcbs)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


# ------------------------------------------------------------------------------ resident decode in one launch
def _same_bits(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.parametrize("block_rows", [4, 8])
@pytest.mark.parametrize("k", [1, 4, 8])
def test_resident_decode_fused(layer, k, block_rows):
    """One launch (the hidden rows handed between its workgroups) against the two launches: the same output bit for
    bit, with no wait given up, and the oracle's result within the layer bar."""
    kind, banks, cbs, dbanks, dcbs = layer
    rng = np.random.default_rng(17 + k)
    x = numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    ids = rng.choice(E, k, replace=False)
    w = numerics.bf16_round(rng.dirichlet(np.ones(k)).astype(np.float32))
    xd, idd, wd = dev(x).view(torch.bfloat16), dev(ids), dev(w)
    want = kernels.resident_decode(xd, idd, wd, dbanks, kind, dcbs, H, I)
    kernels.resident_status(DEV, I)
    got = kernels.resident_decode_fused(xd, dbanks, kind, dcbs, H, I, ids=idd, weights=wd, block_rows=block_rows)
    assert _same_bits(got, want)
    assert kernels.resident_status(DEV, I) == 0
    assert_bf16_close(bits_of(got), ref.resident_decode_ref(x, ids, w, banks, (2 * I, H), kind, cbs))


@pytest.mark.parametrize("n,k,ties", [(E, 4, False), (E, 8, True), (E, 1, False), (256, 6, False), (100, 8, True)])
def test_resident_decode_fused_routed(layer, n, k, ties):
    """The routing inside the one launch: ids, weights and output equal the two-launch routed decode's bit for bit
    (banks padded to n experts with zeros and logits past the first E far below, as in the two-launch test)."""
    kind, banks, cbs, dbanks, dcbs = layer
    if n > E:
        dbanks = [{name: torch.cat([t, t.new_zeros((t.shape[0] // E * (n - E), *t.shape[1:]))]) for name, t in b.items()}
                  for b in dbanks]
    rng = np.random.default_rng(29 + n + k)
    x = numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    lf = rng.integers(-2, 3, n).astype(np.float32) if ties else rng.standard_normal(n).astype(np.float32)
    lf[E:] = -30.0
    xd, lg = dev(x).view(torch.bfloat16), dev(numerics.f32_to_bf16_bits(lf)).view(torch.bfloat16)
    want, wid, ww = kernels.resident_decode_routed(xd, lg, k, dbanks, kind, dcbs, H, I)
    got, gid, gw = kernels.resident_decode_fused(xd, dbanks, kind, dcbs, H, I, logits=lg, k=k)
    assert torch.equal(gid, wid) and torch.equal(gw, ww)
    assert _same_bits(got, want)
    rid, rw = kernels.route(lg.view(1, n), k)
    assert torch.equal(gid, rid) and torch.equal(gw, rw)


@pytest.mark.parametrize("routed", [False, True])
def test_resident_decode_fused_recomputes_exactly(layer, routed):
    """Every wait given up at once (the test hook), and a tiny spin limit: each down workgroup computes the hidden
    rows itself, and the output is still the two launches' bit for bit; the status reports the recomputation."""
    kind, banks, cbs, dbanks, dcbs = layer
    rng = np.random.default_rng(41)
    x = numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))
    xd = dev(x).view(torch.bfloat16)
    if routed:
        lg = dev(numerics.f32_to_bf16_bits(rng.standard_normal(E).astype(np.float32))).view(torch.bfloat16)
        want = kernels.resident_decode_routed(xd, lg, 6, dbanks, kind, dcbs, H, I)
        call = dict(logits=lg, k=6)
    else:
        ids = dev(rng.choice(E, 5, replace=False))
        wts = dev(numerics.bf16_round(rng.dirichlet(np.ones(5)).astype(np.float32)))
        want = (kernels.resident_decode(xd, ids, wts, dbanks, kind, dcbs, H, I),)
        call = dict(ids=ids, weights=wts)
    kernels.resident_status(DEV, I)
    for extra in (dict(recompute_all=True), dict(spin_limit=1, block_rows=8)):
        got = kernels.resident_decode_fused(xd, dbanks, kind, dcbs, H, I, **call, **extra)
        got = got if routed else (got,)
        for a, b in zip(got, want):
            assert _same_bits(a, b) if a.dtype == torch.bfloat16 else torch.equal(a, b)
        status = kernels.resident_status(DEV, I)
        assert status == kernels.RESIDENT_RECOMPUTED if "recompute_all" in extra else status in (0, 1)


def test_resident_decode_fused_graph_replays(layer):
    """The routed one-launch decode captured in a HIP graph: every replay, with new x and logits in place, equals the
    eager two-launch result (the workspace is not cleared between replays: its words carry each launch's epoch)."""
    kind, banks, cbs, dbanks, dcbs = layer
    rng = np.random.default_rng(43)
    xs = [numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32)) for _ in range(4)]
    ls = [numerics.f32_to_bf16_bits(rng.standard_normal(E).astype(np.float32)) for _ in range(4)]
    x_buf = dev(xs[0]).view(torch.bfloat16).clone()
    l_buf = dev(ls[0]).view(torch.bfloat16).clone()
    stream = torch.cuda.Stream(DEV)
    kernels.resident_workspace(DEV, I, stream)  # before capture
    stream.wait_stream(torch.cuda.current_stream(DEV))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            out, ids, w = kernels.resident_decode_fused(x_buf, dbanks, kind, dcbs, H, I, logits=l_buf, k=4)
    torch.cuda.current_stream(DEV).wait_stream(stream)
    for x, lgt in zip(xs, ls):
        x_buf.copy_(dev(x).view(torch.bfloat16))
        l_buf.copy_(dev(lgt).view(torch.bfloat16))
        g.replay()
        torch.cuda.synchronize()
        want, wid, ww = kernels.resident_decode_routed(x_buf, l_buf, 4, dbanks, kind, dcbs, H, I)
        torch.cuda.synchronize()
        assert _same_bits(out, want) and torch.equal(ids, wid) and torch.equal(w, ww)


@pytest.mark.parametrize("kind", ["int8", "w4"])
def test_resident_decode_fused_ffn_512(kind):
    """The reference model's own layer shape (FFN 512): one launch against two, bit for bit."""
    inter = 512
    rng = np.random.default_rng(47)
    gu = rng.standard_normal((E, 2 * inter, H)).astype(np.float32) * 0.02
    dn = rng.standard_normal((E, H, inter)).astype(np.float32) * 0.02
    if kind == "int8":
        banks, cbs = (ref.quantize_int8_convrot(gu), ref.quantize_int8_convrot(dn)), (None, None)
    else:
        (a, ca), (b, cb) = ref.quantize_codes(gu, 4), ref.quantize_codes(dn, 4)
        banks, cbs = (a, b), (ca, cb)
    dbanks = [fields_on(b) for b in banks]
    dcbs = tuple(None if c is None else dev(c) for c in cbs)
    x = dev(numerics.f32_to_bf16_bits(rng.standard_normal((1, H)).astype(np.float32))).view(torch.bfloat16)
    lg = dev(numerics.f32_to_bf16_bits(rng.standard_normal(E).astype(np.float32))).view(torch.bfloat16)
    want = kernels.resident_decode_routed(x, lg, 8, dbanks, kind, dcbs, H, inter)
    for block_rows in (4, 8):
        got = kernels.resident_decode_fused(x, dbanks, kind, dcbs, H, inter, logits=lg, k=8, block_rows=block_rows)
        assert _same_bits(got[0], want[0]) and torch.equal(got[1], want[1]) and torch.equal(got[2], want[2])


@pytest.mark.parametrize("rows,N,K", [(1, 1536, 2048), (3, 1536, 2048), (1, 8 * 1536, 2048), (2, 1024, 512),
                                      (4, 64, 1536)])
def test_fp8_linear_per_row_scale(rows, N, K):
    """An FP8 weight with a bf16 scale per output row (absmax / 448) against bf16 activations, dequantized to bf16 then
    multiplied, as the CPU path runs it (offload.py:163-167, then the linear). The first case is the benchmark's single
    GEMV: x [1, 2048] ~ N(0, 1), W [1536, 2048] ~ N(0, 0.02), seed 0; the third stacks 8 experts' rows (one call for
    experts_decode's gate_up). Every output within one bf16 step of the oracle's float64 sums (the kernel sums in
    float32 in its own order), and nearly all identical."""
    bf16_bits_to_f32 = numerics.bf16_bits_to_f32
    rng = np.random.default_rng(0)
    x = numerics.f32_to_bf16_bits(rng.standard_normal((rows, K)).astype(np.float32))
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    codes, sbits = ref.quantize_fp8_rows(w)
    xt = torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV)
    wt = torch.from_numpy(codes).to(DEV)
    st = torch.from_numpy(sbits.view(np.int16)).view(torch.bfloat16).to(DEV)
    got = kernels.fp8_linear(xt, wt, st)
    assert got.shape == (rows, N) and got.dtype == torch.bfloat16
    gv = bf16_bits_to_f32(got.view(torch.int16).cpu().numpy().view(np.uint16)).astype(np.float64)
    want = bf16_bits_to_f32(ref.fp8_rows_linear_ref(x, codes, sbits)).astype(np.float64)
    # one bf16 step of v is at most 2^-7 |v| (2^(e-7) for v in [2^e, 2^(e+1)))
    assert np.all(np.abs(gv - want) <= 2.0 ** -7 * np.abs(want) + 1e-6), np.abs(gv - want).max()
    assert (gv == want).mean() >= 0.97
    # the float8 view of the weight is taken as well as its bytes
    assert torch.equal(kernels.fp8_linear(xt, wt.view(torch.float8_e4m3fn), st), got)


def test_fp8_linear_rejects_bad_shapes():
    x = torch.zeros((5, 2048), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((16, 2048), dtype=torch.uint8, device=DEV)
    s = torch.ones((16,), dtype=torch.bfloat16, device=DEV)
    with pytest.raises(RuntimeError, match="rows must be"):
        kernels.fp8_linear(x, w, s)
    with pytest.raises(RuntimeError, match="K must be"):
        kernels.fp8_linear(x[:1, :768].contiguous(), w[:, :768].contiguous(), s)
