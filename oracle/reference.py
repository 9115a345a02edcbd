"""Oracle for the reference's own expert kernels and formats (test infrastructure only): drama3/kernels.py's SOURCE
and drama3/offload.py's resident decode / prefill, restated in numpy (float64 sums unless a step is exact in float32).

Only tests/, __graft_entry__.smoke() and bench.py's CPU leg import this, to check results. Every function cites the
reference lines it follows. What pins each one (tests/test_oracle_reference.py):
  e4m3_ref         exhaustive over 256 codes against OCP e4m3fn (torch.float8_e4m3fn) except the NaN codes, which the
                   reference's bit placement reads as +-480 (checked as such)
  route_ref        brute force ranking, ties to the lower index, against a sort; weights against the closed form
  rotate_ref       dense H256 (symmetric, orthogonal) and the butterfly network of kernels.py:241-255 built by hand
  decode_codes_ref exhaustive: every (code, e4m3 scale byte) pair at 4 and 6 bits against the formula, plus the byte /
                   bit-plane layout by planting single codes
  gemv_*_ref       brute-force float64 dot products of the decoded rows; plan / fill / late / took_over semantics on
                   hand-built cases
  fp8_rows_*       the dequantized matrix bit for bit against torch's float8 decode, product and bf16 cast; the
                   linear against torch's bf16 linear on the CPU (within one bf16 step) and an unquantized float64
                   product (within the format's error); a planted transposed scale must fail
  grouped_ref      equal to gemv_*_ref row by row
  resident_*_ref   against an unquantized float64 layer within the formats' quantization error, and a planted
                   gate / up swap that must fail
The quantizers (quantize_int8_convrot, quantize_fp8_block, quantize_codes) make synthetic banks in the reference's
layouts; the reference's own quantizers live in comfy_kitchen, which is not available, so their exact rounding
choices (codebook fitting, scale derivation) are not restated: parity unpinned at that boundary, and no kernel
depends on it (the kernels read whatever bytes a bank holds).
"""
import numpy as np

from .numerics import bf16_bits_to_f32, e4m3_encode, f32_to_bf16_bits, hadamard

ROWS_PER_BLOCK = 16   # kernels.py:590
FP8_BLOCK = 128       # offload.py:36
GROUP = 16            # W4A8 / W6A8 scale group (offload.py:82)
ROT = 256             # ConvRot group (offload.py:80,82)


# ---------------------------------------------------------------------------------------------------------- numerics
def e4m3_ref(codes):
    """kernels.py:25-29: the 7 magnitude bits placed in a float's exponent and mantissa, times 2^120. Exact for every
    code, subnormals included; the NaN codes 0x7F / 0xFF read +-480."""
    c = np.asarray(codes, dtype=np.uint32)
    bits = (((c & 0x80) << 24) | ((c & 0x7F) << 20)).astype(np.uint32)
    return bits.view(np.float32).astype(np.float64) * 2.0 ** 120


def silu(g):
    return g / (1.0 + np.exp(-g))


# ------------------------------------------------------------------------------------------------------------ route
def route_ref(logits_bits, k):
    """kernels.py:39-67 route_experts, per row: the k largest bf16 logits by rank (value, then lower index first);
    weights exp(l - l_max) / sum over the k, in float32, rounded to bf16. Returns ids [rows, k] int64, weights
    [rows, k] float32."""
    v = bf16_bits_to_f32(np.atleast_2d(logits_bits))
    rows, n = v.shape
    ids = np.zeros((rows, k), dtype=np.int64)
    weights = np.zeros((rows, k), dtype=np.float32)
    for r in range(rows):
        rank = np.array([np.sum((v[r] > v[r, i]) | ((v[r] == v[r, i]) & (np.arange(n) < i))) for i in range(n)])
        order = np.argsort(rank)[:k]
        top = v[r, order].astype(np.float32)
        total = np.float32(0)
        for e in range(k):
            total = np.float32(total + np.exp(np.float32(top[e] - top[0])))
        w = (np.exp((top - top[0]).astype(np.float32)) / total).astype(np.float32)
        ids[r] = order
        weights[r] = bf16_bits_to_f32(f32_to_bf16_bits(w))
    return ids, weights


# ----------------------------------------------------------------------------------------------------- weighted sum
def weighted_sum_ref(parts, weights):
    """kernels.py:69-76: out[h] = bf16(sum_e parts[e, h] * weights[e]) -> bf16 bits [1, H] (sum in float64)."""
    acc = (np.asarray(parts, np.float64) * np.asarray(weights, np.float64)[:, None]).sum(0)
    return f32_to_bf16_bits(acc.astype(np.float32))[None, :]


# ----------------------------------------------------------------------------------------------------------- rotate
def rotate_ref(x, swiglu=False):
    """kernels.py:222-258 rotate_rows: rows of x (float; with swiglu [rows, 2K] gate | up, SiLU(gate) * up first)
    times H256 on every 256 columns (H symmetric: row @ H)."""
    x = np.asarray(x, np.float64)
    if swiglu:
        K = x.shape[1] // 2
        x = silu(x[:, :K]) * x[:, K:]
    rows, K = x.shape
    return (x.reshape(rows, K // ROT, ROT) @ hadamard(ROT)).reshape(rows, K)


# ---------------------------------------------------------------------------------------------------- code decoding
def decode_codes_ref(qdata, scale, bits, codebook=None):
    """kernels.py:466-483 decode_codes for whole rows: qdata [R, K * bits / 8] (K/2 nibble bytes, byte b = columns 2b
    (low) and 2b + 1 (high); at 6 bits then K/4 bytes of 2-bit high planes, a little-endian u32 per 16 columns, column
    j at bits 2j), scale [R, K / 16] e4m3 bytes -> int8 [R, K]: clamp(rint(value * scale), +-127) in float32, value =
    codebook[code] (4 bits) or code - 32 (6 bits)."""
    qdata = np.asarray(qdata, np.uint8)
    R = qdata.shape[0]
    K = qdata.shape[1] * 8 // bits
    lo = qdata[:, :K // 2]
    code = np.empty((R, K), np.int32)
    code[:, 0::2] = lo & 0xF
    code[:, 1::2] = lo >> 4
    if bits == 6:
        hi = qdata[:, K // 2:K // 2 + K // 4]
        two = np.stack([(hi >> s) & 3 for s in (0, 2, 4, 6)], axis=-1).reshape(R, K)  # byte i -> columns 4i..4i+3
        code |= two.astype(np.int32) << 4
        value = (code - 32).astype(np.float32)
    else:
        value = np.asarray(codebook, np.float32)[code]
    s = np.repeat(e4m3_ref(scale).astype(np.float32), GROUP, axis=1)
    return np.clip(np.rint((value * s).astype(np.float32)), -127, 127).astype(np.int8)


# -------------------------------------------------------------------------------------------------- decode GEMVs
def _source(fields, slot_fields, plan, e, id_, host, rows, name):
    """Expert e's tensor `name` [rows, ...]: from the host bank (expert id_) or its slot (kernels.py:290-292)."""
    if host:
        return fields[name][id_ * rows:(id_ + 1) * rows]
    slot = plan[e, 0]
    return slot_fields[name][slot * rows:(slot + 1) * rows]


def _fill(slot_fields, plan, e, rows, values):
    slot = plan[e, 0]
    for name, v in values.items():
        slot_fields[name][slot * rows:(slot + 1) * rows] = v


def gemv_int8_ref(x, ids, plan, took_over, late, slot_fields, host_fields, n):
    """kernels.py:260-314 gemv_int8: out [k, n] = (int8 row . x[e or 0]) * row scale. plan[e] = (slot, code): code 0
    reads the slot, 1 the host bank and fills the slot when it has one, 2 gives zeros; with `late` only code 2 runs
    (from the host bank) and only if took_over, the rest give zeros. Slot fields are updated in place."""
    x = np.asarray(x, np.float64)
    plan = np.asarray(plan).reshape(-1, 2)
    k = len(ids)
    out = np.zeros((k, n))
    for e in range(k):
        code = plan[e, 1]
        if (code != 2 or not took_over) if late else code == 2:
            continue
        q = _source(host_fields, slot_fields, plan, e, ids[e], code != 0, n, "_qdata").astype(np.float64)
        s = _source(host_fields, slot_fields, plan, e, ids[e], code != 0, n, "scale").reshape(n).astype(np.float64)
        xr = x[0 if x.shape[0] == 1 else e]
        out[e] = (q @ xr) * s
        if code == 1 and plan[e, 0] >= 0:
            _fill(slot_fields, plan, e, n, {"_qdata": q.astype(np.int8), "scale": s.astype(np.float32).reshape(-1, *slot_fields["scale"].shape[1:])})
    return out


def fp8_rows(weight, scale):
    """Float8 rows [R, C] with 128 x 128 block scales [R / 128, C / 128] -> float64 values (offload.py:163-167, with
    kernels.py's decode)."""
    R, C = weight.shape
    return e4m3_ref(weight) * np.repeat(np.repeat(np.asarray(scale, np.float64), FP8_BLOCK, 0), FP8_BLOCK, 1)[:R, :C]


def quantize_fp8_rows(w):
    """Float weights [N, K] -> (e4m3 codes [N, K], bf16 scale bits [N]) with one scale per output row, absmax / 448
    rounded to bf16, codes = e4m3(w / scale) (round to nearest even)."""
    w = np.asarray(w, dtype=np.float32)
    sbits = f32_to_bf16_bits(np.abs(w).max(axis=1) / np.float32(448.0))
    s = bf16_bits_to_f32(sbits)
    s = np.where(s == 0, np.float32(1), s).astype(np.float32)
    return e4m3_encode((w / s[:, None]).astype(np.float32)), f32_to_bf16_bits(s)


def fp8_rows_dequant(codes, scale_bits):
    """The dequantized weight the CPU path multiplies with, as bf16 values (float32 [N, K]): e4m3(code) * scale, each
    product (exact in float32) rounded to bf16 (offload.py:163-167's .to(dtype), the scale per row)."""
    s = bf16_bits_to_f32(scale_bits).astype(np.float32)
    v = (e4m3_ref(codes).astype(np.float32) * s[:, None]).astype(np.float32)
    return bf16_bits_to_f32(f32_to_bf16_bits(v))


def fp8_rows_linear_ref(x_bits, codes, scale_bits):
    """nn.functional.linear(x, dequantized weight) in bf16 for x [rows, K] (bf16 bits): float64 sums of the bf16
    inputs, one rounding to bf16 (the CPU's bf16 matmul sums in float32, so within one bf16 step of this).
    Returns bf16 bits [rows, N]."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    wd = fp8_rows_dequant(codes, scale_bits).astype(np.float64)
    return f32_to_bf16_bits((x @ wd.T).astype(np.float32))


def gemv_fp8_ref(x, ids, plan, slot_fields, host_fields, n):
    """kernels.py:316-363 gemv_fp8: out [k, n] = sum over columns of e4m3(W) * x * block scale; plan code != 0 reads
    the host bank (and fills the slot when it has one)."""
    x = np.asarray(x, np.float64)
    plan = np.asarray(plan).reshape(-1, 2)
    k = len(ids)
    out = np.zeros((k, n))
    for e in range(k):
        host = plan[e, 1] != 0
        w = _source(host_fields, slot_fields, plan, e, ids[e], host, n, "weight")
        sr = n // FP8_BLOCK
        s = _source(host_fields, slot_fields, plan, e, ids[e], host, sr, "scale")
        out[e] = fp8_rows(w, s) @ x[0 if x.shape[0] == 1 else e]
        if host and plan[e, 0] >= 0:
            _fill(slot_fields, plan, e, n, {"weight": w.copy()})
            _fill(slot_fields, plan, e, sr, {"scale": s.copy()})
    return out


def gemv_codes_ref(x, ids, plan, slot_fields, host_fields, codebook, bits, n):
    """kernels.py:495-536 gemv_codes: out [k, n] = (decoded int8-grid row . x) * s_channel; plan code != 0 reads the
    host bank (and fills the slot when it has one)."""
    x = np.asarray(x, np.float64)
    plan = np.asarray(plan).reshape(-1, 2)
    k = len(ids)
    out = np.zeros((k, n))
    for e in range(k):
        host = plan[e, 1] != 0
        f = {name: _source(host_fields, slot_fields, plan, e, ids[e], host, n, name) for name in ("_qdata", "scale", "s_channel")}
        q = decode_codes_ref(f["_qdata"], f["scale"], bits, codebook).astype(np.float64)
        out[e] = (q @ x[0 if x.shape[0] == 1 else e]) * f["s_channel"].reshape(n)
        if host and plan[e, 0] >= 0:
            _fill(slot_fields, plan, e, n, {name: v.copy() for name, v in f.items()})
    return out


def grouped_ref(kind, x, groups, slot_fields, host_fields, codebook, n):
    """kernels.py:365-464,538-587 grouped_int8 / grouped_fp8 / grouped_codes: group (expert, slot, fill, first, rows)
    reads its slot, or the host bank when it has no slot or fills it (copying it in); out [T, n] rows of the groups
    (others NaN: the kernels leave them unset)."""
    x = np.asarray(x, np.float64)
    out = np.full((x.shape[0], n), np.nan)
    for expert, slot, fill, first, rows in np.asarray(groups).reshape(-1, 5):
        host = slot < 0 or fill
        plan = np.array([[slot, 1 if host else 0]])
        xs = x[first:first + rows]
        if kind == "int8":
            names = ("_qdata", "scale")
        elif kind == "fp8":
            names = ("weight", "scale")
        else:
            names = ("_qdata", "scale", "s_channel")
        f = {}
        for name in names:
            r = n // FP8_BLOCK if (kind == "fp8" and name == "scale") else n
            f[name] = _source(host_fields, slot_fields, plan, 0, expert, host, r, name)
        if kind == "int8":
            w = f["_qdata"].astype(np.float64) * f["scale"].reshape(n, 1)
        elif kind == "fp8":
            w = fp8_rows(f["weight"], f["scale"])
        else:
            w = decode_codes_ref(f["_qdata"], f["scale"], int(kind[1]), codebook).astype(np.float64) * f["s_channel"].reshape(n, 1)
        out[first:first + rows] = xs @ w.T
        if fill:
            for name, v in f.items():
                r = n // FP8_BLOCK if (kind == "fp8" and name == "scale") else n
                slot_fields[name][slot * r:(slot + 1) * r] = v
    return out


def _gemv(kind, x, ids, plan, fields, n, codebook):
    if kind == "int8":
        return gemv_int8_ref(x, ids, plan, False, False, fields, fields, n)
    if kind == "fp8":
        return gemv_fp8_ref(x, ids, plan, fields, fields, n)
    return gemv_codes_ref(x, ids, plan, fields, fields, codebook, int(kind[1]), n)


# ------------------------------------------------------------------------------------------------------ the layer
def resident_decode_ref(x_bits, ids, weights, banks, rows, kind, codebooks):
    """offload.py:108-123 resident_decode: one bf16 row x [1, H] through experts ids [k] of banks held whole (expert e
    in slot e): fp8 -> gemv, SiLU(gate) * up, gemv; int8 / w4 / w6 -> rotate, gemv, rotate(swiglu), gemv; then the
    weighted sum -> bf16 bits [1, H]."""
    ids = np.asarray(ids)
    plan = np.stack([ids, np.zeros_like(ids)], -1).astype(np.int32)
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    (gate_up, down), (gu_rows, dn_rows) = banks, rows
    if kind == "fp8":
        gu = _gemv(kind, x, ids, plan, gate_up, gu_rows, None)
        I = gu_rows // 2
        out = _gemv(kind, silu(gu[:, :I]) * gu[:, I:], ids, plan, down, dn_rows, None)
    else:
        gu = _gemv(kind, rotate_ref(x), ids, plan, gate_up, gu_rows, codebooks[0])
        out = _gemv(kind, rotate_ref(gu, swiglu=True), ids, plan, down, dn_rows, codebooks[1])
    return weighted_sum_ref(out, weights)


def resident_prefill_ref(x_bits, topk_idx, topk_weight, banks, rows, kind, codebooks):
    """offload.py:126-149 resident_prefill: rows x [T, H] (bf16 bits) through their top-k experts, each product scaled
    by its weight and summed over k in k's order -> bf16 bits [T, H]. Each expert's rows go through it together (one
    float64 matrix product per bank), each pair's row as resident_decode_ref computes it."""
    topk_idx = np.asarray(topk_idx)
    T, k = topk_idx.shape
    (gate_up, down), (gu_rows, dn_rows) = banks, rows
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    xin = x if kind == "fp8" else rotate_ref(x)
    w = np.asarray(topk_weight, np.float64)
    pairs = np.zeros((T, k, dn_rows))
    I = gu_rows // 2
    for e in np.unique(topk_idx):
        ts, js = np.nonzero(topk_idx == e)
        wg = expert_rows(kind, gate_up, int(e), gu_rows, codebooks[0])
        wd = expert_rows(kind, down, int(e), dn_rows, codebooks[1])
        gu = xin[ts] @ wg.T
        h = silu(gu[:, :I]) * gu[:, I:]
        if kind != "fp8":
            h = rotate_ref(h)
        pairs[ts, js] = h @ wd.T
    out = np.zeros((T, dn_rows))
    for j in range(k):
        out += pairs[:, j] * w[:, j:j + 1]
    return f32_to_bf16_bits(out.astype(np.float32))


def expert_rows(kind, fields, e, rows, codebook):
    """Float64 rows [rows, K] of expert e of a bank (what the GEMVs multiply x by, scales applied)."""
    if kind == "fp8":
        sr = rows // FP8_BLOCK
        return fp8_rows(fields["weight"][e * rows:(e + 1) * rows], fields["scale"][e * sr:(e + 1) * sr])
    return dequantize_bank(kind, {n: v[e * rows:(e + 1) * rows] for n, v in fields.items()}, codebook)


# ------------------------------------------------------------------------------------ synthetic banks (quantizers)
def convrot(w):
    """Weights [..., K] into the ConvRot basis: W H per 256 columns, so that (W H)(H x) = W x."""
    w = np.asarray(w, np.float64)
    K = w.shape[-1]
    return (w.reshape(*w.shape[:-1], K // ROT, ROT) @ hadamard(ROT)).reshape(w.shape)


def quantize_int8_convrot(w):
    """[E, N, K] float -> {"_qdata": int8 [E * N, K], "scale": float32 [E * N]}: rows in the ConvRot basis, symmetric
    per-row absmax / 127."""
    E, N, K = w.shape
    wr = convrot(w).reshape(E * N, K)
    s = (np.abs(wr).max(1) / 127.0).astype(np.float32)
    s = np.where(s > 0, s, np.float32(1))
    q = np.clip(np.rint(wr / s[:, None]), -127, 127).astype(np.int8)
    return {"_qdata": q, "scale": s}


def quantize_fp8_block(w):
    """[E, N, K] float -> {"weight": e4m3 bytes [E * N, K], "scale": float32 [E * N / 128, K / 128]}, one absmax / 448
    scale per 128 x 128 block (offload.py:163-167 layout)."""
    E, N, K = w.shape
    wb = np.asarray(w, np.float64).reshape(E * N // FP8_BLOCK, FP8_BLOCK, K // FP8_BLOCK, FP8_BLOCK)
    s = (np.abs(wb).max(axis=(1, 3)) / 448.0).astype(np.float32)
    s = np.where(s > 0, s, np.float32(1))
    codes = e4m3_encode((wb / s[:, None, :, None]).astype(np.float32)).reshape(E * N, K)
    return {"weight": codes, "scale": s}


def default_codebook():
    """A 16-entry codebook for synthetic W4A8 banks: normal quantiles scaled to +-8 (the reference fits its own per
    bank; any float table exercises the decode)."""
    from scipy.special import ndtri
    c = ndtri((np.arange(16) + 0.5) / 16)
    return (c / np.abs(c).max() * 8.0).astype(np.float32)


def pack_codes(code, bits):
    """codes [R, K] (0..15 or 0..63) -> qdata [R, K * bits / 8]: nibble plane, then (6 bits) 2-bit high planes."""
    code = np.asarray(code, np.uint32)
    R, K = code.shape
    lo = ((code[:, 0::2] & 0xF) | ((code[:, 1::2] & 0xF) << 4)).astype(np.uint8)
    if bits == 4:
        return lo
    two = ((code >> 4) & 3).reshape(R, K // 4, 4)
    hi = (two[..., 0] | (two[..., 1] << 2) | (two[..., 2] << 4) | (two[..., 3] << 6)).astype(np.uint8)
    return np.concatenate([lo, hi], axis=1)


def quantize_codes(w, bits, codebook=None):
    """[E, N, K] float -> ({"_qdata", "scale" (e4m3 per 16 columns), "s_channel" (float32 per row)}, codebook): rows in
    the ConvRot basis; s_channel = absmax / 127 puts a row on the int8 grid, each 16-column group gets an e4m3 scale
    and codes (nearest codebook entry at 4 bits, rint to -32..31 at 6 bits)."""
    E, N, K = w.shape
    wr = convrot(w).reshape(E * N, K)
    sc = (np.abs(wr).max(1) / 127.0).astype(np.float32)
    sc = np.where(sc > 0, sc, np.float32(1))
    t = wr / sc[:, None]
    tg = t.reshape(E * N, K // GROUP, GROUP)
    gmax = np.abs(tg).max(2)
    if bits == 4:
        codebook = default_codebook() if codebook is None else np.asarray(codebook, np.float32)
        sbyte = e4m3_encode((gmax / np.abs(codebook).max()).astype(np.float32))
        s = e4m3_ref(sbyte)[..., None]
        # nearest codebook entry of t / s (the codebook ascending: compare against the midpoints)
        order = np.argsort(codebook)
        mids = (codebook[order][1:].astype(np.float64) + codebook[order][:-1]) / 2
        with np.errstate(divide="ignore", invalid="ignore"):
            u = np.where(s > 0, tg / s, 0.0)
        code = order[np.searchsorted(mids, u)]
    else:
        sbyte = e4m3_encode((gmax / 31.0).astype(np.float32))
        s = e4m3_ref(sbyte)[..., None]
        with np.errstate(divide="ignore", invalid="ignore"):
            code = np.where(s > 0, np.clip(np.rint(tg / s), -32, 31), 0) + 32
    code = code.reshape(E * N, K).astype(np.uint32)
    fields = {"_qdata": pack_codes(code, bits), "scale": sbyte.reshape(E * N, K // GROUP), "s_channel": sc}
    return fields, (codebook if bits == 4 else None)


def dequantize_bank(kind, fields, codebook=None):
    """Float64 rows [E * N, K] of a bank in the ConvRot basis (int8 / codes) or plain (fp8)."""
    if kind == "int8":
        return fields["_qdata"].astype(np.float64) * fields["scale"].reshape(-1, 1)
    if kind == "fp8":
        return fp8_rows(fields["weight"], fields["scale"])
    return decode_codes_ref(fields["_qdata"], fields["scale"], int(kind[1]), codebook).astype(np.float64) * fields["s_channel"].reshape(-1, 1)
