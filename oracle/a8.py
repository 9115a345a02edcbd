"""Oracle of the fused A8 MoE layer (test infrastructure only): numpy restatement of what d3_moe_a8 computes.

Semantics restated (file:line into the reference where it defines them):
  routing        top-k of the bf16 logits by descending value, ties to the lower index; weights exp(l_i - l_0) /
                 sum_k exp(l_j - l_0), rounded to bf16 (drama3/kernels.py:39-67 route_experts)
  activations    per row: s = absmax / Q, q = rint(x * (Q / absmax)) (int8, Q = 127, clamp +-127) or e4m3(x * (Q /
                 absmax)) (F8, Q = 448); float32 arithmetic, as the kernel does it
  weights        the banks of drama3/formats.py (I8, W4, W6, F8), restated here independently
  expert         gate_up rows [2I, H] (gate first, then up: the split kernels.py:233-236 and offload.py:115 use),
                 h = SiLU(g) * u with g, u dequantized, then down rows [H, I] against h quantized per (expert, row)
  combine        out = bf16(sum_j w_j * part_j), j in routing order (kernels.py:69-76 weighted_sum)
Integer dot products are exact (int64); everything else is float64 until the final bf16 rounding, so the kernels'
float results match within a tolerance and their int32 sums and codes match exactly.
"""
import numpy as np

from .numerics import bf16_bits_to_f32, bf16_round, e4m3_decode, e4m3_encode, f32_to_bf16_bits

FMT_I8, FMT_W4, FMT_W6, FMT_F8 = 0, 1, 2, 3
GROUP = 128


def row_bytes(fmt, cols):
    return cols // 2 if fmt == FMT_W4 else cols * 3 // 4 if fmt == FMT_W6 else cols


# ---------------------------------------------------------------------------------------------------------- routing
def route(logits_bits, k):
    """logits [M, E] bf16 bits -> (ids [M, k] int64, weights [M, k] float32)."""
    v = bf16_bits_to_f32(logits_bits).astype(np.float64)
    M, E = v.shape
    ids = np.zeros((M, k), dtype=np.int64)
    w = np.zeros((M, k), dtype=np.float32)
    for m in range(M):
        order = sorted(range(E), key=lambda e: (-v[m, e], e))[:k]
        top = v[m, order]
        ex = np.exp(top - top[0])
        ids[m] = order
        w[m] = bf16_round((ex / ex.sum()).astype(np.float32))
    return ids, w


# ----------------------------------------------------------------------------------------------------- activations
def quantize_act(x, fmt):
    """x [M, K] float32 -> (codes [M, K] (int8, or e4m3 uint8 for F8), scale [M] float32)."""
    x = np.asarray(x, dtype=np.float32)
    qmax = np.float32(448.0 if fmt == FMT_F8 else 127.0)
    amax = np.abs(x).max(axis=1).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(amax > 0, qmax / amax, np.float32(0)).astype(np.float32)
    scaled = (x * inv[:, None]).astype(np.float32)
    if fmt == FMT_F8:
        q = e4m3_encode(scaled)
    else:
        q = np.clip(np.rint(scaled), -127, 127).astype(np.int8)
    return q, (amax / qmax).astype(np.float32)


def act_values(q, fmt):
    return e4m3_decode(q).astype(np.float64) if fmt == FMT_F8 else q.astype(np.float64)


# ---------------------------------------------------------------------------------------------------------- weights
def quantize_weights(w, fmt):
    """Float weights [R, K] -> (packed uint8 [R, row_bytes], scale bf16 bits [R] or [R, K / 128])."""
    w = np.asarray(w, dtype=np.float32)
    R, K = w.shape
    if fmt in (FMT_I8, FMT_F8):
        qmax = np.float32(127.0 if fmt == FMT_I8 else 448.0)
        sbits = f32_to_bf16_bits(np.abs(w).max(axis=1) / qmax)
        s = bf16_bits_to_f32(sbits)
        s = np.where(s == 0, np.float32(1), s).astype(np.float32)
        sbits = f32_to_bf16_bits(s)
        v = (w / s[:, None]).astype(np.float32)
        if fmt == FMT_I8:
            return np.clip(np.rint(v), -127, 127).astype(np.int8).view(np.uint8), sbits
        return e4m3_encode(v), sbits
    lo, hi = (-8, 7) if fmt == FMT_W4 else (-32, 31)
    g = w.reshape(R, K // GROUP, GROUP)
    s = bf16_bits_to_f32(f32_to_bf16_bits(np.abs(g).max(axis=2) / np.float32(hi)))
    s = np.where(s == 0, np.float32(1), s).astype(np.float32)
    q = np.clip(np.rint((g / s[..., None]).astype(np.float32)), lo, hi).astype(np.int32).reshape(R, K)
    return (pack_w4(q) if fmt == FMT_W4 else pack_w6(q)), f32_to_bf16_bits(s)


def pack_w4(q):
    """codes [R, K] in [-8, 7] -> bytes [R, K / 2]: byte b holds column 2b (low nibble) and 2b + 1 (high)."""
    n = (np.asarray(q) & 0xF).astype(np.uint8)
    return (n[:, 0::2] | (n[:, 1::2] << 4)).astype(np.uint8)


def unpack_w4(b):
    b = np.asarray(b, dtype=np.uint8)
    out = np.empty((b.shape[0], b.shape[1] * 2), dtype=np.int32)
    out[:, 0::2] = b & 0xF
    out[:, 1::2] = b >> 4
    return np.where(out >= 8, out - 16, out).astype(np.int8)


def pack_w6(q):
    """codes [R, K] in [-32, 31] -> bytes [R, 3K / 4]; per 16 columns a 12-byte unit: byte i = (q_i & 63) |
    (((q_{12 + i % 4} & 63) >> (2 * (i // 4))) & 3) << 6."""
    c = (np.asarray(q) & 63).astype(np.uint32)
    R, K = c.shape
    u = c.reshape(R, K // 16, 16)
    out = np.empty((R, K // 16, 12), dtype=np.uint32)
    for i in range(12):
        out[..., i] = u[..., i] | (((u[..., 12 + i % 4] >> (2 * (i // 4))) & 3) << 6)
    return out.astype(np.uint8).reshape(R, K * 3 // 4)


def unpack_w6(b):
    b = np.asarray(b, dtype=np.uint8).astype(np.uint32)
    R, n = b.shape
    u = b.reshape(R, n // 12, 12)
    out = np.empty((R, n // 12, 16), dtype=np.int32)
    out[..., :12] = u & 63
    for m in range(4):
        out[..., 12 + m] = ((u[..., m] >> 6) & 3) | (((u[..., m + 4] >> 6) & 3) << 2) | (((u[..., m + 8] >> 6) & 3) << 4)
    out = np.where(out >= 32, out - 64, out)
    return out.astype(np.int8).reshape(R, n // 12 * 16)


def codes(packed, fmt):
    """Integer codes [R, K] (int8) of packed rows; e4m3 bytes for F8."""
    if fmt == FMT_W4:
        return unpack_w4(packed)
    if fmt == FMT_W6:
        return unpack_w6(packed)
    return np.asarray(packed, dtype=np.uint8).view(np.int8) if fmt == FMT_I8 else np.asarray(packed, dtype=np.uint8)


def dequantize(packed, scale_bits, fmt):
    """Float64 weights [R, K]."""
    if fmt == FMT_F8:
        return e4m3_decode(packed).astype(np.float64) * bf16_bits_to_f32(scale_bits).astype(np.float64)[:, None]
    q = codes(packed, fmt).astype(np.float64)
    s = bf16_bits_to_f32(scale_bits).astype(np.float64)
    if fmt == FMT_I8:
        return q * s[:, None]
    R, K = q.shape
    return (q.reshape(R, K // GROUP, GROUP) * s[..., None]).reshape(R, K)


# ------------------------------------------------------------------------------------------------------------- dots
def group_dots(packed, fmt, act):
    """Per 128-column group dot products of packed rows [R, row_bytes] with activation codes act [C, K]:
    [R, K / 128, C], int64 (I8, W4, W6) or float64 (F8, e4m3 x e4m3), exact either way: the sums run in float64
    (a matrix product per group), which holds them without rounding (int8 x int8 x 128 terms < 2^22; e4m3 products
    are multiples of 2^-18 below 2^18, 128 of them fit 43 bits), so any order of summation gives the same value."""
    w = codes(packed, fmt)
    R, K = w.shape
    C = act.shape[0]
    G = K // GROUP
    if fmt == FMT_F8:
        wv = e4m3_decode(w).astype(np.float64)
        av = e4m3_decode(act).astype(np.float64)
    else:
        wv = w.astype(np.float64)
        av = np.asarray(act).astype(np.float64)
    wv = wv.reshape(R, G, GROUP).transpose(1, 0, 2)   # [G, R, 128]
    av = av.reshape(C, G, GROUP).transpose(1, 2, 0)   # [G, 128, C]
    dots = np.matmul(wv, av).transpose(1, 0, 2)       # [R, G, C]
    return dots if fmt == FMT_F8 else np.rint(dots).astype(np.int64)


def project(packed, scale_bits, fmt, act_codes, act_scale):
    """Rows [R] of a bank against quantized activations [C, K] -> float64 [C, R]: per-group sums scaled by the group
    scale (W4, W6) or the row scale (I8, F8), times the activation scale."""
    dots = group_dots(packed, fmt, act_codes).astype(np.float64)  # [R, G, C]
    s = bf16_bits_to_f32(scale_bits).astype(np.float64)
    if fmt in (FMT_W4, FMT_W6):
        y = np.einsum("rgc,rg->cr", dots, s)
    else:
        y = dots.sum(axis=1).T * s[None, :]
    return y * np.asarray(act_scale, dtype=np.float64)[:, None]


# ------------------------------------------------------------------------------------------------------------ layer
def expert_output(xq, xs, gu, dn, fmt, I):
    """One expert on one row's quantized activations (xq [1, H] codes, xs [1] scale): gate_up, SiLU(gate) * up, the
    hidden row quantized per row, down. gu / dn = (packed rows, scale bits). Returns (out float64 [H], hidden [I])."""
    y = project(gu[0], gu[1], fmt, xq, xs)[0]  # [2I]
    g, u = y[:I], y[I:]
    h = g / (1.0 + np.exp(-g)) * u
    hq, hs = quantize_act(h.astype(np.float32)[None, :], fmt)
    return project(dn[0], dn[1], fmt, hq, hs)[0], h


def experts_output(xq, xs, gu, dn, fmt, I):
    """expert_output for C rows of one expert at once (xq [C, H], xs [C]): (out float64 [C, H], hidden [C, I]). Every
    row's values are those expert_output gives it: the sums are exact and the rest is per row."""
    y = project(gu[0], gu[1], fmt, xq, xs)  # [C, 2I]
    g, u = y[:, :I], y[:, I:]
    h = g / (1.0 + np.exp(-g)) * u
    hq, hs = quantize_act(h.astype(np.float32), fmt)
    return project(dn[0], dn[1], fmt, hq, hs), h


def moe_layer(x_bits, logits_bits, gate_up, down, fmt, topk, fetch, ids=None, weights=None):
    """The fused layer for rows x [M, H] (bf16 bits) and logits [M, E] (bf16 bits), or the routing given as ids /
    weights [M, k] (as Experts.forward receives it, model.py:73).

    gate_up / down: (rows, cols) of the banks; fetch(bank, e) -> (packed rows, scale bits) of expert e, so callers can
    hand over only the experts a test touches. Each expert runs once on all its rows (experts_output). Returns (out
    bf16 bits [M, H], ids [M, k], weights [M, k], hidden float64 [M, k, I])."""
    x = bf16_bits_to_f32(x_bits)
    M, H = x.shape
    if ids is None:
        ids, w = route(logits_bits, topk)
    else:
        ids, w = np.asarray(ids, dtype=np.int64), np.asarray(weights, dtype=np.float32)
    I = down[1]
    xq, xs = quantize_act(x, fmt)
    parts = np.zeros((M, topk, H), dtype=np.float64)
    hidden = np.zeros((M, topk, I), dtype=np.float64)
    for e in np.unique(ids):
        rows, js = np.nonzero(ids == e)
        parts[rows, js], hidden[rows, js] = experts_output(xq[rows], xs[rows], fetch("gate_up", int(e)),
                                                           fetch("down", int(e)), fmt, I)
    out = np.zeros((M, H), dtype=np.float64)
    for j in range(topk):  # routing order, as the per-row sum
        out = out + w[:, j:j + 1].astype(np.float64) * parts[:, j]
    return f32_to_bf16_bits(out.astype(np.float32)), ids, w, hidden


# ------------------------------------------------------------------------------------------------------------ block
def router_logits(x_bits, router_bits):
    """The router's linear (model.py:115): bf16(x . router[e]) [M, E], from float64 sums."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    w = bf16_bits_to_f32(router_bits).astype(np.float64)
    return f32_to_bf16_bits((x @ w.T).astype(np.float32))


def moe_block(x_bits, gate_up, down, fmt, topk, fetch, logits_bits, shared=None, shared_gate_bits=None):
    """SparseMoeBlock.forward for one row (model.py:107-124) on A8 banks: the routed experts as moe_layer, then with
    `shared` = ((gate_up packed, scale bits), (down packed, scale bits)) of one expert and its gate [H] (bf16 bits)
    the sum the block forms from bf16 tensors: out = bf16(experts + bf16(bf16(sigmoid(bf16(x . gate))) *
    bf16(shared(x)))) (model.py:123). Returns (out bf16 bits [1, H], ids, weights)."""
    out_bits, ids, w, _ = moe_layer(x_bits, logits_bits, gate_up, down, fmt, topk, fetch)
    if shared is None:
        return out_bits, ids, w
    x = bf16_bits_to_f32(x_bits)
    xq, xs = quantize_act(x, fmt)
    y, _ = expert_output(xq[0:1], xs[0:1], shared[0], shared[1], fmt, down[1])
    return block_combine(out_bits, f32_to_bf16_bits(y.astype(np.float32))[None, :], x_bits, shared_gate_bits), ids, w


def block_combine(routed_bits, shared_bits, x_bits, gate_bits):
    """model.py:123 on bf16 tensors, rows [M, H]: out = routed + sigmoid(shared_expert_gate(x)) * shared_expert(x),
    every op rounding to bf16 as torch's bf16 ops do: the gate's linear (float sums, one rounding), its sigmoid, the
    product with the shared expert's bf16 output, the sum with the routed experts' bf16 output. Returns bf16 bits."""
    x = bf16_bits_to_f32(x_bits).astype(np.float64)
    g = bf16_bits_to_f32(gate_bits).astype(np.float64).reshape(-1)
    gate = bf16_round((x @ g).astype(np.float32))                                      # [M]
    gw = bf16_round((1.0 / (1.0 + np.exp(-gate.astype(np.float64)))).astype(np.float32))
    prod = bf16_round((gw[:, None] * bf16_bits_to_f32(shared_bits)).astype(np.float32))
    out = bf16_bits_to_f32(routed_bits).astype(np.float32) + prod
    return f32_to_bf16_bits(out.astype(np.float32))
