"""Oracle numerics (test infrastructure only): bfloat16 and float8 e4m3fn conversions and the ConvRot rotation,
restated from their definitions in numpy.

Pinned by tests/test_oracle_numerics.py against torch's own casts (torch.bfloat16, torch.float8_e4m3fn, libraries in
this container) and against the rotation's closed form (Hadamard H256 = kron^4(h4) / 16 is symmetric and orthogonal).
"""
import numpy as np


def bf16_bits_to_f32(bits):
    """uint16 bfloat16 bits -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(v):
    """float32 -> bfloat16 bits, round to nearest, ties to even (kernels.py:33-37 to_bf16); NaN kept quiet."""
    b = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    return np.where(nan, ((b >> 16) | 0x40).astype(np.uint16), rounded)


def bf16_round(v):
    return bf16_bits_to_f32(f32_to_bf16_bits(v))


def _e4m3_table():
    """Values of the 256 e4m3fn codes: 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits; exponent 0 is
    subnormal (2^-6 * m / 8); 0x7F and 0xFF are NaN (no infinities)."""
    codes = np.arange(256)
    sign = np.where(codes & 0x80, -1.0, 1.0)
    exp = (codes >> 3) & 0xF
    man = codes & 7
    mag = np.where(exp == 0, 2.0 ** -6 * man / 8.0, 2.0 ** (exp - 7.0) * (1.0 + man / 8.0))
    val = sign * mag
    val[(codes & 0x7F) == 0x7F] = np.nan
    return val.astype(np.float32)


E4M3 = _e4m3_table()
_POS = E4M3[:127].astype(np.float64)  # codes 0..126: 0 .. 448, increasing


def e4m3_decode(codes):
    return E4M3[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(v):
    """float32 -> e4m3fn codes, round to nearest, ties to even (even mantissa); saturates to +-448 at and beyond the
    midpoint 464 between 448 and the missing 512 step (the kernels' converter does the same)."""
    v = np.asarray(v, dtype=np.float32)
    a = np.abs(v).astype(np.float64)
    hi = np.clip(np.searchsorted(_POS, a, side="left"), 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    dlo, dhi = np.abs(a - _POS[lo]), np.abs(_POS[hi] - a)
    pick_hi = (dhi < dlo) | ((dhi == dlo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo)
    code = np.where(a >= 464.0, 126, code)
    sign = np.where(np.signbit(v), 0x80, 0)
    out = (code | sign).astype(np.uint8)
    return np.where(np.isnan(v), (0x7F | sign).astype(np.uint8), out)


def hadamard(size=256):
    """ConvRot's rotation (drama3/offload.py:170-176): kron of h4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]],
    normalized by sqrt(size)."""
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64)
    h = h4
    while h.shape[0] < size:
        h = np.kron(h, h4)
    return h / np.sqrt(size)
