"""A8 expert banks: the packed layouts the fused layer reads, and torch quantizers that produce them.

The four formats (codes in include/drama3_moe.h):
  I8  int8 rows, one bf16 scale per row: s = bf16(absmax / 127), q = clamp(round(w / s), -127, 127)
  W4  signed int4 two per byte along K (byte b: column 2b low nibble, 2b + 1 high), one bf16 scale per 128 columns:
      s = bf16(absmax / 7), q = clamp(round(w / s), -8, 7)
  W6  signed 6-bit, 16 columns per 12-byte unit along K, one bf16 scale per 128 columns: s = bf16(absmax / 31),
      q = clamp(round(w / s), -32, 31). Unit layout: byte i (0..11) holds q_i & 63 in its low 6 bits and bits
      2 (i >> 2) .. 2 (i >> 2) + 1 of q_{12 + (i & 3)} in its top two.
  F8  float8 e4m3fn rows, one bf16 scale per row: s = bf16(absmax / 448), q = e4m3(w / s)
Rounding is half to even (torch.round), in float32. A bank holds E experts of N rows each, flattened to [E * N, ...]
like the reference's flat banks (drama3/offload.py:72-90, tools/convert.py:179-216).

This module is the converter's side (it replaces comfy_kitchen's quantizers for these formats, tools/convert.py:48-82);
the kernels only read its output.
"""
import dataclasses

import torch

FMT_I8, FMT_W4, FMT_W6, FMT_F8 = 0, 1, 2, 3
NAMES = {FMT_I8: "int8", FMT_W4: "w4a8", FMT_W6: "w6a8", FMT_F8: "fp8"}
GROUP = 128


def row_bytes(fmt, cols):
    return cols // 2 if fmt == FMT_W4 else cols * 3 // 4 if fmt == FMT_W6 else cols


def group_scaled(fmt):
    return fmt in (FMT_W4, FMT_W6)


@dataclasses.dataclass
class A8Bank:
    """E experts of `rows` output rows over `cols` inputs: weight [E * rows, row_bytes] uint8, scale bf16 [E * rows]
    (I8, F8) or [E * rows, cols / 128] (W4, W6)."""
    fmt: int
    weight: torch.Tensor
    scale: torch.Tensor
    experts: int
    rows: int
    cols: int

    def to(self, device):
        return dataclasses.replace(self, weight=self.weight.to(device), scale=self.scale.to(device))

    def expert_bytes(self):
        return (self.weight.numel() + self.scale.numel() * self.scale.element_size()) // self.experts


def _scale(absmax, qmax):
    s = (absmax / qmax).to(torch.bfloat16)
    return torch.where(s == 0, torch.ones_like(s), s)


def pack_w4(q):
    """int codes [..., K] in [-8, 7] -> uint8 [..., K / 2]."""
    n = (q.to(torch.int32) & 0xF).to(torch.uint8)
    return n[..., 0::2] | (n[..., 1::2] << 4)


def unpack_w4(packed):
    b = packed.to(torch.int32)
    lo, hi = b & 0xF, (b >> 4) & 0xF
    q = torch.stack((lo, hi), dim=-1).flatten(-2)
    return torch.where(q >= 8, q - 16, q).to(torch.int8)


def pack_w6(q):
    """int codes [..., K] in [-32, 31] -> uint8 [..., 3K / 4] (16 columns per 12-byte unit)."""
    c = (q.to(torch.int32) & 63).unflatten(-1, (-1, 16))
    low = c[..., :12]
    i = torch.arange(12, device=q.device)
    top = (c[..., 12 + (i & 3)] >> (2 * (i >> 2))) & 3
    return (low | (top << 6)).to(torch.uint8).flatten(-2)


def unpack_w6(packed):
    b = packed.to(torch.int32).unflatten(-1, (-1, 12))
    low = b & 63
    top = (b >> 6) & 3
    high = top[..., 0:4] | (top[..., 4:8] << 2) | (top[..., 8:12] << 4)
    c = torch.cat((low, high), dim=-1)
    return torch.where(c >= 32, c - 64, c).to(torch.int8).flatten(-2)


def pack_w6_le3(q):
    """int codes [..., K] in [-32, 31] -> uint8 [..., 3K / 4] packed 4 per 3 bytes along K, little-endian, low bits
    first: value 4j + i at bits 6i .. 6i + 5 of the 24-bit word in bytes 3j .. 3j + 2 (the layout the W6A8 sweep
    workload is described with; the A8 W6 bank itself packs 16 per 12 bytes, pack_w6)."""
    c = (q.to(torch.int32) & 63).unflatten(-1, (-1, 4))
    word = c[..., 0] | (c[..., 1] << 6) | (c[..., 2] << 12) | (c[..., 3] << 18)
    return torch.stack((word & 0xFF, (word >> 8) & 0xFF, word >> 16), dim=-1).to(torch.uint8).flatten(-2)


def unpack_w6_le3(packed):
    b = packed.to(torch.int32).unflatten(-1, (-1, 3))
    word = b[..., 0] | (b[..., 1] << 8) | (b[..., 2] << 16)
    c = torch.stack([(word >> (6 * i)) & 63 for i in range(4)], dim=-1)
    return torch.where(c >= 32, c - 64, c).to(torch.int8).flatten(-2)


def w6_from_le3(packed):
    """Rows packed 4 per 3 bytes (pack_w6_le3) -> the A8 W6 layout the kernels read (pack_w6): same codes."""
    return pack_w6(unpack_w6_le3(packed))


def w6_to_le3(packed):
    """The A8 W6 layout -> rows packed 4 per 3 bytes: same codes."""
    return pack_w6_le3(unpack_w6(packed))


def quantize(w, fmt):
    """Float weights [E, rows, cols] -> A8Bank (on w's device)."""
    experts, rows, cols = w.shape
    w = w.float().reshape(experts * rows, cols)
    if fmt in (FMT_I8, FMT_F8):
        qmax = 127.0 if fmt == FMT_I8 else 448.0
        scale = _scale(w.abs().amax(dim=-1), qmax)
        v = w / scale.float()[:, None]
        if fmt == FMT_I8:
            weight = torch.round(v).clamp(-127, 127).to(torch.int8).view(torch.uint8)
        else:
            weight = v.to(torch.float8_e4m3fn).view(torch.uint8)
    elif fmt in (FMT_W4, FMT_W6):
        if cols % GROUP:
            raise ValueError("W4 / W6 need cols % 128 == 0")
        lo, hi = (-8, 7) if fmt == FMT_W4 else (-32, 31)
        g = w.view(experts * rows, cols // GROUP, GROUP)
        scale = _scale(g.abs().amax(dim=-1), float(hi))
        q = torch.round(g / scale.float()[..., None]).clamp(lo, hi).to(torch.int32).view(experts * rows, cols)
        weight = pack_w4(q) if fmt == FMT_W4 else pack_w6(q)
    else:
        raise ValueError(f"unknown format {fmt}")
    return A8Bank(fmt, weight.contiguous(), scale.contiguous(), experts, rows, cols)


def codes(bank):
    """The bank's integer codes [E * rows, cols] (int8; e4m3 bytes for F8), the inverse of the packing."""
    if bank.fmt == FMT_W4:
        return unpack_w4(bank.weight)
    if bank.fmt == FMT_W6:
        return unpack_w6(bank.weight)
    return bank.weight.view(torch.int8)


def dequantize(bank):
    """Float32 weights [E, rows, cols] of a bank."""
    n = bank.experts * bank.rows
    if bank.fmt == FMT_F8:
        w = bank.weight.view(torch.float8_e4m3fn).float() * bank.scale.float()[:, None]
    elif bank.fmt == FMT_I8:
        w = bank.weight.view(torch.int8).float() * bank.scale.float()[:, None]
    else:
        q = codes(bank).float().view(n, bank.cols // GROUP, GROUP)
        w = (q * bank.scale.float()[..., None]).view(n, bank.cols)
    return w.view(bank.experts, bank.rows, bank.cols)
