"""A layer's routed experts in the reference's own formats on an MI355X: the entry points model.py imports from
drama3/offload.py (FP8Experts, experts_decode, gather_experts, kernel_bank, resident_decode, resident_prefill), with
the same arguments and results, running the gfx950 kernels of kernels.py.

Storage is an HBM-resident expert table (`ExpertTable`): every layer's banks stay on the device (288 GB holds a
40-layer model's experts many times over), so the decode plan is the identity (slot e = expert e, offload.py:113)
and no lookup or host copy sits on the path. Banks are field dicts of flat tensors, as the reference's kernels read
them (offload.py:72-90, 264-273):
  int8   {"_qdata": int8 [E * N, K], "scale": float32 [E * N]}                 ConvRot basis (H256 per 256 columns)
  fp8    {"weight": uint8 e4m3 [E * N, K], "scale": float32 [E * N / 128, K / 128]}
  w4/w6  {"_qdata": uint8 [E * N, K * bits / 8], "scale": uint8 e4m3 [E * N, K / 16], "s_channel": float32 [E * N]},
         plus a float32 [16] codebook per bank at 4 bits                       ConvRot basis

comfy's QuantizedTensor (comfy.quant_ops) is used when it is importable; without it `kernel_bank` and friends accept
any object with the same `_qdata`, `_params`, `_layout_cls` attributes.
"""
import dataclasses
import time

import torch
import torch.nn as nn

from . import kernels

FP8_BLOCK = 128             # offload.py:36
CPU_EXPERT_US, CPU_ROW_US = 60, 13   # offload.py:37-38: the CPU's cost of one int8 expert, first estimate
PCIE_BYTES_PER_US = 12e3    # offload.py:39
HALF_LIFE = 128             # offload.py:44
MAX_EXPERTS_PER_ROW = 8     # offload.py:46
RESERVE_START, RESERVE_MIN, RESERVE_MAX = 32, 8, 256   # offload.py:49
ADMIT = 6.0                 # offload.py:51
AWAIT_US = 5000             # offload.py:53

try:  # optional: ComfyUI's quantized tensor type
    from comfy.quant_ops import QuantizedTensor
except ImportError:  # pragma: no cover - comfy is not part of this package
    QuantizedTensor = None


def _quantized(weight):
    if QuantizedTensor is not None:
        return isinstance(weight, QuantizedTensor)
    return all(hasattr(weight, a) for a in ("_qdata", "_params", "_layout_cls"))


def pinned(tensor, pin):
    """offload.py:56-60: a contiguous copy, in pinned host memory when `pin`."""
    if not pin:
        return tensor.contiguous()
    out = torch.empty(tensor.shape, dtype=tensor.dtype, pin_memory=True)
    return out.copy_(tensor)


def tensor_fields(weight):
    """offload.py:63-65: the tensors among a quantized weight's parameters."""
    params = weight._params
    return {f.name: getattr(params, f.name) for f in dataclasses.fields(params) if torch.is_tensor(getattr(params, f.name))}


def per_row_fields(weight):
    """offload.py:68-71: the bank's tensors holding one entry per weight row (sliced or gathered with the rows)."""
    rows = weight._qdata.shape[0]
    return {"_qdata": weight._qdata, **{n: v for n, v in tensor_fields(weight).items() if v.ndim >= 1 and v.shape[0] == rows}}


def kernel_bank(weight):
    """offload.py:74-90: (kind, fields) of a flat quantized bank [E * out, ...] the kernels read, or None: "int8"
    (ConvRot 256) with {"_qdata", "scale"}; "w4" (with codebook) or "w6" (without) with {"_qdata", "scale",
    "s_channel"}, group 16, ConvRot 256. In-features above 2048 are not taken (the grouped kernels hold 2048)."""
    if not _quantized(weight) or weight._qdata.ndim != 2:
        return None
    params, fields = weight._params, per_row_fields(weight)
    if params.orig_shape[-1] > 2048:
        return None
    if weight._layout_cls == "TensorWiseINT8Layout":
        if getattr(params, "convrot", False) and params.convrot_groupsize == 256 and set(fields) == {"_qdata", "scale"}:
            return "int8", fields
        return None
    if (weight._layout_cls == "AsymW4A8Int8Layout" and params.group_size == 16 and params.convrot_groupsize == 256
            and params.correction is None and not params.transposed and set(fields) == {"_qdata", "scale", "s_channel"}):
        bits = weight._qdata.shape[1] * 8 // params.orig_shape[-1]
        if (bits, params.codebook is not None) in ((4, True), (6, False)):
            return f"w{bits}", fields
    return None


def swiglu(y):
    """SiLU(gate) * up of rows [.., 2I] (gate first), the split comfy.ops._swiglu_eager makes (offload.py:115)."""
    gate, up = y.chunk(2, dim=-1)
    return nn.functional.silu(gate) * up


def quantized_gemv(kind, x, ids, plan, took_over, late, slot_fields, host_fields, rows, codebook):
    """offload.py:93-98: [k, rows] of a decode row's experts in an int8, W4A8 or W6A8 bank against x (float32,
    rotated)."""
    if kind == "int8":
        return kernels.gemv_int8(x, ids, plan, took_over, late, slot_fields, host_fields, rows)
    return kernels.gemv_codes(x, ids, plan, slot_fields, host_fields, codebook, int(kind[1]), rows)


def quantized_grouped(kind, x, groups, slot_fields, host_fields, rows, codebook):
    """offload.py:101-105: quantized_gemv for a prompt's rows grouped by expert."""
    if kind == "int8":
        return kernels.grouped_int8(x, groups, slot_fields, host_fields, rows)
    return kernels.grouped_codes(x, groups, slot_fields, host_fields, codebook, int(kind[1]), rows)


_consts = {}


def _constants(device):
    """Per device: int32 [0] (took_over: no expert left to the CPU) and [1] (the rotation always runs)."""
    key = (device.type, device.index)
    if key not in _consts:
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            raise RuntimeError("drama3.offload: run one call before capturing a graph (constants must exist)")
        _consts[key] = torch.arange(2, dtype=torch.int32, device=device).split(1)
    return _consts[key]


_FUSED_KINDS = {"int8": 0, "fp8": 1, "w4": 4, "w6": 6}


def resident_decode(x, ids, weights, banks, rows, kind, codebooks):
    """offload.py:108-123: one row x [1, H] through experts `ids` [k] of banks held whole on the GPU (expert e in
    slot e, `rows` per expert): fp8 -> gemv, SiLU(gate) * up, gemv; int8 / w4 / w6 -> rotate, gemv, rotate(swiglu),
    gemv; then the routing-weighted sum, bf16 [1, H]. Nothing waits on the host. Two launches
    (kernels.resident_decode) where the shapes allow, else the reference's five."""
    (gate_up, down), (gate_up_rows, down_rows) = banks, rows
    H, I = down_rows, gate_up_rows // 2
    if H in (1024, 2048) and I in (512, 768, 1024) and ids.shape[0] <= 8 and x.dtype == torch.bfloat16:
        return kernels.resident_decode(x, ids, weights.float(), banks, kind, codebooks, H, I)
    return resident_decode_unfused(x, ids, weights, banks, rows, kind, codebooks)



def routed_decode(x, logits, k, banks, rows, kind, codebooks):
    """kernels.route(logits, k) then resident_decode (model.py:116-118 then offload.py:108-123) for one row:
    (out [1, H] bf16, ids [1, k], weights [1, k]). Two launches where the shapes allow (the routing inside the
    gate_up launch), else route's own launch and resident_decode."""
    (gate_up, down), (gate_up_rows, down_rows) = banks, rows
    H, I = down_rows, gate_up_rows // 2
    experts = _rows(kind, gate_up, 1) // gate_up_rows
    if logits.numel() != experts:
        raise ValueError(f"{logits.numel()} logits for banks of {experts} experts: a routed id past the banks would be "
                         f"read out of bounds")
    if (H in (1024, 2048) and I in (512, 768, 1024) and k <= 8 and k <= logits.numel() <= 256
            and x.dtype == torch.bfloat16 and logits.dtype == torch.bfloat16):
        return kernels.resident_decode_routed(x, logits, k, banks, kind, codebooks, H, I)
    ids, weights = kernels.route(logits.reshape(1, -1), k)
    return resident_decode(x, ids[0], weights[0], banks, rows, kind, codebooks), ids, weights

def resident_decode_unfused(x, ids, weights, banks, rows, kind, codebooks):
    """resident_decode as the reference launches it: rotate, gemv, rotate(SwiGLU), gemv, weighted_sum."""
    (gate_up, down), (gate_up_rows, down_rows) = banks, rows
    plan = torch.stack((ids.to(torch.int32), torch.zeros_like(ids, dtype=torch.int32)), dim=-1)
    if kind == "fp8":
        gate, up = kernels.gemv_fp8(x.float(), ids, plan, gate_up, gate_up, gate_up_rows).chunk(2, dim=-1)
        out = kernels.gemv_fp8(nn.functional.silu(gate) * up, ids, plan, down, down, down_rows)
        return kernels.weighted_sum(out, weights.float())
    took_over, always = _constants(x.device)
    hidden = quantized_gemv(kind, kernels.rotate(x, always), ids, plan, took_over, False, gate_up, gate_up,
                            gate_up_rows, codebooks[0])
    out = quantized_gemv(kind, kernels.rotate(hidden, always, swiglu=True), ids, plan, took_over, False, down, down,
                         down_rows, codebooks[1])
    return kernels.weighted_sum(out, weights.float())


def grouped_experts(sorted_x, groups, slot_banks, host_banks, rows, kind, codebooks, always):
    """offload.py:126-136: [rows, H] float32 of sorted_x's rows through their experts, one grouped kernel per bank;
    `always` is an int32 1 on the GPU."""
    if kind == "fp8":
        gate, up = kernels.grouped_fp8(sorted_x.float(), groups, slot_banks[0], host_banks[0], rows[0]).chunk(2, dim=-1)
        return kernels.grouped_fp8(nn.functional.silu(gate) * up, groups, slot_banks[1], host_banks[1], rows[1])
    hidden = quantized_grouped(kind, kernels.rotate(sorted_x.float(), always), groups, slot_banks[0], host_banks[0],
                               rows[0], codebooks[0])
    return quantized_grouped(kind, kernels.rotate(hidden, always, swiglu=True), groups, slot_banks[1], host_banks[1],
                             rows[1], codebooks[1])


def expert_groups(topk_idx, num_experts):
    """The rows of a prompt's (token, k) pairs sorted by expert, on the device and without a host sync: (order
    [T * k] int64, groups [num_experts, 5] int32 = (expert, expert, 0, first, rows)). Experts without rows keep a group
    of 0 rows, which the grouped kernels skip without reading anything. Replaces offload.py:140-143's
    bincount().tolist(), so a prompt's pass can be captured in a graph."""
    flat = topk_idx.reshape(-1)
    order = torch.sort(flat, stable=True).indices
    counts = torch.zeros(num_experts, dtype=torch.int64, device=flat.device)
    counts.scatter_add_(0, flat, torch.ones_like(flat))
    first = torch.cumsum(counts, 0) - counts
    experts = torch.arange(num_experts, dtype=torch.int64, device=flat.device)
    groups = torch.stack((experts, experts, torch.zeros_like(experts), first, counts), dim=1).to(torch.int32)
    return order, groups


def resident_prefill(x, topk_idx, topk_weight, banks, rows, kind, codebooks, num_experts):
    """offload.py:139-149: many rows x [T, H] through banks held whole on the GPU: one grouped kernel per bank, each
    product scaled by its routing weight and summed over k, in x's dtype."""
    num_tokens, top_k = topk_idx.shape
    order, groups = expert_groups(topk_idx, num_experts)
    _, always = _constants(x.device)
    sorted_out = grouped_experts(x[order // top_k], groups, banks, banks, rows, kind, codebooks, always)
    out = torch.empty_like(sorted_out)
    out[order] = sorted_out * topk_weight.reshape(-1)[order].unsqueeze(1).float()
    return out.view(num_tokens, top_k, -1).sum(dim=1).to(x.dtype)


def gather_experts(weight, ids, num_experts):
    """offload.py:152-160: experts `ids` [k] of a flat [E * out, in] bank as one [k * out, in] weight, on the device.
    A field dict is gathered field by field (per-row fields; block-scale grids by their own row count)."""
    if isinstance(weight, dict):
        return {n: v.view(num_experts, -1, *v.shape[1:]).index_select(0, ids).flatten(0, 1) for n, v in weight.items()}
    if not _quantized(weight):
        return weight.view(num_experts, -1, weight.shape[-1]).index_select(0, ids).flatten(0, 1)
    rows = weight._qdata.shape[0] // num_experts
    picked = {n: v.view(num_experts, rows, *v.shape[1:]).index_select(0, ids).flatten(0, 1)
              for n, v in per_row_fields(weight).items()}
    qdata = picked.pop("_qdata")
    return type(weight)(qdata, weight._layout_cls,
                        dataclasses.replace(weight._params, orig_shape=(len(ids) * rows, weight._params.orig_shape[-1]), **picked))


def dequantize_fp8(weight, scale, dtype):
    """offload.py:163-167: float8 rows [R, C] with a float32 scale per 128 x 128 block [R / 128, C / 128] -> dtype."""
    rows, cols = weight.shape
    blocks = weight.float().view(rows // FP8_BLOCK, FP8_BLOCK, cols // FP8_BLOCK, FP8_BLOCK)
    return (blocks * scale[:, None, :, None]).view(rows, cols).to(dtype)


def hadamard(size):
    """offload.py:170-176: ConvRot's rotation, the regular Hadamard matrix of `size` (a power of 4), normalized."""
    h4 = torch.tensor([[1.0, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]])
    h = h4
    while h.shape[0] < size:
        h = torch.kron(h, h4)
    return h / size ** 0.5


def experts_decode(x, gate_up, down, weights):
    """offload.py:192-199: one row x [1, H] through k experts as two matmuls (gate_up [k * 2I, H], down [k * H, I],
    keeping the diagonal blocks of the second), summed by weights."""
    k = weights.shape[0]
    hidden = swiglu(nn.functional.linear(x, gate_up).view(k, -1))
    out = nn.functional.linear(hidden, down).view(k, k, -1).diagonal(dim1=0, dim2=1).T
    return (out * weights[:, None].to(out.dtype)).sum(0, keepdim=True)


def experts_on_cpu(banks, experts, counts, x, rotation):
    """offload.py:179-189: rows x [rows, H] (bf16, rotated; counts[i] rows for experts[i], in turn) through their int8
    ConvRot experts on the CPU (`banks` = (gate_up, down) QuantHostBank): [rows, H] float32."""
    gate_up, down = banks
    bounds = []
    start = 0
    for expert, n in zip(experts, counts):
        bounds.append((expert, start, start + n))
        start += n
    hidden = swiglu(torch.cat([gate_up.cpu_linear(x[a:b], expert) for expert, a, b in bounds]).float())
    hidden = (hidden.view(len(x), -1, 256) @ rotation).flatten(1).to(torch.bfloat16)
    return torch.cat([down.cpu_linear(hidden[a:b], expert) for expert, a, b in bounds]).float()


# ------------------------------------------------------------------------------------------------------ storage
class HostBank:
    """offload.py:200-218: one expert bank, tensors whose first dimension holds each expert's rows in turn, pinned
    in host memory when `pin`. `kernel` names the kernel family that reads it."""

    kernel = None

    def __init__(self, num_experts, fields, pin):
        self.num_experts = num_experts
        self.fields = {n: pinned(t, pin) for n, t in fields.items()}

    def rows(self, name):
        return self.fields[name].shape[0] // self.num_experts

    def take(self, fields, first, last):
        """Experts [first, last) of `fields`, laid out like this bank's."""
        return {n: t[first * self.rows(n):last * self.rows(n)] for n, t in fields.items()}

    def to_device(self, first, last, device):
        return {n: t.to(device, non_blocking=True) for n, t in self.take(self.fields, first, last).items()}


class QuantHostBank(HostBank):
    """offload.py:221-261 for a bank given as its kind and field dict (int8 ConvRot, W4A8, W6A8) instead of a comfy
    module: the CPU's int8 matmul reads it in place."""

    def __init__(self, num_experts, kind, fields, pin, codebook=None):
        super().__init__(num_experts, fields, pin)
        self.kernel = kind
        self._codebook = codebook
        if kind == "int8":
            self.scale_bf16 = self.fields["scale"].view(-1).to(torch.bfloat16)

    def codebook(self, device):
        return None if self._codebook is None else self._codebook.to(device)

    def cpu_linear(self, x, expert):
        """offload.py:245-249: rows x [M, K] (bf16, rotated) through int8 expert `expert` on the CPU: [M, N]."""
        rows = self.rows("_qdata")
        return torch._weight_int8pack_mm(x, self.fields["_qdata"][expert * rows:(expert + 1) * rows],
                                         self.scale_bf16[expert * rows:(expert + 1) * rows])


class FP8HostBank(HostBank):
    """offload.py:264-273: experts as Fish ships them, float8 rows [E, N, K] and block scales [E, N / 128, K / 128]."""

    kernel = "fp8"

    def __init__(self, weight, scale, pin):
        super().__init__(weight.shape[0], {"weight": weight.view(torch.uint8).flatten(0, 1), "scale": scale.flatten(0, 1)}, pin)

    def weight(self, fields, device):
        return dequantize_fp8(fields["weight"].view(torch.float8_e4m3fn), fields["scale"], torch.bfloat16)


class SlotPool:
    """offload.py:560-700, the device part: `count` expert slots in HBM filled from host banks, the least used expert
    out first. table [L * E] maps a key (layer * E + expert) to its slot, -1, or -2 - slot while the host copies it in
    (pending); owner [count] maps a slot to its key. The state lives on the device, where kernels.resolve keeps it
    (`device_state`); `promote` copies the slots decode steps reserved for the CPU's experts between steps."""

    def __init__(self, banks, count, device):
        self.banks = banks
        self.device = torch.device(device)
        self.layers, self.num_experts = len(banks), banks[0][0].num_experts
        self.rows = [{n: bank.rows(n) for n in bank.fields} for bank in banks[0]]
        self.expert_bytes = sum(t[:bank.rows(n)].nbytes for bank in banks[0] for n, t in bank.fields.items())
        self.count = max(8, min(self.layers * self.num_experts, int(count)))
        self.fields = [{n: torch.zeros((self.count * bank.rows(n), *t.shape[1:]), dtype=t.dtype, device=self.device)
                        for n, t in bank.fields.items()} for bank in banks[0]]
        keys = self.layers * self.num_experts
        dev = self.device
        self.table = torch.full((keys,), -1, dtype=torch.int32, device=dev)
        self.owner = torch.full((self.count,), -1, dtype=torch.int32, device=dev)
        self.score = torch.zeros((keys,), dtype=torch.float32, device=dev)
        self.at = torch.full((keys,), -1, dtype=torch.int32, device=dev)
        self.pending = torch.zeros((self.count,), dtype=torch.int32, device=dev)
        self.clock = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.reads = torch.zeros((3,), dtype=torch.int32, device=dev)
        self.reserve = RESERVE_START
        self.budget = torch.tensor(self._budget(), dtype=torch.int32, device=dev)
        # a layer's step, whether the GPU took over the CPU's experts, a set flag, the GPU's share of missed experts
        self.step, self.took_over, self.always = torch.tensor([[0], [0], [1]], dtype=torch.int32, device=dev)
        self.share = torch.zeros((1,), dtype=torch.float32, device=dev)
        self.reserved, self.copying = [], []
        self.copy_stream = None

    def device_state(self):
        """(table, owner, score, at, pending, clock, budget, reads, step, share) for kernels.resolve."""
        return (self.table, self.owner, self.score, self.at, self.pending, self.clock, self.budget, self.reads,
                self.step, self.share)

    def _budget(self):
        """[slots a decode step may reserve, at most per layer] (offload.py:644-646)."""
        return [self.reserve, max(1, -(-2 * self.reserve // self.layers))]

    def _fill(self, slot, sources):
        for fields, rows, source in zip(self.fields, self.rows, sources):
            for name, target in fields.items():
                target[slot * rows[name]:(slot + 1) * rows[name]].copy_(source[name], non_blocking=True)

    def _map(self, pairs):
        if pairs:
            keys, slots = zip(*pairs)
            keys = torch.tensor(keys, dtype=torch.long, device=self.device)
            slots = torch.tensor(slots, dtype=torch.long, device=self.device)
            self.table[keys] = slots.to(torch.int32)
            self.pending[slots] = 0

    def promote(self):
        """offload.py:624-642: map the slots whose copies landed, copy the experts reserved since the last call into
        theirs on a copy stream, and let the next step reserve as many as the copies kept up with."""
        landed = []
        while self.copying and self.copying[0][0].query():
            landed += self.copying.pop(0)[1]
        self._map(landed)
        lagging = bool(self.copying)
        if self.reserved:
            if self.copy_stream is None:
                self.copy_stream = torch.cuda.Stream(self.device)
            self.copy_stream.wait_stream(torch.cuda.current_stream(self.device))
            with torch.cuda.stream(self.copy_stream):
                for layer, expert, slot in self.reserved:
                    self._fill(slot, [bank.take(bank.fields, expert, expert + 1) for bank in self.banks[layer]])
                event = torch.cuda.Event()
                event.record()
            self.copying.append((event, [(layer * self.num_experts + expert, slot)
                                         for layer, expert, slot in self.reserved]))
            self.reserved = []
        self.reserve = max(RESERVE_MIN, self.reserve * 3 // 4) if lagging else min(RESERVE_MAX, self.reserve * 5 // 4 + 1)
        self.budget.copy_(torch.tensor(self._budget(), dtype=torch.int32), non_blocking=True)

    def settle(self):
        """Every reserved slot copied in and mapped."""
        self.promote()
        if self.copy_stream is not None:
            self.copy_stream.synchronize()
        self._map([pair for _, pairs in self.copying for pair in pairs])
        self.copying = []


class CpuSide:
    """offload.py:276-299: where a decode step's layers hand experts to the CPU. A layer copies its plan, routing,
    rotated row and step here (pinned host memory) and records posted[layer], then waits on the device
    (kernels.await_cpu) for flag[layer] to reach that step; the host (HostExperts.after_layer) runs the experts and
    writes result[layer], then the flag."""

    def __init__(self, layers, k, hidden):
        self.plan = torch.empty((layers, k, 2), dtype=torch.int32, pin_memory=True)
        self.ids = torch.empty((layers, k), dtype=torch.long, pin_memory=True)
        self.weights = torch.empty((layers, k), dtype=torch.float32, pin_memory=True)
        self.rows = torch.empty((layers, 1, hidden), dtype=torch.bfloat16, pin_memory=True)
        self.step = torch.zeros((layers,), dtype=torch.int32, pin_memory=True)
        self.flag = torch.zeros((layers,), dtype=torch.int32, pin_memory=True)
        self.result = torch.empty((layers, hidden), dtype=torch.bfloat16, pin_memory=True)
        self.posted = [torch.cuda.Event() for _ in range(layers)]

    def post(self, layer, plan, ids, weights, rows, step):
        for target, source in ((self.plan[layer], plan), (self.ids[layer], ids), (self.weights[layer], weights),
                               (self.rows[layer], rows), (self.step[layer:layer + 1], step)):
            target.copy_(source, non_blocking=True)
        self.posted[layer].record()

    def wait(self, layer, plan, step, took_over):
        return kernels.await_cpu(plan, self.flag[layer:layer + 1], step, self.result[layer], AWAIT_US, took_over)


class HostExperts:
    """The host-offload option (offload.py:302-452, ExpertStore's decode): every layer's banks in pinned host memory,
    a SlotPool of `slots` experts in HBM. A decode row resolves its experts on the device (kernels.resolve), the GEMVs
    read cached ones from their slots and missed ones straight from host memory, filling their slots on the way; with
    `cpu_side` (int8 banks) the CPU runs part of the missed experts meanwhile (`after_layer` on the host, bounded by
    kernels.await_cpu on the device). Nothing on the device waits on the host beyond AWAIT_US."""

    def __init__(self, kind, layer_banks, num_experts, slots, device, codebooks=None, cpu_side=False, pin=True):
        self.kind = kind
        if kind == "fp8":
            self.banks = [tuple(_FieldBank(num_experts, "fp8", f, pin) for f in banks) for banks in layer_banks]
        else:
            self.banks = [tuple(QuantHostBank(num_experts, kind, f, pin) for f in banks) for banks in layer_banks]
        self.codebooks = [tuple(None if c is None else c.to(device) for c in cb) for cb in codebooks] \
            if codebooks is not None else [(None, None)] * len(self.banks)
        self.cache = SlotPool(self.banks, slots, device)
        self.cpu_side = None
        if cpu_side:
            if kind != "int8":
                raise ValueError("the CPU side runs int8 experts (torch._weight_int8pack_mm)")
            hidden = self.banks[0][0].fields["_qdata"].shape[1]
            self.cpu_side = CpuSide(len(self.banks), MAX_EXPERTS_PER_ROW, hidden)
        self.rotation = hadamard(256)
        self.cpu_expert_us = CPU_EXPERT_US + CPU_ROW_US

    def between_steps(self):
        """offload.py:386-391: copy the experts the CPU ran into their reserved slots; give the GPU the share of
        missed experts that lets both sides finish together."""
        self.cache.promote()
        pcie = self.cache.expert_bytes / PCIE_BYTES_PER_US
        self.cache.share.fill_(self.cpu_expert_us / (self.cpu_expert_us + pcie))

    def decode(self, layer, x, ids, weights):
        """offload.py:403-432: one row x [1, H] through its experts `ids` [k]: [1, H] in x's dtype."""
        gate_up, down = self.banks[layer]
        cache, side = self.cache, self.cpu_side
        plan = kernels.resolve(ids, layer, len(self.banks), gate_up.num_experts, HALF_LIFE, side is not None, ADMIT,
                               *cache.device_state())
        slots_gate_up, slots_down = cache.fields
        weights = weights.float()
        if self.kind == "fp8":
            gate, up = kernels.gemv_fp8(x.float(), ids, plan, slots_gate_up, gate_up.fields,
                                        gate_up.rows("weight")).chunk(2, dim=-1)
            out = kernels.gemv_fp8(nn.functional.silu(gate) * up, ids, plan, slots_down, down.fields,
                                   down.rows("weight"))
            return kernels.weighted_sum(out, weights)
        cb_gu, cb_dn = self.codebooks[layer]

        def experts(late):
            hidden = quantized_gemv(self.kind, rotated, ids, plan, cache.took_over, late, slots_gate_up,
                                    gate_up.fields, gate_up.rows("_qdata"), cb_gu)
            hidden = kernels.rotate(hidden, cache.took_over if late else cache.always, swiglu=True)
            return quantized_gemv(self.kind, hidden, ids, plan, cache.took_over, late, slots_down, down.fields,
                                  down.rows("_qdata"), cb_dn)

        rotated = kernels.rotate(x, cache.always)
        if side is None:
            return kernels.weighted_sum(experts(False), weights)
        side.post(layer, plan, ids, weights, rotated.to(torch.bfloat16), cache.step)
        out = weights @ experts(False) + side.wait(layer, plan, cache.step, cache.took_over)
        return (out + weights @ experts(True)).to(x.dtype)

    def after_layer(self, layer):
        """offload.py:434-452: the host's part of decode layer `layer`, already launched: wait for its routing, run
        the experts it left to the CPU, and hand the result to the layer."""
        side = self.cpu_side
        side.posted[layer].synchronize()
        plan = side.plan[layer].tolist()
        on_cpu = [e for e, (_, code) in enumerate(plan) if code == 2]
        if not on_cpu:
            return
        ids = side.ids[layer].tolist()
        for e in on_cpu:
            if plan[e][0] >= 0:
                self.cache.reserved.append((layer, ids[e], plan[e][0]))
        started = time.perf_counter()
        out = experts_on_cpu(self.banks[layer], [ids[e] for e in on_cpu], [1] * len(on_cpu),
                             side.rows[layer].expand(len(on_cpu), -1), self.rotation)
        side.result[layer].copy_(side.weights[layer, on_cpu] @ out)
        side.flag[layer] = int(side.step[layer])
        self.cpu_expert_us = 0.9 * self.cpu_expert_us + 0.1 * 1e6 * (time.perf_counter() - started) / len(on_cpu)


class _FieldBank(HostBank):
    """A host bank given as its field dict (FP8 {"weight", "scale"} with block scales)."""

    def __init__(self, num_experts, kind, fields, pin):
        super().__init__(num_experts, fields, pin)
        self.kernel = kind


class ExpertTable:
    """Every layer's expert banks resident in HBM: the build's replacement for the reference's slot cache
    (offload.py:560-753). A bank is placed once (`place`); the kernels then read expert e in place (plan (e, 0)).
    `bytes` is what the table holds; `fits` checks it against the device's memory."""

    def __init__(self, device):
        self.device = torch.device(device)
        self.layers = {}

    def place(self, layer, kind, gate_up, down, codebooks=(None, None)):
        on = lambda f: {n: t.to(self.device, non_blocking=True).contiguous() for n, t in f.items()}  # noqa: E731
        cbs = tuple(None if c is None else c.to(self.device) for c in codebooks)
        self.layers[layer] = (kind, (on(gate_up), on(down)), cbs)
        return self.layers[layer]

    @property
    def bytes(self):
        return sum(t.numel() * t.element_size() for _, banks, _ in self.layers.values() for f in banks for t in f.values())

    def fits(self, extra=0):
        free, _ = torch.cuda.mem_get_info(self.device)
        return extra <= free

    def decode(self, layer, x, ids, weights, num_experts):
        kind, banks, cbs = self.layers[layer]
        rows = [_rows(kind, b, num_experts) for b in banks]
        return resident_decode(x, ids, weights, banks, rows, kind, cbs)

    def prefill(self, layer, x, topk_idx, topk_weight, num_experts):
        kind, banks, cbs = self.layers[layer]
        rows = [_rows(kind, b, num_experts) for b in banks]
        return resident_prefill(x, topk_idx, topk_weight, banks, rows, kind, cbs, num_experts)


def _rows(kind, fields, num_experts):
    return fields["weight" if kind == "fp8" else "_qdata"].shape[0] // num_experts


class FP8Experts(nn.Module):
    """offload.py:755-802: routed experts as Fish ships them, float8 e4m3 weights with a float32 scale per 128 x 128
    block. On a gfx950 GPU a decode row runs resident_decode and a prompt resident_prefill; elsewhere the experts a
    use needs are dequantized to the compute dtype."""

    def __init__(self, num_experts, hidden, intermediate, device=None, dtype=None):
        super().__init__()
        self.num_experts = num_experts
        self.dtype = dtype
        for name, rows, cols in (("gate_up", 2 * intermediate, hidden), ("down", hidden, intermediate)):
            self.register_parameter(f"{name}_weight", nn.Parameter(
                torch.empty((num_experts, rows, cols), dtype=torch.float8_e4m3fn, device=device), requires_grad=False))
            self.register_parameter(f"{name}_scale", nn.Parameter(
                torch.empty((num_experts, rows // FP8_BLOCK, cols // FP8_BLOCK), dtype=torch.float32, device=device),
                requires_grad=False))

    def sync_free(self, device):
        """Whether a decode row on `device` runs without waiting on the host."""
        return kernels.available(device)

    def experts(self, name, ids):
        weight = getattr(self, f"{name}_weight").view(torch.uint8).index_select(0, ids).view(torch.float8_e4m3fn)
        return dequantize_fp8(weight.flatten(0, 1), getattr(self, f"{name}_scale").index_select(0, ids).flatten(0, 1),
                              self.dtype)

    def forward(self, x, topk_idx, topk_weight):
        if kernels.available(x.device):
            banks = [{"weight": getattr(self, f"{name}_weight").view(torch.uint8).flatten(0, 1),
                      "scale": getattr(self, f"{name}_scale").flatten(0, 1)} for name in ("gate_up", "down")]
            rows = [getattr(self, f"{name}_weight").shape[1] for name in ("gate_up", "down")]
            if x.shape[0] == 1:
                return resident_decode(x, topk_idx[0], topk_weight[0], banks, rows, "fp8", (None, None))
            return resident_prefill(x, topk_idx, topk_weight, banks, rows, "fp8", (None, None), self.num_experts)
        if x.shape[0] == 1:
            return experts_decode(x, self.experts("gate_up", topk_idx[0]), self.experts("down", topk_idx[0]), topk_weight[0])
        num_tokens, top_k = topk_idx.shape
        order = torch.argsort(topk_idx.reshape(-1))
        counts = torch.bincount(topk_idx.reshape(-1), minlength=self.num_experts).tolist()
        sorted_x = x[order // top_k]
        weight = topk_weight.reshape(-1)[order].unsqueeze(1)
        sorted_out = torch.empty_like(sorted_x)
        start = 0
        for expert, n in enumerate(counts):
            if n == 0:
                continue
            ids = torch.tensor([expert], device=x.device)
            rows = slice(start, start + n)
            hidden = swiglu(nn.functional.linear(sorted_x[rows], self.experts("gate_up", ids)))
            sorted_out[rows] = nn.functional.linear(hidden, self.experts("down", ids)) * weight[rows]
            start += n
        out = torch.empty_like(sorted_out)
        out[order] = sorted_out
        return out.view(num_tokens, top_k, -1).sum(dim=1)
