"""gfx950 kernels for a layer's routed experts, with the reference's call surface (drama3/kernels.py:590-724).

The reference compiles CUDA source with NVRTC at first use and launches it on torch's current stream
(kernels.py:593-601). Here the kernels are HIP for gfx950, compiled ahead of time into libdrama3_moe.so and launched
through its C ABI (include/drama3_moe.h) on the same stream; every function below keeps the reference's name,
arguments, output shape / dtype and allocation (torch.empty on the input's device, so graph capture works), and
nothing waits on the host.

Differences from the reference, by design: float sums run in a different order (results agree within float
tolerance, not bit for bit), and FP8 bytes are decoded by the hardware e4m3fn converter, so the two NaN codes 0x7F /
0xFF read as NaN where the reference's bit trick reads +-480 (kernels.py:25-29); quantized checkpoints never hold
them.
"""
import functools

import torch

from . import _lib

ROWS_PER_BLOCK = 16


@functools.cache
def _gfx950(index):
    return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0] == "gfx950"


def available(device):
    """Whether the kernels run on `device`: a gfx950 GPU. On such a device a missing library is an error, not a
    fallback."""
    if device.type != "cuda" or not torch.cuda.is_available():
        return False
    if not _gfx950(device.index if device.index is not None else torch.cuda.current_device()):
        return False
    _lib.lib()  # raises if libdrama3_moe.so was not built
    return True


def _stream(t):
    return _lib.stream_of(t.device)


def _p(t):
    return None if t is None else t.data_ptr()


def _call(name, *args):
    _lib.check(getattr(_lib.lib(), name)(*args), name)


def route(logits, k):
    """(ids [1, k] int64, weights [1, k] float32) of one row of router logits [1, n] (bfloat16): the k largest, by
    descending logit (ties to the lower index), and their softmax weights renormalized over them, rounded to
    bfloat16."""
    rows, n = logits.shape
    logits = logits.contiguous()
    ids = torch.empty((rows, k), dtype=torch.int64, device=logits.device)
    weights = torch.empty((rows, k), dtype=torch.float32, device=logits.device)
    _call("d3_route", _p(logits), rows, n, k, _p(ids), _p(weights), _stream(logits))
    return ids, weights


def weighted_sum(parts, weights):
    """[1, H] bfloat16: parts [k, H] (float32) summed by weights [k] (float32)."""
    parts = parts.contiguous()
    weights = weights.contiguous()
    out = torch.empty((1, parts.shape[1]), dtype=torch.bfloat16, device=parts.device)
    _call("d3_weighted_sum", _p(parts), _p(weights), parts.shape[0], parts.shape[1], _p(out), _stream(parts))
    return out


def resolve(ids, layer, layers, num_experts, half_life, cpu, admit, table, owner, score, at, pending, clock, budget,
            reads, step, share):
    """plan [k, 2] int32 for the row's experts `ids` [k] (int64) of `layer`: the slot cache's lookup and decayed-LFU
    eviction on the device, state tensors updated in place (kernels.py:78-191)."""
    plan = torch.empty((ids.shape[0], 2), dtype=torch.int32, device=ids.device)
    _call("d3_resolve", _p(ids.contiguous()), ids.shape[0], int(layer), int(layers), int(num_experts), _p(table),
          _p(owner), _p(score), _p(at), _p(pending), owner.shape[0], _p(clock), _p(budget), _p(plan), _p(reads),
          _p(step), _p(share), float(half_life), int(cpu), float(admit), _stream(ids))
    return plan


def await_cpu(plan, flag, step, result, timeout_us, took_over):
    """[1, H] float32: the host's result for the experts `plan` left to the CPU, or zeros when the host is late (then
    took_over is set; kernels.py:193-220). flag and result live in pinned host memory."""
    out = torch.empty((1, result.shape[-1]), dtype=torch.float32, device=plan.device)
    _call("d3_await_cpu", _p(plan), plan.shape[0], _p(flag), _p(step), _p(result), int(timeout_us), _p(out),
          _p(took_over), result.shape[-1], _stream(plan))
    return out


def rotate(x, only_if, swiglu=False):
    """Rows of x [rows, K] (float32 or bfloat16; float32 [rows, 2K] gate | up with `swiglu`, SiLU(gate) * up first) in
    the ConvRot basis: float32 [rows, K]. Only when `only_if` (an int32 on the GPU) is set; otherwise the output is
    left unset."""
    rows, width = x.shape
    k = width // 2 if swiglu else width
    x = x.contiguous()
    if swiglu and x.dtype != torch.float32:
        raise TypeError("rotate(swiglu=True) takes float32 gate | up rows")
    mode = 2 if swiglu else 1 if x.dtype == torch.bfloat16 else 0
    if mode == 0 and x.dtype != torch.float32:
        x = x.float()
    out = torch.empty((rows, k), dtype=torch.float32, device=x.device)
    _call("d3_rotate", _p(x), mode, rows, k, _p(out), _p(only_if), _stream(x))
    return out


def gemv_int8(x, ids, plan, took_over, late, slot_fields, host_fields, n):
    """[k, n] float32: each expert's int8 rows against x [1 or k, K] (float32, rotated); fields are {"_qdata",
    "scale"}."""
    k, width = ids.shape[0], x.shape[1]
    x = x.contiguous()
    out = torch.empty((k, n), dtype=torch.float32, device=x.device)
    _call("d3_gemv_int8", _p(x), x.shape[0], _p(ids), _p(plan), _p(took_over), int(late), _p(slot_fields["_qdata"]),
          _p(slot_fields["scale"]), _p(host_fields["_qdata"]), _p(host_fields["scale"]), _p(out), k, n, width,
          _stream(x))
    return out


def gemv_fp8(x, ids, plan, slot_fields, host_fields, n):
    """[k, n] float32: each expert's float8 rows against x [1 or k, K] float32; fields are {"weight", "scale"}."""
    k, width = ids.shape[0], x.shape[1]
    x = x.contiguous()
    out = torch.empty((k, n), dtype=torch.float32, device=x.device)
    _call("d3_gemv_fp8", _p(x), x.shape[0], _p(ids), _p(plan), _p(slot_fields["weight"]), _p(slot_fields["scale"]),
          _p(host_fields["weight"]), _p(host_fields["scale"]), _p(out), k, n, width, _stream(x))
    return out


def gemv_codes(x, ids, plan, slot_fields, host_fields, codebook, bits, n):
    """gemv_int8 for W4A8/W6A8 banks; fields are {"_qdata", "scale" (e4m3), "s_channel"}, codebook [16] at 4 bits."""
    k, width = ids.shape[0], x.shape[1]
    x = x.contiguous()
    out = torch.empty((k, n), dtype=torch.float32, device=x.device)
    _call("d3_gemv_codes", _p(x), x.shape[0], _p(ids), _p(plan), _p(slot_fields["_qdata"]), _p(slot_fields["scale"]),
          _p(slot_fields["s_channel"]), _p(host_fields["_qdata"]), _p(host_fields["scale"]),
          _p(host_fields["s_channel"]), _p(codebook), int(bits), _p(out), k, n, width, _stream(x))
    return out


GROUPED_KINDS = {"int8": (0, "_qdata"), "fp8": (1, "weight"), "w4": (4, "_qdata"), "w6": (6, "_qdata")}


def _grouped_fields(slot_fields, host_fields, codebook, wkey):
    return (_p(slot_fields[wkey]), _p(slot_fields["scale"]), _p(slot_fields.get("s_channel")), _p(host_fields[wkey]),
            _p(host_fields["scale"]), _p(host_fields.get("s_channel")), _p(codebook))


def grouped_plan(groups, rows):
    """The work list of the grouped products over `rows` sorted rows in `groups` [g, 5] int32: passes of up to 32
    rows, on the device. One plan serves every bank the same rows and groups go through."""
    ints = _lib.lib().d3_grouped_mfma_work_ints(groups.shape[0], rows)
    work = torch.empty(ints, dtype=torch.int32, device=groups.device)
    _call("d3_grouped_plan", _p(groups), groups.shape[0], rows, _p(work), ints, _stream(groups))
    return work


def grouped_fp8_planes(planes, rows, width, groups, work, slot_fields, host_fields, n, fills_first=False, order=None,
                       k=1):
    """[rows, n] float32: the fp8 grouped products on the bf16 matrix cores over planes [1 or 3, R * width] bf16
    (prep_planes / split, or bf16 rows themselves as one plane) and the plan `work` (grouped_plan). Row p of the
    groups' rows is the planes' row p, or with `order` [rows] int64 their row order[p] // k. fills_first: every
    group's first pass before the others, which then read a filled group from its slot."""
    out = torch.empty((rows, n), dtype=torch.float32, device=planes.device)
    if rows == 0:
        return out
    _call("d3_grouped_fp8", _p(planes), planes.shape[0], planes.shape[1], _p(order), int(k), rows, _p(groups),
          groups.shape[0], _p(work), work.shape[0], int(fills_first), _p(slot_fields["weight"]),
          _p(slot_fields["scale"]), _p(host_fields["weight"]), _p(host_fields["scale"]), _p(out), n, width,
          _stream(planes))
    return out


def grouped_i8(kind, planes, scales, rows, width, groups, work, slot_fields, host_fields, codebook, n,
               fills_first=False, order=None, k=1):
    """The grouped products of kind "int8", "w4" or "w6" on the int8 matrix cores, over (planes [3, R * width] int8,
    scales [R] float32) from prep_planes_i8; rows, order, k, work and fills_first as for grouped_fp8_planes."""
    code, wkey = GROUPED_KINDS[kind]
    out = torch.empty((rows, n), dtype=torch.float32, device=planes.device)
    if rows == 0:
        return out
    _call("d3_grouped_i8", code, _p(planes), _p(scales), planes.shape[1], _p(order), int(k), rows, _p(groups),
          groups.shape[0], _p(work), work.shape[0], int(fills_first),
          *_grouped_fields(slot_fields, host_fields, codebook, wkey), _p(out), n, width, _stream(planes))
    return out


def _grouped(kind, x, groups, slot_fields, host_fields, codebook, n, wkey, matrix=None):
    """The grouped products on the matrix cores when n % 64 == 0 or `matrix` (int8 and the codes on the int8 cores
    against x as three int8 planes, fp8 on the bf16 cores against three bf16 planes), else on the vector unit."""
    x = x.contiguous()
    if (matrix if matrix is not None else n % 64 == 0) and x.numel():
        name = {0: "int8", 1: "fp8", 4: "w4", 6: "w6"}[kind]
        work = grouped_plan(groups, x.shape[0])
        if kind != 1:
            planes, scales = prep_planes_i8(x, False)
            return grouped_i8(name, planes, scales, x.shape[0], x.shape[1], groups, work, slot_fields, host_fields,
                              codebook, n)
        planes = torch.empty((3, x.numel()), dtype=torch.bfloat16, device=x.device)
        _call("d3_split_bf16x3", _p(x), x.numel(), _p(planes), _stream(x))
        return grouped_fp8_planes(planes, x.shape[0], x.shape[1], groups, work, slot_fields, host_fields, n)
    out = torch.empty((x.shape[0], n), dtype=torch.float32, device=x.device)
    if x.numel():
        _call("d3_grouped", kind, _p(x), _p(groups), groups.shape[0],
              *_grouped_fields(slot_fields, host_fields, codebook, wkey), _p(out), n, x.shape[1], _stream(x))
    return out


def expert_groups(topk_idx, num_experts, plan=False):
    """(order [P] int64, inverse [P] int32, groups [num_experts, 5] int32) of a prompt's pairs topk_idx [T, k] int64:
    each expert's pairs together, experts ascending; inverse = each pair's place in order; groups (e, e, 0, first,
    rows). With `plan`, also the grouped products' work list over them (grouped_plan's) from the same launch. On the
    device, no host sync."""
    ids = topk_idx.reshape(-1).contiguous()
    if ids.dtype != torch.int64:
        ids = ids.long()
    P = ids.shape[0]
    order = torch.empty(P, dtype=torch.int64, device=ids.device)
    inverse = torch.empty(P, dtype=torch.int32, device=ids.device)
    groups = torch.empty((num_experts, 5), dtype=torch.int32, device=ids.device)
    work, ints = None, 0
    if plan:
        ints = _lib.lib().d3_grouped_mfma_work_ints(num_experts, P)
        work = torch.empty(ints, dtype=torch.int32, device=ids.device)
    _call("d3_expert_groups", _p(ids), P, num_experts, _p(order), _p(inverse), _p(groups), _p(work), ints,
          _stream(ids))
    return (order, inverse, groups, work) if plan else (order, inverse, groups)


def prep_planes(x, rotate, order=None, k=1, swiglu=False, n_planes=3):
    """planes [n_planes, P * K] bf16 for grouped_fp8_planes: row p is x's row order[p] // k (x's row p without order),
    through SiLU(gate) * up first with `swiglu` (x float32 gate | up [., 2K]), in the ConvRot basis with `rotate`.
    n_planes 1 takes bf16 rows as they are (no rotation, no SwiGLU); 3 splits float32 values into hi + mid + lo."""
    x = x.contiguous()
    width = x.shape[1] // 2 if swiglu else x.shape[1]
    if swiglu:
        if x.dtype != torch.float32:
            raise TypeError("prep_planes(swiglu=True) takes float32 gate | up rows")
        mode = 2
    elif x.dtype == torch.bfloat16:
        mode = 1
    else:
        x, mode = x.float(), 0
    P = order.shape[0] if order is not None else x.shape[0]
    planes = torch.empty((n_planes, P * width), dtype=torch.bfloat16, device=x.device)
    _call("d3_prep_planes", mode, int(rotate), n_planes, _p(x), _p(order), int(k), P, width, _p(planes), _stream(x))
    return planes


def prep_planes_i8(x, rotate, order=None, k=1, swiglu=False):
    """(planes [3, P * K] int8, scales [P] float32) for grouped_i8, rows as for prep_planes: v / S = a0 + a1 / 254 +
    a2 / 254^2 to within 0.5 / 254^2, S the row's power-of-two scale (max |v| <= 127 S)."""
    x = x.contiguous()
    width = x.shape[1] // 2 if swiglu else x.shape[1]
    if swiglu:
        if x.dtype != torch.float32:
            raise TypeError("prep_planes_i8(swiglu=True) takes float32 gate | up rows")
        mode = 2
    elif x.dtype == torch.bfloat16:
        mode = 1
    else:
        x, mode = x.float(), 0
    P = order.shape[0] if order is not None else x.shape[0]
    planes = torch.empty((3, P * width), dtype=torch.int8, device=x.device)
    scales = torch.empty(P, dtype=torch.float32, device=x.device)
    _call("d3_prep_planes_i8", mode, int(rotate), _p(x), _p(order), int(k), P, width, _p(planes), _p(scales),
          _stream(x))
    return planes, scales


def expert_groups_prep_i8(topk_idx, num_experts, x, rotate):
    """expert_groups(topk_idx, num_experts, plan=True) and prep_planes_i8(x, rotate) (x [T, K] float32 or bf16 token
    rows) in one launch: (order, inverse, groups, work, planes, scales)."""
    ids = topk_idx.reshape(-1).contiguous()
    if ids.dtype != torch.int64:
        ids = ids.long()
    x = x.contiguous()
    if x.dtype != torch.bfloat16:
        x = x.float()
    P, (T, K) = ids.shape[0], x.shape
    order = torch.empty(P, dtype=torch.int64, device=ids.device)
    inverse = torch.empty(P, dtype=torch.int32, device=ids.device)
    groups = torch.empty((num_experts, 5), dtype=torch.int32, device=ids.device)
    ints = _lib.lib().d3_grouped_mfma_work_ints(num_experts, P)
    work = torch.empty(ints, dtype=torch.int32, device=ids.device)
    planes = torch.empty((3, T * K), dtype=torch.int8, device=x.device)
    scales = torch.empty(T, dtype=torch.float32, device=x.device)
    _call("d3_expert_groups_prep_i8", _p(ids), P, num_experts, _p(order), _p(inverse), _p(groups), _p(work), ints,
          int(x.dtype == torch.bfloat16), int(rotate), _p(x), T, K, _p(planes), _p(scales), _stream(ids))
    return order, inverse, groups, work, planes, scales


_OUT_TYPES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def combine_rows(sorted_out, inverse, topk_weight, dtype):
    """[T, H] of `dtype` (float32, bfloat16 or float16): sum over j of topk_weight[t, j] * sorted_out[inverse[t k +
    j]], in float32, j in order."""
    T, k = topk_weight.shape
    H = sorted_out.shape[1]
    w = topk_weight.contiguous()
    if w.dtype not in (torch.bfloat16, torch.float32):
        w = w.float()
    out = torch.empty((T, H), dtype=dtype, device=sorted_out.device)
    _call("d3_combine_rows", _p(sorted_out.contiguous()), _p(inverse), _p(w), int(w.dtype == torch.bfloat16), T, k,
          H, _p(out), _OUT_TYPES[dtype], _stream(sorted_out))
    return out


def grouped_int8(x, groups, slot_fields, host_fields, n):
    """[rows, n] float32 for x's rows (float32, rotated, sorted by expert) through their experts; groups [g, 5] int32
    (expert, slot, fill, first row, rows). Rows outside every group are left unset."""
    return _grouped(0, x, groups, slot_fields, host_fields, None, n, "_qdata")


def grouped_fp8(x, groups, slot_fields, host_fields, n):
    """grouped_int8 for float8 experts, against float32 rows x."""
    return _grouped(1, x, groups, slot_fields, host_fields, None, n, "weight")


def grouped_codes(x, groups, slot_fields, host_fields, codebook, bits, n):
    """grouped_int8 for W4A8/W6A8 banks (see gemv_codes)."""
    return _grouped(int(bits), x, groups, slot_fields, host_fields, codebook, n, "_qdata")


_RESIDENT_KINDS = GROUPED_KINDS


def resident_decode(x, ids, weights, banks, kind, codebooks, H, I):
    """[1, H] bfloat16: offload.resident_decode's product in two launches (gate_up with x rotated in its prologue and
    SiLU(gate) * up in its epilogue; down with the hidden rows rotated in its prologue and the routing-weighted sum),
    banks resident, expert e in slot e. weights float32 [k]."""
    code, wkey = _RESIDENT_KINDS[kind]
    gate_up, down = banks
    k = ids.shape[0]
    gu = torch.empty((k, I), dtype=torch.float32, device=x.device)  # the hidden rows
    out = torch.empty((1, H), dtype=torch.bfloat16, device=x.device)
    _call("d3_resident_decode", code, _p(x.contiguous()), _p(ids.contiguous()), _p(weights.contiguous()), k,
          _p(gate_up[wkey]), _p(gate_up["scale"]), _p(gate_up.get("s_channel")), _p(down[wkey]), _p(down["scale"]),
          _p(down.get("s_channel")), _p(codebooks[0]), _p(codebooks[1]), _p(gu), _p(out), H, I, _stream(x))
    return out



def resident_decode_routed(x, logits, k, banks, kind, codebooks, H, I):
    """(out [1, H] bfloat16, ids [1, k] int64, weights [1, k] float32): route(logits, k) and resident_decode in two
    launches, the routing in the gate_up launch's prologue (logits [n] or [1, n] bfloat16, k <= n <= 256). ids and
    weights equal route's for the same logits."""
    code, wkey = _RESIDENT_KINDS[kind]
    gate_up, down = banks
    lg = logits.reshape(-1).contiguous()
    experts = gate_up[wkey].shape[0] // (2 * I)
    if lg.shape[0] != experts or down[wkey].shape[0] != experts * H:
        raise ValueError(f"{lg.shape[0]} logits for banks of {experts} experts: a routed id past the banks would be "
                         f"read out of bounds")
    gu = torch.empty((k, I), dtype=torch.float32, device=x.device)  # the hidden rows
    out = torch.empty((1, H), dtype=torch.bfloat16, device=x.device)
    ids = torch.empty((1, k), dtype=torch.int64, device=x.device)
    weights = torch.empty((1, k), dtype=torch.float32, device=x.device)
    _call("d3_resident_decode_routed", code, _p(x.contiguous()), _p(lg), lg.shape[0], k, _p(ids), _p(weights),
          _p(gate_up[wkey]), _p(gate_up["scale"]), _p(gate_up.get("s_channel")), _p(down[wkey]), _p(down["scale"]),
          _p(down.get("s_channel")), _p(codebooks[0]), _p(codebooks[1]), _p(gu), _p(out), H, I, _stream(x))
    return out, ids, weights

# The one-launch resident decode hands the hidden rows between its workgroups through a workspace per (device,
# stream): zeroed once, never cleared again (every word carries its launch's epoch). One first met under graph capture
# is allocated and zeroed in the graph (a fill kernel, so each replay clears it again, which changes nothing).
RESIDENT_MAX_K = 8
_resident_ws = {}


def resident_workspace(device, I, stream=None):
    """The zeroed workspace of the one-launch resident decode for (device, stream) and FFN size I."""
    device = torch.device(device)
    stream = stream if stream is not None else torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream, I)
    ws = _resident_ws.get(key)
    if ws is None:
        with torch.cuda.stream(stream):
            ws = torch.empty(int(_lib.lib().d3_resident_workspace_bytes(RESIDENT_MAX_K, I)), dtype=torch.uint8,
                             device=device).zero_()
        _resident_ws[key] = ws
    return ws


RESIDENT_RECOMPUTED = 1  # a down workgroup stopped waiting and computed the hidden rows itself (the output is exact)


def resident_status(device, I, stream=None):
    """The resident workspace's status bits since the last call (synchronizes, then clears them): 0 or
    RESIDENT_RECOMPUTED."""
    import ctypes
    ws = resident_workspace(device, I, stream)
    torch.cuda.synchronize(ws.device)
    value = ctypes.c_uint32(0)
    _lib.check(_lib.lib().d3_resident_status(ctypes.c_void_p(ws.data_ptr()), ctypes.byref(value)),
               "d3_resident_status")
    return value.value


def resident_fused_fits(kind, H, I, k):
    """Whether resident_decode_fused takes this layer shape."""
    return kind in _RESIDENT_KINDS and H == 2048 and I in (512, 768) and 1 <= k <= RESIDENT_MAX_K


def resident_decode_fused(x, banks, kind, codebooks, H, I, ids=None, weights=None, logits=None, k=None,
                          spin_limit=0, block_rows=0, recompute_all=False):
    """resident_decode (ids [k] int64, weights [k] float32 given) or resident_decode_routed (logits [n] or [1, n]
    bfloat16 and k given) in one launch, with the same output, ids and weights bit for bit. Returns out [1, H]
    bfloat16, or (out, ids [1, k], weights [1, k]) when routed."""
    code, wkey = _RESIDENT_KINDS[kind]
    gate_up, down = banks
    routed = logits is not None
    out = torch.empty((1, H), dtype=torch.bfloat16, device=x.device)
    if routed:
        lg = logits.reshape(-1).contiguous()
        experts = gate_up[wkey].shape[0] // (2 * I)
        if lg.shape[0] != experts or down[wkey].shape[0] != experts * H:
            raise ValueError(f"{lg.shape[0]} logits for banks of {experts} experts: a routed id past the banks would "
                             f"be read out of bounds")
        n = lg.shape[0]
        ids = torch.empty((1, k), dtype=torch.int64, device=x.device)
        weights = torch.empty((1, k), dtype=torch.float32, device=x.device)
    else:
        lg, n = None, 0
        ids, weights = ids.contiguous(), weights.contiguous()
        k = ids.shape[-1]
    ws = resident_workspace(x.device, I)
    _call("d3_resident_decode_fused", code, _p(x.contiguous()), _p(lg), n, k, _p(ids), _p(weights),
          _p(gate_up[wkey]), _p(gate_up["scale"]), _p(gate_up.get("s_channel")), _p(down[wkey]), _p(down["scale"]),
          _p(down.get("s_channel")), _p(codebooks[0]), _p(codebooks[1]), _p(ws), ws.numel(), int(spin_limit),
          int(block_rows), int(bool(recompute_all)), _p(out), H, I, _stream(x))
    return (out, ids, weights) if routed else out


def fp8_linear(x, weight, scale):
    """nn.functional.linear(x, dequantized weight) for an FP8 weight with one bf16 scale per output row, as the CPU
    path computes it (offload.py:163-167 dequantize_fp8, then the bf16 linear): x [rows, K] bf16 (rows <= 4), weight
    [N, K] float8_e4m3fn (or its bytes), scale [N] bf16 -> [rows, N] bf16. Each weight is rounded to bf16 after its
    scale, as the dequantized matrix holds it; sums in float32."""
    if x.dtype != torch.bfloat16 or scale.dtype != torch.bfloat16:
        raise TypeError("x and scale must be bfloat16")
    if weight.dtype not in (torch.float8_e4m3fn, torch.uint8):
        raise TypeError(f"weight must be float8_e4m3fn (or its uint8 bytes), not {weight.dtype}")
    if x.device.type != "cuda" or weight.device != x.device or scale.device != x.device:
        raise ValueError(f"x, weight and scale must be on one GPU (got {x.device}, {weight.device}, {scale.device})")
    rows, K = x.shape
    N = weight.shape[0]
    if weight.shape != (N, K) or scale.numel() != N:
        raise ValueError("weight [N, K] and scale [N] expected")
    x = x.contiguous()
    w = weight.contiguous().view(torch.uint8)
    out = torch.empty((rows, N), dtype=torch.bfloat16, device=x.device)
    _call("d3_gemv_fp8_rows", _p(x), rows, _p(w), _p(scale.contiguous()), _p(out), N, K, _stream(x))
    return out


def decode_codes(qdata, scale, codebook, bits, table=False):
    """int8 [R, K]: W4A8 / W6A8 rows decoded to the int8 grid exactly as gemv_codes / grouped_codes decode them
    (a check of kernels.py:466-483's decode_codes; no counterpart in the reference's call surface). table: 4-bit rows
    through the per-scale-byte tables of the resident decode kernels instead."""
    R = qdata.shape[0]
    K = qdata.shape[1] * 8 // bits
    out = torch.empty((R, K), dtype=torch.int8, device=qdata.device)
    mode = _lib.DECODE_TABLE_W4 if table else int(bits)
    if table and bits != 4:
        raise ValueError("the table decode is for 4-bit rows")
    _call("d3_decode_codes", mode, _p(qdata.contiguous()), _p(scale.contiguous()), _p(codebook), R, K, _p(out),
          _stream(qdata))
    return out
