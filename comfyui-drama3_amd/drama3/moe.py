"""The fused routed-expert MoE layer on A8 banks: one launch per layer for M <= 16 rows.

`moe_layer(x, logits, gate_up, down, topk)` does what the reference's SparseMoeBlock.forward does for its routed
experts (drama3/model.py:107-122: router softmax / top-k / renormalization, then Experts.forward ->
offload.resident_decode, drama3/offload.py:108-123), for every row of a batch of decode lines at once, in one kernel
(include/drama3_moe.h, d3_moe_a8). The shared expert and the router's linear stay with the caller, as in the
reference (model.py:115,123).

Each (device, stream) pair gets a workspace, zeroed once and never cleared again: every word the kernel hands from one
workgroup to another carries the launch's epoch (its dispatch ID plus a salt from its queue), so words a previous
launch left behind are told apart without a reset, and a graph captured on one stream may be replayed on another.
Launches that overlap on one workspace race. Allocate it before capturing a graph (`prepare`).

A workgroup that waits for another's result past `spin_limit` polls (one that is not resident because another kernel
holds part of the device, or a deliberately tiny limit) computes the result itself, bit for bit what the producer
would have published, so the output stays exact; `status` reports that this happened.
"""
import ctypes
import threading

import torch

from . import _lib
from .formats import FMT_W4, FMT_W6, A8Bank

MAX_ROWS = 16
MAX_TOPK = 8
_workspaces = {}
_lock = threading.Lock()


def _workspace_bytes(H, I):
    return int(_lib.lib().d3_moe_a8_workspace_bytes(MAX_ROWS, MAX_TOPK, H, I))


def workspace(device, H, I, stream=None):
    """The zeroed workspace for (device, stream); created on first use, outside graph capture."""
    device = torch.device(device)
    stream = stream if stream is not None else torch.cuda.current_stream(device)
    key = (device.index, stream.cuda_stream, H, I)
    with _lock:
        ws = _workspaces.get(key)
        if ws is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("drama3.moe: call prepare() before capturing a graph (the workspace must exist)")
            with torch.cuda.stream(stream):
                ws = torch.zeros(_workspace_bytes(H, I), dtype=torch.uint8, device=device)
            _workspaces[key] = ws
    return ws


def prepare(device, H, I, stream=None):
    """Create the workspace for `stream` (default: the current one) ahead of graph capture."""
    workspace(device, H, I, stream)


STATUS_RECOMPUTED = 1   # a wait gave up and its workgroup computed the missing values itself (the output is exact)
STATUS_INVALID = 2      # a wait still failed after that: the output of that launch is not valid


def status(device, H, I, stream=None):
    """The workspace's status bits since the last call (synchronizes, then clears them): 0, STATUS_RECOMPUTED,
    STATUS_INVALID."""
    ws = workspace(device, H, I, stream)
    torch.cuda.synchronize(ws.device)
    value = ctypes.c_uint32(0)
    _lib.check(_lib.lib().d3_moe_a8_status(ctypes.c_void_p(ws.data_ptr()), ctypes.byref(value)), "d3_moe_a8_status")
    return value.value


# From this many rows on, moe_layer runs the grouped path (d3_moe_a8_prefill): its persistent grouped products read
# each expert once for all rows and keep the memory busy, where the fused kernel's items for several rows queue up
# behind each other. Measured on MI355X (us per layer, fused / grouped): int8 5 rows 49.8 / 58.3, 6 rows 57.4 /
# 56.7, 7 rows 63.0 / 60.9, 8 rows 69.4 / 65.3, 16 rows 143 / 92; FP8 6 rows 56.5 / 56.4, 7 rows 61.7 / 60.8; W4A8
# 6 rows 44.4 / 46.1, 7 rows 48.1 / 49.2, 8 rows 52.8 / 52.6, 16 rows 116 / 70; W6A8 6 rows 53.7 / 56.5, 7 rows
# 59.1 / 60.9, 8 rows 63.9 / 66.1. GROUPED_FROM_ROWS holds for int8 and FP8; the 4- and 6-bit formats switch later.
GROUPED_FROM_ROWS = 6
GROUPED_FROM_ROWS_BY_FORMAT = {FMT_W4: 8, FMT_W6: 9}


def grouped_from_rows(fmt):
    """The row count from which moe_layer runs the grouped path for banks of format `fmt`."""
    return GROUPED_FROM_ROWS_BY_FORMAT.get(fmt, GROUPED_FROM_ROWS)


def moe_layer(x, logits, gate_up: A8Bank, down: A8Bank, topk, *, routing=False, spin_limit=0, grid=0, out=None,
              fused=None, item_units=0, recompute_all=False):
    """x [M, H] bf16 and router logits [M, E] bf16 (M <= 16) through the routed experts: [M, H] bf16, and with
    `routing` also (ids [M, topk] int64 in descending logit order, weights [M, topk] float32). Fewer than
    grouped_from_rows(format) rows run the fused one-launch kernel (d3_moe_a8), more the grouped path (moe_prefill);
    `fused` forces either. `item_units` (8 or 16; 0 picks) sets the one-row schedule's hidden units per gate_up workgroup.
    `spin_limit` bounds a workgroup's wait for another's result (0: the library's default; see the module's
    docstring for what happens past it). `recompute_all` is a test hook: every such wait gives up at once."""
    if fused is None:
        fused = x.shape[0] < grouped_from_rows(gate_up.fmt)
    if not fused:
        return moe_prefill(x, gate_up, down, topk, logits=logits, routing=routing, out=out)
    if x.dtype != torch.bfloat16 or logits.dtype != torch.bfloat16:
        raise TypeError("x and logits must be bfloat16")
    if x.dim() != 2 or logits.dim() != 2 or x.shape[0] != logits.shape[0]:
        raise ValueError("x [M, H] and logits [M, E] expected")
    M, H = x.shape
    E = logits.shape[1]
    if gate_up.fmt != down.fmt or gate_up.experts != E or down.experts != E:
        raise ValueError("banks must share the format and hold one expert per logit")
    if gate_up.cols != H or down.rows != H or gate_up.rows != 2 * down.cols:
        raise ValueError("gate_up [E * 2I, H] and down [E * H, I] expected")
    I = down.cols
    device = x.device
    x = x.contiguous()
    logits = logits.contiguous()
    if out is None:
        out = torch.empty((M, H), dtype=torch.bfloat16, device=device)
    ids = torch.empty((M, topk), dtype=torch.int64, device=device) if routing else None
    weights = torch.empty((M, topk), dtype=torch.float32, device=device) if routing else None
    ws = workspace(device, H, I)
    desc = _lib.MoeA8Desc(
        x=x.data_ptr(), logits=logits.data_ptr(), gate_up=gate_up.weight.data_ptr(),
        gate_up_scale=gate_up.scale.data_ptr(), down=down.weight.data_ptr(), down_scale=down.scale.data_ptr(),
        out=out.data_ptr(), ids_out=_lib.ptr(ids), weights_out=_lib.ptr(weights), workspace=ws.data_ptr(),
        workspace_bytes=ws.numel(), format=gate_up.fmt, M=M, H=H, I=I, E=E, topk=topk, spin_limit=spin_limit,
        grid=grid, item_units=item_units, recompute_all=int(recompute_all))
    _lib.check(_lib.lib().d3_moe_a8(ctypes.byref(desc), _lib.stream_of(device)), "d3_moe_a8")
    return (out, ids, weights) if routing else out


def _check_shared(shared, shared_gate, gate_up, H, I):
    if shared is None:
        return None, None, None
    sg, sd = shared
    if (sg.fmt, sd.fmt) != (gate_up.fmt, gate_up.fmt) or sg.experts != 1 or sd.experts != 1 or \
            (sg.rows, sg.cols, sd.rows, sd.cols) != (2 * I, H, H, I):
        raise ValueError("the shared expert: one expert of the layer's format and shape")
    if shared_gate is None or shared_gate.dtype != torch.bfloat16 or shared_gate.numel() != H:
        raise ValueError("shared_gate [H] bfloat16 expected")
    return sg, sd, shared_gate.contiguous()


_ZERO_LOGITS = {}


def _one_expert_logits(device, M):
    """[M, 1] bf16 zeros: every row's only expert, at weight 1. Kept per (device, M) once made outside a graph
    capture (a tensor first made inside one is filled only when the graph replays)."""
    key = (device.type, device.index, M)
    t = _ZERO_LOGITS.get(key)
    if t is None:
        t = torch.zeros((M, 1), dtype=torch.bfloat16, device=device)
        if not torch.cuda.is_current_stream_capturing():
            _ZERO_LOGITS[key] = t
    return t


def router_logits(x, router):
    """The router's logits of every row, model.py:115's self.gate(flat): [M, E] bf16 from x [M, H] and router [E, H]
    bf16, float sums in the one-row block's order, so each row's logits equal what that block computes."""
    M, H = x.shape
    out = torch.empty((M, router.shape[0]), dtype=torch.bfloat16, device=x.device)
    _lib.check(_lib.lib().d3_router_logits(x.data_ptr(), router.data_ptr(), M, H, router.shape[0], out.data_ptr(),
                                           _lib.stream_of(x.device)), "d3_router_logits")
    return out


def moe_block(x, gate_up: A8Bank, down: A8Bank, topk, *, router=None, logits=None, shared=None, shared_gate=None,
              routing=False, return_logits=False, out=None, item_units=0, spin_limit=0, recompute_all=False):
    """SparseMoeBlock.forward (drama3/model.py:107-124) for decode rows: x [M, H] bf16 -> [M, H] bf16.

    The router: `router` [E, H] bf16 (its logits computed on the device, model.py:115) or given `logits` [M, E] bf16.
    The shared expert: `shared` = (gate_up, down) A8Banks of one expert in the layer's format and shape, and
    `shared_gate` [H] bf16; it is added as model.py:123 does (both terms bf16). With `routing` also returns ids and
    weights [M, topk], with `return_logits` the router's logits [M, E] bf16. `item_units`, `spin_limit` and
    `recompute_all` as for moe_layer.

    One row runs in one launch (router, routed experts, shared expert, sum). More rows run in four, each over all the
    rows at once: the router's logits (router_logits), the routed layer (moe_layer: one launch, each expert read
    once), the shared expert as a layer of one expert at weight 1 (its banks read once), and the sum
    (d3_block_combine). Each row's output, routing and logits equal the one-row block's on that row bit for bit
    while the routed layer runs fused (fewer than grouped_from_rows(format) rows); from there on the grouped path's
    own summation order applies."""
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.shape[0] < 1:
        raise ValueError("x [M, H] bfloat16 expected")
    M, H = x.shape
    E = gate_up.experts
    if gate_up.fmt != down.fmt or down.experts != E or gate_up.cols != H or down.rows != H or gate_up.rows != 2 * down.cols:
        raise ValueError("gate_up [E * 2I, H] and down [E * H, I] of one format expected")
    I = down.cols
    device = x.device
    if (router is None) == (logits is None):
        raise ValueError("router or logits, one of them")
    if router is not None:
        if router.dtype != torch.bfloat16 or router.shape != (E, H):
            raise ValueError("router [E, H] bfloat16 expected")
        router = router.contiguous()
    else:
        if logits.dtype != torch.bfloat16 or logits.shape != (M, E):
            raise ValueError(f"logits [{M}, {E}] bfloat16 expected")
        logits = logits.contiguous()
    sg, sd, shared_gate = _check_shared(shared, shared_gate, gate_up, H, I)
    if out is not None and (out.shape != x.shape or out.dtype != torch.bfloat16 or not out.is_contiguous()):
        raise ValueError("out [M, H] bfloat16, contiguous, expected")
    x = x.contiguous()
    if M > 1:
        lg = router_logits(x, router) if router is not None else logits
        res = moe_layer(x, lg, gate_up, down, topk, routing=routing, spin_limit=spin_limit,
                        out=None if sg is not None else out, recompute_all=recompute_all)
        routed, ids, weights = res if routing else (res, None, None)
        if sg is None:
            out = routed
        else:
            ys = moe_layer(x, _one_expert_logits(device, M), sg, sd, 1, spin_limit=spin_limit,
                           recompute_all=recompute_all)
            out = torch.empty_like(x) if out is None else out
            _lib.check(_lib.lib().d3_block_combine(x.data_ptr(), shared_gate.data_ptr(), routed.data_ptr(),
                                                   ys.data_ptr(), M, H, out.data_ptr(), _lib.stream_of(device)),
                       "d3_block_combine")
        res = (out,)
        if routing:
            res += (ids, weights)
        if return_logits:
            res += (lg if router is not None else logits,)
        return res if len(res) > 1 else out
    if out is None:
        out = torch.empty((1, H), dtype=torch.bfloat16, device=device)
    ids = torch.empty((1, topk), dtype=torch.int64, device=device) if routing else None
    weights = torch.empty((1, topk), dtype=torch.float32, device=device) if routing else None
    lg_out = torch.empty((1, E), dtype=torch.bfloat16, device=device) if return_logits else None
    ws = workspace(device, H, I)
    desc = _lib.MoeA8Desc(
        x=x.data_ptr(), logits=_lib.ptr(logits), gate_up=gate_up.weight.data_ptr(),
        gate_up_scale=gate_up.scale.data_ptr(), down=down.weight.data_ptr(), down_scale=down.scale.data_ptr(),
        out=out.data_ptr(), ids_out=_lib.ptr(ids), weights_out=_lib.ptr(weights), workspace=ws.data_ptr(),
        workspace_bytes=ws.numel(), format=gate_up.fmt, M=1, H=H, I=I, E=E, topk=topk, spin_limit=spin_limit, grid=0,
        router=_lib.ptr(router), logits_out=_lib.ptr(lg_out),
        shared_gate_up=_lib.ptr(sg.weight if sg is not None else None),
        shared_gate_up_scale=_lib.ptr(sg.scale if sg is not None else None),
        shared_down=_lib.ptr(sd.weight if sd is not None else None),
        shared_down_scale=_lib.ptr(sd.scale if sd is not None else None), shared_gate=_lib.ptr(shared_gate),
        item_units=item_units, recompute_all=int(recompute_all))
    _lib.check(_lib.lib().d3_moe_a8(ctypes.byref(desc), _lib.stream_of(device)), "d3_moe_a8")
    res = (out,)
    if routing:
        res += (ids, weights)
    if return_logits:
        res += (lg_out,)
    return res if len(res) > 1 else out


def moe_prefill(x, gate_up: A8Bank, down: A8Bank, topk, *, logits=None, topk_idx=None, topk_weight=None,
                routing=False, out=None):
    """Many rows x [T, H] bf16 through the routed experts of A8 banks: [T, H] bf16 (d3_moe_a8_prefill). Routing from
    router `logits` [T, E] bf16 (as moe_layer; with `routing` also returns ids and weights), or given as `topk_idx`
    [T, k] int64 with `topk_weight` [T, k] (as Experts.forward receives them, drama3/model.py:73). The (row, expert)
    pairs are grouped by expert on the device; nothing waits on the host."""
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise TypeError("x must be bfloat16 [T, H]")
    T, H = x.shape
    E = gate_up.experts
    if gate_up.fmt != down.fmt or down.experts != E:
        raise ValueError("banks must share the format and the expert count")
    if gate_up.cols != H or down.rows != H or gate_up.rows != 2 * down.cols:
        raise ValueError("gate_up [E * 2I, H] and down [E * H, I] expected")
    I = down.cols
    device = x.device
    x = x.contiguous()
    if logits is not None:
        if logits.dtype != torch.bfloat16 or logits.shape != (T, E):
            raise ValueError("logits [T, E] bfloat16 expected")
        logits = logits.contiguous()
        ids_in = weights_in = None
    else:
        if topk_idx is None or topk_weight is None:
            raise ValueError("logits, or topk_idx and topk_weight")
        ids_in = topk_idx.to(torch.int64).contiguous()
        weights_in = topk_weight.to(torch.float32).contiguous()
        if ids_in.shape != (T, topk) or weights_in.shape != (T, topk):
            raise ValueError("topk_idx / topk_weight [T, topk] expected")
    if out is None:
        out = torch.empty((T, H), dtype=torch.bfloat16, device=device)
    ids = torch.empty((T, topk), dtype=torch.int64, device=device) if routing and logits is not None else None
    weights = torch.empty((T, topk), dtype=torch.float32, device=device) if ids is not None else None
    nbytes = int(_lib.lib().d3_moe_a8_prefill_workspace_bytes(T, topk, H, I, E))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    desc = _lib.MoeA8PrefillDesc(
        x=x.data_ptr(), logits=_lib.ptr(logits), ids_in=_lib.ptr(ids_in), weights_in=_lib.ptr(weights_in),
        gate_up=gate_up.weight.data_ptr(), gate_up_scale=gate_up.scale.data_ptr(), down=down.weight.data_ptr(),
        down_scale=down.scale.data_ptr(), out=out.data_ptr(), ids_out=_lib.ptr(ids), weights_out=_lib.ptr(weights),
        workspace=ws.data_ptr(), workspace_bytes=nbytes, format=gate_up.fmt, T=T, H=H, I=I, E=E, topk=topk)
    _lib.check(_lib.lib().d3_moe_a8_prefill(ctypes.byref(desc), _lib.stream_of(device)), "d3_moe_a8_prefill")
    return (out, ids, weights) if ids is not None else out


def gemv_groups(bank_rows, fmt, cols, act):
    """Exact per-group dot products of packed rows [R, row_bytes] with act [C, cols] (int8, or e4m3 bytes for F8):
    [R, cols / 128, C] int32 (float32 for F8). Runs the fused layer's MFMA step on its own."""
    R = bank_rows.shape[0]
    C = act.shape[0]
    dtype = torch.float32 if fmt == 3 else torch.int32
    acc = torch.empty((R, cols // 128, C), dtype=dtype, device=bank_rows.device)
    _lib.check(_lib.lib().d3_gemv_a8_groups(fmt, bank_rows.data_ptr(), R, cols, act.contiguous().data_ptr(), C,
                                            acc.data_ptr(), _lib.stream_of(bank_rows.device)), "d3_gemv_a8_groups")
    return acc


def cvt_fp8(values, hardware=True):
    """float32 -> float8 e4m3fn codes (uint8) by the converter the kernels quantize activations with (hardware) or by
    the format's definition, round to nearest, ties to even."""
    values = values.contiguous()
    n = values.numel()
    out = torch.empty(n, dtype=torch.uint8, device=values.device)
    _lib.check(_lib.lib().d3_cvt_fp8(values.data_ptr(), n, out.data_ptr(), int(hardware),
                                     _lib.stream_of(values.device)), "d3_cvt_fp8")
    return out


def unpack_rows(bank_rows, fmt, cols):
    """The int8 codes [R, cols] the fused layer's W4 / W6 unpacking feeds the MFMA."""
    R = bank_rows.shape[0]
    codes = torch.empty((R, cols), dtype=torch.int8, device=bank_rows.device)
    _lib.check(_lib.lib().d3_unpack_rows(fmt, bank_rows.data_ptr(), R, cols, codes.data_ptr(),
                                         _lib.stream_of(bank_rows.device)), "d3_unpack_rows")
    return codes
