"""The reference's CPU expert path, restated in torch (test infrastructure and bench.py's cpu_baseline leg only).

What the reference runs when experts are computed on the host (drama3/offload.py:179-189 experts_on_cpu, 245-249
QuantHostBank.cpu_linear, 192-199 experts_decode, 163-167 dequantize_fp8): per routed expert, a matmul straight from
the quantized bank - torch._weight_int8pack_mm for int8 rows with their per-row scales, or the weights dequantized to
bf16 on every call for the other formats - then SwiGLU (gate first) and the down projection, and the routing-weighted
sum. Activations stay bf16 as there. The ConvRot rotation of the reference's int8 files is not part of these banks.
"""
import torch


def _swiglu(y):
    gate, up = y.chunk(2, dim=-1)
    return torch.nn.functional.silu(gate) * up


def dequantize_rows(weight, scale, fmt, cols):
    """bf16 weights [rows, cols] of one expert's rows (packed weight [rows, row_bytes], scales), decoded per call as
    the reference decodes FP8 experts per use (drama3/offload.py:771-773)."""
    if fmt == 3:
        return (weight.view(torch.float8_e4m3fn).float() * scale.float()[:, None]).to(torch.bfloat16)
    if fmt == 0:
        return (weight.view(torch.int8).float() * scale.float()[:, None]).to(torch.bfloat16)
    from drama3 import formats  # the packed layouts' inverse
    q = (formats.unpack_w4(weight) if fmt == 1 else formats.unpack_w6(weight)).float()
    q = q.view(weight.shape[0], cols // 128, 128) * scale.float()[..., None]
    return q.view(weight.shape[0], cols).to(torch.bfloat16)


def expert_rows(bank_weight, bank_scale, rows, e):
    return bank_weight[e * rows:(e + 1) * rows], bank_scale[e * rows:(e + 1) * rows]


def layer(x, ids, weights, gate_up, down, fmt, H, I):
    """One decode row x [1, H] bf16 through experts ids [k] with routing weights [k] on the CPU: [1, H] float32.
    gate_up = (weight [E * 2I, row_bytes(H)], scale), down = (weight [E * H, row_bytes(I)], scale)."""
    outs = []
    for e in ids.tolist():
        gw, gs = expert_rows(*gate_up, 2 * I, e)
        dw, ds = expert_rows(*down, H, e)
        if fmt == 0:
            hidden = _swiglu(torch._weight_int8pack_mm(x, gw.view(torch.int8), gs).float()).to(torch.bfloat16)
            outs.append(torch._weight_int8pack_mm(hidden, dw.view(torch.int8), ds).float())
        else:
            hidden = _swiglu(torch.nn.functional.linear(x, dequantize_rows(gw, gs, fmt, H)).float()).to(torch.bfloat16)
            outs.append(torch.nn.functional.linear(hidden, dequantize_rows(dw, ds, fmt, I)).float())
    return weights.float() @ torch.cat(outs)


def grouped_layer(x, ids, weights, gate_up, down, fmt, H, I):
    """Many rows x [T, H] bf16 through their experts ids [T, k] on the CPU, one expert at a time over the rows that
    chose it, as FP8Experts.forward's prompt branch runs (drama3/offload.py:783-802): [T, H] float32."""
    T, k = ids.shape
    flat = ids.reshape(-1)
    out = torch.zeros((T * k, H), dtype=torch.float32)
    for e in torch.unique(flat).tolist():
        sel = (flat == e).nonzero().flatten()
        rows = x[sel // k]
        gw, gs = expert_rows(*gate_up, 2 * I, e)
        dw, ds = expert_rows(*down, H, e)
        if fmt == 0:
            hidden = _swiglu(torch._weight_int8pack_mm(rows, gw.view(torch.int8), gs).float()).to(torch.bfloat16)
            y = torch._weight_int8pack_mm(hidden, dw.view(torch.int8), ds).float()
        else:
            hidden = _swiglu(torch.nn.functional.linear(rows, dequantize_rows(gw, gs, fmt, H)).float()).to(torch.bfloat16)
            y = torch.nn.functional.linear(hidden, dequantize_rows(dw, ds, fmt, I)).float()
        out[sel] = y * weights.reshape(-1)[sel].float()[:, None]
    return out.view(T, k, H).sum(1)


def fp8_rows_linear(x, weight, scale):
    """x [rows, K] bf16 times an FP8 weight [N, K] (float8_e4m3fn) with one bf16 scale per output row, dequantized to
    bf16 on every call and multiplied in bf16 (drama3/offload.py:163-167, then the linear): [rows, N] bf16."""
    wd = (weight.float() * scale.float()[:, None]).to(torch.bfloat16)
    return torch.nn.functional.linear(x, wd)
