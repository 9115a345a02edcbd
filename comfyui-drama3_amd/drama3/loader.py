"""The expert banks of a converted Drama 3 checkpoint (the reference's tools/convert.py output, read by its
drama3/loader.py:106-137), loaded into the field dicts the kernels read, without ComfyUI.

Keys and layouts per layer l, as tools/convert.py:179-216 writes them (E experts stacked on the first dimension):
  fp8    model.layers.l.mlp.experts.{gate_up,down}_weight   float8_e4m3fn [E, N, K]
         model.layers.l.mlp.experts.{gate_up,down}_scale    float32 [E, N / 128, K / 128]
  int8   model.layers.l.mlp.experts.{gate_up,down}_proj.weight        int8 [E, N, K]   (ConvRot basis)
                                                       .weight_scale  float32 [E, N, 1]
                                                       .comfy_quant   uint8 JSON {"format": "int8_tensorwise", ...}
  w4/w6  ...{gate_up,down}_proj.weight             uint8 [E, N, K * bits / 8]  (nibble plane, then 2-bit planes)
                               .weight_s_rel       uint8 (e4m3) [E, N, K / 16]
                               .weight_s_channel   float32 [E, N] (or [E, N, 1])
                               .weight_codebook    float32 [16] (4 bits only)
                               .comfy_quant        uint8 JSON {"format": "asym_w4a8_int8" | "w6a8_int8", ...}
and the file's metadata "drama3_format" (fp8, int8, w4a8, w6a8) and "drama3_config" (the model config JSON).

Banks come back flat ([E * N, ...], the slot-cache layout the kernels index, offload.py:72-90): {"weight", "scale"}
for fp8, {"_qdata", "scale"} for int8, {"_qdata", "scale", "s_channel"} plus a codebook for w4 / w6. Files are read
with safetensors (nothing executes from a file).
"""
import json

import torch
from safetensors import safe_open

PREFIX = "model.layers.{layer}.mlp.experts."
KINDS = {"fp8": "fp8", "int8": "int8", "w4a8": "w4", "w6a8": "w6"}
QUANT_FORMATS = {"int8_tensorwise": "int8", "asym_w4a8_int8": "w4", "w6a8_int8": "w6"}


def read_metadata(path):
    with safe_open(str(path), framework="pt") as f:
        return f.metadata() or {}


def file_kind(path):
    """The expert format of a converted file ("fp8", "int8", "w4", "w6")."""
    meta = read_metadata(path)
    fmt = meta.get("drama3_format")
    if fmt not in KINDS:
        raise ValueError(f"{path} is not a converted Drama 3 file (drama3_format {fmt!r})")
    return KINDS[fmt]


def expert_layers(path):
    """Layer numbers that hold expert banks."""
    layers = set()
    with safe_open(str(path), framework="pt") as f:
        for key in f.keys():
            if ".mlp.experts." in key and key.startswith("model.layers."):
                layers.add(int(key.split(".")[2]))
    return sorted(layers)


def _flat(t):
    return t.reshape(t.shape[0] * t.shape[1], *t.shape[2:])


def load_layer(path, layer, device="cpu"):
    """(kind, (gate_up fields, down fields), (gate_up codebook, down codebook)) of one layer's expert banks."""
    kind = file_kind(path)
    p = PREFIX.format(layer=layer)
    banks, codebooks = [], []
    with safe_open(str(path), framework="pt", device="cpu") as f:
        for bank in ("gate_up", "down"):
            if kind == "fp8":
                weight = f.get_tensor(f"{p}{bank}_weight")
                scale = f.get_tensor(f"{p}{bank}_scale")
                fields = {"weight": _flat(weight.view(torch.uint8)), "scale": _flat(scale.float())}
                cb = None
            else:
                m = f"{p}{bank}_proj."
                conf = json.loads(bytes(f.get_tensor(m + "comfy_quant").tolist()).decode())
                if QUANT_FORMATS.get(conf.get("format")) != kind:
                    raise ValueError(f"layer {layer} {bank}: comfy_quant format {conf.get('format')!r} in a {kind} file")
                if conf.get("convrot_groupsize", 256) != 256:
                    raise ValueError("the kernels take ConvRot groups of 256")
                qdata = f.get_tensor(m + "weight")
                if kind == "int8":
                    fields = {"_qdata": _flat(qdata.view(torch.int8)),
                              "scale": _flat(f.get_tensor(m + "weight_scale").float()).reshape(-1)}
                    cb = None
                else:
                    if conf.get("group_size", 16) != 16:
                        raise ValueError("the kernels take W4A8 / W6A8 scale groups of 16")
                    fields = {"_qdata": _flat(qdata.view(torch.uint8)),
                              "scale": _flat(f.get_tensor(m + "weight_s_rel").view(torch.uint8)),
                              "s_channel": _flat(f.get_tensor(m + "weight_s_channel").float()).reshape(-1)}
                    keys = set(f.keys())
                    cb = f.get_tensor(m + "weight_codebook").float() if m + "weight_codebook" in keys else None
                    if (kind == "w4") != (cb is not None):
                        raise ValueError("4-bit banks carry a codebook, 6-bit banks none")
            banks.append({n: t.to(device).contiguous() for n, t in fields.items()})
            codebooks.append(None if cb is None else cb.to(device))
    return kind, tuple(banks), tuple(codebooks)


def load_experts(path, device="cpu", layers=None):
    """{layer: (kind, banks, codebooks)} for every expert layer of the file (or `layers`)."""
    return {layer: load_layer(path, layer, device) for layer in (layers if layers is not None else expert_layers(path))}


def write_experts(path, kind, layers, config=None):
    """Write banks in the converted-file layout (the inverse of load_layer): layers = {layer: ((gate_up fields, down
    fields), (codebooks)), ...} with flat fields and `experts` rows per bank given by the fields' first dimension /
    experts in config["num_experts"]."""
    from safetensors.torch import save_file
    experts = int(config["num_experts"])
    out = {}
    for layer, (banks, codebooks) in layers.items():
        p = PREFIX.format(layer=layer)
        for bank, fields, cb in zip(("gate_up", "down"), banks, codebooks):
            def stack(t):
                return t.reshape(experts, t.shape[0] // experts, *t.shape[1:]).contiguous()
            if kind == "fp8":
                out[f"{p}{bank}_weight"] = stack(fields["weight"]).view(torch.float8_e4m3fn)
                out[f"{p}{bank}_scale"] = stack(fields["scale"].float())
                continue
            m = f"{p}{bank}_proj."
            if kind == "int8":
                out[m + "weight"] = stack(fields["_qdata"].view(torch.int8))
                out[m + "weight_scale"] = stack(fields["scale"].float().reshape(-1, 1))
                conf = {"format": "int8_tensorwise", "convrot": True, "convrot_groupsize": 256, "num_experts": experts}
            else:
                out[m + "weight"] = stack(fields["_qdata"])
                out[m + "weight_s_rel"] = stack(fields["scale"])
                out[m + "weight_s_channel"] = stack(fields["s_channel"].float().reshape(-1))
                if cb is not None:
                    out[m + "weight_codebook"] = cb.float().contiguous()
                conf = {"format": "asym_w4a8_int8" if kind == "w4" else "w6a8_int8", "group_size": 16,
                        "convrot_groupsize": 256, "num_experts": experts}
            out[m + "comfy_quant"] = torch.tensor(list(json.dumps(conf).encode()), dtype=torch.uint8)
    fmt = {v: k for k, v in KINDS.items()}[kind]
    save_file(out, str(path), metadata={"drama3_format": fmt, "drama3_config": json.dumps(config or {})})
