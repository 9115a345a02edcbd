"""The converted-checkpoint loader (drama3/loader.py) on files laid out as the reference's tools/convert.py:179-216
writes them: a file assembled by hand here, key by key, loads into the kernels' field dicts; write_experts and
load_experts round-trip every format bit for bit. CPU only."""
import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from drama3 import loader
from oracle import reference as ref

E, N, K = 4, 256, 512


def conf_tensor(conf):
    return torch.tensor(list(json.dumps(conf).encode()), dtype=torch.uint8)


def test_hand_built_w4a8_file(tmp_path):
    """Keys, dtypes and shapes as convert.py's w4a8_bank / write produce them (weight [E, N, K/2] uint8, s_rel as
    uint8 e4m3 [E, N, K/16], s_channel float32 [E, N], codebook [16], comfy_quant JSON bytes)."""
    rng = np.random.default_rng(0)
    tensors = {}
    want = {}
    for bank, (n, k) in (("gate_up", (2 * N, K)), ("down", (K, N))):
        q = rng.integers(0, 256, size=(E, n, k // 2), dtype=np.uint8)
        s = rng.integers(0x20, 0x40, size=(E, n, k // 16), dtype=np.uint8)
        c = rng.uniform(1e-3, 1e-2, size=(E, n)).astype(np.float32)
        cb = np.linspace(-8, 7, 16).astype(np.float32)
        m = f"model.layers.3.mlp.experts.{bank}_proj."
        tensors[m + "weight"] = torch.from_numpy(q)
        tensors[m + "weight_s_rel"] = torch.from_numpy(s)
        tensors[m + "weight_s_channel"] = torch.from_numpy(c)
        tensors[m + "weight_codebook"] = torch.from_numpy(cb)
        tensors[m + "comfy_quant"] = conf_tensor({"format": "asym_w4a8_int8", "group_size": 16, "convrot_groupsize": 256,
                                                  "num_experts": E})
        want[bank] = (q.reshape(E * n, -1), s.reshape(E * n, -1), c.reshape(-1), cb)
    path = tmp_path / "w4.safetensors"
    save_file(tensors, str(path), metadata={"drama3_format": "w4a8", "drama3_config": "{}"})
    assert loader.expert_layers(path) == [3]
    kind, banks, cbs = loader.load_layer(path, 3)
    assert kind == "w4"
    for bank, fields, cb in zip(("gate_up", "down"), banks, cbs):
        q, s, c, table = want[bank]
        assert np.array_equal(fields["_qdata"].numpy(), q) and np.array_equal(fields["scale"].numpy(), s)
        assert np.array_equal(fields["s_channel"].numpy(), c) and np.array_equal(cb.numpy(), table)


def test_hand_built_fp8_and_int8_files(tmp_path):
    rng = np.random.default_rng(1)
    w = rng.integers(0, 0x7E, size=(E, 2 * N, K), dtype=np.uint8)
    sc = rng.uniform(0.5, 2, size=(E, 2 * N // 128, K // 128)).astype(np.float32)
    tensors = {"model.layers.0.mlp.experts.gate_up_weight": torch.from_numpy(w).view(torch.float8_e4m3fn),
               "model.layers.0.mlp.experts.gate_up_scale": torch.from_numpy(sc),
               "model.layers.0.mlp.experts.down_weight": torch.from_numpy(w[:, :K, :N].copy()).view(torch.float8_e4m3fn),
               "model.layers.0.mlp.experts.down_scale": torch.from_numpy(sc[:, :K // 128, :N // 128].copy())}
    path = tmp_path / "fp8.safetensors"
    save_file(tensors, str(path), metadata={"drama3_format": "fp8", "drama3_config": "{}"})
    kind, (gu, dn), _ = loader.load_layer(path, 0)
    assert kind == "fp8" and gu["weight"].dtype == torch.uint8 and gu["weight"].shape == (E * 2 * N, K)
    assert np.array_equal(gu["weight"].numpy(), w.reshape(E * 2 * N, K))
    assert np.array_equal(gu["scale"].numpy(), sc.reshape(E * 2 * N // 128, K // 128))

    q = rng.integers(-127, 128, size=(E, 2 * N, K), dtype=np.int8)
    s = rng.uniform(1e-3, 1e-2, size=(E, 2 * N, 1)).astype(np.float32)  # int8_convrot's [out, 1] scales
    tensors = {}
    for bank, (qq, ss) in (("gate_up", (q, s)), ("down", (q[:, :K, :N].copy(), s[:, :K].copy()))):
        m = f"model.layers.1.mlp.experts.{bank}_proj."
        tensors[m + "weight"] = torch.from_numpy(qq)
        tensors[m + "weight_scale"] = torch.from_numpy(ss)
        tensors[m + "comfy_quant"] = conf_tensor({"format": "int8_tensorwise", "convrot": True,
                                                  "convrot_groupsize": 256, "num_experts": E})
    path = tmp_path / "int8.safetensors"
    save_file(tensors, str(path), metadata={"drama3_format": "int8", "drama3_config": "{}"})
    kind, (gu, dn), _ = loader.load_layer(path, 1)
    assert kind == "int8" and gu["_qdata"].dtype == torch.int8
    assert np.array_equal(gu["_qdata"].numpy(), q.reshape(E * 2 * N, K))
    assert np.array_equal(gu["scale"].numpy(), s.reshape(-1)) and dn["scale"].shape == (E * K,)


@pytest.mark.parametrize("kind", ["fp8", "int8", "w4", "w6"])
def test_write_load_round_trip(tmp_path, kind):
    rng = np.random.default_rng(2)
    layers = {}
    for layer in (0, 2):
        gu = rng.standard_normal((E, 2 * N, K)) * 0.02
        dn = rng.standard_normal((E, K, N)) * 0.02
        if kind == "fp8":
            banks, cbs = (ref.quantize_fp8_block(gu), ref.quantize_fp8_block(dn)), (None, None)
        elif kind == "int8":
            banks, cbs = (ref.quantize_int8_convrot(gu), ref.quantize_int8_convrot(dn)), (None, None)
        else:
            (a, ca), (b, cb) = ref.quantize_codes(gu, int(kind[1])), ref.quantize_codes(dn, int(kind[1]))
            banks, cbs = (a, b), (ca, cb)
        layers[layer] = (tuple({n: torch.from_numpy(np.ascontiguousarray(v)) for n, v in b.items()} for b in banks),
                         tuple(None if c is None else torch.from_numpy(c) for c in cbs))
    path = tmp_path / f"{kind}.safetensors"
    loader.write_experts(path, kind, layers, {"num_experts": E})
    got = loader.load_experts(path)
    assert sorted(got) == [0, 2]
    for layer, (banks, cbs) in layers.items():
        k2, banks2, cbs2 = got[layer]
        assert k2 == kind
        for f1, f2 in zip(banks, banks2):
            assert set(f1) == set(f2)
            for n in f1:
                assert torch.equal(f1[n].reshape(f2[n].shape).view(f2[n].dtype), f2[n]), n
        for c1, c2 in zip(cbs, cbs2):
            assert (c1 is None) == (c2 is None) and (c1 is None or torch.equal(c1, c2))


def test_rejects_other_files(tmp_path):
    path = tmp_path / "x.safetensors"
    save_file({"a": torch.zeros(1)}, str(path), metadata={"format": "pt"})
    with pytest.raises(ValueError):
        loader.load_layer(path, 0)
