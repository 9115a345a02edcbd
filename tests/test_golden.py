"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): the oracle must reproduce them (CPU),
and the kernels must meet them (GPU) to the same bars as the parity tests."""
import pathlib

import numpy as np
import pytest
import torch

from oracle import a8, numerics
from oracle import reference as ref

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
A8 = [("i8", a8.FMT_I8), ("w4", a8.FMT_W4), ("w6", a8.FMT_W6), ("f8", a8.FMT_F8)]


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


# ------------------------------------------------------------------------------------------- the oracle (CPU)
def test_oracle_route():
    g = load("route")
    ids, w = ref.route_ref(g["logits"], int(g["k"]))
    assert np.array_equal(ids, g["ids"]) and np.array_equal(w, g["weights"])


def test_oracle_rotate():
    g = load("rotate")
    assert np.allclose(ref.rotate_ref(g["x"]), g["out"], rtol=0, atol=1e-6)
    assert np.allclose(ref.rotate_ref(g["gate_up"], swiglu=True), g["swiglu_out"], rtol=0, atol=1e-6)


@pytest.mark.parametrize("bits", [4, 6])
def test_oracle_decode(bits):
    g = load(f"decode_w{bits}")
    assert np.array_equal(ref.decode_codes_ref(g["qdata"], g["scale"], bits, g["codebook"]), g["codes"])


def test_oracle_gemv_int8():
    g = load("gemv_int8")
    slot = {"_qdata": g["slot_q"].copy(), "scale": g["slot_s"].copy()}
    out = ref.gemv_int8_ref(g["x"], g["ids"], g["plan"], False, False, slot,
                            {"_qdata": g["host_q"], "scale": g["host_s"]}, g["out"].shape[1])
    assert np.allclose(out, g["out"], rtol=1e-12, atol=0)
    assert np.array_equal(slot["_qdata"], g["slot_q_after"]) and np.array_equal(slot["scale"], g["slot_s_after"])


@pytest.mark.parametrize("name,fmt", A8)
def test_oracle_a8(name, fmt):
    g = load(f"a8_{name}")
    assert np.array_equal(a8.codes(g["rows"], fmt), g["codes"])
    assert np.array_equal(a8.group_dots(g["rows"], fmt, g["act"]), g["dots"])


# ------------------------------------------------------------------------------------------- the kernels (GPU)
DEV = torch.device("cuda:0")


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.gpu
def test_kernels_route():
    from drama3 import kernels
    g = load("route")
    ids, w = kernels.route(dev(g["logits"]).view(torch.bfloat16), int(g["k"]))
    assert np.array_equal(ids.cpu().numpy(), g["ids"])
    assert np.all(np.abs(w.cpu().numpy() - g["weights"]) <= 2.0 ** -8 * g["weights"] + 1e-7)


@pytest.mark.gpu
def test_kernels_rotate():
    from drama3 import kernels
    g = load("rotate")
    always = torch.ones(1, dtype=torch.int32, device=DEV)
    got = kernels.rotate(dev(g["x"]), always).cpu().numpy()
    assert np.abs(got - g["out"]).max() <= 2e-6 * np.abs(g["out"]).max()
    got = kernels.rotate(dev(g["gate_up"]), always, swiglu=True).cpu().numpy()
    assert np.abs(got - g["swiglu_out"]).max() <= 2e-6 * np.abs(g["swiglu_out"]).max()


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [4, 6])
def test_kernels_decode(bits):
    from drama3 import kernels
    g = load(f"decode_w{bits}")
    got = kernels.decode_codes(dev(g["qdata"]), dev(g["scale"]), dev(g["codebook"]), bits).cpu().numpy()
    assert np.array_equal(got, g["codes"])


@pytest.mark.gpu
def test_kernels_gemv_int8():
    from drama3 import kernels
    g = load("gemv_int8")
    n = g["out"].shape[1]
    slot = {"_qdata": dev(g["slot_q"]), "scale": dev(g["slot_s"])}
    host = {"_qdata": dev(g["host_q"]), "scale": dev(g["host_s"])}
    took = torch.zeros(1, dtype=torch.int32, device=DEV)
    got = kernels.gemv_int8(dev(g["x"]), dev(g["ids"]), dev(g["plan"]), took, False, slot, host, n).cpu().numpy()
    absw = np.abs(g["host_q"].astype(np.float64)) * g["host_s"][:, None]
    for j, e in enumerate(g["ids"]):
        bound = 3e-5 * (absw[e * n:(e + 1) * n] @ np.abs(g["x"][0])) + 1e-30
        assert np.all(np.abs(got[j] - g["out"][j]) <= bound)
    assert np.array_equal(slot["_qdata"].cpu().numpy(), g["slot_q_after"])
    assert np.array_equal(slot["scale"].cpu().numpy(), g["slot_s_after"])


@pytest.mark.gpu
@pytest.mark.parametrize("name,fmt", A8)
def test_kernels_a8(name, fmt):
    from drama3 import moe
    g = load(f"a8_{name}")
    K = g["act"].shape[1]
    if fmt in (a8.FMT_W4, a8.FMT_W6):
        assert np.array_equal(moe.unpack_rows(dev(g["rows"]), fmt, K).cpu().numpy(), g["codes"])
    got = moe.gemv_groups(dev(g["rows"]), fmt, K, dev(g["act"])).cpu().numpy()
    if fmt == a8.FMT_F8:
        assert np.abs(got - g["dots"]).max() <= 1e-4 * np.abs(g["dots"]).max()
    else:
        assert np.array_equal(got.astype(np.int64), g["dots"])
