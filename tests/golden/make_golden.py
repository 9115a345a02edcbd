"""Writes the golden fixtures of tests/test_golden.py: small seeded inputs and the oracle's outputs (oracle/), as
.npz files without pickles. The reference's own tests hold no vectors for this path, so these pin the oracle against
regressions and give the kernels fixed cases to meet.

    python tests/golden/make_golden.py
"""
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "comfyui-drama3_amd"))

from oracle import a8, numerics  # noqa: E402
from oracle import reference as ref  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent


def save(name, **arrays):
    np.savez_compressed(OUT / f"{name}.npz", **arrays)
    print(name, {k: v.shape for k, v in arrays.items()})


def main():
    rng = np.random.default_rng(2024)
    # routing: 6 rows of 128 logits with many ties (kernels.py:39-67)
    v = (rng.integers(-5, 5, size=(6, 128)) * 0.375).astype(np.float32)
    logits = numerics.f32_to_bf16_bits(v)
    ids, w = ref.route_ref(logits, 8)
    save("route", logits=logits, k=np.int32(8), ids=ids, weights=w)

    # rotation, float rows and SwiGLU rows (kernels.py:222-258)
    x = rng.standard_normal((3, 512)).astype(np.float32)
    gu = rng.standard_normal((2, 1024)).astype(np.float32)
    save("rotate", x=x, out=ref.rotate_ref(x).astype(np.float32), gate_up=gu,
         swiglu_out=ref.rotate_ref(gu, swiglu=True).astype(np.float32))

    # W4A8 / W6A8 decode to the int8 grid (kernels.py:466-483), every code with a spread of scale bytes
    cb = ref.default_codebook()
    for bits in (4, 6):
        K = 512
        q = rng.integers(0, 256, size=(8, K * bits // 8)).astype(np.uint8)
        s = rng.integers(0, 0x7F, size=(8, K // 16)).astype(np.uint8)
        save(f"decode_w{bits}", qdata=q, scale=s, codebook=cb, codes=ref.decode_codes_ref(q, s, bits, cb))

    # gemv_int8 with a slot plan (kernels.py:260-314): cached, filling, slot-less and CPU experts
    E, N, K, slots = 5, 32, 256, 3
    host_q = rng.integers(-127, 128, size=(E * N, K), dtype=np.int8)
    host_s = rng.uniform(1e-3, 1e-2, size=E * N).astype(np.float32)
    slot = {"_qdata": np.zeros((slots * N, K), np.int8), "scale": np.zeros(slots * N, np.float32)}
    slot["_qdata"][N:2 * N] = host_q[4 * N:5 * N]
    slot["scale"][N:2 * N] = host_s[4 * N:5 * N]
    xg = rng.standard_normal((1, K)).astype(np.float32)
    gids = np.array([4, 2, 3, 0])
    plan = np.array([[1, 0], [2, 1], [-1, 1], [0, 2]], np.int32)
    slot_q0, slot_s0 = slot["_qdata"].copy(), slot["scale"].copy()
    out = ref.gemv_int8_ref(xg, gids, plan, False, False, slot, {"_qdata": host_q, "scale": host_s}, N)
    save("gemv_int8", x=xg, ids=gids, plan=plan, host_q=host_q, host_s=host_s, slot_q=slot_q0, slot_s=slot_s0,
         out=out, slot_q_after=slot["_qdata"], slot_s_after=slot["scale"])

    # A8 formats: unpacked codes and exact group dot products (the fused kernel's MFMA step)
    for fmt, name in ((a8.FMT_I8, "i8"), (a8.FMT_W4, "w4"), (a8.FMT_W6, "w6"), (a8.FMT_F8, "f8")):
        K = 768
        rows = rng.integers(0, 256, size=(32, a8.row_bytes(fmt, K))).astype(np.uint8)
        if fmt == a8.FMT_F8:
            rows[(rows & 0x7F) == 0x7F] = 0x38
            act = rng.integers(0, 256, size=(5, K)).astype(np.uint8)
            act[(act & 0x7F) == 0x7F] = 0x38
        else:
            act = rng.integers(-127, 128, size=(5, K)).astype(np.int8)
        save(f"a8_{name}", rows=rows, act=act, codes=a8.codes(rows, fmt), dots=a8.group_dots(rows, fmt, act))


if __name__ == "__main__":
    main()
