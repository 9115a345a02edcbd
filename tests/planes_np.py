"""numpy restatement of the int8-plane split of d3_prep_planes_i8, for the tests: the GPU test compares the kernel's
planes with it bit for bit, and test_planes_np.py pins it by the bounds the split must meet."""
import numpy as np


def split_i8_np(v):
    """(a0, a1, a2 float32 [P, K], S [P]) of float32 rows v [P, K] as d3_prep_planes_i8 splits them: S the smallest
    power of two with max |v| <= 127 S, a0 = rint(v / S), d = v / S - a0, a1 = rint(f32(254 d)), a2 = rint(f32(254
    f32(254 d - a1))) with 254 d - a1 from the exact product (float64 holds it). An all-zero row gets S = 0, a row
    holding inf or NaN S = NaN, both with zero planes."""
    v = np.asarray(v, np.float32)
    finite = np.isfinite(v).all(axis=1)
    m = np.where(finite, np.abs(np.where(np.isfinite(v), v, 0)).max(axis=1), 0).astype(np.float32)
    split = finite & (m > 0)
    m = np.where(split, m, np.float32(1))
    v = np.where(split[:, None], v, np.float32(0))
    e = np.frexp(m)[1].astype(np.int64) - 7
    e = np.maximum(e, -149)
    e = np.where(m > np.ldexp(np.float32(127), e).astype(np.float32), e + 1, e)
    a = np.ldexp(v, -e[:, None]).astype(np.float32)
    a0 = np.rint(a)
    d = (a - a0).astype(np.float32)
    a1 = np.rint((d * np.float32(254)).astype(np.float32))
    r2 = (d.astype(np.float64) * 254 - a1).astype(np.float32)
    a2 = np.rint((r2 * np.float32(254)).astype(np.float32))
    S = np.where(split, np.ldexp(np.float32(1), e), np.where(finite, np.float32(0), np.float32(np.nan)))
    return a0, a1, a2, S.astype(np.float32)
