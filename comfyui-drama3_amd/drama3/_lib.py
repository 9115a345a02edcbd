"""ctypes binding of libdrama3_moe.so, the gfx950 kernels behind kernels.py and moe.py.

Replaces the reference's NVRTC path (drama3/kernels.py:593-601: `_kernel` compiles SOURCE per device, `_launch` runs
it on torch.cuda.current_stream). Here the kernels are compiled ahead of time into one shared library with a C ABI
(include/drama3_moe.h); every entry point takes device pointers, sizes and the HIP stream.

torch is imported first: the library's HIP runtime dependency (libamdhip64.so.7) then resolves to the runtime torch
already loaded, so both share devices and streams.
"""
import ctypes
import functools
import os
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "_lib" / "libdrama3_moe.so"
DECODE_TABLE_W4 = 0x104  # d3_decode_codes: 4-bit rows through the resident kernels' tables (D3_DECODE_TABLE_W4)

c_int32, c_int64, c_uint32, c_void_p = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_void_p


class MoeA8Desc(ctypes.Structure):
    """d3_moe_a8_desc (include/drama3_moe.h)."""
    _fields_ = [
        ("x", c_void_p), ("logits", c_void_p), ("gate_up", c_void_p), ("gate_up_scale", c_void_p),
        ("down", c_void_p), ("down_scale", c_void_p), ("out", c_void_p), ("ids_out", c_void_p),
        ("weights_out", c_void_p), ("workspace", c_void_p), ("workspace_bytes", c_int64), ("format", c_int32),
        ("M", c_int32), ("H", c_int32), ("I", c_int32), ("E", c_int32), ("topk", c_int32), ("spin_limit", c_uint32),
        ("grid", c_int32), ("router", c_void_p), ("logits_out", c_void_p), ("shared_gate_up", c_void_p),
        ("shared_gate_up_scale", c_void_p), ("shared_down", c_void_p), ("shared_down_scale", c_void_p),
        ("shared_gate", c_void_p), ("item_units", c_int32), ("recompute_all", c_int32),
    ]


class MoeA8PrefillDesc(ctypes.Structure):
    """d3_moe_a8_prefill_desc (include/drama3_moe.h)."""
    _fields_ = [
        ("x", c_void_p), ("logits", c_void_p), ("ids_in", c_void_p), ("weights_in", c_void_p), ("gate_up", c_void_p),
        ("gate_up_scale", c_void_p), ("down", c_void_p), ("down_scale", c_void_p), ("out", c_void_p),
        ("ids_out", c_void_p), ("weights_out", c_void_p), ("workspace", c_void_p), ("workspace_bytes", c_int64),
        ("format", c_int32), ("T", c_int32), ("H", c_int32), ("I", c_int32), ("E", c_int32), ("topk", c_int32),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "d3_last_error": (ctypes.c_char_p, []),
    "d3_version": (c_int32, []),
    "d3_moe_a8_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32, c_int32]),
    "d3_moe_a8": (c_int32, [ctypes.POINTER(MoeA8Desc), c_void_p]),
    "d3_moe_a8_noalloc": (c_int32, [ctypes.POINTER(MoeA8Desc), c_void_p]),
    "d3_moe_a8_status": (c_int32, [c_void_p, ctypes.POINTER(c_uint32)]),
    "d3_moe_a8_noalloc_status": (c_int32, [ctypes.POINTER(c_uint32)]),
    "d3_moe_a8_prefill_workspace_bytes": (c_int64, [c_int32, c_int32, c_int32, c_int32, c_int32]),
    "d3_moe_a8_prefill": (c_int32, [ctypes.POINTER(MoeA8PrefillDesc), c_void_p]),
    "d3_gemv_a8_groups": (c_int32, [c_int32, c_void_p, c_int32, c_int32, c_void_p, c_int32, c_void_p, c_void_p]),
    "d3_unpack_rows": (c_int32, [c_int32, c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
    "d3_cvt_fp8": (c_int32, [c_void_p, c_int32, c_void_p, c_int32, c_void_p]),
    "d3_stream_read": (c_int32, [c_void_p, c_int64, c_void_p, c_int32, c_void_p]),
    "d3_router_logits": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p]),
    "d3_block_combine": (c_int32, [c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
    "d3_empty_launch": (c_int32, [c_int32, c_void_p]),
    "d3_gemv_fp8_rows": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "d3_route": (c_int32, [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "d3_weighted_sum": (c_int32, [c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
    "d3_rotate": (c_int32, [c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "d3_gemv_int8": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                               c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p]),
    "d3_gemv_fp8": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                              c_int32, c_int32, c_int32, c_void_p]),
    "d3_gemv_codes": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_int32, c_void_p, c_int32, c_int32, c_int32, c_void_p]),
    "d3_grouped": (c_int32, [c_int32, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                             c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "d3_split_bf16x3": (c_int32, [c_void_p, c_int64, c_void_p, c_void_p]),
    "d3_grouped_mfma_work_ints": (c_int64, [c_int32, c_int64]),
    "d3_grouped_plan": (c_int32, [c_void_p, c_int32, c_int64, c_void_p, c_int64, c_void_p]),
    "d3_grouped_fp8": (c_int32, [c_void_p, c_int32, c_int64, c_void_p, c_int32, c_int32, c_void_p, c_int32, c_void_p,
                                 c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32, c_int32,
                                 c_void_p]),
    "d3_expert_groups": (c_int32, [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                   c_void_p]),
    "d3_prep_planes": (c_int32, [c_int32, c_int32, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p,
                                 c_void_p]),
    "d3_prep_planes_i8": (c_int32, [c_int32, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p,
                                    c_void_p, c_void_p]),
    "d3_expert_groups_prep_i8": (c_int32, [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
                                           c_int32, c_int32, c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "d3_grouped_i8": (c_int32, [c_int32, c_void_p, c_void_p, c_int64, c_void_p, c_int32, c_int32, c_void_p, c_int32,
                                c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "d3_combine_rows": (c_int32, [c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p,
                                  c_int32, c_void_p]),
    "d3_decode_codes": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
    "d3_resident_decode": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
                                     c_int32, c_void_p]),
    "d3_resident_decode_routed": (c_int32, [c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p,
                                            c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                            c_void_p, c_void_p, c_void_p, c_int32, c_int32, c_void_p]),
    "d3_resident_workspace_bytes": (c_int64, [c_int32, c_int32]),
    "d3_resident_decode_fused": (c_int32, [c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p,
                                           c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                           c_void_p, c_void_p, c_int64, ctypes.c_uint32, c_int32, c_int32, c_void_p,
                                           c_int32, c_int32, c_void_p]),
    "d3_resident_status": (c_int32, [c_void_p, c_void_p]),
    "d3_resolve": (c_int32, [c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
                             c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                             ctypes.c_double, c_int32, ctypes.c_double, c_void_p]),
    "d3_await_cpu": (c_int32, [c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int32,
                               c_void_p]),
}

_lock = threading.Lock()


@functools.cache
def lib():
    """The loaded library; raises if it was not built (python comfyui-drama3_amd/csrc/build.py)."""
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is missing: build it with comfyui-drama3_amd/csrc/build.py")
    with _lock:
        handle = ctypes.CDLL(os.fspath(LIB_PATH))
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype, fn.argtypes = restype, argtypes
    return handle


def check(rc, what):
    """Raise RuntimeError for a non-zero return code of entry point `what`."""
    if rc != 0:
        message = lib().d3_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {message}")


def ptr(tensor):
    """Device (or pinned host) address of a tensor, or None for None."""
    return None if tensor is None else tensor.data_ptr()


def stream_of(device):
    """The HIP stream handle of torch's current stream on `device`."""
    return c_void_p(torch.cuda.current_stream(device).cuda_stream)
