"""ctypes binding of libi4moe.so, the C ABI declared in include/i4moe.h.

Only plain pointers, sizes and a hipStream_t cross the boundary.  torch is used
by the callers for device memory and the current stream; nothing here falls
back to a CPU or torch implementation: if the library is missing or was built
for another ABI version, every entry point raises.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libi4moe.so"
ABI_VERSION = 9

# element types and layouts (include/i4moe.h)
F32, F16, BF16 = 0, 1, 2
LAYOUT_CT, LAYOUT_AWQ, LAYOUT_TILE = 0, 1, 2
LAYOUTS = {"ct": LAYOUT_CT, "awq": LAYOUT_AWQ, "tile": LAYOUT_TILE}

_DT = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}


class QWeightC(ctypes.Structure):
    """struct i4_qweight"""

    _fields_ = [
        ("packed", c_void_p),
        ("scale", c_void_p),
        ("zeros", c_void_p),
        ("packed_estride", c_int64),
        ("scale_estride", c_int64),
        ("zeros_estride", c_int64),
        ("layout", c_int32),
        ("group", c_int32),
        ("scale_dtype", c_int32),
        ("E", c_int32),
        ("N", c_int32),
        ("K", c_int32),
    ]


class MoeWeightsC(ctypes.Structure):
    """struct i4_moe_weights"""

    _fields_ = [("gate_up", QWeightC), ("down", QWeightC), ("router_w", c_void_p),
                ("norm_w", c_void_p), ("norm_eps", ctypes.c_float),
                ("gate_up_tile", QWeightC), ("down_tile", QWeightC)]


class DWeightC(ctypes.Structure):
    """struct i4_dweight"""

    _fields_ = [("data", c_void_p), ("scale", c_void_p), ("E", c_int32), ("N", c_int32),
                ("K", c_int32)]


class DmoeWeightsC(ctypes.Structure):
    """struct i4_dmoe_weights"""

    _fields_ = [("gate_up", DWeightC), ("down", DWeightC), ("router_w", c_void_p),
                ("shared_gate_up", DWeightC), ("shared_down", DWeightC),
                ("shared_gate_w", c_void_p)]


class ThinkerLayerC(ctypes.Structure):
    """struct i4_thinker_layer"""

    _fields_ = [("in_norm_w", c_void_p), ("q_norm_w", c_void_p), ("k_norm_w", c_void_p),
                ("k_cache", c_void_p), ("v_cache", c_void_p), ("eps", ctypes.c_float),
                ("qkv", QWeightC), ("o", QWeightC), ("moe", MoeWeightsC)]


# name -> (restype, argtypes); every function declared in include/i4moe.h
SIGNATURES = {
    "i4_abi_version": (c_int, []),
    "i4_strerror": (c_char_p, [c_int]),
    "i4_dq_gemv": (c_int, [c_void_p, c_int, c_int64, POINTER(QWeightC), c_void_p, c_int,
                           c_void_p, c_int, c_void_p, c_size_t, c_void_p]),
    "i4_dq_gemv_workspace_bytes": (c_size_t, [POINTER(QWeightC), c_int]),
    "i4_dq_gemv_bounded": (c_int, [c_void_p, c_int, c_int64, POINTER(QWeightC), c_void_p, c_int,
                                   c_void_p, c_int, c_void_p, c_size_t, c_int, c_int, c_void_p]),
    "i4_linear": (c_int, [c_void_p, c_int, c_int, POINTER(QWeightC), c_void_p, c_void_p, c_int,
                          c_void_p, c_size_t, c_void_p]),
    "i4_linear_workspace_bytes": (c_size_t, [POINTER(QWeightC), c_int]),
    "i4_unpack": (c_int, [POINTER(QWeightC), c_void_p, c_void_p]),
    "i4_dequant": (c_int, [POINTER(QWeightC), c_void_p, c_int, c_void_p]),
    "i4_repack_awq_to_ct": (c_int, [POINTER(QWeightC), c_void_p, c_void_p, c_void_p, c_int, c_int,
                                    c_void_p]),
    "i4_repack_tile": (c_int, [POINTER(QWeightC), c_void_p, c_void_p, c_void_p, c_int, c_int,
                               c_void_p]),
    "i4_router_logits": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, c_int, c_void_p,
                                 ctypes.c_float, c_void_p, c_void_p, c_void_p]),
    "i4_route_topk": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                              c_void_p, c_int, c_void_p]),
    "i4_moe_forward": (c_int, [c_void_p, c_int, c_int, POINTER(MoeWeightsC), c_int, c_int,
                               c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                               c_size_t, c_void_p]),
    "i4_moe_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "i4_moe_forward_bounded": (c_int, [c_void_p, c_int, c_int, POINTER(MoeWeightsC), c_int,
                                       c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_size_t,
                                       c_int, c_int, c_void_p]),
    "i4_moe_status_offset": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "i4_moe_forward_noalloc": (c_int, [c_void_p, c_int, c_int, POINTER(MoeWeightsC), c_int, c_int,
                                       c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_void_p]),
    "i4_moe_down_wait": (c_int, [c_void_p, c_int, POINTER(QWeightC), c_void_p, c_int, c_int, c_int,
                                 c_void_p, c_void_p, c_void_p, c_int, c_void_p]),
    "i4_moe_gate_up": (c_int, [c_void_p, c_int, POINTER(QWeightC), c_void_p, c_int, c_void_p,
                               c_void_p]),
    "i4_moe_route_gate_up": (c_int, [c_void_p, c_int, POINTER(QWeightC), c_void_p, c_int, c_int,
                                     c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "i4_moe_down_combine": (c_int, [c_void_p, c_int, POINTER(QWeightC), c_void_p, c_void_p, c_int,
                                    c_void_p, c_void_p, c_void_p]),
    "i4_moe_stack_forward": (c_int, [c_void_p, c_int, c_int, POINTER(MoeWeightsC), c_int, c_int,
                                     c_int, c_void_p, c_void_p, c_size_t, c_void_p]),
    "i4_moe_stack_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "i4_moe_route_sum": (c_int, [c_void_p, c_int, c_void_p, POINTER(MoeWeightsC), c_int, c_void_p,
                                 c_int, c_void_p, c_size_t, c_void_p]),
    "i4_moe_experts_x": (c_int, [c_void_p, c_int, POINTER(MoeWeightsC), c_int, c_int, c_void_p,
                                 c_int, c_int, c_void_p, c_size_t, c_void_p]),
    "i4_moe_sum": (c_int, [c_void_p, c_int, c_void_p, POINTER(MoeWeightsC), c_int, c_void_p,
                           c_void_p, c_size_t, c_void_p]),
    "i4_rmsnorm_linear": (c_int, [c_void_p, c_int, c_int, c_void_p, ctypes.c_float,
                                  POINTER(QWeightC), c_void_p, c_void_p, c_int, c_void_p]),
    "i4_rmsnorm": (c_int, [c_void_p, c_int, c_int, c_int, c_void_p, ctypes.c_float, c_void_p,
                           c_void_p]),
    "i4_attn_decode": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                               ctypes.c_float, c_void_p, c_int, c_void_p, c_void_p, c_int,
                               c_void_p, c_void_p, c_size_t, c_void_p]),
    "i4_attn_decode_at": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                  ctypes.c_float, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
                                  c_void_p, c_void_p, c_size_t, c_void_p]),
    "i4_attn_decode_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "i4_attn_decode_o": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p,
                                 ctypes.c_float, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                                 c_int, POINTER(QWeightC), c_void_p, c_void_p, c_void_p,
                                 c_size_t, c_void_p]),
    "i4_attn_decode_o_workspace_bytes": (c_size_t, [c_int, c_int, c_int]),
    "i4_attn_decode_o_status_offset": (c_size_t, [c_int, c_int, c_int]),
    "i4_attn_decode_qkv_o": (c_int, [c_void_p, c_int, c_void_p, ctypes.c_float,
                                     POINTER(QWeightC), c_int, c_int, c_int, c_void_p, c_void_p,
                                     c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_int,
                                     POINTER(QWeightC), c_void_p, c_void_p, c_size_t, c_void_p]),
    "i4_attn_decode_qkv_o_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int]),
    "i4_thinker_layer_decode": (c_int, [c_void_p, c_int, c_void_p, ctypes.c_float,
                                        POINTER(QWeightC), c_int, c_int, c_int, c_void_p,
                                        c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p,
                                        c_int, POINTER(QWeightC), POINTER(MoeWeightsC), c_int,
                                        c_int, c_void_p, c_void_p, c_size_t, c_void_p]),
    "i4_thinker_layer_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int,
                                                    c_int, c_int]),
    "i4_thinker_decode_step": (c_int, [c_void_p, c_int, POINTER(ThinkerLayerC), c_int, c_int,
                                       c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_int,
                                       c_int, c_void_p, c_void_p, c_size_t, c_void_p]),
    "i4_thinker_decode_step_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int,
                                                          c_int, c_int, c_int]),
    "i4_dmoe_forward": (c_int, [c_void_p, c_int, c_int, POINTER(DmoeWeightsC), c_int, c_int,
                                c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_size_t, c_void_p]),
    "i4_dmoe_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "i4_dmoe_status_offset": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "i4_dmoe_down_wait": (c_int, [c_void_p, c_int, POINTER(DmoeWeightsC), c_int, c_int,
                                  c_void_p, c_void_p, c_void_p, c_void_p, c_size_t, c_int,
                                  c_void_p]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """Load libi4moe.so once and declare every signature."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built: run __graft_entry__.build() (hipcc, gfx950) first")
        lb = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lb, name)
            fn.restype = res
            fn.argtypes = args
        ver = lb.i4_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"libi4moe ABI {ver}, package expects {ABI_VERSION}")
        _lib = lb
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(lib().i4_strerror(rc).decode())


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DT[dt]
    except KeyError:
        raise RuntimeError(f"unsupported dtype {dt}") from None


def half_code(dt: torch.dtype) -> int:
    if dt not in (torch.float16, torch.bfloat16):
        raise RuntimeError(f"activations must be float16 or bfloat16, got {dt}")
    return _DT[dt]


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*ts: torch.Tensor | None) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError("libi4moe operates on HIP device tensors only "
                               f"(got a tensor on {t.device})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("all tensors must be on the same device")
    if dev is None:
        raise RuntimeError("no device tensor given")
    return dev
