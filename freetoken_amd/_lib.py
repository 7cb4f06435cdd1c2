"""ctypes binding of ``libftmoe.so`` (the C ABI declared in include/ftmoe.h).

The library is built in-tree by ``freetoken_amd.build``; there is no fallback:
if it is missing or fails to load, every entry point raises.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libftmoe.so"

FTMOE_OK = 0
FTMOE_ERR_INVALID = -1
FTMOE_ERR_UNSUPPORTED = -2
FTMOE_ERR_HIP = -3
FTMOE_ERR_WORKSPACE = -4
FTMOE_ERR_BUSY = -5
FTMOE_ERR_TIMEOUT = -6

DTYPE_F32, DTYPE_BF16 = 0, 1
FMT_NONE, FMT_BF16, FMT_FP8_B128, FMT_MXFP4 = -1, 0, 1, 2
ACT = {"silu": 0, "gelu": 1, "gelu_tanh": 2}

# Every symbol include/ftmoe.h declares, with (restype, argtypes).
_vp, _i, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
_ip = ctypes.POINTER(ctypes.c_int)


class FtmoeBank(ctypes.Structure):
    _fields_ = [
        ("format", ctypes.c_int),
        ("num_rows", ctypes.c_int),
        ("hidden", ctypes.c_int),
        ("inter", ctypes.c_int),
        ("gate_up", ctypes.c_void_p),
        ("gate_up_scale", ctypes.c_void_p),
        ("down", ctypes.c_void_p),
        ("down_scale", ctypes.c_void_p),
        ("swiglu_limit", ctypes.c_float),
    ]


_bp = ctypes.POINTER(FtmoeBank)


ROUTER_SOFTMAX_TOPK, ROUTER_GROUPED_SIGMOID = 0, 1


class FtmoeRouter(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int),
        ("logits", ctypes.c_void_p),
        ("logits_dtype", ctypes.c_int),
        ("num_experts", ctypes.c_int),
        ("renormalize", ctypes.c_int),
        ("bias", ctypes.c_void_p),
        ("n_group", ctypes.c_int),
        ("topk_group", ctypes.c_int),
        ("routed_scaling_factor", ctypes.c_float),
    ]


class FtmoeFetchBank(ctypes.Structure):
    _fields_ = [
        ("host_rows", ctypes.c_void_p),
        ("slot_bank", ctypes.c_void_p),
        ("row_bytes", ctypes.c_size_t),
    ]


_fbp = ctypes.POINTER(FtmoeFetchBank)

SIGNATURES = {
    "ftmoe_last_error": (ctypes.c_char_p, []),
    "ftmoe_version": (_i, []),
    "ftmoe_route_softmax_topk": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp]),
    "ftmoe_route_grouped_sigmoid": (_i, [_vp, _vp, _i, _i, _i, _i, _i, _i, _f, _vp, _vp, _vp]),
    "ftmoe_align_sizes": (None, [_i, _i, _i, _ip, _ip]),
    "ftmoe_align": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "ftmoe_slot_map": (_i, [_vp, _i, _vp, _i, _vp, _vp, _vp, _vp]),
    "ftmoe_route_histogram": (_i, [_vp, _i, _i, _vp, _vp]),
    "ftmoe_lru_ensure": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _vp, _i, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp,
                              _vp, _vp]),
    "ftmoe_fetch_experts": (_i, [_fbp, _i, _vp, _vp, _vp, _i, _vp]),
    "ftmoe_prefill_hit_compact": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "ftmoe_host_alloc": (_i, [ctypes.c_size_t, ctypes.POINTER(_vp)]),
    "ftmoe_host_free": (_i, [_vp]),
    "ftmoe_materialize_layer": (_i, [_i, _i, _i, _vp, _vp, _vp, _vp, _i, _vp, _vp, _vp, _vp]),
    "ftmoe_release_slots": (_i, [_i, _i, _i, _i, _vp, _vp, _vp, _i, _vp]),
    "ftmoe_act_quant_fp8": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "ftmoe_experts_decode_workspace": (_sz, [_i, _i, _bp, _bp]),
    "ftmoe_experts_decode": (_i, [_vp, _i, _i, _vp, _vp, _bp, _bp, _i, _i, _vp, _vp, _sz, _vp]),
    "ftmoe_experts_decode_noalloc": (_i, [_vp, _i, _i, _vp, _vp, _bp, _bp, _i, _i, _vp, _vp]),
    "ftmoe_experts_decode_noalloc_capacity": (_sz, []),
    "ftmoe_experts_decode_cached": (_i, [_vp, _i, _i, _vp, _vp, _vp, _i, _vp, _vp, _vp, _bp, _bp, _i, _i, _vp, _vp, _sz,
                                         _vp]),
    "ftmoe_experts_decode_routed": (_i, [_vp, _i, _i, ctypes.POINTER(FtmoeRouter), _vp, _vp, _vp, _i, _vp, _vp, _vp,
                                         _bp, _bp, _i, _i, _vp, _vp, _sz, _vp]),
    "ftmoe_experts_prefill_workspace": (_sz, [_i, _i, _bp, _bp]),
    "ftmoe_experts_prefill": (_i, [_vp, _i, _i, _vp, _vp, _bp, _bp, _i, _vp, _vp, _sz, _vp]),
    "ftmoe_cpu_executor_create": (_vp, [_i]),
    "ftmoe_cpu_executor_destroy": (_i, [_vp, _i]),
    "ftmoe_cpu_executor_healthy": (_i, [_vp]),
    "ftmoe_cpu_executor_set_handshake": (_i, [_vp, _i]),
    "ftmoe_cpu_executor_handshake": (_i, [_vp]),
    "ftmoe_cpu_executor_set_watchdog": (None, [_vp, _i]),
    "ftmoe_cpu_executor_hold": (None, [_vp, _i]),
    "ftmoe_cpu_executor_isa": (ctypes.c_char_p, [_vp]),
    "ftmoe_cpu_experts": (_i, [_vp, _bp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "ftmoe_cpu_experts_submit": (_i, [_vp, _bp, _vp, _vp, _vp, _i, _i, _i, _vp, _vp, ctypes.POINTER(_vp)]),
    "ftmoe_cpu_experts_wait": (_i, [_vp, _vp, _vp]),
    "ftmoe_stage_timing_begin": (_i, []),
    "ftmoe_stage_timing_end": (_i, [ctypes.POINTER(ctypes.c_double), _i, _ip, _ip]),
}


class FtmoeError(RuntimeError):
    pass


_LIB = None


def lib():
    """Loads the library once; raises if it was not built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FtmoeError(
                f"{LIB_PATH} is missing: build it with `python -m freetoken_amd.build` "
                "(the MI355X MoE path has no CPU fallback)"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def check(rc: int, what: str) -> None:
    if rc == FTMOE_OK:
        return
    msg = lib().ftmoe_last_error().decode(errors="replace")
    if rc in (FTMOE_ERR_INVALID, FTMOE_ERR_UNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise FtmoeError(f"{what} failed ({rc}): {msg}")
