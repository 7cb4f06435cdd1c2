"""The C-ABI library loads and exports every symbol include/ftmoe.h declares;
host-side argument validation and size queries (no kernel launches)."""

import ctypes
import re
from pathlib import Path

import pytest

from freetoken_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "ftmoe.h"


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(ftmoe_[a-z0-9_]+)\s*\(", text)))


def test_library_built_and_loads():
    assert _lib.LIB_PATH.exists(), "run freetoken_amd.build first"
    assert _lib.lib().ftmoe_version() == 1


def test_exports_every_declared_symbol():
    syms = declared_symbols()
    assert len(syms) >= 9
    handle = _lib.lib()
    for s in syms:
        assert hasattr(handle, s), s
        assert s in _lib.SIGNATURES, f"{s} has no ctypes signature"


def test_validation_errors_without_launch():
    L = _lib.lib()
    w = ctypes.c_void_p(16)
    rc = L.ftmoe_route_softmax_topk(w, 0, 4, 2000, 8, 1, w, w, None)
    assert rc == _lib.FTMOE_ERR_UNSUPPORTED
    assert b"E=2000" in L.ftmoe_last_error()
    rc = L.ftmoe_route_grouped_sigmoid(w, None, 4, 256, 7, 4, 8, 1, 2.5, w, w, None)
    assert rc == _lib.FTMOE_ERR_UNSUPPORTED
    rc = L.ftmoe_align(None, 8, 16, 4, w, w, w, None)
    assert rc == _lib.FTMOE_ERR_INVALID
    bank = _lib.FtmoeBank(_lib.FMT_FP8_B128, 8, 1000, 256, 16, None, 16, None)
    rc = L.ftmoe_experts_decode(w, 1, 8, w, w, ctypes.byref(bank), None, 0, 0, w, w, 1 << 20, None)
    assert rc == _lib.FTMOE_ERR_UNSUPPORTED  # hidden not a multiple of 128
    # miss path: admission tables beyond one workgroup's LDS, unaligned gather rows
    rc = L.ftmoe_lru_ensure(w, 8, 0, 1, 256, w, w, w, w, 9000, None, -1, 0, w, w, 8, w, w, None, None, None, None)
    assert rc == _lib.FTMOE_ERR_UNSUPPORTED and b"S=9000" in L.ftmoe_last_error()
    rc = L.ftmoe_lru_ensure(w, 8, 2, 2, 256, w, w, w, w, 64, None, -1, 0, w, w, 8, w, w, None, None, None, None)
    assert rc == _lib.FTMOE_ERR_UNSUPPORTED  # layer outside [0, num_layers)
    rc = L.ftmoe_lru_ensure(w, 8, 0, 1, 256, None, w, w, w, 64, None, -1, 0, w, w, 8, w, w, None, None, None, None)
    assert rc == _lib.FTMOE_ERR_INVALID
    rc = L.ftmoe_lru_ensure(w, 8, 0, 1, 256, w, w, w, w, 64, None, -1, 70000, w, w, 8, w, w, None, None, None, None)
    assert rc == _lib.FTMOE_ERR_UNSUPPORTED and b"frac_q16=70000" in L.ftmoe_last_error()
    rc = L.ftmoe_lru_ensure(None, 8, 0, 1, 256, w, w, w, w, 64, None, -1, 0, w, w, 8, w, w, None, None, None, None)
    assert rc == _lib.FTMOE_ERR_INVALID
    fb = (_lib.FtmoeFetchBank * 1)(_lib.FtmoeFetchBank(16, 16, 24))
    rc = L.ftmoe_fetch_experts(fb, 1, w, w, w, 4, None)
    assert rc == _lib.FTMOE_ERR_UNSUPPORTED and b"16-byte" in L.ftmoe_last_error()
    rc = L.ftmoe_fetch_experts(fb, 9, w, w, w, 4, None)
    assert rc == _lib.FTMOE_ERR_UNSUPPORTED


def test_align_sizes_formula():
    from freetoken_amd.ops import align_sizes

    assert align_sizes(12, 4, 4) == (27, 7)  # numel + (E+1)(BM-1)
    assert align_sizes(3, 16, 8) == (24, 3)  # numel < E+1: numel * BM


def test_workspace_query():
    L = _lib.lib()
    bank = _lib.FtmoeBank(_lib.FMT_FP8_B128, 64, 7168, 2048, 16, 16, 16, 16)
    sh = _lib.FtmoeBank(_lib.FMT_FP8_B128, 1, 7168, 2048, 16, 16, 16, 16)
    n = L.ftmoe_experts_decode_workspace(64, 8, ctypes.byref(bank), ctypes.byref(sh))
    # act rows (M*k + M) * I bf16 + ic3 M*k*H bf16 + shared out M*H bf16, plus small index arrays
    assert n >= (576 * 2048 + 512 * 7168 + 64 * 7168) * 2


def test_ops_reject_cpu_tensors():
    import torch

    from freetoken_amd import ops

    with pytest.raises(ValueError):
        ops.route_softmax_topk(torch.zeros(2, 8), 2, True)


def test_empty_batch_is_a_noop():
    """M = 0 (empty tensors, NULL data pointers) returns OK from every router
    and expert entry point without reading a pointer or launching; M < 0 is an
    error.  Runs without a GPU: a launch or a dereference would fail here."""
    L = _lib.lib()
    w = ctypes.c_void_p(16)
    bank = _lib.FtmoeBank(_lib.FMT_FP8_B128, 8, 256, 256, 16, 16, 16, 16)
    bp = ctypes.byref(bank)
    shared = _lib.FtmoeBank(_lib.FMT_FP8_B128, 1, 256, 256, 16, 16, 16, 16)
    sp = ctypes.byref(shared)
    assert L.ftmoe_route_softmax_topk(None, _lib.DTYPE_F32, 0, 64, 8, 1, None, None, None) == 0
    assert L.ftmoe_route_grouped_sigmoid(None, None, 0, 256, 8, 4, 8, 1, 2.5, None, None, None) == 0
    assert L.ftmoe_experts_decode(None, 0, 8, None, None, bp, sp, 0, 0, None, None, 0, None) == 0
    assert L.ftmoe_experts_decode_noalloc(None, 0, 8, None, None, bp, None, 0, 0, None, None) == 0
    assert L.ftmoe_experts_prefill(None, 0, 8, None, None, bp, sp, 0, None, None, 0, None) == 0
    assert L.ftmoe_experts_decode_cached(None, 0, 8, None, None, None, 64, None, None, None, bp, None, 0, 0, None,
                                         None, 0, None) == 0
    for kind in (_lib.ROUTER_SOFTMAX_TOPK, _lib.ROUTER_GROUPED_SIGMOID):
        r = _lib.FtmoeRouter(kind, None, _lib.DTYPE_F32, 8, 1, None, 1, 1, 1.0)
        assert L.ftmoe_experts_decode_routed(None, 0, 8, ctypes.byref(r), None, None, None, 0, None, None, None, bp,
                                             None, 0, 0, None, None, 0, None) == 0
    assert L.ftmoe_experts_decode_workspace(0, 8, bp, None) == 0
    assert L.ftmoe_experts_prefill_workspace(0, 8, bp, None) == 0
    # negative sizes and invalid configurations still fail with M = 0
    assert L.ftmoe_route_softmax_topk(w, _lib.DTYPE_F32, -1, 64, 8, 1, w, w, None) == _lib.FTMOE_ERR_INVALID
    assert L.ftmoe_route_softmax_topk(None, _lib.DTYPE_F32, 0, 64, 80, 1, None, None, None) == _lib.FTMOE_ERR_UNSUPPORTED
    assert L.ftmoe_experts_decode(w, -1, 8, w, w, bp, None, 0, 0, w, w, 1 << 20, None) == _lib.FTMOE_ERR_INVALID
    assert L.ftmoe_experts_prefill(w, -1, 8, w, w, bp, None, 0, w, w, 1 << 20, None) == _lib.FTMOE_ERR_INVALID
    assert L.ftmoe_experts_decode_noalloc(w, -1, 8, w, w, bp, None, 0, 0, w, None) == _lib.FTMOE_ERR_INVALID
    assert L.ftmoe_experts_decode(None, 0, 0, None, None, bp, None, 0, 0, None, None, 0, None) == _lib.FTMOE_ERR_INVALID
    bad = _lib.FtmoeBank(_lib.FMT_FP8_B128, 8, 1000, 256, 16, None, 16, None)
    assert L.ftmoe_experts_decode(None, 0, 8, None, None, ctypes.byref(bad), None, 0, 0, None, None, 0,
                                  None) == _lib.FTMOE_ERR_UNSUPPORTED
    r = _lib.FtmoeRouter(7, None, _lib.DTYPE_F32, 8, 1, None, 1, 1, 1.0)
    assert L.ftmoe_experts_decode_routed(None, 0, 8, ctypes.byref(r), None, None, None, 0, None, None, None, bp, None,
                                         0, 0, None, None, 0, None) == _lib.FTMOE_ERR_UNSUPPORTED
