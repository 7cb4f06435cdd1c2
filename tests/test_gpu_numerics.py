"""Device numerics helpers of the library checked exhaustively on the GPU.

f32_to_bf16 / pack_bf16x2 (freetoken_amd/csrc/ftmoe_common.h) round with
gfx950's conversion instruction; every kernel epilogue rounds through them
(the reference's bf16 rounding points, e.g. kernel/triton/fused_moe.py:142-153,
cpu_moe_ext.cpp:61-68).  The oracle rounds with the integer formula
(u + 0x7fff + ((u >> 16) & 1)) >> 16 (oracle/numerics.py bf16_round); the two
must agree on every finite and infinite float32, and NaN must stay NaN."""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest

HELPER = Path(__file__).resolve().parent / "gpu_helpers" / "libbf16check.so"


def _helper():
    if not HELPER.exists():
        from tests.gpu_helpers import build_helpers  # built by __graft_entry__.build(); rebuilt if absent

        build_helpers.build()
    lib = ctypes.CDLL(str(HELPER))
    lib.ftmoe_test_bf16_rounding.restype = ctypes.c_int
    lib.ftmoe_test_bf16_rounding.argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    return lib


@pytest.mark.gpu
def test_bf16_rounding_matches_oracle_on_all_floats():
    import torch

    assert torch.cuda.is_available()
    counts = (ctypes.c_ulonglong * 2)()
    rc = _helper().ftmoe_test_bf16_rounding(counts)
    assert rc == 0, f"HIP error {rc}"
    assert counts[0] == 0, f"{counts[0]} finite/infinite inputs round differently from the oracle"
    assert counts[1] == 0, f"{counts[1]} NaN inputs did not stay NaN"


def test_helper_source_uses_the_library_header():
    src = (Path(__file__).resolve().parent / "gpu_helpers" / "bf16_rounding.hip").read_text()
    assert '#include "ftmoe_common.h"' in src and "ftmoe::f32_to_bf16" in src and "ftmoe::pack_bf16x2" in src
