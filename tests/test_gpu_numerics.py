"""Device numerics helpers of the library checked exhaustively on the GPU.

f32_to_bf16 / pack_bf16x2 (freetoken_amd/csrc/ftmoe_common.h) round with
gfx950's conversion instruction; every kernel epilogue rounds through them
(the reference's bf16 rounding points, e.g. kernel/triton/fused_moe.py:142-153,
cpu_moe_ext.cpp:61-68).  The oracle rounds with the integer formula
(u + 0x7fff + ((u >> 16) & 1)) >> 16 (oracle/numerics.py bf16_round); the two
must agree on every finite and infinite float32, and NaN must stay NaN.

The activation quantisation (freetoken_amd/csrc/quant.h, reference
per_token_group_quant_fp8, kernel/triton/fp8_block_linear.py:53-59) divides by
the group scale s = max(amax, 1e-10)/448 as a multiplication by RN(1/s) with
an FMA correction; over every pair of bf16 values (amax, x) with |x| <= amax
its e4m3 codes must equal those of the IEEE quotient, and its float32 results
may differ only where the quotient is far below e4m3's range (the residual
underflows).  The same algorithm is checked in C on the CPU."""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
HELPER = HERE / "gpu_helpers" / "libbf16check.so"
QUANT_HELPER = HERE / "gpu_helpers" / "libquantcheck.so"


def _load(path, fn):
    if not path.exists():
        from tests.gpu_helpers import build_helpers  # built by __graft_entry__.build(); rebuilt if absent

        build_helpers.build()
    lib = ctypes.CDLL(str(path))
    getattr(lib, fn).restype = ctypes.c_int
    getattr(lib, fn).argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    return lib


def _helper():
    return _load(HELPER, "ftmoe_test_bf16_rounding")


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


# float32 results of the quantisation division that differ from the IEEE
# quotient on the CPU (all with |x / s| < 2^-71; recorded by the C check)
CPU_TINY_MISMATCHES = 3474188


@pytest.mark.gpu
def test_quant_division_matches_ieee_on_all_bf16_pairs():
    import torch

    assert torch.cuda.is_available()
    counts = (ctypes.c_ulonglong * 3)()
    rc = _load(QUANT_HELPER, "ftmoe_test_quant_division").ftmoe_test_quant_division(counts)
    assert rc == 0, f"HIP error {rc}"
    assert counts[0] == 0, f"{counts[0]} pairs give e4m3 codes different from the IEEE division"
    assert counts[1] == 0, f"{counts[1]} pairs differ in float32 where |x / s| >= 2^-64"
    # the device's FMA and denormal handling match the CPU's on this domain
    assert counts[2] == CPU_TINY_MISMATCHES, counts[2]


def test_quant_division_algorithm_on_the_cpu(tmp_path):
    """The same algorithm in C (tests/cpu_helpers/quant_division.c) over the
    same 1.07e9 pairs: no mismatch with |x / s| >= 2^-64, none of another sign."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no gcc")
    exe = tmp_path / "quant_division"
    subprocess.run([gcc, "-O3", "-fopenmp", "-ffp-contract=off", str(HERE / "cpu_helpers" / "quant_division.c"),
                    "-o", str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe)], stdout=subprocess.PIPE, text=True, timeout=300)
    assert r.returncode == 0, r.stdout
    f = r.stdout.split()
    assert f[0] == "pairs" and int(f[1]) == 1065402240, r.stdout
    assert int(f[3]) == CPU_TINY_MISMATCHES and int(f[5]) == 0 and int(f[7]) == 0, r.stdout


def test_quant_helper_source_uses_the_library_header():
    src = (HERE / "gpu_helpers" / "quant_division.hip").read_text()
    assert '#include "quant.h"' in src and "ftmoe::group_scale<0>" in src and "ftmoe::quant_value<0>" in src
