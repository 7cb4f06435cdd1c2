"""The HBM read bandwidth a plain streaming kernel reaches on this GPU
(tests/gpu_helpers/read_bw.hip): the practical ceiling against which the
decode GEMVs' bandwidth (bench.py's `roofline`, priced against the 8 TB/s
nominal peak) can be read.  Printed with -s; the assertions only check that
the measurement ran and lies between a sane floor and the nominal peak."""

from __future__ import annotations

import ctypes
from pathlib import Path

import pytest

HELPER = Path(__file__).resolve().parent / "gpu_helpers" / "libreadbw.so"


@pytest.mark.gpu
def test_hbm_read_ceiling(dev):
    if not HELPER.exists():
        from tests.gpu_helpers import build_helpers  # built by __graft_entry__.build(); rebuilt if absent

        build_helpers.build()
    lib = ctypes.CDLL(str(HELPER))
    lib.ftmoe_test_read_bandwidth.restype = ctypes.c_int
    lib.ftmoe_test_read_bandwidth.argtypes = [ctypes.POINTER(ctypes.c_double)]
    best = (ctypes.c_double * 4)()
    rc = lib.ftmoe_test_read_bandwidth(best)
    assert rc == 0, f"HIP error {rc}"
    print(f"HBM read ceiling: {best[0]:.2f} TB/s (grid {int(best[1])}, {int(best[2])} loads in flight per thread, "
          f"{'nontemporal' if best[3] else 'plain'} loads) = {best[0] / 8.0:.1%} of the 8 TB/s nominal peak")
    assert 3.0 < best[0] < 8.0, best[0]
