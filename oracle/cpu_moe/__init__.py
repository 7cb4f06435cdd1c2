"""ctypes wrapper of the CPU MoE executor restatement (libcpumoe.so).

Test infrastructure: the CPU baseline of bench.py and a second checker of the
oracle's bf16 / MXFP4 decode math.  Built by ``make`` in this directory (done by
``__graft_entry__.build()``).
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "libcpumoe.so"
FMT = {"bf16": 0, "mxfp4": 1}


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


_L = None


def lib():
    global _L
    if _L is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        vp, i = ctypes.c_void_p, ctypes.c_int
        L.cpumoe_create.restype = vp
        L.cpumoe_create.argtypes = [i, i, i, i, i, ctypes.POINTER(ctypes.c_int), i]
        L.cpumoe_isa.restype = ctypes.c_char_p
        L.cpumoe_isa.argtypes = [vp]
        L.cpumoe_set_bank.argtypes = [vp, vp, vp, vp, vp]
        L.cpumoe_run.argtypes = [vp, vp, vp, vp, i, vp]
        L.cpumoe_destroy.argtypes = [vp]
        L.cpumoe_fill_bf16.argtypes = [vp, ctypes.c_size_t, ctypes.c_float, ctypes.c_uint64, i]
        _L = L
    return _L


def physical_cores() -> list[int]:
    """One logical CPU per physical core among the CPUs this process may use."""
    allowed = sorted(os.sched_getaffinity(0))
    seen, out = set(), []
    for cpu in allowed:
        try:
            core = Path(f"/sys/devices/system/cpu/cpu{cpu}/topology/core_id").read_text().strip()
            pkg = Path(f"/sys/devices/system/cpu/cpu{cpu}/topology/physical_package_id").read_text().strip()
            key = (pkg, core)
        except OSError:
            key = (cpu,)
        if key not in seen:
            seen.add(key)
            out.append(cpu)
    return out


class CpuMoe:
    """Two-pass CPU decode over host banks (bf16 [E,2I,H]/[E,H,I] as uint16, or
    MXFP4 packed + e8m0 scales)."""

    def __init__(self, hidden, inter, top_k, num_experts, fmt="bf16", cpus=None):
        self.cpus = list(cpus) if cpus is not None else physical_cores()
        arr = (ctypes.c_int * len(self.cpus))(*self.cpus)
        self.h = lib().cpumoe_create(hidden, inter, top_k, num_experts, FMT[fmt], arr, len(self.cpus))
        self.H, self.I, self.k, self.E, self.fmt = hidden, inter, top_k, num_experts, fmt
        self._keep = None

    @property
    def isa(self) -> str:
        return lib().cpumoe_isa(self.h).decode()

    def set_bank(self, gate_up, down, gate_up_scale=None, down_scale=None):
        self._keep = [np.ascontiguousarray(a) if a is not None else None
                      for a in (gate_up, down, gate_up_scale, down_scale)]
        ptr = lambda a: None if a is None else a.ctypes.data  # noqa: E731
        lib().cpumoe_set_bank(self.h, *[ptr(a) for a in self._keep])

    def run(self, x_bits: np.ndarray, w: np.ndarray, ids: np.ndarray) -> np.ndarray:
        x_bits = np.ascontiguousarray(x_bits, dtype=np.uint16)
        w = np.ascontiguousarray(w, dtype=np.float32)
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        m = x_bits.shape[0]
        y = np.empty((m, self.H), dtype=np.uint16)
        lib().cpumoe_run(self.h, x_bits.ctypes.data, w.ctypes.data, ids.ctypes.data, m, y.ctypes.data)
        return y

    def close(self):
        if self.h:
            lib().cpumoe_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
