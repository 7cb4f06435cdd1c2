"""Shared helpers of the GPU parity tests: upload oracle banks, run layers."""

from __future__ import annotations

import numpy as np
import torch

from freetoken_amd.ops import ExpertBank
from oracle.experts import Bank

_FMT = {"bf16": "bf16", "fp8": "fp8_block", "mxfp4": "mxfp4"}


def code_bank(fmt: str, rows: int, hidden: int, inter: int, rng: np.random.Generator) -> Bank:
    """A quantised bank straight from random codes (every e4m3 code but NaN,
    every e2m1 code) and random positive scales: full-size shapes in seconds,
    where quantising normal weights takes minutes.  The oracle dequantises the
    same bytes, so the comparison is unchanged."""
    shapes = ((rows, 2 * inter, hidden), (rows, hidden, inter))
    if fmt == "fp8":
        mats, scales = [], []
        for n, k in ((2 * inter, hidden), (hidden, inter)):
            q = rng.integers(0, 256, size=(rows, n, k), dtype=np.uint8)
            q[(q & 0x7F) == 0x7F] -= 1  # no NaN codes
            mats.append(q)
            scales.append(rng.uniform(0.5e-4, 1.5e-4, size=(rows, n // 128, k // 128)).astype(np.float32))
        return Bank("fp8", mats[0], mats[1], scales[0], scales[1])
    assert fmt == "mxfp4", fmt
    mats, codes = [], []
    for r, n, k in shapes:
        mats.append(rng.integers(0, 256, size=(r, n, k // 2), dtype=np.uint8))
        codes.append(rng.integers(118, 122, size=(r, n, k // 32), dtype=np.uint8))
    return Bank("mxfp4", mats[0], mats[1], codes[0], codes[1])


def to_device_bank(bank: Bank, dev, rows=None) -> ExpertBank:
    sl = slice(None) if rows is None else rows

    def t(a, dtype=None):
        x = torch.from_numpy(np.ascontiguousarray(a[sl])).to(dev)
        return x.to(dtype) if dtype is not None else x

    lim = getattr(bank, "swiglu_limit", 0.0)
    if bank.fmt == "bf16":
        return ExpertBank("bf16", t(bank.gate_up, torch.bfloat16), t(bank.down, torch.bfloat16), swiglu_limit=lim)
    if bank.fmt == "fp8":
        return ExpertBank(
            "fp8_block",
            t(bank.gate_up).view(torch.float8_e4m3fn),
            t(bank.down).view(torch.float8_e4m3fn),
            t(bank.gate_up_scale),
            t(bank.down_scale),
            swiglu_limit=lim,
        )
    return ExpertBank("mxfp4", t(bank.gate_up), t(bank.down), t(bank.gate_up_scale), t(bank.down_scale),
                      swiglu_limit=lim)


def bf16_dev(a, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev).to(torch.bfloat16)


def to_np(t: torch.Tensor) -> np.ndarray:
    if t.dtype == torch.bfloat16:
        t = t.float()
    return t.detach().cpu().numpy()


def sub_bank(bank: Bank, rows) -> Bank:
    """Rows of a bank (e.g. the resident experts of a slot cache)."""
    f = (lambda a: None if a is None else np.ascontiguousarray(a[rows]))
    return Bank(bank.fmt, f(bank.gate_up), f(bank.down), f(bank.gate_up_scale), f(bank.down_scale),
                getattr(bank, "swiglu_limit", 0.0))
