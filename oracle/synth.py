"""Seeded synthetic inputs shaped like BASELINE.json's configs (numpy, CPU).

Test infrastructure: used by tests/ and tests/golden/make_golden.py to build
identical inputs for the oracle and the HIP path.  Weights are N(0, std)
before quantisation; activations N(0, 1) rounded to bf16.
"""

from __future__ import annotations

import numpy as np

from .experts import Bank, quantize_fp8_block, quantize_mxfp4
from .numerics import bf16_round


def normal(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def make_bank(fmt: str, rows: int, hidden: int, inter: int, rng: np.random.Generator, std: float = 0.02) -> Bank:
    gu = normal(rng, (rows, 2 * inter, hidden), std)
    dn = normal(rng, (rows, hidden, inter), std)
    if fmt == "bf16":
        return Bank("bf16", bf16_round(gu), bf16_round(dn))
    if fmt == "fp8":
        gq, gs = quantize_fp8_block(gu)
        dq, ds = quantize_fp8_block(dn)
        return Bank("fp8", gq, dq, gs, ds)
    if fmt == "mxfp4":
        gq, gs = quantize_mxfp4(gu)
        dq, ds = quantize_mxfp4(dn)
        return Bank("mxfp4", gq, dq, gs, ds)
    raise ValueError(fmt)


def activations(rng: np.random.Generator, m: int, hidden: int) -> np.ndarray:
    return bf16_round(normal(rng, (m, hidden)))


def tied_logits(rng: np.random.Generator, m: int, e: int, bf16: bool = True) -> np.ndarray:
    """N(0,1) router logits with deliberate exact ties (copied values) so the
    lowest-index tie rule is exercised on every row."""
    lg = normal(rng, (m, e))
    for r in range(m):
        src = rng.integers(0, e, size=max(1, e // 8))
        dst = rng.integers(0, e, size=src.size)
        lg[r, dst] = lg[r, src]
    return bf16_round(lg) if bf16 else lg


def zipf_bias(rng: np.random.Generator, e: int, s: float = 1.1) -> np.ndarray:
    """log p_e with p_e proportional to rank^-s over a seeded permutation."""
    ranks = rng.permutation(e) + 1
    p = ranks.astype(np.float64) ** -s
    p /= p.sum()
    return np.log(p).astype(np.float32)
