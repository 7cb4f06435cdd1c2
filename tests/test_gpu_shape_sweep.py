"""Seeded random sweep of decode and prefill shapes against the oracle:
formats, shared-expert formats and sizes, expert counts from 1, hidden and
intermediate sizes that are multiples of 128 but not of 256 (the MXFP4 register
path), batches from 1 token to several route chunks per expert, top-k from 1,
and routes with skipped ids (-1, the sentinel id == num_experts, out of range)
as the reference's layers pass them (layers/moe.py:116-194).  Tolerance as the
other parity tests (max-rel 2e-2, cosine 0.9995)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import synth
from freetoken_amd import ops

from _helpers import bf16_dev, to_device_bank, to_np
from test_gpu_parity import COS_TOL, MAX_REL_TOL, cosine, max_rel

N_DECODE, N_PREFILL = 24, 12


def _decode_config(i: int):
    rng = np.random.default_rng(7000 + i)
    fmt = ("bf16", "fp8", "mxfp4")[i % 3]
    sfmt = (None, fmt, "bf16")[(i // 3) % 3]
    E = int(rng.choice([1, 2, 5, 17, 40, 70]))
    H = int(rng.choice([128, 384, 640, 1152]))
    I = int(rng.choice([128, 256, 384, 640]))
    sI = int(rng.choice([128, 384])) if sfmt else 0
    k = int(rng.integers(1, min(8, E) + 1))
    M = int(rng.choice([1, 2, 3, 5, 9, 17, 31, 63, 130]))
    return rng, fmt, sfmt, E, H, I, sI, k, M


def _ids(rng, M, E, k, skips=True):
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
    if skips and M * k >= 4:
        flat = ids.reshape(-1)
        pos = rng.choice(flat.size, 3, replace=False)
        flat[pos[0]] = -1
        flat[pos[1]] = E  # the sentinel bucket: no expert
        flat[pos[2]] = E + 7
    return ids


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(N_DECODE))
def test_decode_shape_sweep(dev, i):
    rng, fmt, sfmt, E, H, I, sI, k, M = _decode_config(i)
    bank = synth.make_bank(fmt, E, H, I, rng)
    shared = synth.make_bank(sfmt, 1, H, sI, rng) if sfmt else None
    x = synth.activations(rng, M, H)
    ids = _ids(rng, M, E, k)
    w = rng.random((M, k), dtype=np.float32) + 0.05
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, shared)
    y = ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                           to_device_bank(bank, dev), to_device_bank(shared, dev) if shared else None)
    got = to_np(y)
    case = (fmt, sfmt, E, H, I, sI, k, M)
    assert np.isfinite(got).all(), case
    assert max_rel(got, y_ref) <= MAX_REL_TOL, (case, max_rel(got, y_ref))
    assert cosine(got, y_ref) >= COS_TOL, (case, cosine(got, y_ref))


def _prefill_config(i: int):
    rng = np.random.default_rng(8000 + i)
    fmt = ("fp8", "mxfp4", "bf16")[i % 3]
    shared = bool((i // 3) % 2)
    E = int(rng.choice([1, 3, 9, 24, 40]))
    H = int(rng.choice([128, 384, 640]))
    I = int(rng.choice([128, 256, 384]))
    k = int(rng.integers(1, min(8, E) + 1))
    M = int(rng.choice([1, 7, 100, 300, 700]))
    return rng, fmt, shared, E, H, I, k, M


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(N_PREFILL))
def test_prefill_shape_sweep(dev, i):
    rng, fmt, shared, E, H, I, k, M = _prefill_config(i)
    bank = synth.make_bank(fmt, E, H, I, rng)
    sh = synth.make_bank(fmt, 1, H, I, rng) if shared else None
    x = synth.activations(rng, M, H)
    ids = _ids(rng, M, E, k)
    w = rng.random((M, k), dtype=np.float32) + 0.05
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    y_ref = oracle.experts.moe_layer("prefill", x, w, ids, bank, sh)
    y = ops.experts_prefill(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                            to_device_bank(bank, dev), to_device_bank(sh, dev) if sh else None)
    got = to_np(y)
    case = (fmt, shared, E, H, I, k, M)
    assert np.isfinite(got).all(), case
    assert max_rel(got, y_ref) <= MAX_REL_TOL, (case, max_rel(got, y_ref))
    assert cosine(got, y_ref) >= COS_TOL, (case, cosine(got, y_ref))


def test_sweep_covers_the_corners():
    """The seeded configurations reach the corners the sweep is for (CPU only)."""
    dec = [_decode_config(i)[1:] for i in range(N_DECODE)]
    pre = [_prefill_config(i)[1:] for i in range(N_PREFILL)]
    assert {d[0] for d in dec} == {"bf16", "fp8", "mxfp4"} and {d[1] for d in dec} >= {None, "bf16"}
    assert any(d[2] == 1 for d in dec) and any(d[6] == 1 for d in dec)  # one expert, top-1
    assert any(d[7] == 1 for d in dec) and any(d[7] >= 63 for d in dec)  # one token, many
    assert any(d[0] == "mxfp4" and (d[3] % 256 or d[4] % 256) for d in dec)  # MXFP4, K not a multiple of 256
    assert {p[0] for p in pre} == {"fp8", "mxfp4", "bf16"} and any(p[1] for p in pre)
    assert any(p[6] >= 300 for p in pre) and any(p[6] == 1 for p in pre)
