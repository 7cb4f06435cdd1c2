"""The clamped SwiGLU of the DeepSeek-V4 ds_fp4 experts (``swiglu_limit``;
reference moe/fused_ds_fp4.py:105-124,192-226 and kernel/triton/dsv4/
fused_moe.py:121-141: silu(min(gate, L)) * clamp(up, -L, L) on the bf16 gate
and up values) in the decode and prefill epilogues, against the oracle layer
at limit 0 (no clamp), 7 (the DeepSeek-V4 default range, rarely binding on
these activations) and 0.75 (binding on a large share of the values); the
shared expert carries a limit of its own.  Also through the reference-named
entry points of moe/fused_ds_fp4.py."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import synth
from freetoken_amd import ops
from freetoken_amd.moe import fused_ds_fp4

from _helpers import bf16_dev, to_device_bank, to_np
from conftest import COS_TOL, MAX_REL_TOL, cosine, max_rel

pytestmark = pytest.mark.gpu

LIMITS = [0.0, 7.0, 0.75]


def _banks(fmt, sfmt, E, H, I, lim, rng):
    bank = synth.make_bank(fmt, E, H, I, rng)
    bank.swiglu_limit = lim
    shared = None
    if sfmt:
        shared = synth.make_bank(sfmt, 1, H, I, rng)
        shared.swiglu_limit = lim
    return bank, shared


def _routing(rng, M, E, k):
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
    w = rng.random((M, k), dtype=np.float32)
    return (w / w.sum(1, keepdims=True)).astype(np.float32), ids


@pytest.mark.parametrize("lim", LIMITS)
@pytest.mark.parametrize("fmt,sfmt", [("mxfp4", "bf16"), ("fp8", "fp8")])
@pytest.mark.parametrize("M", [1, 33])
def test_decode_swiglu_limit(dev, fmt, sfmt, M, lim):
    rng = np.random.default_rng(700 + M + int(lim * 8))
    E, H, I, k = 20, 1280, 384, 8
    bank, shared = _banks(fmt, sfmt, E, H, I, lim, rng)
    x = synth.activations(rng, M, H)
    w, ids = _routing(rng, M, E, k)
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, shared)
    y = ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                           to_device_bank(bank, dev), to_device_bank(shared, dev))
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL and cosine(got, y_ref) >= COS_TOL, (fmt, M, lim, max_rel(got, y_ref))
    if lim == 0.75:  # the clamp binds: the unclamped layer is far from this one
        bank.swiglu_limit = shared.swiglu_limit = 0.0
        assert max_rel(oracle.experts.moe_layer("decode", x, w, ids, bank, shared), y_ref) > 4 * MAX_REL_TOL


@pytest.mark.parametrize("lim", LIMITS)
@pytest.mark.parametrize("fmt", ["mxfp4", "fp8", "bf16"])
def test_prefill_swiglu_limit(dev, fmt, lim):
    rng = np.random.default_rng(800 + int(lim * 8))
    E, H, I, M, k = 16, 1024, 256, 300, 4
    bank, shared = _banks(fmt, fmt, E, H, I, lim, rng)
    x = synth.activations(rng, M, H)
    w, ids = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
    y_ref = oracle.experts.moe_layer("prefill", x, w, ids, bank, shared)
    y = ops.experts_prefill(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                            to_device_bank(bank, dev), to_device_bank(shared, dev))
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL and cosine(got, y_ref) >= COS_TOL, (fmt, lim, max_rel(got, y_ref))


@pytest.mark.parametrize("lim", [7.0, 0.75])
def test_ds_fp4_entry_points_take_the_limit(dev, lim):
    """routed_experts_fp4 (decode) and routed_experts_fp4_prefill with the
    reference's argument order: the banks' limit reaches both epilogues."""
    rng = np.random.default_rng(900 + int(lim))
    E, H, I, k = 16, 1024, 256, 8
    bank, _ = _banks("mxfp4", None, E, H, I, lim, rng)
    db = to_device_bank(bank, dev)
    for regime, M in (("decode", 3), ("prefill", 160)):
        x = synth.activations(rng, M, H)
        w, ids = _routing(rng, M, E, k)
        y_ref = oracle.experts.moe_layer(regime, x, w, ids, bank, None)
        args = (bf16_dev(x, dev), torch.from_numpy(ids).to(dev), torch.from_numpy(w).to(dev), db.gate_up,
                db.gate_up_scale, db.down, db.down_scale, lim)
        y = fused_ds_fp4.routed_experts_fp4(*args) if regime == "decode" else \
            fused_ds_fp4.routed_experts_fp4_prefill(*args, E)
        got = to_np(y)
        assert max_rel(got, y_ref) <= MAX_REL_TOL and cosine(got, y_ref) >= COS_TOL, (regime, lim)
    with pytest.raises(ValueError, match="silu"):
        ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev), db,
                           activation="gelu")
