"""GPU parity of the prefill path (activation quantisation and grouped GEMMs)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import synth
from oracle.numerics import bf16_round
from freetoken_amd import ops

from _helpers import bf16_dev, to_device_bank, to_np
from conftest import COS_TOL, MAX_REL_TOL, cosine, max_rel

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,K", [(1, 128), (37, 1024), (513, 7168)])
def test_act_quant_fp8_exact(dev, rows, K):
    rng = np.random.default_rng(rows)
    x = bf16_round(synth.activations(rng, rows, K) * np.float32(rng.uniform(0.01, 30)))
    x[0, :128] = 0.0  # all-zero group: amax clamp
    q_ref, s_ref = oracle.experts.per_token_group_quant_fp8(x)
    q, s = ops.act_quant_fp8(bf16_dev(x, dev), 0)
    np.testing.assert_array_equal(to_np(s), s_ref)
    np.testing.assert_array_equal(to_np(q), q_ref)


@pytest.mark.parametrize("rows,K", [(3, 256), (129, 2048)])
def test_act_quant_ue8m0_exact(dev, rows, K):
    rng = np.random.default_rng(rows + 1)
    x = bf16_round(synth.activations(rng, rows, K) * np.float32(3.0))
    x[1, 128:256] = bf16_round(np.float32(1e-6))  # below the 1e-4 amax floor
    q_ref, c_ref = oracle.experts.act_quant_ue8m0(x)
    q, c = ops.act_quant_fp8(bf16_dev(x, dev), 1)
    np.testing.assert_array_equal(to_np(c), c_ref)
    np.testing.assert_array_equal(to_np(q), q_ref)


def _prefill_case(fmt, E, H, I, M, k, shared, seed, grouped=True):
    rng = np.random.default_rng(seed)
    bank = synth.make_bank(fmt, E, H, I, rng)
    sh = synth.make_bank(fmt, 1, H, I, rng) if shared else None
    x = synth.activations(rng, M, H)
    if grouped:
        lg = synth.normal(rng, (M, E)) + synth.zipf_bias(rng, E)[None, :]
        w, ids = oracle.routing.grouped_sigmoid_topk(lg, synth.normal(rng, (E,), 0.05), 8, 4, k, True, 2.5)
    else:
        lg = synth.normal(rng, (M, E))
        w, ids = oracle.routing.softmax_topk(lg, k, True)
    return bank, sh, x, w, ids


PREFILL_CASES = [
    ("fp8_shared", "fp8", 32, 1024, 256, 512, 8, True),
    ("mxfp4_shared", "mxfp4", 32, 1024, 256, 512, 8, True),
    ("fp8_noshared_small", "fp8", 16, 512, 384, 37, 8, False),
    ("bf16", "bf16", 16, 512, 256, 300, 2, False),
    # every token on 8 of 16 experts: experts of up to 10 M blocks, so the
    # tile schedule's chunks of 8 (FP8 gate_up) and 2 (down) run full and
    # with a remainder
    ("fp8_hot_experts", "fp8", 16, 512, 256, 2560, 8, True),
    ("mxfp4_hot_experts", "mxfp4", 16, 512, 256, 2560, 8, False),
]


@pytest.mark.parametrize("case", PREFILL_CASES, ids=[c[0] for c in PREFILL_CASES])
def test_prefill_parity(dev, case):
    name, fmt, E, H, I, M, k, shared = case
    bank, sh, x, w, ids = _prefill_case(fmt, E, H, I, M, k, shared, seed=len(name), grouped=(E % 8 == 0 and k == 8))
    y_ref = oracle.experts.moe_layer("prefill", x, w, ids, bank, sh)
    y = ops.experts_prefill(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                            to_device_bank(bank, dev), to_device_bank(sh, dev) if sh else None)
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL, (name, max_rel(got, y_ref))
    assert cosine(got, y_ref) >= COS_TOL, (name, cosine(got, y_ref))


def test_prefill_skipped_ids_and_sentinel(dev):
    bank, sh, x, w, ids = _prefill_case("fp8", 16, 512, 256, 64, 4, True, seed=3, grouped=False)
    ids[0, 0] = -1
    ids[5, 2] = 16  # == num_experts: the align sentinel bucket, no expert
    ids[7, 1] = 99
    y_ref = oracle.experts.moe_layer("prefill", x, w, ids, bank, sh)
    y = ops.experts_prefill(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                            to_device_bank(bank, dev), to_device_bank(sh, dev))
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL
    assert cosine(got, y_ref) >= COS_TOL


def test_prefill_deterministic(dev):
    bank, sh, x, w, ids = _prefill_case("fp8", 32, 1024, 256, 256, 8, True, seed=4)
    args = (bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
            to_device_bank(bank, dev), to_device_bank(sh, dev))
    a = ops.experts_prefill(*args).clone()
    b = ops.experts_prefill(*args)
    assert torch.equal(a, b)


def test_decode_and_prefill_agree_on_bf16(dev):
    """The two regimes compute the same bf16 math (reference decode-vs-grouped
    check, tests/moe/test_fused_moe.py:101-156, tolerance 2e-2)."""
    bank, _, x, w, ids = _prefill_case("bf16", 16, 512, 256, 24, 4, False, seed=5, grouped=False)
    args = (bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev), to_device_bank(bank, dev))
    a = to_np(ops.experts_prefill(*args))
    b = to_np(ops.experts_decode(*args))
    assert max_rel(a, b) <= 2e-2 and cosine(a, b) >= COS_TOL


@pytest.mark.parametrize("activation", ["gelu", "gelu_tanh"])
@pytest.mark.parametrize("fmt", ["fp8", "mxfp4", "bf16"])
def test_prefill_activation_variants(dev, fmt, activation):
    """The gelu forms of the gate/up epilogue (reference kernel/triton/
    activation.py:99-109), which takes the runtime-kind branch of the
    quantised GEMMs' epilogue (SiLU has its own straight-line code)."""
    bank, sh, x, w, ids = _prefill_case(fmt, 16, 512, 256, 300, 4, fmt != "bf16", seed=11, grouped=False)
    y_ref = oracle.experts.moe_layer("prefill", x, w, ids, bank, sh, activation=activation)
    y = ops.experts_prefill(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                            to_device_bank(bank, dev), to_device_bank(sh, dev) if sh else None, activation=activation)
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL, (fmt, activation, max_rel(got, y_ref))
    assert cosine(got, y_ref) >= COS_TOL, (fmt, activation, cosine(got, y_ref))
    y_silu = oracle.experts.moe_layer("prefill", x, w, ids, bank, sh)
    assert max_rel(y_silu, y_ref) > 4 * MAX_REL_TOL
