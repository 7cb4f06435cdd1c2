"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: every fixture still matches the generator and the oracle (weight banks by
SHA-256, routing exactly, expected outputs to float tolerance), and the KATs
hold the hand-derived answers.  GPU: the HIP path reproduces every fixture --
routing, slot map and permutation bit-exactly, layer outputs within the
north-star bar (max-rel 2e-2, cosine 0.9995)."""

from __future__ import annotations

import ast
import importlib.util
import os

import numpy as np
import pytest

import oracle
from oracle.numerics import bf16_bits, bf16_from_bits

from conftest import COS_TOL, MAX_REL_TOL, cosine, max_rel

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
_spec = importlib.util.spec_from_file_location("make_golden", os.path.join(HERE, "make_golden.py"))
golden = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(golden)

LAYER_CASES = list(golden.RECIPES)


def load(name: str) -> dict:
    with np.load(os.path.join(HERE, f"{name}.npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def meta_of(fx: dict) -> dict:
    return dict(ast.literal_eval(str(fx["meta"])))


# ----------------------------------------------------------------- CPU: fixtures vs generator and oracle


@pytest.mark.parametrize("name", LAYER_CASES)
def test_fixture_matches_generator_and_oracle(name):
    fx = load(name)
    inputs, banks, meta = golden.build(name)
    assert meta == meta_of(fx)
    for bname, b in banks.items():
        assert golden.bank_digest(b) == str(fx[f"sha256_{bname}"]), f"{name}: bank {bname} changed"
    np.testing.assert_array_equal(bf16_bits(inputs["x"]), fx["x_bits"])
    for k, v in inputs.items():
        if k != "x":
            np.testing.assert_array_equal(v, fx[f"in_{k}"])
    out = golden.run(name, inputs, banks, meta)
    np.testing.assert_array_equal(out["topk_ids"], fx["out_topk_ids"])
    np.testing.assert_allclose(out["topk_w"], fx["out_topk_w"], rtol=1e-6, atol=0)
    for k in ("slot_ids", "miss_mask", "slot_stats"):
        if f"out_{k}" in fx:
            np.testing.assert_array_equal(out[k], fx[f"out_{k}"])
    # float32 accumulation order of the host BLAS may move a bf16 rounding
    y, y_ref = bf16_from_bits(out["y_bits"]), bf16_from_bits(fx["out_y_bits"])
    assert max_rel(y, y_ref) <= 5e-3 and cosine(y, y_ref) >= 0.99999, name


def test_kat_align_docstring_and_regression():
    kat = load("kat_align")
    # reference moe/fused.py:113-126: stable order per expert, sentinel 12
    np.testing.assert_array_equal(kat["doc_sorted"][:16], [3, 6, 9, 12, 0, 4, 10, 12, 1, 7, 11, 12, 2, 5, 8, 12])
    s, e, n = oracle.align.moe_align_block_size(kat["doc_ids"], 4, 4)
    np.testing.assert_array_equal(s, kat["doc_sorted"])
    np.testing.assert_array_equal(e, kat["doc_expert_ids"])
    np.testing.assert_array_equal(n, kat["doc_ntpp"])
    s, e, n = oracle.align.moe_align_block_size(kat["rand_ids"], 8, 16)
    np.testing.assert_array_equal(s, kat["rand_sorted"])
    np.testing.assert_array_equal(e, kat["rand_expert_ids"])
    np.testing.assert_array_equal(n, kat["rand_ntpp"])


def test_kat_routing_hand_answers_and_regression():
    kat = load("kat_routing")
    # all-equal row: ties go to the lowest indices
    np.testing.assert_array_equal(kat["softmax_renorm_ids"][0], np.arange(8))
    np.testing.assert_allclose(kat["softmax_renorm_w"][0], np.full(8, 1 / 8, np.float32), rtol=1e-6)
    # one large logit, the rest equal: 17 first, then 0..6
    np.testing.assert_array_equal(kat["softmax_renorm_ids"][1], [17, 0, 1, 2, 3, 4, 5, 6])
    # grouped sigmoid, every score equal: groups 0..3 kept, experts 0..7
    np.testing.assert_array_equal(kat["sigmoid_nobias_ids"][0], np.arange(8))
    # the bias lifts expert 5 to rank 0 while its weight stays sigmoid(0) based
    assert kat["sigmoid_ids"][0, 0] == 5
    w, ids = oracle.routing.softmax_topk(kat["softmax_logits"], 8, True)
    np.testing.assert_array_equal(ids, kat["softmax_renorm_ids"])
    np.testing.assert_array_equal(w, kat["softmax_renorm_w"])
    w, ids = oracle.routing.softmax_topk(kat["softmax_logits"], 8, False)
    np.testing.assert_array_equal(ids, kat["softmax_ids"])
    w, ids = oracle.routing.grouped_sigmoid_topk(kat["sigmoid_logits"], kat["sigmoid_bias"], 8, 4, 8, True, 2.5)
    np.testing.assert_array_equal(ids, kat["sigmoid_ids"])
    np.testing.assert_array_equal(w, kat["sigmoid_w"])


# ----------------------------------------------------------------- GPU: HIP path vs fixtures


@pytest.mark.gpu
def test_gpu_kat_routing(dev):
    import torch

    from freetoken_amd import ops
    from _helpers import to_np

    kat = load("kat_routing")
    for renorm, wk, ik in ((True, "softmax_renorm_w", "softmax_renorm_ids"), (False, "softmax_w", "softmax_ids")):
        w, ids = ops.route_softmax_topk(torch.from_numpy(kat["softmax_logits"]).to(dev), 8, renorm)
        np.testing.assert_array_equal(to_np(ids), kat[ik])
        np.testing.assert_allclose(to_np(w), kat[wk], rtol=2e-6, atol=1e-7)
    for bias_key, wk, ik in ((True, "sigmoid_w", "sigmoid_ids"), (False, "sigmoid_nobias_w", "sigmoid_nobias_ids")):
        bias = kat["sigmoid_bias"] if bias_key else np.zeros(32, np.float32)
        w, ids = ops.route_grouped_sigmoid(torch.from_numpy(kat["sigmoid_logits"]).to(dev),
                                           torch.from_numpy(bias).to(dev), 8, 4, 8, True, 2.5)
        np.testing.assert_array_equal(to_np(ids), kat[ik])
        np.testing.assert_allclose(to_np(w), kat[wk], rtol=1e-6, atol=1e-7)


@pytest.mark.gpu
def test_gpu_kat_align(dev):
    import torch

    from freetoken_amd import ops
    from _helpers import to_np

    kat = load("kat_align")
    for key, bs, e in (("doc", 4, 4), ("rand", 8, 16)):
        s, eids, n = ops.align(torch.from_numpy(kat[f"{key}_ids"]).to(dev), bs, e)
        np.testing.assert_array_equal(to_np(s), kat[f"{key}_sorted"])
        np.testing.assert_array_equal(to_np(eids), kat[f"{key}_expert_ids"])
        np.testing.assert_array_equal(to_np(n), kat[f"{key}_ntpp"])


@pytest.mark.gpu
@pytest.mark.parametrize("name", LAYER_CASES)
def test_gpu_layer_matches_fixture(dev, name):
    import torch

    from freetoken_amd import ops
    from _helpers import bf16_dev, to_device_bank, to_np

    fx = load(name)
    inputs, banks, meta = golden.build(name)
    for bname, b in banks.items():
        assert golden.bank_digest(b) == str(fx[f"sha256_{bname}"])
    logits = torch.from_numpy(fx["in_logits"]).to(dev)
    if meta["router"] == "softmax":
        w, ids = ops.route_softmax_topk(logits, meta["k"], bool(meta["renorm"]))
    else:
        w, ids = ops.route_grouped_sigmoid(logits, torch.from_numpy(fx["in_bias"]).to(dev), meta["n_group"],
                                           meta["topk_group"], meta["k"], bool(meta["renorm"]), meta["scale"])
    np.testing.assert_array_equal(to_np(ids), fx["out_topk_ids"])
    np.testing.assert_allclose(to_np(w), fx["out_topk_w"], rtol=1e-6, atol=1e-7)
    if "in_slot_for_id" in fx:
        stats = torch.zeros(4, dtype=torch.int64, device=dev)
        miss = torch.empty(ids.shape, dtype=torch.uint8, device=dev)
        ops.slot_map(ids, torch.from_numpy(fx["in_slot_for_id"]).to(dev), out=ids, miss_mask=miss, stats=stats)
        np.testing.assert_array_equal(to_np(ids), fx["out_slot_ids"])
        np.testing.assert_array_equal(to_np(miss), fx["out_miss_mask"])
        np.testing.assert_array_equal(to_np(stats), fx["out_slot_stats"])
    x = bf16_dev(bf16_from_bits(fx["x_bits"]), dev)
    bank = to_device_bank(banks["bank"], dev)
    shared = to_device_bank(banks["shared"], dev) if "shared" in banks else None
    if meta["regime"] == "decode":
        y = ops.experts_decode(x, w, ids, bank, shared)
    else:
        y = ops.experts_prefill(x, w, ids, bank, shared)
    got, ref = to_np(y), bf16_from_bits(fx["out_y_bits"])
    assert max_rel(got, ref) <= MAX_REL_TOL, (name, max_rel(got, ref))
    assert cosine(got, ref) >= COS_TOL, (name, cosine(got, ref))
