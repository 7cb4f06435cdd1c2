"""ftmoe_experts_decode_routed (router logits -> decode output in one call)
against the separate calls it replaces: the router entry point followed by
ftmoe_experts_decode / ftmoe_experts_decode_cached.  Same kernels after the
router, so weights, ids, slot ids, counters and outputs must be bit-identical,
both where the router and the permutation share one launch (at most 16 tokens
and 64 routes) and where they do not.  Reference: MoELayer.forward decode
(layers/moe.py:166-194), the DeepSeek-V3 block (models/glm4_moe/moe.py:53-83)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import synth
from freetoken_amd import ops

from _helpers import bf16_dev, code_bank, to_device_bank, to_np


def _same(a, b, what):
    assert torch.equal(a, b), what


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 3, 8, 9, 40])
@pytest.mark.parametrize("logit_dtype", [torch.float32, torch.bfloat16])
def test_softmax_routed_matches_separate_calls(dev, M, logit_dtype):
    rng = np.random.default_rng(M)
    E, H, I, k = 128, 512, 256, 8 if M <= 8 else 4
    bank = to_device_bank(synth.make_bank("fp8", E, H, I, rng), dev)
    x = bf16_dev(synth.activations(rng, M, H), dev)
    logits = torch.from_numpy(synth.normal(rng, (M, E))).to(dev).to(logit_dtype)
    y, w, ids = ops.experts_decode_routed(x, logits, ops.Router("softmax", k, True), bank)
    w2, ids2 = ops.route_softmax_topk(logits, k, True)
    y2 = ops.experts_decode(x, w2, ids2, bank)
    torch.cuda.synchronize()
    _same(ids, ids2, "ids")
    _same(w, w2, "weights")
    _same(y, y2, "y")
    # and the routing itself against the oracle
    w_ref, ids_ref = oracle.routing.softmax_topk(logits.float().cpu().numpy(), k, True)
    np.testing.assert_array_equal(to_np(ids), ids_ref)


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 3, 4, 8, 16, 33, 96, 160])
@pytest.mark.parametrize("fmts", [("fp8", "fp8"), ("mxfp4", "bf16")])
def test_grouped_routed_cached_matches_separate_calls(dev, M, fmts):
    """C4-shaped router (256 experts, 8 groups, top-4 groups, k 8) over a
    64-slot table with misses, with a shared expert (FP8 beside FP8, bf16 beside
    MXFP4 as in C3).  Up to 4 tokens the shared expert's gate_up runs in the
    router's launch; from 17 tokens the router and the permutation run in
    separate launches (M = 33: the gate_up K split four ways; 96: the FP8
    K-unsplit kernel; 160: the FP8 wide kernel).  The outputs must equal the
    separate calls bit for bit."""
    rng = np.random.default_rng(100 + M)
    E, S, H, I, k = 256, 64, 512, 256, 8
    bank = to_device_bank(code_bank(fmts[0], S, H, I, rng), dev)
    if fmts[1] == "bf16":
        shared = to_device_bank(synth.make_bank("bf16", 1, H, 384, rng), dev)  # its own intermediate size
    else:
        shared = to_device_bank(code_bank(fmts[1], 1, H, I, rng), dev)
    table = np.full(E, -1, dtype=np.int32)
    table[np.sort(rng.choice(E, S, replace=False))] = np.arange(S, dtype=np.int32)
    t_dev = torch.from_numpy(table).to(dev)
    bias = torch.from_numpy(synth.normal(rng, (E,), 0.1)).to(dev)
    x = bf16_dev(synth.activations(rng, M, H), dev)
    logits = torch.from_numpy(synth.normal(rng, (M, E))).to(dev)
    router = ops.Router("grouped_sigmoid", k, True, bias, 8, 4, 2.5)
    st1 = torch.zeros(4, dtype=torch.int64, device=dev)
    st2 = torch.zeros(4, dtype=torch.int64, device=dev)
    miss1 = torch.zeros((M, k), dtype=torch.uint8, device=dev)
    miss2 = torch.zeros((M, k), dtype=torch.uint8, device=dev)
    y, w, ids = ops.experts_decode_routed(x, logits, router, bank, shared=shared, slot_for_id=t_dev, miss_mask=miss1,
                                          stats=st1)
    w2, ids2 = ops.route_grouped_sigmoid(logits, bias, 8, 4, k, True, 2.5)
    y2 = ops.experts_decode(x, w2, ids2, bank, shared=shared, slot_for_id=t_dev, miss_mask=miss2, stats=st2)
    torch.cuda.synchronize()
    _same(w, w2, "weights")
    _same(ids, ids2, "slot ids")
    _same(miss1, miss2, "miss mask")
    _same(st1, st2, "counters")
    _same(y, y2, "y")
    w_ref, ids_ref = oracle.routing.grouped_sigmoid_topk(logits.cpu().numpy(), bias.cpu().numpy(), 8, 4, k, True, 2.5)
    slots_ref, _, _ = oracle.slots.slot_map(ids_ref, table)
    np.testing.assert_array_equal(to_np(ids), slots_ref)


# ----------------------------------------------------------------- front-end routers under ties
# The decode front ends (router + permutation in one launch: up to 16 tokens
# and 64 routes; with a grouped router and a shared expert up to 4 tokens
# beside the shared gate_up) select each token's experts in a wave of their
# own launch, and align up to 16 routes by counting ranks instead of sorting.
# On logits full of exact ties (copied values, whole rows equal, tied groups,
# -0.0 against +0.0, a bias that flips the choice) their ids must equal the
# oracle's and their weights the standalone router's bit for bit, with the
# permutation after them.


def _tie_rows(rng, M, E, bf16):
    lg = synth.tied_logits(rng, M, E, bf16=bf16)
    lg[0] = 0.25  # a whole row tied: lowest groups, lowest experts
    if M > 1:
        lg[1, : E // 2] = -0.0
        lg[1, E // 2:] = 0.0  # -0.0 equals +0.0: the lower index wins
    if M > 2:
        lg[2] = np.tile(np.arange(8, dtype=np.float32), E // 8)  # repeating pattern: every group ties
    return lg


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 3, 16])
@pytest.mark.parametrize("E,k,renorm,bf16", [(16, 2, True, True), (128, 8, True, False), (160, 8, False, False),
                                             (256, 8, True, True), (256, 6, False, True)])
def test_front_end_softmax_ties(dev, M, E, k, renorm, bf16):
    rng = np.random.default_rng(E + 7 * M + k)
    k = min(k, 64 // M)
    H, I = 128, 128
    bank = to_device_bank(synth.make_bank("bf16", E, H, I, rng), dev)
    lg = _tie_rows(rng, M, E, bf16)
    t = torch.from_numpy(lg).to(dev)
    t = t.to(torch.bfloat16) if bf16 else t
    x = bf16_dev(synth.activations(rng, M, H), dev)
    y, w, ids = ops.experts_decode_routed(x, t, ops.Router("softmax", k, renorm), bank)
    w2, ids2 = ops.route_softmax_topk(t, k, renorm)
    y2 = ops.experts_decode(x, w2, ids2, bank)
    torch.cuda.synchronize()
    _, ids_ref = oracle.routing.softmax_topk(t.float().cpu().numpy(), k, renorm)
    np.testing.assert_array_equal(to_np(ids), ids_ref)
    _same(w, w2, "weights")
    _same(y, y2, "y")


@pytest.mark.gpu
@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 16])
@pytest.mark.parametrize("E,ng,tg,k", [(256, 8, 4, 8), (64, 8, 4, 4), (160, 1, 1, 8), (96, 8, 4, 4), (256, 16, 4, 2)])
@pytest.mark.parametrize("shared", [False, True])
def test_front_end_grouped_ties(dev, M, E, ng, tg, k, shared):
    """Grouped router front ends (lane-block group scores, and the LDS scan for
    groups of 12), with and without a slot table, and with a shared expert (its
    gate_up in the router's launch up to 4 tokens)."""
    rng = np.random.default_rng(E * 3 + M + ng)
    k = min(k, 64 // M)
    H, I, S = 128, 128, E // 2
    bank = to_device_bank(synth.make_bank("bf16", S, H, I, rng), dev)
    sh = to_device_bank(synth.make_bank("bf16", 1, H, I, rng), dev) if shared else None
    table = np.full(E, -1, dtype=np.int32)
    table[np.sort(rng.choice(E, S, replace=False))] = np.arange(S, dtype=np.int32)
    t_dev = torch.from_numpy(table).to(dev)
    lg = _tie_rows(rng, M, E, False)
    bias = synth.normal(rng, (E,), 0.05)
    bias[E - 1] = 5.0  # flips the choice towards the last expert
    for b in (None, bias):
        tb = None if b is None else torch.from_numpy(b).to(dev)
        router = ops.Router("grouped_sigmoid", k, True, tb, ng, tg, 2.5)
        x = bf16_dev(synth.activations(rng, M, H), dev)
        logits = torch.from_numpy(lg).to(dev)
        st1 = torch.zeros(4, dtype=torch.int64, device=dev)
        st2 = torch.zeros(4, dtype=torch.int64, device=dev)
        y, w, slots = ops.experts_decode_routed(x, logits, router, bank, shared=sh, slot_for_id=t_dev, stats=st1)
        w2, ids2 = ops.route_grouped_sigmoid(logits, tb, ng, tg, k, True, 2.5)
        y2 = ops.experts_decode(x, w2, ids2, bank, shared=sh, slot_for_id=t_dev, stats=st2)
        torch.cuda.synchronize()
        _, ids_ref = oracle.routing.grouped_sigmoid_topk(lg, b, ng, tg, k, True, 2.5)
        slots_ref, _, stats_ref = oracle.slots.slot_map(ids_ref, table)
        np.testing.assert_array_equal(to_np(slots), slots_ref)
        np.testing.assert_array_equal(to_np(st1), stats_ref)
        _same(w, w2, "weights")
        _same(slots, ids2, "slot ids")
        _same(st1, st2, "counters")
        _same(y, y2, "y")
