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
@pytest.mark.parametrize("M", [1, 2, 4, 8, 16, 33])
@pytest.mark.parametrize("fmts", [("fp8", "fp8"), ("mxfp4", "bf16")])
def test_grouped_routed_cached_matches_separate_calls(dev, M, fmts):
    """C4-shaped router (256 experts, 8 groups, top-4 groups, k 8) over a
    64-slot table with misses, with a shared expert (FP8 beside FP8, bf16 beside
    MXFP4 as in C3).  Up to 2 tokens the shared expert's gate_up runs in the
    router's launch; the outputs must still equal the separate calls bit for
    bit."""
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
