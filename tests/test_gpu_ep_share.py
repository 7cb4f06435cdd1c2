"""Expert-parallel shares of a decode layer on one GPU (the per-GPU part of
the path's EP sharding; the all-to-alls are not on one GPU): the experts are
split over `ep` banks, each share receives the tokens with at least one route
to its experts (other routes as -1) and runs the ordinary decode entry point.
Each share must match the oracle on its own routes, and the sum of the shares'
outputs, scattered back to the tokens, the whole layer (routes summed across
shares in float32 before the bf16 rounding of the reference's combine, so only
within tolerance)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import synth
from freetoken_amd import ops

from _helpers import bf16_dev, sub_bank, to_device_bank, to_np
from test_gpu_parity import COS_TOL, MAX_REL_TOL, cosine, max_rel


@pytest.mark.gpu
@pytest.mark.parametrize("ep,B", [(4, 48), (8, 300)])
def test_ep_shares_sum_to_the_layer(dev, ep, B):
    rng = np.random.default_rng(40 + ep)
    E, H, I, k = 64, 512, 256, 8
    bank = synth.make_bank("fp8", E, H, I, rng)
    x = synth.activations(rng, B, H)
    w, ids = oracle.routing.grouped_sigmoid_topk(synth.normal(rng, (B, E)), synth.normal(rng, (E,), 0.1), 8, 4, k,
                                                 True, 2.5)
    y_full = oracle.experts.moe_layer("decode", x, w, ids, bank, None)
    e_loc = E // ep
    acc = np.zeros((B, H), dtype=np.float32)
    for g in range(ep):
        lo = g * e_loc
        local = (ids >= lo) & (ids < lo + e_loc)
        tok = np.nonzero(local.any(1))[0]
        if tok.size == 0:
            continue
        ids_g = np.where(local[tok], ids[tok] - lo, -1).astype(np.int32)
        share = sub_bank(bank, np.arange(lo, lo + e_loc))
        y = ops.experts_decode(bf16_dev(x[tok], dev), torch.from_numpy(w[tok].copy()).to(dev),
                               torch.from_numpy(ids_g).to(dev), to_device_bank(share, dev))
        got = to_np(y)
        ref = oracle.experts.moe_layer("decode", x[tok], w[tok], ids_g, share, None)
        assert max_rel(got, ref) <= MAX_REL_TOL and cosine(got, ref) >= COS_TOL, (g, max_rel(got, ref))
        acc[tok] += got
    assert max_rel(acc, y_full) <= MAX_REL_TOL, max_rel(acc, y_full)
    assert cosine(acc, y_full) >= COS_TOL, cosine(acc, y_full)
