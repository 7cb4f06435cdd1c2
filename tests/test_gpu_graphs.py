"""Decode calls captured in HIP graphs and replayed: the router + shared
expert launch (grouped router, up to four tokens), the router and the
permutation in separate launches (40 and 96 tokens), and the wide FP8
segments of calls from 144 tokens.  Every replay, with new inputs written into the
captured buffers and an eager call of the same layer between replays, must
equal the eager call bit for bit (the decode path is fixed-shape and free of
host synchronisation, as the reference's captured decode requires,
engine/graph.py:127-187)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import synth
from freetoken_amd import ops

from _helpers import bf16_dev, code_bank, to_device_bank


@pytest.mark.gpu
@pytest.mark.parametrize("M,fmts", [(1, ("fp8", "fp8")), (2, ("mxfp4", "bf16")), (4, ("fp8", "fp8")),
                                    (40, ("mxfp4", "bf16")), (96, ("fp8", "fp8")), (160, ("fp8", "fp8")),
                                    (256, ("fp8", "fp8"))])
def test_routed_decode_graph_replays_equal_eager(dev, M, fmts):
    rng = np.random.default_rng(900 + M)
    E, S, H, I, k = 256, 64, 512, 256, 8
    bank = to_device_bank(code_bank(fmts[0], S, H, I, rng), dev)
    if fmts[1] == "bf16":
        shared = to_device_bank(synth.make_bank("bf16", 1, H, 384, rng), dev)
    else:
        shared = to_device_bank(code_bank(fmts[1], 1, H, I, rng), dev)
    table = np.full(E, -1, dtype=np.int32)
    table[np.sort(rng.choice(E, S, replace=False))] = np.arange(S, dtype=np.int32)
    t_dev = torch.from_numpy(table).to(dev)
    bias = torch.from_numpy(synth.normal(rng, (E,), 0.1)).to(dev)
    router = ops.Router("grouped_sigmoid", k, True, bias, 8, 4, 2.5)

    def inputs():
        x = bf16_dev(synth.activations(rng, M, H), dev)
        # logits biased towards the resident experts, so most routes are served
        logits = synth.normal(rng, (M, E)) + 2.0 * (table >= 0)[None, :]
        return x, torch.from_numpy(logits.astype(np.float32)).to(dev)

    x_buf = torch.zeros((M, H), dtype=torch.bfloat16, device=dev)
    l_buf = torch.zeros((M, E), dtype=torch.float32, device=dev)
    y_buf = torch.empty((M, H), dtype=torch.bfloat16, device=dev)
    w_buf = torch.empty((M, k), dtype=torch.float32, device=dev)
    i_buf = torch.empty((M, k), dtype=torch.int32, device=dev)
    x, lg = inputs()
    x_buf.copy_(x)
    l_buf.copy_(lg)

    def call(xx, ll, out, w, ids):
        return ops.experts_decode_routed(xx, ll, router, bank, shared=shared, out=out, slot_for_id=t_dev,
                                         topk_w=w, topk_ids=ids)

    call(x_buf, l_buf, y_buf, w_buf, i_buf)  # eager call sizes the workspace
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            call(x_buf, l_buf, y_buf, w_buf, i_buf)
    torch.cuda.synchronize()
    for rep in range(3):
        x, lg = inputs()
        x_buf.copy_(x)
        l_buf.copy_(lg)
        y_e, w_e, i_e = call(x.clone(), lg.clone(), None, None, None)  # eager, other buffers
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(i_buf, i_e), ("slot ids", rep)
        assert torch.equal(w_buf, w_e), ("weights", rep)
        assert torch.equal(y_buf, y_e), ("y", rep)
        assert bool(torch.isfinite(y_buf.float()).all())
    del graph
