"""The decode routing histogram (ftmoe_route_histogram; reference
OffloadMoeCache.decode_freq, moe/offload_cache.py:230-236,803-807) against
numpy's bincount: ids outside [0, E) skipped, counts accumulated over calls,
counted from the raw expert ids by every decode path of OffloadMoELayer (the
fused slot lookup rewrites them to slots in the same call), and kept counting
in a replayed graph."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import synth
from freetoken_amd import ops
from freetoken_amd.moe.offload_cache import ExpertSlotCache
from freetoken_amd.layers.moe import OffloadMoELayer

from _helpers import bf16_dev, to_device_bank, to_np

pytestmark = pytest.mark.gpu


def _bincount(ids, E):
    v = ids.reshape(-1)
    return np.bincount(v[(v >= 0) & (v < E)], minlength=E).astype(np.int64)


@pytest.mark.parametrize("numel,E", [(1, 256), (8, 256), (2048, 256), (70000, 160), (5000, 16384)])
def test_route_histogram_matches_bincount(dev, numel, E):
    rng = np.random.default_rng(numel + E)
    ids = rng.integers(-3, E + 3, size=numel).astype(np.int32)
    freq = torch.zeros(E, dtype=torch.int64, device=dev)
    t = torch.from_numpy(ids).to(dev)
    ops.route_histogram(t, freq)
    ops.route_histogram(t, freq)  # accumulates
    np.testing.assert_array_equal(to_np(freq), 2 * _bincount(ids, E))


def test_offload_layer_counts_raw_ids_and_replays(dev):
    rng = np.random.default_rng(5)
    E, S, H, I, k, M = 32, 8, 512, 256, 4, 6
    bank = synth.make_bank("fp8", E, H, I, rng)
    resident = np.sort(rng.choice(E, S, replace=False))
    cache = ExpertSlotCache(2, E, S, "fp8_block", device=dev)
    db = to_device_bank(bank, dev, resident)
    cache.set_bank_caches(gate_up=db.gate_up, gate_up_scale=db.gate_up_scale, down=db.down, down_scale=db.down_scale)
    cache.assign(1, resident, np.arange(S))
    cache.collect_decode_freq = True
    layer = OffloadMoELayer(1, E, k, H, I, device=dev)
    layer.offload_cache = cache
    x_buf = bf16_dev(synth.activations(rng, M, H), dev)
    w_buf = torch.full((M, k), 0.25, dtype=torch.float32, device=dev)
    i_buf = torch.zeros((M, k), dtype=torch.int32, device=dev)
    raw_src = torch.zeros((M, k), dtype=torch.int32, device=dev)
    want = np.zeros(E, np.int64)

    def new_ids():
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
        raw_src.copy_(torch.from_numpy(ids))
        return ids

    ids = new_ids()
    i_buf.copy_(raw_src)
    layer.routed_forward(x_buf, w_buf, i_buf)  # eager: sizes the workspace
    want += _bincount(ids, E)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(to_np(cache.decode_freq[1]), want)
    assert int(cache.decode_freq[0].sum()) == 0
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            i_buf.copy_(raw_src)
            layer.routed_forward(x_buf, w_buf, i_buf)
    torch.cuda.synchronize()
    for _ in range(3):
        ids = new_ids()
        graph.replay()
        torch.cuda.synchronize()
        want += _bincount(ids, E)
        np.testing.assert_array_equal(to_np(cache.decode_freq[1]), want)
    del graph
    st = cache.decode_routing_stats()
    assert st["working_set_max"] == int((want > 0).sum())
    assert abs(st["slots_per_layer"] - S / 2) < 1e-12
