"""The module interface (drop-in boundary) end to end: ``MoELayer``,
``OffloadMoELayer`` over an ``ExpertSlotCache``, ``make_moe_layer`` and the
backend registry, against the CPU oracle (routing bit-exact; bf16 outputs
within max-rel 2e-2 and cosine 0.9995).  Reference: ``layers/moe.py:29-194,
197-636``, ``moe/__init__.py:16-65``, ``moe/offload_cache.py:155-175,800-810``."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle
from oracle import synth
from freetoken_amd import ops
from freetoken_amd.core import moe_phase
from freetoken_amd.layers.moe import MoELayer, OffloadMoELayer, make_moe_layer
from freetoken_amd.moe import SUPPORTED_MOE_BACKENDS, create_moe_backend, is_offload_moe_backend
from freetoken_amd.moe.offload_cache import ExpertSlotCache

from _helpers import bf16_dev, to_device_bank, to_np
from conftest import COS_TOL, MAX_REL_TOL, cosine, max_rel

_LAYER_FMT = {"bf16": "bf16", "fp8": "fp8_block", "mxfp4": "ds_fp4"}


def _load_layer(layer: MoELayer, bank) -> None:
    """Copies an oracle bank into the layer's weight attributes."""
    dev = layer.device
    if bank.fmt == "bf16":
        layer.gate_up_proj.copy_(torch.from_numpy(bank.gate_up).to(dev).to(torch.bfloat16))
        layer.down_proj.copy_(torch.from_numpy(bank.down).to(dev).to(torch.bfloat16))
    elif bank.fmt == "fp8":
        layer.gate_up_proj.copy_(torch.from_numpy(bank.gate_up).to(dev).view(torch.float8_e4m3fn))
        layer.down_proj.copy_(torch.from_numpy(bank.down).to(dev).view(torch.float8_e4m3fn))
        layer.gate_up_scale_inv.copy_(torch.from_numpy(bank.gate_up_scale).to(dev))
        layer.down_scale_inv.copy_(torch.from_numpy(bank.down_scale).to(dev))
    else:
        layer.gate_up_proj.copy_(torch.from_numpy(bank.gate_up).to(dev))
        layer.down_proj.copy_(torch.from_numpy(bank.down).to(dev))
        layer.gate_up_scale.copy_(torch.from_numpy(bank.gate_up_scale).to(dev))
        layer.down_scale.copy_(torch.from_numpy(bank.down_scale).to(dev))


def _check(got: torch.Tensor, ref: np.ndarray, what) -> None:
    g = to_np(got)
    assert max_rel(g, ref) <= MAX_REL_TOL, (what, max_rel(g, ref))
    assert cosine(g, ref) >= COS_TOL, (what, cosine(g, ref))


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["bf16", "fp8", "mxfp4"])
@pytest.mark.parametrize("phase,M", [("decode", 6), ("prefill", 40)])
@pytest.mark.parametrize("with_shared", [False, True])
def test_moe_layer_forward(dev, fmt, phase, M, with_shared):
    rng = np.random.default_rng(M + (3 if with_shared else 0))
    E, H, I, k = 16, 512, 256, 4
    bank = synth.make_bank(fmt, E, H, I, rng)
    shared = synth.make_bank(fmt, 1, H, I, rng) if with_shared else None
    layer = MoELayer(E, k, H, I, renormalize=True, weight_format=_LAYER_FMT[fmt], device=dev)
    _load_layer(layer, bank)
    if shared is not None:
        layer.shared_expert = to_device_bank(shared, dev)
    x = synth.activations(rng, M, H)
    logits = synth.normal(rng, (M, E))
    w_ref, ids_ref = oracle.routing.softmax_topk(logits, k, True)
    y_ref = oracle.experts.moe_layer(phase, x, w_ref, ids_ref, bank, shared)
    with moe_phase(phase):
        y = layer.forward(bf16_dev(x, dev), torch.from_numpy(logits).to(dev))
    _check(y, y_ref, (fmt, phase, with_shared))


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
def test_moe_layer_routed_forward_grouped_sigmoid(dev, fmt):
    """The DeepSeek-V3 block: grouped-sigmoid routing from the model code, then
    routed_forward with a shared expert (decode and prefill)."""
    rng = np.random.default_rng(31)
    E, H, I, k = 32, 512, 256, 8
    bank = synth.make_bank(fmt, E, H, I, rng)
    shared = synth.make_bank(fmt, 1, H, I, rng)
    layer = MoELayer(E, k, H, I, weight_format=_LAYER_FMT[fmt], device=dev)
    _load_layer(layer, bank)
    layer.shared_expert = to_device_bank(shared, dev)
    bias = synth.normal(rng, (E,), 0.1)
    for phase, M in (("decode", 8), ("prefill", 48)):
        x = synth.activations(rng, M, H)
        logits = synth.normal(rng, (M, E))
        w_ref, ids_ref = oracle.routing.grouped_sigmoid_topk(logits, bias, 8, 4, k, True, 2.5)
        w, ids = ops.route_grouped_sigmoid(torch.from_numpy(logits).to(dev), torch.from_numpy(bias).to(dev), 8, 4, k,
                                           True, 2.5)
        np.testing.assert_array_equal(to_np(ids), ids_ref)
        y_ref = oracle.experts.moe_layer(phase, x, w_ref, ids_ref, bank, shared)
        with moe_phase(phase):
            y = layer.routed_forward(bf16_dev(x, dev), w, ids)
        _check(y, y_ref, (fmt, phase))


def _offload_layer(dev, fmt, E, S, H, I, k, rng, resident):
    bank = synth.make_bank(fmt, E, H, I, rng)
    cache = ExpertSlotCache(2, E, S, _LAYER_FMT[fmt], device=dev)
    rows = np.asarray(resident)
    dbank = to_device_bank(bank, dev, rows)
    names = ("gate_up", "down") if fmt == "bf16" else ("gate_up", "gate_up_scale", "down", "down_scale")
    tensors = ((dbank.gate_up, dbank.down) if fmt == "bf16"
               else (dbank.gate_up, dbank.gate_up_scale, dbank.down, dbank.down_scale))
    cache.set_bank_caches(**dict(zip(names, tensors)))
    cache.assign(1, rows, np.arange(len(rows)))
    layer = OffloadMoELayer(1, E, k, H, I, device=dev)
    layer.offload_cache = cache
    return layer, cache, bank


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
def test_offload_layer_decode_with_misses(dev, fmt):
    """Decode over 8 resident slots of 32 experts: ids are rewritten to slots in
    place, misses are skipped and counted (layer 1's counters)."""
    rng = np.random.default_rng(41)
    E, S, H, I, k, M = 32, 8, 512, 256, 4, 12
    resident = np.sort(rng.choice(E, S, replace=False))
    layer, cache, bank = _offload_layer(dev, fmt, E, S, H, I, k, rng, resident)
    table = np.full(E, -1, dtype=np.int32)
    table[resident] = np.arange(S, dtype=np.int32)
    x = synth.activations(rng, M, H)
    logits = synth.normal(rng, (M, E))
    w_ref, ids_ref = oracle.routing.softmax_topk(logits, k, True)
    slots_ref, _, stats_ref = oracle.slots.slot_map(ids_ref, table)
    sub = oracle.experts.Bank(bank.fmt, bank.gate_up[resident], bank.down[resident],
                              None if bank.gate_up_scale is None else bank.gate_up_scale[resident],
                              None if bank.down_scale is None else bank.down_scale[resident])
    y_ref = oracle.experts.moe_layer("decode", x, w_ref, slots_ref, sub, None)
    ids = torch.from_numpy(ids_ref.copy()).to(dev)
    with moe_phase("decode", backend="offload"):
        y = layer.routed_forward(bf16_dev(x, dev), torch.from_numpy(w_ref).to(dev), ids)
    np.testing.assert_array_equal(to_np(ids), slots_ref)
    np.testing.assert_array_equal(to_np(cache.lru_stats[1]), stats_ref)
    assert int(cache.lru_stats[0].abs().sum()) == 0
    _check(y, y_ref, fmt)
    st = cache.decode_miss_stats()
    assert st["layer_calls"] == 1 and st["missed_routes"] == int(stats_ref[3])


@pytest.mark.gpu
def test_offload_layer_prefill_materialised(dev):
    """Prefill reads the first num_experts slot rows (slot == expert)."""
    rng = np.random.default_rng(43)
    E, H, I, k, M = 16, 512, 256, 4, 40
    layer, _, bank = _offload_layer(dev, "fp8", E, E, H, I, k, rng, np.arange(E))
    x = synth.activations(rng, M, H)
    logits = synth.normal(rng, (M, E))
    w_ref, ids_ref = oracle.routing.softmax_topk(logits, k, True)
    y_ref = oracle.experts.moe_layer("prefill", x, w_ref, ids_ref, bank, None)
    with moe_phase("prefill", backend="offload"):
        y = layer.routed_forward(bf16_dev(x, dev), torch.from_numpy(w_ref).to(dev),
                                 torch.from_numpy(ids_ref).to(dev))
    _check(y, y_ref, "offload prefill")


@pytest.mark.gpu
def test_fused_backend_forward(dev):
    """SUPPORTED_MOE_BACKENDS["fused"]().forward (reference moe/fused.py:426-452)."""
    rng = np.random.default_rng(47)
    E, H, I, k, M = 16, 512, 256, 2, 5
    bank = synth.make_bank("bf16", E, H, I, rng)
    x = synth.activations(rng, M, H)
    logits = synth.normal(rng, (M, E))
    w_ref, ids_ref = oracle.routing.softmax_topk(logits, k, True)
    y_ref = oracle.experts.moe_layer("decode", x, w_ref, ids_ref, bank, None)
    be = create_moe_backend("fused")
    y = be.forward(bf16_dev(x, dev), torch.from_numpy(bank.gate_up).to(dev).to(torch.bfloat16),
                   torch.from_numpy(bank.down).to(dev).to(torch.bfloat16), torch.from_numpy(logits).to(dev), k, True)
    _check(y, y_ref, "fused backend")


# ----------------------------------------------------------------- host logic (CPU)


def test_registry_and_construction_seam():
    assert {"fused", "mi355x", "offload"} <= set(SUPPORTED_MOE_BACKENDS.keys())
    assert is_offload_moe_backend("offload") and not is_offload_moe_backend("fused")
    with pytest.raises(KeyError):
        create_moe_backend("nope")
    with pytest.raises(RuntimeError):
        create_moe_backend("offload").forward(None, None, None, None, 1, True, "silu", False)
    cfg = SimpleNamespace(num_experts=8, num_experts_per_tok=2, hidden_size=256, moe_intermediate_size=128,
                          norm_topk_prob=True, moe_backend="fused")
    layer = make_moe_layer(cfg, weight_format="fp8_block", extra_attrs={"tag": 7})
    assert type(layer) is MoELayer and layer.tag == 7
    assert layer.gate_up_proj.shape == (8, 256, 256) and layer.gate_up_proj.dtype == torch.float8_e4m3fn
    assert layer.gate_up_scale_inv.shape == (8, 2, 2) and layer.down_scale_inv.shape == (8, 2, 1)
    cfg.moe_backend = "offload"
    off = make_moe_layer(cfg, layer_id=3)
    assert type(off) is OffloadMoELayer and off.layer_id == 3 and not hasattr(off, "gate_up_proj")
    with pytest.raises(AssertionError):
        make_moe_layer(cfg)  # offload layers need their layer id


@pytest.mark.gpu
def test_graph_replay_after_workspace_growth(dev, monkeypatch):
    """Capture-then-prefill (the reference's engine/graph.py:127-187 order):
    decode captured in a graph, then an eager prefill that needs a larger
    workspace, then replays.  The buffer the graph captured must stay owned by
    the workspace: a tensor allocated after the growth is never written by a
    replay, and every replay and the prefill match the oracle."""
    monkeypatch.setattr(ops, "_WS", ops._Workspace())  # start from an empty workspace
    rng = np.random.default_rng(131)
    E, H, I, k, M, Mp = 32, 1024, 512, 8, 8, 512
    bank = synth.make_bank("fp8", E, H, I, rng)
    shared = synth.make_bank("fp8", 1, H, I, rng)
    dbank, dshared = to_device_bank(bank, dev), to_device_bank(shared, dev)
    x_buf = torch.zeros((M, H), dtype=torch.bfloat16, device=dev)
    w_buf = torch.zeros((M, k), dtype=torch.float32, device=dev)
    ids_buf = torch.zeros((M, k), dtype=torch.int32, device=dev)

    def routing(m):
        w_ref, ids_ref = oracle.routing.softmax_topk(synth.normal(rng, (m, E)), k, True)
        return synth.activations(rng, m, H), w_ref, ids_ref

    x, w_ref, ids_ref = routing(M)
    x_buf.copy_(bf16_dev(x, dev))
    w_buf.copy_(torch.from_numpy(w_ref))
    ids_buf.copy_(torch.from_numpy(ids_ref))
    ops.experts_decode(x_buf, w_buf, ids_buf, dbank, dshared)  # eager call sizes the workspace
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream(device=dev)
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            y = ops.experts_decode(x_buf, w_buf, ids_buf, dbank, dshared)
    torch.cuda.synchronize()
    captured = ops._WS.buf[dev.index or 0]
    cap_ptr, cap_bytes = captured.data_ptr(), captured.numel()
    del captured

    xp, wp, idp = routing(Mp)
    yp = ops.experts_prefill(bf16_dev(xp, dev), torch.from_numpy(wp).to(dev), torch.from_numpy(idp).to(dev),
                             dbank, dshared)
    torch.cuda.synchronize()
    assert ops._WS.buf[dev.index or 0].data_ptr() != cap_ptr, "the prefill should have grown the workspace"
    # memory freed by the growth would be handed to the next allocation of its size
    junk = torch.full((cap_bytes,), 0x5A, dtype=torch.uint8, device=dev)
    _check(yp, oracle.experts.moe_layer("prefill", xp, wp, idp, bank, shared), "prefill after capture")
    for rep in range(3):
        x, w_ref, ids_ref = routing(M)
        x_buf.copy_(bf16_dev(x, dev))
        w_buf.copy_(torch.from_numpy(w_ref))
        ids_buf.copy_(torch.from_numpy(ids_ref))
        graph.replay()
        torch.cuda.synchronize()
        _check(y, oracle.experts.moe_layer("decode", x, w_ref, ids_ref, bank, shared), ("replay", rep))
        assert bool((junk == 0x5A).all()), f"replay {rep} wrote into memory released by the workspace"
    del graph
    ops.release_retired_workspaces()
