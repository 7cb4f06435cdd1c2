"""Hybrid CPU/GPU decode (reference layers/moe.py:325-372, moe/cpu_executor.py:
538-600): the capped admission with its CPU split bit-exact against the
oracle (offload_kernels.py:128-188, the balance rule of :160-164 and its test
tests/moe/test_hybrid_fetch.py:89-115), and offload layers whose decode
splits each step between the GPU slot cache and the CPU executor computing
what the oracle computes -- eagerly and replayed in a captured graph."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import slots as S
from oracle import synth
from freetoken_amd.core import moe_phase
from freetoken_amd.layers.moe import OffloadMoELayer
from freetoken_amd.moe.cpu_decode import CpuMoeDecoder
from freetoken_amd.moe.offload_cache import ExpertSlotCache

from _helpers import bf16_dev, to_device_bank, to_np
from conftest import COS_TOL, MAX_REL_TOL, cosine, max_rel

Q16 = 1 << 16


@pytest.mark.gpu
@pytest.mark.parametrize("frac,max_fetch", [(0.415, 32), (0.0, 1), (0.0, 0), (1.0, 32)])
def test_hybrid_admission_and_split_match_oracle(dev, frac, max_fetch):
    L, E, Sz, k = 2, 32, 40, 8
    st = S.CacheState(L, E, Sz)
    cache = ExpertSlotCache(L, E, Sz, "fp8_block", device=dev, decode_target="hybrid", hybrid_max_fetch=max_fetch,
                            hybrid_fetch_fraction=frac)
    cache.sources = {"_": []}  # admission only: no gather in this test
    fq = min(Q16, max(0, round(frac * Q16)))
    rng = np.random.default_rng(int(frac * 1000) + max_fetch)
    for step in range(64):
        layer = step % L
        ids = rng.permutation(E)[:k].astype(np.int32).reshape(2, k // 2)
        if step % 9 == 4:
            ids[0, 0] = E + 3  # outside [0, E): skipped, never given to the CPU
        out_ref, evict, src, nmiss, _ = S.lru_ensure(st, layer, ids, max_fetch=max_fetch, by_recency=True,
                                                     capacity=min(E, Sz), frac_q16=fq)
        t = torch.from_numpy(ids.copy()).to(dev)
        cpu = torch.full_like(t, -9)
        cache.ensure_experts_hybrid(layer, t, cpu_ids=cpu)
        np.testing.assert_array_equal(to_np(t), out_ref, err_msg=f"step {step}")
        np.testing.assert_array_equal(to_np(cpu), S.hybrid_split(ids, out_ref, E), err_msg=f"step {step}")
        n = int(cache.num_indices.item())
        assert n == evict.size and int(cache.num_missing_full.item()) == nmiss
        np.testing.assert_array_equal(to_np(cache.evict_slots)[:n], evict)
        np.testing.assert_array_equal(to_np(cache.src_indices)[:n], src)
        np.testing.assert_array_equal(to_np(cache.slot_for_id), st.slot_for_id)
        np.testing.assert_array_equal(to_np(cache.expert_recency), st.recency)


def _pinned(bank):
    arrays = (bank.gate_up, bank.gate_up_scale, bank.down, bank.down_scale)
    return [torch.from_numpy(np.ascontiguousarray(a)).pin_memory() for a in arrays]


def _hybrid_setup(dev, fmt, L, E, Sz, H, I, k, rng, decode_target="hybrid", handshake="host", **kw):
    banks = [synth.make_bank(fmt, E, H, I, rng) for _ in range(L)]
    qfmt = {"fp8": "fp8_block", "mxfp4": "ds_fp4"}[fmt]
    cache = ExpertSlotCache(L, E, Sz, qfmt, device=dev, decode_target=decode_target, **kw)
    eb = to_device_bank(banks[0], dev, rows=np.arange(Sz))
    cache.set_bank_caches(gate_up=eb.gate_up, gate_up_scale=eb.gate_up_scale, down=eb.down, down_scale=eb.down_scale)
    for t in cache.banks.values():
        t.view(torch.uint8).fill_(0)
    names = ("gate_up", "gate_up_scale", "down", "down_scale")
    per_layer = [_pinned(b) for b in banks]
    cache.set_bank_sources({n: [per_layer[l][j] for l in range(L)] for j, n in enumerate(names)})
    cache.reset()
    dec = CpuMoeDecoder(cache, k, threads=8, handshake=handshake)
    if handshake == "flags":  # the stream memory operations passed their probe on this device
        assert dec.executor.handshake.startswith("flags"), dec.executor.handshake
    cache.set_cpu_executor(dec)
    layers = [OffloadMoELayer(l, E, k, H, I, device=dev) for l in range(L)]
    for lay in layers:
        lay.offload_cache = cache
    return banks, cache, layers


def _expected(st, layer, x, w, ids, bank, E, max_fetch, frac_q16, capacity, shared=None):
    """Oracle of one hybrid step: admission, then the GPU partial (routes with a
    slot, plus the shared expert) and the CPU partial (unfetched misses) added
    in bf16 (layers/moe.py:372)."""
    out, *_ = S.lru_ensure(st, layer, ids, max_fetch=max_fetch, by_recency=True, capacity=capacity,
                           frac_q16=frac_q16)
    cpu_ids = S.hybrid_split(ids, out, E)
    gpu_ids = np.where(out >= 0, ids, -1).astype(np.int32)
    y_gpu = oracle.experts.moe_layer("decode", x, w, gpu_ids, bank, shared)
    y_cpu = oracle.experts.moe_layer("decode", x, w, cpu_ids, bank, None)
    return out, cpu_ids, oracle.numerics.bf16_round(y_gpu + y_cpu)


@pytest.mark.gpu
@pytest.mark.parametrize("handshake", ["host", "flags"])
@pytest.mark.parametrize("fmt,max_fetch,frac,with_shared", [("fp8", 1, 0.0, False), ("mxfp4", 2, 0.0, False),
                                                            ("fp8", 8, 0.4, False), ("fp8", 1, 0.0, True)])
def test_hybrid_layer_matches_oracle(dev, fmt, max_fetch, frac, with_shared, handshake):
    """Two layers share 6 slots over 16 experts; every step fetches at most the
    cap of its misses and the CPU computes the rest (with a shared expert: on
    the GPU, in the GPU partial).  Both handshakes of the CPU share: host
    functions, and the stream memory operations' flags."""
    rng = np.random.default_rng(71 + max_fetch)
    L, E, Sz, H, I, k, M = 2, 16, 6, 512, 256, 4, 3
    banks, cache, layers = _hybrid_setup(dev, fmt, L, E, Sz, H, I, k, rng, hybrid_max_fetch=max_fetch,
                                         hybrid_fetch_fraction=frac, handshake=handshake)
    shared = synth.make_bank(fmt, 1, H, I, rng) if with_shared else None
    if shared is not None:
        for lay in layers:
            lay.shared_expert = to_device_bank(shared, dev)
    st = S.CacheState(L, E, Sz)
    fq = round(frac * Q16)
    cpu_routes = 0
    for call in range(8):
        l = call % L
        x = synth.activations(rng, M, H)
        w_ref, ids_ref = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
        out, cpu_ids, y_ref = _expected(st, l, x, w_ref, ids_ref, banks[l], E, max_fetch, fq, min(E, Sz), shared)
        cpu_routes += int((cpu_ids >= 0).sum())
        ids = torch.from_numpy(ids_ref.copy()).to(dev)
        with moe_phase("decode", backend="hybrid"):
            y = layers[l].routed_forward(bf16_dev(x, dev), torch.from_numpy(w_ref).to(dev), ids)
        np.testing.assert_array_equal(to_np(ids), out, err_msg=f"call {call}")
        g = to_np(y)
        assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, (fmt, call, max_rel(g, y_ref))
        y_all = oracle.experts.moe_layer("decode", x, w_ref, ids_ref, banks[l], shared)
        assert cosine(g, y_all) >= COS_TOL, (fmt, call)
    assert cpu_routes > 0  # the CPU share was exercised
    np.testing.assert_array_equal(to_np(cache.slot_for_id), st.slot_for_id)
    cache.cpu_executor.close()


@pytest.mark.gpu
@pytest.mark.parametrize("with_shared", [False, True])
def test_cpu_layer_matches_oracle(dev, with_shared):
    """A layer listed in cpu_layer_ids decodes on the CPU from its host banks;
    the slot cache is not touched (layers/moe.py:307-310); a shared expert
    runs on the GPU meanwhile."""
    rng = np.random.default_rng(83)
    L, E, Sz, H, I, k, M = 2, 16, 4, 512, 256, 4, 5
    banks, cache, layers = _hybrid_setup(dev, "fp8", L, E, Sz, H, I, k, rng, decode_target="cpu")
    cache.cpu_layer_ids = frozenset({1})
    shared = synth.make_bank("fp8", 1, H, I, rng) if with_shared else None
    if shared is not None:
        layers[1].shared_expert = to_device_bank(shared, dev)
    x = synth.activations(rng, M, H)
    w_ref, ids_ref = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
    y_ref = oracle.experts.moe_layer("decode", x, w_ref, ids_ref, banks[1], shared)
    ids = torch.from_numpy(ids_ref.copy()).to(dev)
    with moe_phase("decode", backend="cpu"):
        y = layers[1].routed_forward(bf16_dev(x, dev), torch.from_numpy(w_ref).to(dev), ids)
    g = to_np(y)
    assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, max_rel(g, y_ref)
    np.testing.assert_array_equal(to_np(ids), ids_ref)  # raw ids, no slot rewrite
    assert (to_np(cache.slot_for_id) == -1).all() and int(cache.step.item()) == 0
    cache.cpu_executor.close()


@pytest.mark.gpu
@pytest.mark.parametrize("handshake", ["host", "flags"])
def test_hybrid_replays_in_a_graph(dev, handshake):
    """Admission, CPU submit, gather, GPU experts and CPU wait captured once and
    replayed with a new routing each time, with eager work between replays:
    every replay matches the oracle step (host nodes, or stream memory
    operations where they capture, carry the CPU share)."""
    rng = np.random.default_rng(89)
    L, E, Sz, H, I, k, M = 1, 16, 4, 512, 256, 4, 2
    banks, cache, layers = _hybrid_setup(dev, "fp8", L, E, Sz, H, I, k, rng, hybrid_max_fetch=1,
                                         handshake=handshake)
    print("handshake:", cache.cpu_executor.executor.handshake, flush=True)
    layer = layers[0]
    x_buf = torch.zeros((M, H), dtype=torch.bfloat16, device=dev)
    w_buf = torch.zeros((M, k), dtype=torch.float32, device=dev)
    ids_buf = torch.zeros((M, k), dtype=torch.int32, device=dev)

    def call():
        ids = ids_buf.clone()
        with moe_phase("decode", backend="hybrid"):
            return layer.routed_forward(x_buf, w_buf, ids)

    st = S.CacheState(L, E, Sz)
    warm = np.array([[0, 1, 2, 3], [4, 5, 6, 7]], dtype=np.int32)
    ids_buf.copy_(torch.from_numpy(warm))  # eager warm-up: workspace and pinned IO of this batch size
    call()
    torch.cuda.synchronize()
    S.lru_ensure(st, 0, warm, max_fetch=1, by_recency=True, capacity=min(E, Sz))
    stream = torch.cuda.Stream(device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            y = call()
    torch.cuda.synchronize()
    cpu_routes = 0
    for rep in range(5):
        x = synth.activations(rng, M, H)
        w_ref, ids_ref = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
        _, cpu_ids, y_ref = _expected(st, 0, x, w_ref, ids_ref, banks[0], E, 1, 0, min(E, Sz))
        x_buf.copy_(bf16_dev(x, dev))
        w_buf.copy_(torch.from_numpy(w_ref))
        ids_buf.copy_(torch.from_numpy(ids_ref))
        graph.replay()
        torch.cuda.synchronize()
        g = to_np(y)
        assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, (rep, max_rel(g, y_ref))
        cpu_routes += int((cpu_ids >= 0).sum())
        _ = (x_buf * 2).sum().item()  # eager work and a synchronisation between replays
    assert cpu_routes > 0
    np.testing.assert_array_equal(to_np(cache.slot_for_id), st.slot_for_id)
    del graph
    torch.cuda.synchronize()
    cache.cpu_executor.close(graphs_released=True)


@pytest.mark.gpu
def test_stream_wait_unblocks_on_watchdog(dev):
    """The stream-ordered CPU job with a stalled pool (held from the host): the
    stream's wait host function returns after the watchdog period instead of
    blocking the stream for ever, later stream work runs, and the executor
    reports the failure (moe/cpu_executor.py:602-656)."""
    import time

    from freetoken_amd import ops

    rng = np.random.default_rng(97)
    E, H, I, M, k = 4, 256, 128, 2, 2
    bank = synth.make_bank("bf16", E, H, I, rng)
    hb = to_device_bank(bank, "cpu")
    x = torch.from_numpy(synth.activations(rng, M, H)).to(torch.bfloat16).pin_memory()
    w = torch.full((M, k), 0.5, dtype=torch.float32).pin_memory()
    ids = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32).pin_memory()
    y = torch.zeros((M, H), dtype=torch.bfloat16).pin_memory()
    ex = ops.CpuExecutor(threads=2, watchdog_s=0.3)
    ex.hold(True)
    marker = torch.zeros(1, device=dev)
    t0 = time.monotonic()
    job = ex.submit(hb, x, w, ids, y, device=dev)
    ex.wait(job, device=dev)
    marker += 1  # stream work after the wait
    torch.cuda.synchronize()
    assert 0.25 <= time.monotonic() - t0 < 10.0
    assert float(marker.item()) == 1.0 and not ex.healthy
    with pytest.raises(RuntimeError, match="watchdog fired"):
        ex.raise_if_unhealthy()
    ex.hold(False)
    ex.close()


@pytest.mark.gpu
def test_flag_wait_unblocks_on_watchdog(dev):
    """The flag handshake with a stalled pool (held from the host): the
    executor's coordinator fails the job after the watchdog period and raises
    its done flag, so the stream's wait ends, later stream work runs, and the
    executor reports the failure; a healthy executor's flag jobs replay a
    second time on the same records."""
    import time

    from freetoken_amd import ops

    rng = np.random.default_rng(101)
    E, H, I, M, k = 4, 256, 128, 2, 2
    bank = synth.make_bank("bf16", E, H, I, rng)
    hb = to_device_bank(bank, "cpu")
    x = torch.from_numpy(synth.activations(rng, M, H)).to(torch.bfloat16).pin_memory()
    w = torch.full((M, k), 0.5, dtype=torch.float32).pin_memory()
    ids = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32).pin_memory()
    y = torch.zeros((M, H), dtype=torch.bfloat16).pin_memory()
    ex = ops.CpuExecutor(threads=2, watchdog_s=0.3)
    assert ex.set_handshake("flags"), "stream memory operations failed their probe"
    # a working pool first: two jobs in a row through the flags, against the synchronous run
    y_ref = ex.run(hb, x, w, ids)
    for _ in range(2):
        y.zero_()
        job = ex.submit(hb, x, w, ids, y, device=dev)
        ex.wait(job, device=dev)
        torch.cuda.synchronize()
        assert torch.equal(y, y_ref)
    ex.hold(True)
    marker = torch.zeros(1, device=dev)
    t0 = time.monotonic()
    job = ex.submit(hb, x, w, ids, y, device=dev)
    ex.wait(job, device=dev)
    marker += 1  # stream work after the wait
    torch.cuda.synchronize()
    assert 0.25 <= time.monotonic() - t0 < 10.0
    assert float(marker.item()) == 1.0 and not ex.healthy
    ex.hold(False)
    ex.close()
