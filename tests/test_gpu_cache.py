"""The expert-cache miss path on the GPU: LRU admission (ftmoe_lru_ensure)
bit-exact against the oracle's restatement of the reference's CPU mirror
(moe/offload_kernels.py:128-188) over multi-step, multi-layer sequences; the
PCIe gather (ftmoe_fetch_experts) byte-exact; and an offload layer that admits
and fetches its misses computing what the all-resident layer computes
(layers/moe.py:288-320)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import slots as S
from oracle import synth
from freetoken_amd import ops
from freetoken_amd.core import moe_phase
from freetoken_amd.layers.moe import OffloadMoELayer
from freetoken_amd.moe.offload_cache import ExpertSlotCache

from _helpers import bf16_dev, to_device_bank, to_np
from conftest import COS_TOL, MAX_REL_TOL, cosine, max_rel


class _DevCache:
    """Device copy of an oracle CacheState plus the admission outputs."""

    def __init__(self, st: S.CacheState, dev, capacity: int):
        self.slot_for_id = torch.from_numpy(st.slot_for_id.copy()).to(dev)
        self.id_of_slot = torch.from_numpy(st.id_of_slot.copy()).to(dev)
        self.usage = torch.from_numpy(st.usage.copy()).to(dev)
        self.step = torch.tensor([st.step], dtype=torch.int64, device=dev)
        self.recency = torch.from_numpy(st.recency.copy()).to(dev)
        self.evict = torch.full((capacity,), -7, dtype=torch.int32, device=dev)
        self.src = torch.full((capacity,), -7, dtype=torch.int32, device=dev)
        self.n = torch.zeros(1, dtype=torch.int32, device=dev)
        self.nmiss = torch.zeros(1, dtype=torch.int32, device=dev)
        self.stats = torch.zeros(4, dtype=torch.int64, device=dev)
        self.unserved = torch.zeros(st.L, dtype=torch.int64, device=dev)

    def ensure(self, layer, ids, max_fetch, by_recency):
        t = torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int32)).to(self.slot_for_id.device)
        ops.lru_ensure(t, layer, self.slot_for_id, self.id_of_slot, self.usage, self.step, self.evict, self.src,
                       self.n, self.nmiss, recency=self.recency[layer] if by_recency else None,
                       max_fetch=max_fetch, stats=self.stats, unserved=self.unserved[layer:layer + 1])
        return t

    def check(self, st: S.CacheState, by_recency: bool):
        np.testing.assert_array_equal(to_np(self.slot_for_id), st.slot_for_id)
        np.testing.assert_array_equal(to_np(self.id_of_slot), st.id_of_slot)
        np.testing.assert_array_equal(to_np(self.usage), st.usage)
        assert int(self.step.item()) == st.step
        if by_recency:
            np.testing.assert_array_equal(to_np(self.recency), st.recency)
        np.testing.assert_array_equal(to_np(self.unserved), st.unserved)


@pytest.mark.gpu
@pytest.mark.parametrize("L,E,Sz,max_k,max_fetch,by_recency", [
    (1, 16, 4, 6, -1, False),      # more misses than free slots: only the free ones are taken
    (2, 32, 5, 12, -1, True),      # likewise, most recent first
    (3, 64, 24, 12, -1, False),
    (2, 256, 64, 64, -1, False),   # C4-like table, decode batch 8
    (2, 128, 40, 40, 5, True),     # capped, most recent first
    (4, 160, 160, 64, 3, False),   # capped, lowest id first
    (1, 1024, 300, 512, -1, True), # a prefill-sized call
])
def test_lru_ensure_matches_oracle(dev, L, E, Sz, max_k, max_fetch, by_recency):
    rng = np.random.default_rng(E + Sz + max_k)
    st = S.CacheState(L, E, Sz)
    cap = E  # every miss of a call fits the lists
    dc = _DevCache(st, dev, cap)
    acc = np.zeros(4, dtype=np.int64)
    for call in range(25):
        layer = int(rng.integers(L))
        n = int(rng.integers(1, max_k + 1))
        # skewed ids so that hits, misses and evictions all occur
        ids = np.minimum((rng.pareto(1.2, size=n) * E / 8).astype(np.int64), E - 1).astype(np.int32)
        if call % 7 == 3:
            ids[0] = -1  # an id outside [0, E) is skipped
        out_ref, evict, src, nmiss, stats = S.lru_ensure(st, layer, ids, max_fetch=max_fetch, by_recency=by_recency,
                                                         capacity=cap)
        acc += stats
        out = dc.ensure(layer, ids, max_fetch, by_recency)
        np.testing.assert_array_equal(to_np(out), out_ref, err_msg=f"call {call}")
        k = int(dc.n.item())
        assert k == evict.size and int(dc.nmiss.item()) == nmiss, (call, k, evict.size)
        np.testing.assert_array_equal(to_np(dc.evict)[:k], evict)
        np.testing.assert_array_equal(to_np(dc.src)[:k], src)
        assert np.unique(evict).size == evict.size, (call, evict)  # no slot taken twice
        dc.check(st, by_recency)
    np.testing.assert_array_equal(to_np(dc.stats), acc)


@pytest.mark.gpu
@pytest.mark.parametrize("n,exact", [(0, False), (1, False), (5, False), (5, True)])
def test_fetch_experts_copies_rows(dev, n, exact):
    """exact: host rows in ops.alloc_pinned_tensor memory (hipHostMalloc)."""
    rng = np.random.default_rng(11 + n)
    E, Sz = 12, 8
    shapes = [(E, 96, 64), (E, 3, 16), (E, 40000)]  # rows of 6 KiB, 48 B and 40 KB (a partial chunk)
    host = [torch.from_numpy(rng.integers(0, 256, size=s, dtype=np.uint8)).pin_memory() for s in shapes]
    if exact:
        exact_host = [ops.alloc_pinned_tensor(*h.shape, dtype=h.dtype) for h in host]
        for a, b in zip(exact_host, host):
            a.copy_(b)
            assert a.is_pinned() and a.untyped_storage().nbytes() == b.numel()
        host = exact_host
    slots = [torch.full((Sz,) + s[1:], 0xEE, dtype=torch.uint8, device=dev) for s in shapes]
    evict = torch.tensor(list(rng.permutation(Sz)[:6]), dtype=torch.int32, device=dev)
    src = torch.tensor(list(rng.permutation(E)[:6]), dtype=torch.int32, device=dev)
    num = torch.tensor([n], dtype=torch.int32, device=dev)
    ops.fetch_experts(host, slots, evict, src, num)
    torch.cuda.synchronize()
    ev, sr = evict.tolist(), src.tolist()
    for h, d in zip(host, slots):
        got = d.cpu()
        for s in range(Sz):
            if s in ev[:n]:
                assert torch.equal(got[s], h[sr[ev.index(s)]]), s
            else:
                assert (got[s] == 0xEE).all(), s


def _pinned_bank_sources(bank):
    names = ("gate_up", "gate_up_scale", "down", "down_scale")
    arrays = (bank.gate_up, bank.gate_up_scale, bank.down, bank.down_scale)
    return names, [torch.from_numpy(np.ascontiguousarray(a)).pin_memory() for a in arrays]


@pytest.mark.gpu
@pytest.mark.parametrize("fmt", ["fp8", "mxfp4"])
def test_offload_layer_admits_and_fetches_misses(dev, fmt):
    """Two layers share 6 slots over 16 experts; every decode call admits its
    misses, gathers them over PCIe and must equal the all-resident layer."""
    rng = np.random.default_rng(61)
    L, E, Sz, H, I, k, M = 2, 16, 6, 512, 256, 2, 3
    banks = [synth.make_bank(fmt, E, H, I, rng) for _ in range(L)]
    cache = ExpertSlotCache(L, E, Sz, {"fp8": "fp8_block", "mxfp4": "ds_fp4"}[fmt], device=dev)
    # slot banks with the decode dtypes (contents arrive by the gather)
    eb = to_device_bank(banks[0], dev, rows=np.arange(Sz))
    cache.set_bank_caches(gate_up=eb.gate_up, gate_up_scale=eb.gate_up_scale, down=eb.down, down_scale=eb.down_scale)
    for t in cache.banks.values():
        t.view(torch.uint8).fill_(0)
    names = ("gate_up", "gate_up_scale", "down", "down_scale")
    per_layer = [_pinned_bank_sources(b)[1] for b in banks]
    cache.set_bank_sources({n: [per_layer[l][j] for l in range(L)] for j, n in enumerate(names)})
    cache.reset()
    layers = [OffloadMoELayer(l, E, k, H, I, device=dev) for l in range(L)]
    for lay in layers:
        lay.offload_cache = cache
    for call in range(6):
        l = call % L
        x = synth.activations(rng, M, H)
        logits = synth.normal(rng, (M, E))
        w_ref, ids_ref = oracle.routing.softmax_topk(logits, k, True)
        y_ref = oracle.experts.moe_layer("decode", x, w_ref, ids_ref, banks[l], None)
        ids = torch.from_numpy(ids_ref.copy()).to(dev)
        with moe_phase("decode", backend="offload"):
            y = layers[l].routed_forward(bf16_dev(x, dev), torch.from_numpy(w_ref).to(dev), ids)
        slots_now = to_np(ids)
        assert (slots_now >= 0).all() and (slots_now < Sz).all()
        sft = to_np(cache.slot_for_id)
        np.testing.assert_array_equal(slots_now, sft[l][ids_ref])
        g = to_np(y)
        assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, (fmt, call, max_rel(g, y_ref))
    st = cache.decode_miss_stats()
    assert st["layer_calls"] == 6 and st["missing_per_layer"] > 0 and st["unserved_experts"] == 0
    cache.check_capacity()


@pytest.mark.gpu
def test_undersized_cache_counts_unserved_misses(dev):
    """A call routed to more distinct experts than the cache has slots: the free
    slots are taken once each (no slot admitted twice in the call), the misses
    left over are skipped and counted, and check_capacity raises.  The served
    routes equal the oracle with the unserved ones skipped."""
    rng = np.random.default_rng(71)
    E, Sz, H, I, k, M = 16, 4, 512, 256, 2, 3
    bank = synth.make_bank("fp8", E, H, I, rng)
    cache = ExpertSlotCache(1, E, Sz, "fp8_block", device=dev)
    eb = to_device_bank(bank, dev, rows=np.arange(Sz))
    cache.set_bank_caches(gate_up=eb.gate_up, gate_up_scale=eb.gate_up_scale, down=eb.down, down_scale=eb.down_scale)
    names, host = _pinned_bank_sources(bank)
    cache.set_bank_sources({n: [h] for n, h in zip(names, host)})
    cache.reset()
    layer = OffloadMoELayer(0, E, k, H, I, device=dev)
    layer.offload_cache = cache
    ids_ref = np.array([[0, 1], [2, 3], [4, 5]], dtype=np.int32)
    w_ref = np.full((M, k), 0.5, dtype=np.float32)
    x = synth.activations(rng, M, H)
    ids = torch.from_numpy(ids_ref.copy()).to(dev)
    with moe_phase("decode", backend="offload"):
        y = layer.routed_forward(bf16_dev(x, dev), torch.from_numpy(w_ref).to(dev), ids)
    torch.cuda.synchronize()
    got_ids = to_np(ids)
    assert got_ids[:2].tolist() == [[0, 1], [2, 3]] and got_ids[2].tolist() == [-1, -1]
    served = np.where(got_ids >= 0, ids_ref, -1).astype(np.int32)
    y_ref = oracle.experts.moe_layer("decode", x, w_ref, served, bank, None)
    g = to_np(y)
    assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL
    assert cache.decode_miss_stats()["unserved_experts"] == 2
    with pytest.raises(RuntimeError, match="expert cache too small"):
        cache.check_capacity()
    cache.reset_stats()
    cache.check_capacity()


@pytest.mark.gpu
def test_miss_path_replays_in_a_graph(dev):
    """Admission, gather and experts captured once (the decode graph of the
    reference, engine/graph.py:127-187) and replayed with a new routing each
    time: every replay admits that call's misses and matches the oracle."""
    rng = np.random.default_rng(67)
    E, Sz, H, I, k, M = 16, 4, 512, 256, 2, 2
    bank = synth.make_bank("fp8", E, H, I, rng)
    cache = ExpertSlotCache(1, E, Sz, "fp8_block", device=dev)
    eb = to_device_bank(bank, dev, rows=np.arange(Sz))
    cache.set_bank_caches(gate_up=eb.gate_up, gate_up_scale=eb.gate_up_scale, down=eb.down, down_scale=eb.down_scale)
    names, host = _pinned_bank_sources(bank)
    cache.set_bank_sources({n: [h] for n, h in zip(names, host)})
    cache.reset()
    layer = OffloadMoELayer(0, E, k, H, I, device=dev)
    layer.offload_cache = cache
    x_buf = torch.zeros((M, H), dtype=torch.bfloat16, device=dev)
    w_buf = torch.zeros((M, k), dtype=torch.float32, device=dev)
    ids_buf = torch.zeros((M, k), dtype=torch.int32, device=dev)

    def call():
        ids = ids_buf.clone()
        with moe_phase("decode", backend="offload"):
            return layer.routed_forward(x_buf, w_buf, ids)

    ids_buf.copy_(torch.tensor([[0, 1], [2, 3]], dtype=torch.int32))  # warm-up call (eager) sizes the workspace
    call()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=dev)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            y = call()
    torch.cuda.synchronize()
    for rep in range(5):
        x = synth.activations(rng, M, H)
        logits = synth.normal(rng, (M, E))
        w_ref, ids_ref = oracle.routing.softmax_topk(logits, k, True)
        x_buf.copy_(bf16_dev(x, dev))
        w_buf.copy_(torch.from_numpy(w_ref))
        ids_buf.copy_(torch.from_numpy(ids_ref))
        graph.replay()
        torch.cuda.synchronize()
        y_ref = oracle.experts.moe_layer("decode", x, w_ref, ids_ref, bank, None)
        g = to_np(y)
        assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, (rep, max_rel(g, y_ref))
        sft = to_np(cache.slot_for_id)[0]
        assert (sft[np.unique(ids_ref)] >= 0).all(), rep


@pytest.mark.gpu
def test_materialize_and_release_match_oracle(dev):
    """Admissions, whole-layer placements and slot releases interleaved over
    three layers keep the device tables equal to the oracle's
    (offload_kernels.py:250-281, offload_cache.py:592-600)."""
    rng = np.random.default_rng(97)
    L, E, Sz = 3, 24, 56
    st = S.CacheState(L, E, Sz)
    dc = _DevCache(st, dev, E)
    for call in range(30):
        layer = int(rng.integers(L))
        kind = call % 5
        if kind == 3:
            ev_ref, src_ref = S.materialize_layer(st, layer)
            ops.materialize_layer(layer, dc.slot_for_id, dc.id_of_slot, dc.usage, dc.step, dc.evict, dc.src, dc.n)
            assert int(dc.n.item()) == E
            np.testing.assert_array_equal(to_np(dc.evict)[:E], ev_ref)
            np.testing.assert_array_equal(to_np(dc.src)[:E], src_ref)
        elif kind == 4:
            b = int(rng.integers(Sz))
            e = int(rng.integers(b, Sz + 1))
            S.release_slots(st, b, e)
            ops.release_slots(b, e, dc.slot_for_id, dc.id_of_slot, dc.usage)
        else:
            ids = rng.integers(0, E, size=int(rng.integers(1, 12))).astype(np.int32)
            S.lru_ensure(st, layer, ids, capacity=E)
            dc.ensure(layer, ids, -1, False)
        dc.check(st, False)


def _prefill_cache(dev, banks, E, Sz, overlap):
    cache = ExpertSlotCache(len(banks), E, Sz, "fp8_block", device=dev, prefill_overlap=overlap)
    eb = to_device_bank(banks[0], dev, rows=np.arange(Sz) % E)
    cache.set_bank_caches(gate_up=eb.gate_up, gate_up_scale=eb.gate_up_scale, down=eb.down, down_scale=eb.down_scale)
    for t in cache.banks.values():
        t.view(torch.uint8).fill_(0)
    names, _ = _pinned_bank_sources(banks[0])
    per_layer = [_pinned_bank_sources(b)[1] for b in banks]
    cache.set_bank_sources({n: [per_layer[l][j] for l in range(len(banks))] for j, n in enumerate(names)})
    cache.reset()
    return cache


@pytest.mark.gpu
@pytest.mark.parametrize("overlap", [False, True])
def test_offload_prefill_moves_layers(dev, overlap):
    """Prefill over three layers whose experts live only in pinned host memory:
    materialized and gathered per layer, or double-buffered with layer l+1's
    copy behind layer l's GEMMs (layers/moe.py:374-423).  Two passes over the
    layers (the second reuses released buffers); each output equals the
    oracle's prefill layer."""
    rng = np.random.default_rng(101)
    L, E, H, I, k, M = 3, 8, 512, 256, 2, 300
    Sz = 2 * E + 4
    banks = [synth.make_bank("fp8", E, H, I, rng) for _ in range(L)]
    cache = _prefill_cache(dev, banks, E, Sz, overlap)
    layers = [OffloadMoELayer(l, E, k, H, I, device=dev) for l in range(L)]
    for lay in layers:
        lay.offload_cache = cache
    for rep in range(2):
        for l in range(L):
            x = synth.activations(rng, M, H)
            w_ref, ids_ref = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
            y_ref = oracle.experts.moe_layer("prefill", x, w_ref, ids_ref, banks[l], None)
            with moe_phase("prefill", backend="offload"):
                y = layers[l].routed_forward(bf16_dev(x, dev), torch.from_numpy(w_ref).to(dev),
                                             torch.from_numpy(ids_ref.copy()).to(dev))
            g = to_np(y)
            assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, (overlap, rep, l)
    torch.cuda.synchronize()
    if not overlap:  # the last layer stays materialized at slot == expert id
        np.testing.assert_array_equal(to_np(cache.slot_for_id)[L - 1], np.arange(E))


@pytest.mark.gpu
@pytest.mark.parametrize("per_layer", [True, False])
def test_offload_layer_from_ftw_banks(dev, tmp_path, per_layer):
    """Expert banks written as an FTW checkpoint (bf16 block scales, as the
    reference's FP8 banks are stored), loaded into pinned host memory with the
    scales widened, and served to an offload layer's decode through the miss
    path: outputs equal the oracle on the same (bf16-rounded-scale) banks."""
    from freetoken_amd.checkpoint import load_ftw_banks, save_ftw_banks
    from oracle.numerics import bf16_round

    rng = np.random.default_rng(107)
    L, E, Sz, H, I, k, M = 2, 12, 6, 512, 256, 2, 3  # slots >= the distinct experts of a call
    banks = [synth.make_bank("fp8", E, H, I, rng) for _ in range(L)]
    for b in banks:
        b.gate_up_scale = bf16_round(b.gate_up_scale)
        b.down_scale = bf16_round(b.down_scale)
    src = {
        "gate_up": [torch.from_numpy(b.gate_up).view(torch.float8_e4m3fn) for b in banks],
        "gate_up_scale": [torch.from_numpy(b.gate_up_scale).to(torch.bfloat16) for b in banks],
        "down": [torch.from_numpy(b.down).view(torch.float8_e4m3fn) for b in banks],
        "down_scale": [torch.from_numpy(b.down_scale).to(torch.bfloat16) for b in banks],
    }
    save_ftw_banks(str(tmp_path), "fp8_block", src, per_layer=per_layer, shard_limit=1 << 20)
    fmt, sources, _ = load_ftw_banks(str(tmp_path), L)
    assert fmt == "fp8_block" and all(t.is_pinned() for ts in sources.values() for t in ts)
    cache = ExpertSlotCache(L, E, Sz, fmt, device=dev)
    cache.set_bank_caches(**{n: torch.zeros((Sz,) + ts[0].shape[1:], dtype=ts[0].dtype, device=dev)
                             for n, ts in sources.items()})
    cache.set_bank_sources(sources)
    cache.reset()
    layers = [OffloadMoELayer(l, E, k, H, I, device=dev) for l in range(L)]
    for lay in layers:
        lay.offload_cache = cache
    for call in range(4):
        l = call % L
        x = synth.activations(rng, M, H)
        w_ref, ids_ref = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
        y_ref = oracle.experts.moe_layer("decode", x, w_ref, ids_ref, banks[l], None)
        with moe_phase("decode", backend="offload"):
            y = layers[l].routed_forward(bf16_dev(x, dev), torch.from_numpy(w_ref).to(dev),
                                         torch.from_numpy(ids_ref.copy()).to(dev))
        g = to_np(y)
        assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, (per_layer, call)


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["fp8", "bf16"])
def test_offload_layer_from_hf_checkpoint(dev, tmp_path, mode):
    """Expert banks read from a block-FP8 HF safetensors checkpoint into pinned
    host memory (models/qwen3_5_moe/weight.py:834-1055; mode "bf16" is the
    FREETOKEN_FP8_EXPERTS=bf16 dequant route) and served to an offload layer's
    decode through the miss path: outputs equal the oracle on the same banks."""
    from freetoken_amd.checkpoint.hf import load_hf_expert_banks
    from oracle.experts import Bank, dequant_fp8_block
    from oracle.numerics import bf16_round
    from test_hf_checkpoint import write_hf_checkpoint

    rng = np.random.default_rng(113)
    L, E, Sz, H, I, k, M = 2, 8, 6, 512, 256, 2, 3
    banks = write_hf_checkpoint(tmp_path, "model.layers", 1, L, E, H, I, seed=3)
    fmt, sources, lay = load_hf_expert_banks(str(tmp_path), mode=mode)
    assert all(t.is_pinned() for ts in sources.values() for t in ts)
    if mode == "bf16":
        banks = [Bank("bf16", bf16_round(dequant_fp8_block(b.gate_up, b.gate_up_scale)),
                      bf16_round(dequant_fp8_block(b.down, b.down_scale))) for b in banks]
    cache = ExpertSlotCache(L, E, Sz, fmt, device=dev)
    cache.set_bank_caches(**{n: torch.zeros((Sz,) + ts[0].shape[1:], dtype=ts[0].dtype, device=dev)
                             for n, ts in sources.items()})
    cache.set_bank_sources(sources)
    cache.reset()
    layers = [OffloadMoELayer(l, E, k, H, I, device=dev) for l in range(L)]
    for lay_ in layers:
        lay_.offload_cache = cache
    for call in range(4):
        l = call % L
        x = synth.activations(rng, M, H)
        w_ref, ids_ref = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
        y_ref = oracle.experts.moe_layer("decode", x, w_ref, ids_ref, banks[l], None)
        with moe_phase("decode", backend="offload"):
            y = layers[l].routed_forward(bf16_dev(x, dev), torch.from_numpy(w_ref).to(dev),
                                         torch.from_numpy(ids_ref.copy()).to(dev))
        g = to_np(y)
        assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, (mode, call, max_rel(g, y_ref))
    cache.check_capacity()


@pytest.mark.gpu
def test_offload_prefill_hit_miss_split(dev):
    """The double buffer's hit/miss split (moe/offload_cache.py:703-773): experts
    already resident outside the buffers (slots >= 2E) are gathered device to
    device, only the others cross PCIe.  The host rows of the resident experts
    are zeroed after their placement, so any of them taken from the host would
    change the output; every layer's prefill must still equal the oracle, and
    the hit counters must count exactly the placed experts."""
    rng = np.random.default_rng(131)
    L, E, H, I, k, M = 3, 8, 512, 256, 2, 300
    Sz = 2 * E + 6
    banks = [synth.make_bank("fp8", E, H, I, rng) for _ in range(L)]
    cache = ExpertSlotCache(L, E, Sz, "fp8_block", device=dev, prefill_overlap=True, prefill_hit_d2d=True)
    eb = to_device_bank(banks[0], dev, rows=np.arange(Sz) % E)
    cache.set_bank_caches(gate_up=eb.gate_up, gate_up_scale=eb.gate_up_scale, down=eb.down, down_scale=eb.down_scale)
    for t in cache.banks.values():
        t.view(torch.uint8).fill_(0)
    names, _ = _pinned_bank_sources(banks[0])
    per_layer = [_pinned_bank_sources(b)[1] for b in banks]
    sources = {n: [per_layer[l][j] for l in range(L)] for j, n in enumerate(names)}
    cache.set_bank_sources(sources)
    cache.reset()
    placed = {1: ([1, 4, 6], [16, 17, 18]), 2: ([3], [20])}
    for layer, (experts, slots) in placed.items():
        for e, s in zip(experts, slots):
            for n in names:
                cache.banks[n][s].view(torch.uint8).copy_(sources[n][layer][e].view(torch.uint8))
        cache.assign(layer, experts, slots)
    torch.cuda.synchronize()
    for layer, (experts, _) in placed.items():
        for e in experts:
            for n in names:
                sources[n][layer][e].view(torch.uint8).zero_()
    layers = [OffloadMoELayer(l, E, k, H, I, device=dev) for l in range(L)]
    for lay in layers:
        lay.offload_cache = cache
    for rep in range(2):
        for l in range(L):
            x = synth.activations(rng, M, H)
            w_ref, ids_ref = oracle.routing.softmax_topk(synth.normal(rng, (M, E)), k, True)
            y_ref = oracle.experts.moe_layer("prefill", x, w_ref, ids_ref, banks[l], None)
            with moe_phase("prefill", backend="offload"):
                y = layers[l].routed_forward(bf16_dev(x, dev), torch.from_numpy(w_ref).to(dev),
                                             torch.from_numpy(ids_ref.copy()).to(dev))
            g = to_np(y)
            assert max_rel(g, y_ref) <= MAX_REL_TOL and cosine(g, y_ref) >= COS_TOL, (rep, l, max_rel(g, y_ref))
    torch.cuda.synchronize()
    assert cache.prefill_total_rows == 2 * L * E
    assert cache.prefill_hit_rows == 2 * 4, cache.prefill_hit_rows
    sft = to_np(cache.slot_for_id)  # the placed experts stay where they were
    assert sft[1][[1, 4, 6]].tolist() == [16, 17, 18] and sft[2][3] == 20
