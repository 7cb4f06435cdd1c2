"""Pins of the LRU admission of oracle/slots.py (restating the reference's CPU
mirror of its admission kernel, moe/offload_kernels.py:128-188).

The reference's own invariants (tests/moe/test_offload.py:379-404 and
:522-602) are restated on the oracle's tables, and the admission is checked
against properties that do not retype its loop: the victims of a call are the
least recently used slots in (usage, slot) order, resident experts keep their
slots, caps and the recency order behave as documented."""

from __future__ import annotations

import numpy as np

from oracle import slots as S


def _inverse_ok(st: S.CacheState) -> bool:
    flat = st.slot_for_id.reshape(-1)
    for s, f in enumerate(st.id_of_slot.tolist()):
        if f >= 0 and flat[f] != s:
            return False
    for f, s in enumerate(flat.tolist()):
        if s >= 0 and st.id_of_slot[s] != f:
            return False
    return True


def test_large_miss_batch_unique_slots():
    # tests/moe/test_offload.py:379-404
    st = S.CacheState(40, 256, 1664)
    ids = np.arange(256, dtype=np.int32).reshape(32, 8)
    out, evict, src, nmiss, _ = S.lru_ensure(st, 0, ids)
    assert nmiss == 256 and evict.size == 256
    assert out.min() >= 0 and out.max() < 1664
    assert np.unique(evict).size == 256 and evict.min() >= 0 and evict.max() < 1664
    assert src.tolist() == list(range(256))
    # a fresh cache hands out slots in index order (all usages 0)
    assert evict.tolist() == list(range(256))
    assert (out.reshape(-1) == np.arange(256)).all()


def test_tables_stay_inverse_across_layers():
    # tests/moe/test_offload.py:522-602 (layer 1 fills the cache, layer 0 then evicts two of its slots)
    L, E = 2, 8
    st = S.CacheState(L, E, 8)
    S.lru_ensure(st, 0, [3, 5])
    assert _inverse_ok(st)
    S.lru_ensure(st, 1, list(range(E)))
    assert _inverse_ok(st)
    out, evict, src, nmiss, _ = S.lru_ensure(st, 0, [3, 5])
    assert _inverse_ok(st) and evict.size == nmiss
    out3, _, _, _, _ = S.lru_ensure(st, 1, [1, 2])
    assert _inverse_ok(st)
    for e, s in zip([1, 2], out3.tolist()):
        assert st.id_of_slot[s] == 1 * E + e


def test_victims_are_least_recently_used():
    rng = np.random.default_rng(5)
    L, E, Sz = 3, 32, 12
    st = S.CacheState(L, E, Sz)
    for call in range(60):
        layer = int(rng.integers(L))
        ids = rng.integers(0, E, size=int(rng.integers(1, 9)))
        before = st.copy()
        out, evict, src, nmiss, stats = S.lru_ensure(st, layer, ids)
        seen = sorted(set(ids.tolist()))
        resident = [e for e in seen if before.slot_for_id[layer, e] >= 0]
        missing = [e for e in seen if before.slot_for_id[layer, e] < 0]
        assert src.tolist() == missing and nmiss == len(missing)
        # untouched slots ranked by (usage, slot); the misses take the first ones
        touched = {int(before.slot_for_id[layer, e]) for e in resident}
        free = sorted((int(before.usage[s]), s) for s in range(Sz) if s not in touched)
        if len(missing) <= len(free):
            assert evict.tolist() == [s for _, s in free[: len(missing)]]
        # resident experts keep their slots, every seen expert ends resident
        for e in resident:
            assert st.slot_for_id[layer, e] == before.slot_for_id[layer, e]
        if len(seen) <= Sz:
            assert (out >= 0).all()
            for e, s in zip(ids.tolist(), out.tolist()):
                assert st.id_of_slot[s] == layer * E + e
        assert _inverse_ok(st)
        assert stats.tolist() == [len(seen), len(missing), 1, sum(1 for e in ids.tolist() if e in missing)]
        assert st.step == call + 1
        assert all(st.usage[s] == st.step for s in out.tolist() if s >= 0)


def test_cap_and_recency_order():
    E = 16
    st = S.CacheState(1, E, 8)
    S.lru_ensure(st, 0, [9], by_recency=True)  # step 1: expert 9 seen (resident)
    S.lru_ensure(st, 0, [4], by_recency=True)  # step 2: expert 4 seen
    st.slot_for_id[:] = -1                     # drop everything: all three below miss
    st.id_of_slot[:] = -1
    out, evict, src, nmiss, _ = S.lru_ensure(st, 0, [1, 9, 4], max_fetch=2, by_recency=True)
    # most recently seen first (4 at step 2, 9 at step 1), then 1 (never seen); capped at 2
    assert nmiss == 3 and src.tolist() == [4, 9]
    assert out.tolist()[0] == -1 and out.tolist()[1] >= 0 and out.tolist()[2] >= 0
    st2 = S.CacheState(1, E, 8)
    out, evict, src, nmiss, _ = S.lru_ensure(st2, 0, [7, 3, 5], max_fetch=2)
    assert src.tolist() == [3, 5] and out.tolist() == [-1, 0, 1]


def test_out_of_range_ids_are_not_seen():
    st = S.CacheState(1, 8, 4)
    out, evict, src, nmiss, stats = S.lru_ensure(st, 0, [-1, 8, 2])
    assert out.tolist() == [-1, -1, 0] and src.tolist() == [2] and stats.tolist() == [1, 1, 1, 1]


def test_more_misses_than_slots_admits_only_free_slots():
    # every free slot is taken in (usage, slot) order; the misses after them get
    # no slot (never one admitted in the same call) and are counted as unserved
    st = S.CacheState(1, 8, 2)
    out, evict, src, nmiss, _ = S.lru_ensure(st, 0, [0, 1, 2, 3])
    assert evict.tolist() == [0, 1] and src.tolist() == [0, 1] and nmiss == 4
    assert out.tolist() == [0, 1, -1, -1]
    assert st.unserved.tolist() == [2]
    assert _inverse_ok(st)


def test_resident_experts_of_the_call_are_never_victims():
    # S = 4 with experts 6 and 7 resident; a call routed to {0, 1, 2, 3, 6, 7}
    # has two free slots: 0 and 1 take them, 2 and 3 stay unserved, 6 and 7 keep
    # their slots, every victim is distinct (tests/moe/test_offload.py:379-404)
    st = S.CacheState(1, 8, 4)
    S.lru_ensure(st, 0, [6, 7])
    before = st.slot_for_id[0].copy()
    out, evict, src, nmiss, _ = S.lru_ensure(st, 0, [0, 1, 2, 3, 6, 7])
    assert nmiss == 4 and src.tolist() == [0, 1]
    assert np.unique(evict).size == evict.size == 2
    assert not set(evict.tolist()) & {int(before[6]), int(before[7])}
    assert out.tolist()[4:] == [int(before[6]), int(before[7])] and out.tolist()[2:4] == [-1, -1]
    assert st.unserved.tolist() == [2]
    assert _inverse_ok(st)


def test_victims_unique_under_random_pressure():
    rng = np.random.default_rng(12)
    for L, E, Sz in ((1, 16, 4), (2, 32, 6), (3, 64, 16)):
        st = S.CacheState(L, E, Sz)
        for _ in range(80):
            layer = int(rng.integers(L))
            ids = rng.integers(0, E, size=int(rng.integers(1, 3 * Sz)))
            before = st.copy()
            out, evict, src, nmiss, _ = S.lru_ensure(st, layer, ids, max_fetch=int(rng.integers(-1, 4)))
            assert np.unique(evict).size == evict.size
            seen = set(ids.tolist())
            held = {int(before.slot_for_id[layer, e]) for e in seen if before.slot_for_id[layer, e] >= 0}
            assert not set(evict.tolist()) & held
            for e, s in zip(ids.tolist(), out.tolist()):
                assert s == -1 or st.id_of_slot[s] == layer * E + e
            assert _inverse_ok(st)


def test_fraction_cap_known_answers():
    # tests/moe/test_hybrid_fetch.py:29-41: rounding to the balanced neighbour, not up
    q = 1 << 16
    assert S.fraction_cap(3, round(0.415 * q)) == 1
    assert S.fraction_cap(4, round(0.415 * q)) == 2
    for frac in (0.1, 0.415, 0.454, 0.7, 1.0):
        fq = round(frac * q)
        for m in range(65):
            n = S.fraction_cap(m, fq)
            assert 0 <= n <= m and abs(n - frac * m) <= 1.0
            # brute force: the lowest n in [0, m] minimising the slower overlapped side
            costs = [max(f * (q - fq), (m - f) * fq) for f in range(m + 1)]
            assert n == costs.index(min(costs)), (frac, m)


def test_fraction_cap_admission_and_split():
    """The fraction replaces the fixed cap; the CPU split holds exactly the
    unfetched misses (tests/moe/test_hybrid_fetch.py:89-115 on the oracle)."""
    rng = np.random.default_rng(2)
    st = S.CacheState(2, 32, 40)
    fq = round(0.415 * (1 << 16))
    for _ in range(64):
        ids = rng.permutation(32)[:8].astype(np.int32)
        out, evict, src, nmiss, _ = S.lru_ensure(st, 0, ids, max_fetch=32, by_recency=True, frac_q16=fq)
        assert evict.size == S.fraction_cap(nmiss, fq)
        assert (out >= 0).sum() == len(set(ids.tolist())) - (nmiss - evict.size)
        cpu = S.hybrid_split(ids, out, 32)
        assert ((cpu >= 0) == (out < 0)).all() and (cpu[cpu >= 0] == ids[cpu >= 0]).all()
        assert _inverse_ok(st)
    assert S.hybrid_split([-1, 40, 3], [-1, -1, -1], 32).tolist() == [-1, -1, 3]


def test_materialize_layer_invariants():
    """Position == expert id for the layer; the tables stay inverse; experts of
    other layers outside [0, E) keep their slots; the layer's old slots are
    freed (usage 0) and are the next LRU victims."""
    L, E, Sz = 3, 8, 20
    st = S.CacheState(L, E, Sz)
    S.lru_ensure(st, 1, list(range(8)))          # layer 1 fills slots 0..7
    S.lru_ensure(st, 2, [0, 1, 2])               # layer 2 in 8..10
    S.lru_ensure(st, 0, [5, 6])                  # layer 0 in 11..12
    before = st.copy()
    evict, src = S.materialize_layer(st, 0)
    assert evict.tolist() == list(range(E)) and src.tolist() == list(range(E))
    assert st.slot_for_id[0].tolist() == list(range(E)) and _inverse_ok(st)
    assert (st.slot_for_id[1] == -1).all()       # evicted from slots 0..7
    assert st.slot_for_id[2].tolist()[:3] == before.slot_for_id[2].tolist()[:3]  # untouched
    assert st.id_of_slot[11] == -1 and st.id_of_slot[12] == -1 and st.usage[11] == 0 and st.usage[12] == 0
    assert st.step == before.step + 1 and (st.usage[:E] == st.step).all()
    # the freed slots (and the never-used ones) are taken first by the next admission
    _, ev, _, _, _ = S.lru_ensure(st, 2, [7])
    assert ev.tolist() == [11]


def test_release_slots_unmaps():
    st = S.CacheState(2, 8, 16)
    S.lru_ensure(st, 0, list(range(8)))
    S.lru_ensure(st, 1, [3, 4])
    S.release_slots(st, 4, 9)
    assert _inverse_ok(st)
    assert (st.id_of_slot[4:9] == -1).all() and (st.usage[4:9] == 0).all()
    assert st.slot_for_id[0].tolist() == [0, 1, 2, 3, -1, -1, -1, -1]
    assert st.slot_for_id[1, 3] == -1 and st.slot_for_id[1, 4] == 9


def test_decode_routing_stats_closed_forms():
    """ExpertSlotCache.decode_routing_stats (reference moe/offload_cache.py:936-966)
    on hand-built histograms: a uniform layer (entropy log E, 90% of the routes
    on 15 of 16 experts, hit rate slots/E), a one-expert layer (entropy 0, one
    expert covers everything) and an unrouted layer that takes no part."""
    import torch

    from freetoken_amd.moe.offload_cache import ExpertSlotCache

    cache = ExpertSlotCache(3, 16, 12, "fp8_block", device="cpu")
    assert cache.decode_routing_stats() == {}
    cache.decode_freq[0] = 3
    cache.decode_freq[1, 5] = 40
    st = cache.decode_routing_stats()
    assert st["slots_per_layer"] == 4.0
    assert st["working_set_mean"] == 8.5 and st["working_set_max"] == 16
    assert st["experts_for_90pct"] == 8.0  # (15 + 1) / 2
    assert abs(st["oracle_hit_at_slots"] - (4 / 16 + 1.0) / 2) < 1e-12
    assert abs(st["norm_entropy"] - 0.5) < 1e-12
    cache.reset_decode_freq()
    assert int(cache.decode_freq.sum()) == 0 and isinstance(cache.decode_freq, torch.Tensor)
