"""Expert-cache slot indirection: lookup + miss report, and LRU admission.

``OffloadMoeCache.slot_for_id`` is an int32 [L, E] table with -1 for a
non-resident expert (``moe/offload_cache.py:155-175``); decode rewrites each
routed expert id to its slot (``ensure_experts``, ``:800-810``; CPU mirror of
the rewrite at ``moe/offload_kernels.py:185-188``).  ``slot_map`` is the
lookup alone (misses reported, not fetched); ``lru_ensure`` adds the
admission of the misses.  Miss statistics follow the reference's counters
(``moe/offload_cache.py:861-934``): distinct active experts, distinct missing
experts and calls, plus the number of routes that missed.

Pins of ``slot_map`` (tests/test_oracle_experts.py): closed-form table lookups
on hand-built tables (identity, permutation, partial residency, all-miss) and
the invariant slot_for_id[id_of_slot[s]] == s.

``lru_ensure`` restates the admission of the miss path from the reference's
CPU mirror of its admission kernel (``moe/offload_kernels.py:128-188``,
``_ensure_experts_hybrid_cpu``, which the reference holds bit-identical to its
GPU kernel; fixed cap, ``frac_q16 == 0``), limited to the slots its GPU
kernel may take (``:369-387``: none holding an expert of the call or admitted
by it), with the miss order "lowest_id"
(``by_recency=False``) or "recency" (``:9-16``).  The uncapped lowest-id form
stands for flashlib's ``lru_ensure`` (``:19-40``), whose own order is not
available (third-party, absent): parity with flashlib is unpinned; the form
is pinned by the reference's invariants (tests/moe/test_offload.py:379-404:
unique victim slots, src rows = the missing ids in order; :522-602: the slot
tables stay inverse of each other across layers) and by a brute-force
properties checked in tests/test_oracle_slots.py (LRU victims, residency,
caps, recency order).
"""

from __future__ import annotations

import numpy as np

STAT_ACTIVE, STAT_MISS, STAT_CALLS, STAT_MISSED_ROUTES = range(4)


def slot_map(topk_ids, slot_for_id):
    ids = np.asarray(topk_ids, dtype=np.int32)
    table = np.asarray(slot_for_id, dtype=np.int32).reshape(-1)
    e = table.size
    valid = (ids >= 0) & (ids < e)
    slots = np.where(valid, table[np.clip(ids, 0, e - 1)], -1).astype(np.int32)
    miss = valid & (slots < 0)
    uniq = np.unique(ids[valid])
    stats = np.zeros(4, dtype=np.int64)
    stats[STAT_ACTIVE] = uniq.size
    stats[STAT_MISS] = int((table[uniq] < 0).sum()) if uniq.size else 0
    stats[STAT_CALLS] = 1
    stats[STAT_MISSED_ROUTES] = int(miss.sum())
    return slots, miss.astype(np.uint8), stats


class CacheState:
    """Mutable admission state of one slot cache (``moe/offload_cache.py:155-175``):
    ``slot_for_id`` [L, E], ``id_of_slot`` [S] (flat ``layer * E + expert``),
    ``usage`` [S] (step of last use), ``step``, ``recency`` [L, E]."""

    def __init__(self, num_layers: int, num_experts: int, cache_size: int):
        self.L, self.E, self.S = num_layers, num_experts, cache_size
        self.slot_for_id = np.full((num_layers, num_experts), -1, dtype=np.int32)
        self.id_of_slot = np.full(cache_size, -1, dtype=np.int32)
        self.usage = np.zeros(cache_size, dtype=np.int64)
        self.step = 0
        self.recency = np.zeros((num_layers, num_experts), dtype=np.int64)
        self.unserved = np.zeros(num_layers, dtype=np.int64)

    def copy(self) -> "CacheState":
        c = CacheState(self.L, self.E, self.S)
        c.slot_for_id = self.slot_for_id.copy()
        c.id_of_slot = self.id_of_slot.copy()
        c.usage = self.usage.copy()
        c.step = self.step
        c.recency = self.recency.copy()
        c.unserved = self.unserved.copy()
        return c


def fraction_cap(num_missing: int, frac_q16: int) -> int:
    """Bandwidth-matched fetch count (``moe/offload_kernels.py:160-164``): with
    m misses and f = frac_q16 / 2^16, the n in {floor(m f), floor(m f) + 1}
    whose max(n (1 - f), (m - n) f) is smaller, the lower one on a tie, then
    at most m.  Pinned (tests/test_oracle_slots.py) against the brute-force
    argmin of that cost over every n in [0, m]."""
    m, q = num_missing, 1 << 16
    lo = (m * frac_q16) >> 16

    def cost(f):
        return max(f * (q - frac_q16), (m - f) * frac_q16)

    return min(m, lo if cost(lo) <= cost(lo + 1) else lo + 1)


def hybrid_split(raw_ids, slot_ids, num_experts: int):
    """Routes the CPU computes in the hybrid decode (``layers/moe.py:350-352``):
    the raw expert id where admission left no slot (an unfetched miss), -1
    where the GPU computes the route or the id is outside [0, E)."""
    raw = np.asarray(raw_ids, dtype=np.int32)
    valid = (raw >= 0) & (raw < num_experts)
    return np.where(valid & (np.asarray(slot_ids) < 0), raw, -1).astype(np.int32)


def materialize_layer(state: CacheState, layer: int):
    """Whole-layer placement (``_materialize_layer_kernel``,
    ``moe/offload_kernels.py:250-281``): slots holding this layer's experts
    are emptied (usage 0), other layers' experts in slots [0, E) lose their
    mapping, step += 1, and expert e takes slot e with usage = step.  Returns
    the gather entries (evict_slots, src_indices) = (0..E-1, 0..E-1).

    Pinned (tests/test_oracle_slots.py) by invariants: tables stay inverse,
    position == expert id for the layer, untouched experts of other layers
    keep their slots, freed slots are the next LRU victims."""
    E, S = state.E, state.S
    assert S >= E, "materialize needs cache_size >= num_experts"
    base = layer * E
    flat = state.slot_for_id.reshape(-1)
    old = state.id_of_slot.copy()
    for s in range(S):
        o = int(old[s])
        if base <= o < base + E:
            state.id_of_slot[s] = -1
            state.usage[s] = 0
        elif s < E and o >= 0:
            flat[o] = -1
    state.step += 1
    for e in range(E):
        state.id_of_slot[e] = base + e
        flat[base + e] = e
        state.usage[e] = state.step
    return np.arange(E, dtype=np.int32), np.arange(E, dtype=np.int32)


def release_slots(state: CacheState, begin: int, end: int) -> None:
    """Empties slots [begin, end) and unmaps their experts (the prefill double
    buffer's ``_invalidate_prefill_buffer``, ``moe/offload_cache.py:592-600``)."""
    flat = state.slot_for_id.reshape(-1)
    for s in range(begin, end):
        o = int(state.id_of_slot[s])
        if o >= 0:
            flat[o] = -1
        state.id_of_slot[s] = -1
        state.usage[s] = 0


def lru_ensure(state: CacheState, layer: int, expert_ids, max_fetch: int = -1, by_recency: bool = False,
               capacity: int | None = None, frac_q16: int = 0):
    """One admission call (``moe/offload_kernels.py:128-188``); mutates ``state``.
    ``frac_q16`` > 0 replaces ``max_fetch`` by ``fraction_cap``.

    Returns (slot ids [same shape], evict_slots, src_indices, num_missing, stats).
    Ids outside [0, E) are not seen and map to -1."""
    ids = np.asarray(expert_ids, dtype=np.int32)
    flat = ids.reshape(-1)
    E = state.E
    seen = []
    for e in flat.tolist():  # first appearance order (:135-138)
        if 0 <= e < E and e not in seen:
            seen.append(e)
    state.step += 1
    step = state.step
    for e in seen:  # touch the resident ones (:143-146)
        s = int(state.slot_for_id[layer, e])
        if s != -1:
            state.usage[s] = step
    missing = [e for e in seen if int(state.slot_for_id[layer, e]) == -1]
    if by_recency:
        rec = state.recency[layer]
        missing.sort(key=lambda e: (-int(rec[e]), e))
    else:
        missing.sort()
    n = len(missing) if max_fetch < 0 else min(len(missing), max_fetch)
    if frac_q16 > 0:
        n = fraction_cap(len(missing), frac_q16)
    wanted = n
    if capacity is not None:
        n = min(n, capacity)
    # only slots that hold no expert of this call and were not admitted by it
    # (usage < step) may be taken: the exclusion of the reference's GPU kernel
    # (offload_kernels.py:369-387).  Its CPU mirror (:163-174) takes the
    # smallest (usage, slot) unconditionally, which re-picks a slot admitted in
    # the same call once the free slots run out; both agree while they last.
    n = min(n, int((state.usage < step).sum()))
    state.unserved[layer] += wanted - n
    evict, src = [], []
    miss_set = set(missing)
    for idx in range(n):  # one victim after the other (:163-174)
        expert = missing[idx]
        victim = min(range(state.S), key=lambda s: (int(state.usage[s]), s))
        old = int(state.id_of_slot[victim])
        if old >= 0:
            state.slot_for_id.reshape(-1)[old] = -1
        state.id_of_slot[victim] = layer * E + expert
        state.slot_for_id[layer, expert] = victim
        state.usage[victim] = step
        evict.append(victim)
        src.append(expert)
    if by_recency:  # (:176-178)
        for e in seen:
            state.recency[layer, e] = step
    out = np.array([int(state.slot_for_id[layer, e]) if 0 <= e < E else -1 for e in flat.tolist()],
                   dtype=np.int32).reshape(ids.shape)
    stats = np.zeros(4, dtype=np.int64)
    stats[STAT_ACTIVE] = len(seen)
    stats[STAT_MISS] = len(missing)
    stats[STAT_CALLS] = 1
    stats[STAT_MISSED_ROUTES] = sum(1 for e in flat.tolist() if e in miss_set)
    return out, np.array(evict, dtype=np.int32), np.array(src, dtype=np.int32), len(missing), stats
