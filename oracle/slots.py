"""Expert-cache slot indirection (lookup + miss report, no admission).

``OffloadMoeCache.slot_for_id`` is an int32 [L, E] table with -1 for a
non-resident expert (``moe/offload_cache.py:155-175``); decode rewrites each
routed expert id to its slot (``ensure_experts``, ``:800-810``; CPU mirror of
the rewrite at ``moe/offload_kernels.py:185-188``).  This build keeps the
lookup and reports misses instead of fetching them (fetching is the next
step of the miss path).  Miss statistics follow the reference's counters
(``moe/offload_cache.py:861-934``): distinct active experts, distinct missing
experts and calls, plus the number of routes that missed.

Pins (tests/test_oracle_slots.py): closed-form table lookups on hand-built
tables (identity, permutation, partial residency, all-miss) and the
invariant slot_for_id[id_of_slot[s]] == s.
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
