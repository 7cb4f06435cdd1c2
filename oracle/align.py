"""Token -> expert histogram, padded prefix sum and permutation
(``moe_align_block_size``; ``moe/fused.py:88-158``,
``kernel/triton/moe_align.py:1-44,216-325``).

Contract restated:
  * effective_E = num_experts + 1; ids outside [0, effective_E) are ignored
    (``moe_align.py:75-77``);
  * buffer sizes: max_padded = numel*BM if numel < E+1 else numel+(E+1)*(BM-1)
    (``fused.py:139-147``);
  * cumsum[0] = 0, cumsum[i] = cumsum[i-1] + ceil(count[i-1]/BM)*BM;
    num_tokens_post_pad = cumsum[effective_E];
  * expert_ids[b] = expert owning block b for b < num_tokens_post_pad/BM;
  * sorted_ids: route indices scattered into [cumsum[e], cumsum[e]+count[e]);
    unwritten slots hold the sentinel ``numel``.

Canonical order: the reference ranks routes inside an expert with atomics
(``moe_align.py:19-20,104-105,206-209``), so its intra-expert order is not
defined.  This build fixes it to ascending flattened route index (stable),
which is the order of the docstring example (``fused.py:113-126``); per
expert the reference agrees with it as a set.  Positions the reference leaves
unwritten are defined here: sorted_ids beyond num_tokens_post_pad hold the
sentinel and expert_ids beyond the used blocks hold -1.

Pins (tests/test_oracle_align.py): the docstring KAT; brute force against a
sort-based construction on random tiny inputs; invariants (every valid route
appears exactly once, padding holds the sentinel, regions are BM-aligned).
"""

from __future__ import annotations

import numpy as np


def buffer_sizes(numel: int, num_experts: int, block_size: int):
    if numel < num_experts + 1:
        max_padded = numel * block_size
    else:
        max_padded = numel + (num_experts + 1) * (block_size - 1)
    return max_padded, -(-max_padded // block_size)


def moe_align_block_size(topk_ids, block_size: int, num_experts: int):
    ids = np.asarray(topk_ids, dtype=np.int32).reshape(-1)
    numel = ids.size
    eff = num_experts + 1
    max_padded, max_blocks = buffer_sizes(numel, num_experts, block_size)
    valid = (ids >= 0) & (ids < eff)
    counts = np.bincount(ids[valid], minlength=eff).astype(np.int64)
    nblk = -(-counts // block_size)
    cumsum = np.zeros(eff + 1, dtype=np.int64)
    cumsum[1:] = np.cumsum(nblk * block_size)
    total = int(cumsum[eff])
    sorted_ids = np.full(max_padded, numel, dtype=np.int32)
    expert_ids = np.full(max_blocks, -1, dtype=np.int32)
    for e in range(eff):
        routes = np.nonzero(ids == e)[0]
        sorted_ids[cumsum[e] : cumsum[e] + routes.size] = routes
        b0 = cumsum[e] // block_size
        expert_ids[b0 : b0 + nblk[e]] = e
    return sorted_ids, expert_ids, np.array([total], dtype=np.int32)


def expert_segments(topk_ids, num_experts: int):
    """Compact per-expert route lists used by the decode kernels: for every
    expert with at least one route (ascending expert id), its id, the start of
    its routes in ``routes`` and their count; ``routes`` holds the route
    indices in the canonical stable order.  Ids outside [0, num_experts) are
    ignored (skipped routes / cache misses)."""
    ids = np.asarray(topk_ids, dtype=np.int32).reshape(-1)
    valid = (ids >= 0) & (ids < num_experts)
    order = np.argsort(np.where(valid, ids, num_experts), kind="stable")
    routes = order[: int(valid.sum())].astype(np.int32)
    seg_expert, seg_start, seg_count = [], [], []
    pos = 0
    for e in range(num_experts):
        c = int((ids[valid] == e).sum())
        if c:
            seg_expert.append(e)
            seg_start.append(pos)
            seg_count.append(c)
            pos += c
    return (
        np.array(seg_expert, dtype=np.int32),
        np.array(seg_start, dtype=np.int32),
        np.array(seg_count, dtype=np.int32),
        routes,
    )
