"""Expert-cache slot indirection (the lookup half of FreeToken's
``OffloadMoeCache``, ``moe/offload_cache.py``).

``slot_for_id`` [L, E] int32 maps (layer, expert) to a GPU slot or -1;
``id_of_slot`` [S] holds the flat id ``layer * E + expert`` of each slot
(``:155-175``).  The slot banks are one ``[S, ...]`` tensor per bank
(``bank_views``, ``:555-561``).  ``ensure_experts`` rewrites routed expert
ids to slot ids in place (``:800-810``); experts that are not resident are
reported as misses (slot -1, skipped by the expert kernels) instead of being
fetched -- the PCIe miss path and its LRU admission are not part of this
build.  Miss statistics accumulate on the device, graph-safe, in the
reference's layout (``:205-229,861-934``).
"""

from __future__ import annotations

from collections import OrderedDict

import torch

from .. import ops

STAT_ACTIVE, STAT_MISS, STAT_CALLS, STAT_MISSED_ROUTES = range(4)
N_STATS = 4


class ExpertSlotCache:
    def __init__(self, num_layers: int, num_experts: int, cache_size: int, quant_format: str,
                 device: torch.device | str = "cuda"):
        assert quant_format in ("bf16", "fp8_block", "ds_fp4"), quant_format
        self.num_layers = num_layers
        self.num_experts = num_experts
        self.cache_size = cache_size
        self.quant_format = quant_format
        self.device = torch.device(device)
        self.slot_for_id = torch.full((num_layers, num_experts), -1, dtype=torch.int32, device=self.device)
        self.id_of_slot = torch.full((cache_size,), -1, dtype=torch.int32, device=self.device)
        self.collect_stats = True
        self.lru_stats = torch.zeros((num_layers, N_STATS), dtype=torch.int64, device=self.device)
        self.banks: "OrderedDict[str, torch.Tensor]" = OrderedDict()

    # -------------------------------------------------------------- setup (host)
    def set_bank_caches(self, **banks: torch.Tensor) -> None:
        """Registers the slot banks in order, e.g. gate_up, gate_up_scale, down,
        down_scale; each is ``[cache_size, ...]``."""
        for name, t in banks.items():
            assert t.shape[0] == self.cache_size, (name, t.shape)
            self.banks[name] = t

    def assign(self, layer_id: int, experts, slots) -> None:
        """Marks ``experts`` of ``layer_id`` resident in ``slots`` (the caller
        copies their weights into the slot banks)."""
        experts = torch.as_tensor(experts, dtype=torch.int64)
        slots = torch.as_tensor(slots, dtype=torch.int64)
        old = self.id_of_slot[slots.to(self.device)]
        for flat in old.tolist():
            if flat >= 0:
                self.slot_for_id.view(-1)[flat] = -1
        self.slot_for_id[layer_id, experts.to(self.device)] = slots.to(self.device, torch.int32)
        self.id_of_slot[slots.to(self.device)] = (layer_id * self.num_experts + experts).to(self.device, torch.int32)

    def bank_views(self, n: int | None = None) -> tuple[torch.Tensor, ...]:
        assert self.banks, "set_bank_caches must register the banks first"
        if n is None:
            return tuple(self.banks.values())
        return tuple(t[:n] for t in self.banks.values())

    # -------------------------------------------------------------- hot path
    def ensure_experts(self, layer_id: int, expert_ids: torch.Tensor,
                       miss_mask: torch.Tensor | None = None) -> torch.Tensor:
        """Rewrites ``expert_ids`` (int32, any shape) to slot ids in place."""
        stats = self.lru_stats[layer_id] if self.collect_stats else None
        ops.slot_map(expert_ids, self.slot_for_id[layer_id], out=expert_ids, miss_mask=miss_mask, stats=stats)
        return expert_ids

    def slot_lookup(self, layer_id: int) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(slot table, stats counters or None) of a layer, for decode calls that
        do the ``ensure_experts`` rewrite themselves (``ops.experts_decode``
        with ``slot_for_id``)."""
        return self.slot_for_id[layer_id], (self.lru_stats[layer_id] if self.collect_stats else None)

    # -------------------------------------------------------------- statistics
    def reset_stats(self) -> None:
        self.lru_stats.zero_()

    def decode_miss_stats(self) -> dict:
        active, missing, calls, missed_routes = (int(x) for x in self.lru_stats.sum(0))
        return {
            "layer_calls": calls,
            "active_per_layer": active / calls if calls else 0.0,
            "missing_per_layer": missing / calls if calls else 0.0,
            "miss_rate": missing / active if active else 0.0,
            "missed_routes": missed_routes,
        }
