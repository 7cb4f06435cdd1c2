"""Expert-cache slot indirection (the lookup half of FreeToken's
``OffloadMoeCache``, ``moe/offload_cache.py``).

``slot_for_id`` [L, E] int32 maps (layer, expert) to a GPU slot or -1;
``id_of_slot`` [S] holds the flat id ``layer * E + expert`` of each slot
(``:155-175``).  The slot banks are one ``[S, ...]`` tensor per bank
(``bank_views``, ``:555-561``).  ``ensure_experts`` rewrites routed expert
ids to slot ids in place (``:800-810``).  With host sources registered
(``set_bank_sources``, pinned per-layer ``[E, ...]`` tensors, ``:419-470``) it
also admits the missing experts into least-recently-used slots
(``lru_ensure``, ``moe/offload_kernels.py:19-40``) and ``copy_missing``
gathers their rows over PCIe (``:968-1010``); without sources, misses are
reported (slot -1, skipped by the expert kernels).  ``ensure_experts_hybrid``
is the capped admission (``offload_kernels.py:43-60``) of the hybrid decode,
whose unfetched misses a CPU executor computes (``decode_target``
"hybrid"; "cpu" layers decode on the CPU entirely, ``:117-150,513-526``).
Everything runs on the device without host synchronisation; miss statistics
accumulate in the reference's layout (``:205-229,861-934``).
"""

from __future__ import annotations

from collections import OrderedDict

import numpy as np
import torch

from .. import ops

STAT_ACTIVE, STAT_MISS, STAT_CALLS, STAT_MISSED_ROUTES = range(4)
N_STATS = 4


def bank_from_views(quant_format: str, views, swiglu_limit: float | None = None) -> ops.ExpertBank:
    """An ``ExpertBank`` over bank tensors in registration order: (gate_up,
    down) for bf16, (gate_up, gate_up_scale, down, down_scale) otherwise.
    ``swiglu_limit`` (the layer's DeepSeek-V4 SwiGLU clamp) applies to the
    ds_fp4 format, as the reference passes it to ``routed_experts_fp4`` only
    (``layers/moe.py:556-573``)."""
    if quant_format == "bf16":
        gate_up, down = views
        return ops.ExpertBank("bf16", gate_up, down)
    gate_up, gate_up_scale, down, down_scale = views
    if quant_format == "fp8_block":
        return ops.ExpertBank("fp8_block", gate_up, down, gate_up_scale, down_scale)
    return ops.ExpertBank("mxfp4", gate_up, down, gate_up_scale, down_scale, swiglu_limit=float(swiglu_limit or 0.0))


class ExpertSlotCache:
    def __init__(self, num_layers: int, num_experts: int, cache_size: int, quant_format: str,
                 device: torch.device | str = "cuda", decode_target: str = "gpu", hybrid_max_fetch: int = 1,
                 hybrid_fetch_fraction: float = 0.0, prefill_overlap: bool = False, prefill_hit_d2d: bool = False):
        assert quant_format in ("bf16", "fp8_block", "ds_fp4"), quant_format
        assert decode_target in ("gpu", "cpu", "hybrid"), decode_target
        # decode placement (moe/offload_cache.py:117-136): "gpu" fetches every
        # miss; "hybrid" fetches at most hybrid_max_fetch (or the
        # hybrid_fetch_fraction share) of a step's misses and the CPU executor
        # computes the rest; cpu_layer_ids decode on the CPU entirely
        self.decode_target = decode_target
        self.hybrid_max_fetch = hybrid_max_fetch
        self.hybrid_fetch_fraction = hybrid_fetch_fraction
        self.cpu_executor = None
        self.cpu_layer_ids: frozenset = frozenset()
        # prefill movement (:563-798): with prefill_overlap two full-layer
        # buffers borrow slots [0, 2E) and layer l+1's host copy runs on a copy
        # stream behind layer l's GEMMs; otherwise materialize_layer stages the
        # layer into slots [0, E) before its GEMMs
        assert not prefill_overlap or cache_size >= 2 * num_experts, \
            "prefill overlap borrows two expert layers of slots: cache_size >= 2 * num_experts"
        self.prefill_overlap = prefill_overlap
        # hit/miss split of the double buffer (:703-773): experts resident
        # outside the buffers (slot >= 2E) reach the buffer device to device,
        # only the others cross PCIe; needs slots beyond the two buffers
        self.prefill_hit_d2d = prefill_hit_d2d
        self._pf_split = False
        self.prefill_hit_rows = 0
        self.prefill_total_rows = 0
        self._pf_views: list[torch.Tensor] | None = None
        self._pf_layer: list[int | None] = [None, None]
        self._pf_released = [True, True]
        self._pf_has_release = [False, False]
        self.prefill_copy_stream = None
        self.num_layers = num_layers
        self.num_experts = num_experts
        self.cache_size = cache_size
        self.quant_format = quant_format
        self.device = torch.device(device)
        self.slot_for_id = torch.full((num_layers, num_experts), -1, dtype=torch.int32, device=self.device)
        self.id_of_slot = torch.full((cache_size,), -1, dtype=torch.int32, device=self.device)
        self.collect_stats = True
        self.lru_stats = torch.zeros((num_layers, N_STATS), dtype=torch.int64, device=self.device)
        # opt-in decode routing histogram per (layer, expert), for cache-skew
        # analysis (:230-236): counted on the device from the raw expert ids
        # before their rewrite to slots, so replayed graphs keep counting
        self.collect_decode_freq = False
        self.decode_freq = torch.zeros((num_layers, num_experts), dtype=torch.int64, device=self.device)
        # misses left without a slot because every slot held an expert of the same call
        self.unserved = torch.zeros((num_layers,), dtype=torch.int64, device=self.device)
        self.banks: "OrderedDict[str, torch.Tensor]" = OrderedDict()
        # admission state (moe/offload_cache.py:155-200)
        dev = self.device
        self.usage = torch.zeros((cache_size,), dtype=torch.int64, device=dev)
        self.step = torch.zeros((1,), dtype=torch.int64, device=dev)
        self.expert_recency = torch.zeros((num_layers, num_experts), dtype=torch.int64, device=dev)
        cap = min(num_experts, cache_size)
        self.evict_slots = torch.zeros((cap,), dtype=torch.int32, device=dev)
        self.src_indices = torch.zeros((cap,), dtype=torch.int32, device=dev)
        self.num_indices = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.num_missing_full = torch.zeros((1,), dtype=torch.int32, device=dev)
        self.sources: "OrderedDict[str, list[torch.Tensor]]" = OrderedDict()
        self._pending_src_layer: int | None = None

    # -------------------------------------------------------------- setup (host)
    def set_bank_caches(self, **banks: torch.Tensor) -> None:
        """Registers the slot banks in order, e.g. gate_up, gate_up_scale, down,
        down_scale; each is ``[cache_size, ...]``."""
        for name, t in banks.items():
            assert t.shape[0] == self.cache_size, (name, t.shape)
            self.banks[name] = t

    def set_bank_sources(self, sources: dict) -> None:
        """Registers the host copy of every bank: ``name -> [per-layer tensor]``
        with each tensor ``[num_experts, ...]`` in pinned host memory and the
        same row shape as the slot bank of that name (``:419-470``)."""
        assert set(sources) == set(self.banks), (sorted(sources), sorted(self.banks))
        for name, layers in sources.items():
            assert len(layers) == self.num_layers, (name, len(layers))
            for t in layers:
                assert t.device.type == "cpu" and t.is_pinned() and t.is_contiguous(), name
                assert t.shape[0] == self.num_experts and t.shape[1:] == self.banks[name].shape[1:], (name, t.shape)
                assert t.element_size() == self.banks[name].element_size(), (name, t.dtype, self.banks[name].dtype)
        self.sources = OrderedDict((name, list(sources[name])) for name in self.banks)

    def set_cpu_executor(self, executor) -> None:
        """Attaches the CPU share of the decode (a ``CpuMoeDecoder`` reading
        this cache's host sources; ``:513-522``)."""
        assert self.decode_target in ("cpu", "hybrid"), "set_cpu_executor requires decode_target cpu or hybrid"
        self.cpu_executor = executor

    def is_cpu_layer(self, layer_id: int) -> bool:
        return layer_id in self.cpu_layer_ids

    def host_bank_tensors(self, layer_id: int) -> tuple[torch.Tensor, ...]:
        """The pinned host rows of one layer, in bank order."""
        assert self.sources, "set_bank_sources must register the host banks first"
        return tuple(layers[layer_id] for layers in self.sources.values())

    def reset(self) -> None:
        """Empties the cache: no expert resident, usage and step cleared."""
        self.slot_for_id.fill_(-1)
        self.id_of_slot.fill_(-1)
        self.usage.zero_()
        self.step.zero_()
        self.expert_recency.zero_()
        self.num_indices.zero_()
        self._pending_src_layer = None

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
        """Rewrites ``expert_ids`` (int32, any shape) to slot ids in place.
        With host sources, the missing experts are first admitted (lowest id
        first, into the least recently used slots) and staged for
        ``copy_missing``; without, they map to -1 (``miss_mask`` marks them)."""
        stats = self.lru_stats[layer_id] if self.collect_stats else None
        self.note_decode_routing(layer_id, expert_ids)
        if not self.sources:
            ops.slot_map(expert_ids, self.slot_for_id[layer_id], out=expert_ids, miss_mask=miss_mask, stats=stats)
            return expert_ids
        assert miss_mask is None, "every expert is admitted when host sources are registered"
        return self._admit(layer_id, expert_ids, -1, None, stats)

    def ensure_experts_hybrid(self, layer_id: int, expert_ids: torch.Tensor, max_fetch: int | None = None,
                              by_recency: bool = True, fetch_fraction: float | None = None,
                              cpu_ids: torch.Tensor | None = None) -> torch.Tensor:
        """Capped admission (``offload_kernels.py:43-60``, ``offload_cache.py:812-831``):
        at most ``max_fetch`` (default ``hybrid_max_fetch``; or the
        ``fetch_fraction`` share, default ``hybrid_fetch_fraction``) of the
        missing experts, most recently seen first with ``by_recency`` (else
        lowest id first), are admitted; the others map to -1 and, with
        ``cpu_ids``, are listed there by expert id for the CPU."""
        assert self.sources, "set_bank_sources must register the host banks first"
        stats = self.lru_stats[layer_id] if self.collect_stats else None
        self.note_decode_routing(layer_id, expert_ids)
        rec = self.expert_recency[layer_id] if by_recency else None
        max_fetch = self.hybrid_max_fetch if max_fetch is None else max_fetch
        frac = self.hybrid_fetch_fraction if fetch_fraction is None else fetch_fraction
        return self._admit(layer_id, expert_ids, max_fetch, rec, stats, frac, cpu_ids)

    def _admit(self, layer_id, expert_ids, max_fetch, recency, stats, fetch_fraction=0.0, cpu_ids=None):
        ops.lru_ensure(expert_ids, layer_id, self.slot_for_id, self.id_of_slot, self.usage, self.step,
                       self.evict_slots, self.src_indices, self.num_indices, self.num_missing_full,
                       recency=recency, max_fetch=max_fetch, stats=stats, fetch_fraction=fetch_fraction,
                       cpu_ids=cpu_ids, unserved=self.unserved[layer_id:layer_id + 1])
        self._pending_src_layer = layer_id
        return expert_ids

    def copy_missing(self) -> None:
        """Copies the experts staged by the last admission from their host rows
        into their slots (``:968-1010``); the count stays on the device."""
        assert self.sources, "set_bank_sources must register the host banks first"
        layer_id = self._pending_src_layer
        assert layer_id is not None, "no staged misses (ensure_experts first)"
        ops.fetch_experts([layers[layer_id] for layers in self.sources.values()], list(self.banks.values()),
                          self.evict_slots, self.src_indices, self.num_indices)

    def materialize_layer(self, layer_id: int) -> None:
        """Stages the whole layer at slot == expert id for a prefill
        (``:833-838``); ``copy_missing`` then moves it over PCIe."""
        assert self.cache_size >= self.num_experts, "materialize needs cache_size >= num_experts"
        ops.materialize_layer(layer_id, self.slot_for_id, self.id_of_slot, self.usage, self.step, self.evict_slots,
                              self.src_indices, self.num_indices)
        self._pending_src_layer = layer_id

    # -------------------------------------------------------------- prefill double buffer
    def _prefill_buffers(self) -> list[torch.Tensor]:
        if self._pf_views is None:
            assert self.sources, "set_bank_sources must register the host banks first"
            E = self.num_experts
            self._pf_views = [t[: 2 * E].view(2, E, *t.shape[1:]) for t in self.banks.values()]
            self.prefill_copy_stream = torch.cuda.Stream(device=self.device)
            self._pf_ready = [torch.cuda.Event() for _ in range(2)]
            self._pf_release = [torch.cuda.Event() for _ in range(2)]
            self._pf_begin = torch.cuda.Event()
            dev = self.device
            self._pf_snapshot = torch.empty((self.num_layers, E), dtype=torch.int32, pin_memory=True)
            self._pf_hit_dst = torch.empty((E,), dtype=torch.int32, device=dev)
            self._pf_hit_src = torch.empty((E,), dtype=torch.int32, device=dev)
            self._pf_hit_num = torch.zeros((1,), dtype=torch.int32, device=dev)
        return self._pf_views

    def begin_prefill(self) -> None:
        """Fences the copy stream behind the work already queued on the current
        stream (a running decode may read the slots the buffers borrow; :602-624).
        With the hit/miss split, snapshots the slot table once for the chunk
        (one host synchronisation; the per-layer miss lists are host math)."""
        if not self.prefill_overlap:
            return
        self._prefill_buffers()
        self._pf_layer = [None, None]
        self._pf_released = [True, True]
        self._pf_begin.record(torch.cuda.current_stream(self.device))
        self.prefill_copy_stream.wait_event(self._pf_begin)
        self._pf_split = self.prefill_hit_d2d and self.cache_size > 2 * self.num_experts
        if self._pf_split:
            with torch.cuda.stream(self.prefill_copy_stream):
                self._pf_snapshot.copy_(self.slot_for_id, non_blocking=True)
            self.prefill_copy_stream.synchronize()

    def prefetch_prefill_layer(self, layer_id: int) -> None:
        """Starts the host copy of a whole layer into buffer ``layer_id % 2`` on
        the copy stream, after that buffer's previous layer was released; the
        buffer's slots are emptied first (``:625-658``)."""
        if not self.prefill_overlap or layer_id >= self.num_layers:
            return
        if layer_id < 0:
            raise ValueError(f"invalid prefill layer id {layer_id}")
        buf = layer_id % 2
        if self._pf_layer[buf] == layer_id:
            return
        assert self._pf_layer[buf] is None or self._pf_released[buf], "prefill buffer reused before release"
        views = self._prefill_buffers()
        E = self.num_experts
        if self._pf_split:
            self._prefetch_split(layer_id, buf)
        else:
            with torch.cuda.stream(self.prefill_copy_stream):
                if self._pf_has_release[buf]:
                    self.prefill_copy_stream.wait_event(self._pf_release[buf])
                ops.release_slots(buf * E, (buf + 1) * E, self.slot_for_id, self.id_of_slot, self.usage)
                for layers, v in zip(self.sources.values(), views):  # bytes, whatever the dtypes
                    v[buf].view(torch.uint8).copy_(layers[layer_id].view(torch.uint8), non_blocking=True)
                self._pf_ready[buf].record(self.prefill_copy_stream)
        self._pf_layer[buf] = layer_id
        self._pf_released[buf] = False

    def _prefetch_split(self, layer_id: int, buf: int) -> None:
        """Hit/miss split of one layer's move into buffer ``buf`` (``:703-773``).
        Hits -- experts resident at slots >= 2E, outside the buffers -- are
        listed on the device from the live slot table and gathered slot bank ->
        buffer on the current stream (ordered after the buffer's earlier
        GEMMs).  Misses (slots below 2E belong to the buffers and count as
        misses) are listed from the chunk's snapshot and gathered host -> buffer
        on the copy stream after the buffer's release and the emptying of its
        slots.  The two row sets are disjoint; the live table and the snapshot
        agree on them, since the only writer during a prefill chunk empties
        buffer slots, which are below 2E on both sides."""
        E = self.num_experts
        banks = list(self.banks.values())
        snap = self._pf_snapshot[layer_id]
        hit = snap >= 2 * E
        n_hit = int(hit.sum())
        self.prefill_hit_rows += n_hit
        self.prefill_total_rows += E
        if n_hit:
            ops.prefill_hit_compact(self.slot_for_id[layer_id], 2 * E, buf * E, self._pf_hit_dst, self._pf_hit_src,
                                    self._pf_hit_num)
            ops.fetch_experts(banks, banks, self._pf_hit_dst, self._pf_hit_src, self._pf_hit_num, max_entries=E)
        miss = torch.nonzero(~hit).flatten().to(torch.int32)
        with torch.cuda.stream(self.prefill_copy_stream):
            if self._pf_has_release[buf]:
                self.prefill_copy_stream.wait_event(self._pf_release[buf])
            ops.release_slots(buf * E, (buf + 1) * E, self.slot_for_id, self.id_of_slot, self.usage)
            if miss.numel():
                # host-built lists (pinned, fresh per call: the pinned allocator keeps a block
                # until the copy that reads it has run)
                lists = torch.stack([miss + buf * E, miss, torch.full_like(miss, miss.numel())]).pin_memory()
                dev_lists = lists.to(self.device, non_blocking=True)
                ops.fetch_experts([layers[layer_id] for layers in self.sources.values()], banks, dev_lists[0],
                                  dev_lists[1], dev_lists[2, :1], max_entries=int(miss.numel()))
            self._pf_ready[buf].record(self.prefill_copy_stream)

    def wait_prefill_layer(self, layer_id: int) -> tuple[torch.Tensor, ...]:
        """The layer's full ``[E, ...]`` bank views, the current stream made to
        wait for their copy (``:775-787``)."""
        assert self.prefill_overlap
        self.prefetch_prefill_layer(layer_id)
        buf = layer_id % 2
        assert self._pf_layer[buf] == layer_id
        torch.cuda.current_stream(self.device).wait_event(self._pf_ready[buf])
        return tuple(v[buf] for v in self._pf_views)

    def release_prefill_layer(self, layer_id: int) -> None:
        """Marks the layer's buffer free once the current stream's work queued so
        far (its GEMMs) is done (``:789-798``)."""
        if not self.prefill_overlap:
            return
        buf = layer_id % 2
        if self._pf_layer[buf] != layer_id:
            return
        self._pf_release[buf].record(torch.cuda.current_stream(self.device))
        self._pf_has_release[buf] = True
        self._pf_released[buf] = True

    def slot_lookup(self, layer_id: int,
                    expert_ids: torch.Tensor | None = None) -> tuple[torch.Tensor, torch.Tensor | None]:
        """(slot table, stats counters or None) of a layer, for decode calls that
        do the ``ensure_experts`` rewrite themselves (``ops.experts_decode``
        with ``slot_for_id``); ``expert_ids``, the call's raw ids, feed the
        routing histogram as ``ensure_experts`` would."""
        if expert_ids is not None:
            self.note_decode_routing(layer_id, expert_ids)
        return self.slot_for_id[layer_id], (self.lru_stats[layer_id] if self.collect_stats else None)

    def note_decode_routing(self, layer_id: int, expert_ids: torch.Tensor) -> None:
        """Adds a decode step's raw expert ids to the layer's routing histogram
        when ``collect_decode_freq`` is on (``:803-807``): one small device
        launch, no host synchronisation."""
        if self.collect_decode_freq:
            ops.route_histogram(expert_ids.reshape(-1), self.decode_freq[layer_id])

    # -------------------------------------------------------------- statistics
    def reset_stats(self) -> None:
        self.lru_stats.zero_()
        self.unserved.zero_()

    def check_capacity(self) -> None:
        """Raises when an admission since the last ``reset_stats`` left misses
        without a slot (a call routed to more distinct experts than the cache
        holds: their routes were skipped).  Synchronises with the device."""
        n = int(self.unserved.sum())
        if n:
            raise RuntimeError(f"expert cache too small: {n} missing experts found no free slot "
                               f"(cache_size {self.cache_size}); their routes were skipped")

    def prefill_hit_rate(self) -> float:
        """Share of the layers' experts the hit/miss split gathered device to
        device since construction (the counters of ``:275-276,729``)."""
        return self.prefill_hit_rows / self.prefill_total_rows if self.prefill_total_rows else 0.0

    def decode_routing_stats(self) -> dict:
        """Per-layer routing concentration of the decode histogram
        (``decode_routing_stats``, ``:936-966``; same keys and definitions),
        averaged over the layers that saw routes: the working set (experts
        routed at least once), the experts covering 90% of the routes, the
        best hit rate a per-layer cache of ``cache_size / num_layers`` slots
        holding the most frequent experts could reach on this distribution,
        and the routing entropy normalised by log(E).  Reads the histogram
        back to the host once."""
        freq = self.decode_freq.detach().to("cpu", torch.float64).numpy()
        total = freq.sum(axis=1)
        valid = total > 0
        if not valid.any():
            return {}
        f, tot = freq[valid], total[valid]
        slots_per_layer = self.cache_size / self.num_layers
        c = max(1, int(round(slots_per_layer)))
        ranked = -np.sort(-f, axis=1)
        share = ranked / tot[:, None]
        cover90 = (np.cumsum(share, axis=1) < 0.9).sum(axis=1) + 1
        p = f / tot[:, None]
        with np.errstate(divide="ignore", invalid="ignore"):
            ent = -np.where(p > 0, p * np.log(p), 0.0).sum(axis=1)
        working = (f > 0).sum(axis=1)
        return {
            "slots_per_layer": slots_per_layer,
            "working_set_mean": float(working.mean()),
            "working_set_max": int(working.max()),
            "experts_for_90pct": float(cover90.mean()),
            "oracle_hit_at_slots": float((ranked[:, :c].sum(axis=1) / tot).mean()),
            "norm_entropy": float((ent / np.log(self.num_experts)).mean()),
        }

    def reset_decode_freq(self) -> None:
        self.decode_freq.zero_()

    def decode_miss_stats(self) -> dict:
        active, missing, calls, missed_routes = (int(x) for x in self.lru_stats.sum(0))
        return {
            "layer_calls": calls,
            "active_per_layer": active / calls if calls else 0.0,
            "missing_per_layer": missing / calls if calls else 0.0,
            "miss_rate": missing / active if active else 0.0,
            "missed_routes": missed_routes,
            "unserved_experts": int(self.unserved.sum()),
        }
