"""CPU share of the MoE decode (reference ``moe/cpu_executor.py:523-600``).

``CpuMoeDecoder`` owns the host executor (``ftmoe_cpu_experts_*``), one set
of pinned IO buffers per decode batch size and the host banks of every layer
(the cache's pinned sources, read in place).  ``decode_submit`` copies the
step's activations and routing to the pinned buffers and enqueues the CPU job
on the current stream; ``decode_sync`` makes the stream wait for it and
copies the result back.  Everything is stream-ordered, so GPU work enqueued
between the two runs while the CPU computes, and the whole sequence replays
in a captured graph (the first call of a batch size must be eager: it
allocates that size's pinned buffers).
"""

from __future__ import annotations

import os

import torch

from .. import ops
from .offload_cache import ExpertSlotCache, bank_from_views


def hybrid_fetch_fraction(pcie_gbs: float, cpu_gbs: float, overlapped: bool = True) -> float | None:
    """Bandwidth-matched share of a step's misses to fetch over PCIe, so that
    the fetch and the CPU's share finish together (reference
    ``load_hybrid_fetch_fraction``, ``moe/bench_profile.py:156-191``): from
    rates measured while both run, pcie / (pcie + cpu); from standalone rates,
    under full DRAM contention, pcie / cpu.  Clamped to [0, 1]; None without
    both rates.  The result is ``ExpertSlotCache.hybrid_fetch_fraction``."""
    if not pcie_gbs or not cpu_gbs or pcie_gbs <= 0 or cpu_gbs <= 0:
        return None
    return min(1.0, pcie_gbs / (pcie_gbs + cpu_gbs) if overlapped else pcie_gbs / cpu_gbs)


class CpuMoeDecoder:
    """``handshake``: ``"flags"`` (the default, as the reference's
    ``FREETOKEN_CPU_MOE_FLAG_SYNC``; ``FTMOE_CPU_FLAG_SYNC=0`` opts out) rides
    stream memory operations where their probe passes, else host functions;
    ``"host"`` keeps host functions."""

    def __init__(self, cache: ExpertSlotCache, top_k: int, threads: int = 0, activation: str = "silu",
                 watchdog_s: float | None = None, swiglu_limit: float | None = None, handshake: str | None = None):
        assert cache.sources, "the CPU share reads the cache's host sources: set_bank_sources first"
        self.cache = cache
        self.top_k = top_k
        self.activation = activation
        self.swiglu_limit = swiglu_limit  # the layers' ds_fp4 SwiGLU clamp (cpu_moe_ext.cpp:1769-1781)
        self.executor = ops.CpuExecutor(threads, watchdog_s=watchdog_s)
        if handshake is None:
            handshake = "host" if os.environ.get("FTMOE_CPU_FLAG_SYNC", "1") == "0" else "flags"
        if handshake == "flags" and torch.cuda.is_available():
            self.executor.set_handshake("flags")
        self._io: dict[int, dict[str, torch.Tensor]] = {}
        self._banks: dict[int, ops.ExpertBank] = {}

    def host_bank(self, layer_id: int) -> ops.ExpertBank:
        bank = self._banks.get(layer_id)
        if bank is None:
            bank = bank_from_views(self.cache.quant_format, self.cache.host_bank_tensors(layer_id), self.swiglu_limit)
            self._banks[layer_id] = bank
        return bank

    def _io_for(self, bs: int, hidden: int) -> dict[str, torch.Tensor]:
        io = self._io.get(bs)
        if io is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError(f"no pinned IO buffers for decode batch {bs}: run one eager call before capture")
            k = self.top_k
            io = {
                "x": torch.empty((bs, hidden), dtype=torch.bfloat16, pin_memory=True),
                "ids": torch.empty((bs, k), dtype=torch.int32, pin_memory=True),
                "w": torch.empty((bs, k), dtype=torch.float32, pin_memory=True),
                "y": torch.empty((bs, hidden), dtype=torch.bfloat16, pin_memory=True),
            }
            self._io[bs] = io
        return io

    def decode_submit(self, layer_id: int, hidden_states: torch.Tensor, topk_weights: torch.Tensor,
                      topk_ids: torch.Tensor) -> tuple:
        """Ships the step to pinned memory and starts the CPU job; routes with
        id -1 are skipped by the CPU.  Returns the handle for ``decode_sync``."""
        bs, hidden = hidden_states.shape
        if topk_ids.shape != (bs, self.top_k):
            raise ValueError(f"topk_ids {tuple(topk_ids.shape)} != ({bs}, {self.top_k})")
        self.raise_if_unhealthy()
        io = self._io_for(bs, hidden)
        io["x"].copy_(hidden_states, non_blocking=True)
        io["ids"].copy_(topk_ids, non_blocking=True)
        io["w"].copy_(topk_weights, non_blocking=True)
        job = self.executor.submit(self.host_bank(layer_id), io["x"], io["w"], io["ids"], io["y"],
                                   activation=self.activation, device=hidden_states.device)
        out = torch.empty_like(hidden_states)
        return io, job, out

    def decode_sync(self, pending: tuple) -> torch.Tensor:
        io, job, out = pending
        self.executor.wait(job, device=out.device)
        out.copy_(io["y"], non_blocking=True)
        return out

    def decode(self, layer_id: int, hidden_states, topk_weights, topk_ids) -> torch.Tensor:
        return self.decode_sync(self.decode_submit(layer_id, hidden_states, topk_weights, topk_ids))

    def raise_if_unhealthy(self) -> None:
        """Raises once the executor's watchdog has fired (a host read, no
        device synchronisation): callers replaying captured steps check it
        once per step, as the reference's engine does (moe/cpu_executor.py:643-656)."""
        self.executor.raise_if_unhealthy()

    def close(self, graphs_released: bool = False) -> None:
        self.executor.close(graphs_released=graphs_released)
