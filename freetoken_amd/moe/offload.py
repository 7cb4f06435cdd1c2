"""Offload-family backend markers (reference ``moe/offload.py``,
``moe/cpu_offload.py``): the work is done by ``OffloadMoELayer``, never by the
backend object."""

from __future__ import annotations

import torch

from .base import BaseMoeBackend


class OffloadMoeBackend(BaseMoeBackend):
    def forward(self, hidden_states: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                gating_output: torch.Tensor, topk: int, renormalize: bool, activation: str,
                apply_router_weight_on_input: bool) -> torch.Tensor:
        raise RuntimeError("Offload MoE is handled by OffloadMoELayer")


class CpuOffloadMoeBackend(BaseMoeBackend):
    """Decode on the CPU executor from the pinned host banks."""

    def forward(self, hidden_states, w1, w2, gating_output, topk, renormalize, activation,
                apply_router_weight_on_input) -> torch.Tensor:
        raise RuntimeError("CPU-offload MoE is handled by OffloadMoELayer")


class HybridMoeBackend(BaseMoeBackend):
    """Decode split between the GPU slot cache and the CPU executor."""

    def forward(self, hidden_states, w1, w2, gating_output, topk, renormalize, activation,
                apply_router_weight_on_input) -> torch.Tensor:
        raise RuntimeError("Hybrid MoE is handled by OffloadMoELayer")
