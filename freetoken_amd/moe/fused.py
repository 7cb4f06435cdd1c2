"""Resident-expert MoE entry points with the reference's names and contracts
(``moe/fused.py`` of FreeToken), backed by the gfx950 kernels of libftmoe.so.

Routing: ``fused_topk`` (softmax) and ``grouped_topk`` (DeepSeek-V3 grouped
sigmoid, the router of ``models/glm4_moe/moe.py:53-75``).  Permutation:
``moe_align_block_size`` (stable order).  Experts: ``fused_experts_impl``
(grouped, overwrites ``hidden_states``) and ``fused_experts_decode_impl``
(allocates its output).
"""

from __future__ import annotations

from typing import Tuple

import torch

from .. import ops
from . import BaseMoeBackend

# Above this many routes the grouped (prefill) kernels beat the expert-major
# GEMV; below it the GEMV reads each touched expert exactly once.
GROUPED_MIN_ROUTES = 4096


def _mask_padded(topk_ids: torch.Tensor, num_token_non_padded: torch.Tensor | None) -> None:
    if num_token_non_padded is not None:
        idx = torch.arange(0, topk_ids.shape[0], device=topk_ids.device)
        topk_ids[idx >= num_token_non_padded, :] = -1


def fused_topk(
    hidden_states: torch.Tensor,
    gating_output: torch.Tensor,
    topk: int,
    renormalize: bool,
    num_token_non_padded: torch.Tensor | None = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Softmax top-k routing (reference ``moe/fused.py:38-85``): weights fp32
    [M,k], ids int32 [M,k], ties to the lower expert index."""
    assert hidden_states.shape[0] == gating_output.shape[0], "Number of tokens mismatch"
    topk_weights, topk_ids = ops.route_softmax_topk(gating_output.contiguous(), topk, renormalize)
    _mask_padded(topk_ids, num_token_non_padded)
    return topk_weights, topk_ids


def grouped_topk(
    hidden_states: torch.Tensor,
    gating_output: torch.Tensor,
    topk: int,
    renormalize: bool,
    num_expert_group: int,
    topk_group: int,
    correction_bias: torch.Tensor | None = None,
    routed_scaling_factor: float = 1.0,
    num_token_non_padded: torch.Tensor | None = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """DeepSeek-V3 ``noaux_tc`` routing (reference ``models/glm4_moe/moe.py:53-75``):
    sigmoid scores, bias for selection only, group-limited top-k, renorm, scale."""
    assert hidden_states.shape[0] == gating_output.shape[0], "Number of tokens mismatch"
    topk_weights, topk_ids = ops.route_grouped_sigmoid(
        gating_output, correction_bias, num_expert_group, topk_group, topk, renormalize, routed_scaling_factor
    )
    _mask_padded(topk_ids, num_token_non_padded)
    return topk_weights, topk_ids


def moe_align_block_size(
    topk_ids: torch.Tensor, block_size: int, num_experts: int
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Reference ``moe/fused.py:88-158`` with the canonical stable order inside
    each expert (the reference's atomic order is unspecified)."""
    assert topk_ids.dtype == torch.int32
    return ops.align(topk_ids.contiguous(), block_size, num_experts)


def _check_bf16_experts(hidden_states, w1, w2, topk_weights, topk_ids, activation):
    assert hidden_states.shape[1] == w1.shape[2], "Hidden size mismatch"
    assert w1.shape[0] == w2.shape[0], "Expert cache size mismatch"
    assert w1.shape[1] == 2 * w2.shape[2], "Intermediate size mismatch"
    assert w2.shape[1] == hidden_states.shape[1], "Output hidden size mismatch"
    assert topk_weights.shape == topk_ids.shape, "topk shape mismatch"
    assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
    assert w1.is_contiguous(), "Expert weights1 must be contiguous"
    assert w2.is_contiguous(), "Expert weights2 must be contiguous"
    assert hidden_states.dtype == torch.bfloat16, "the gfx950 path computes in bf16"
    assert w1.dtype == hidden_states.dtype and w2.dtype == hidden_states.dtype
    assert topk_weights.dtype == torch.float32
    assert topk_ids.dtype == torch.int32
    if activation not in ("silu", "gelu", "gelu_tanh"):
        raise ValueError(f"Unsupported activation: {activation}")


def fused_experts_impl(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
) -> torch.Tensor:
    """bf16 experts; returns ``hidden_states`` itself, overwritten with the routed
    output (reference contract, ``moe/fused.py:242-245,333-337``)."""
    _check_bf16_experts(hidden_states, w1, w2, topk_weights, topk_ids, activation)
    bank = ops.ExpertBank("bf16", w1, w2)
    if topk_ids.numel() >= GROUPED_MIN_ROUTES and not apply_router_weight_on_input:
        out = ops.experts_prefill(hidden_states, topk_weights, topk_ids, bank, activation=activation)
    else:
        out = ops.experts_decode(hidden_states, topk_weights, topk_ids, bank, activation=activation,
                                 apply_router_weight_on_input=apply_router_weight_on_input)
    hidden_states.copy_(out)
    return hidden_states


def fused_experts_decode_impl(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
) -> torch.Tensor:
    """bf16 decode experts (reference ``moe/fused.py:340-423``): ids index bank
    rows (experts or cache slots); the output is freshly allocated."""
    _check_bf16_experts(hidden_states, w1, w2, topk_weights, topk_ids, activation)
    assert topk_weights.is_contiguous(), "topk_weights must be contiguous"
    assert topk_ids.is_contiguous(), "topk_ids must be contiguous"
    return ops.experts_decode(hidden_states, topk_weights, topk_ids, ops.ExpertBank("bf16", w1, w2),
                              activation=activation, apply_router_weight_on_input=apply_router_weight_on_input)


class FusedMoe(BaseMoeBackend):
    """Backend ``"fused"`` (reference ``moe/fused.py:426-452``)."""

    def forward(
        self,
        hidden_states: torch.Tensor,
        w1: torch.Tensor,
        w2: torch.Tensor,
        gating_output: torch.Tensor,
        topk: int,
        renormalize: bool,
        activation: str = "silu",
        apply_router_weight_on_input: bool = False,
    ) -> torch.Tensor:
        topk_weights, topk_ids = fused_topk(hidden_states, gating_output, topk, renormalize)
        return fused_experts_impl(hidden_states, w1, w2, topk_weights, topk_ids, activation,
                                  apply_router_weight_on_input=apply_router_weight_on_input)
