"""Block-FP8 (e4m3 + 128x128 scales) routed experts (reference
``moe/fused_fp8_block.py``): W8A8 grouped GEMM for prefill, W8A16
expert-major GEMV for decode.  ``topk_ids`` index bank rows (experts when
resident, cache slots when offloaded)."""

from __future__ import annotations

import torch

from .. import ops


def _bank(gate_up, gate_up_scale, down, down_scale) -> ops.ExpertBank:
    return ops.ExpertBank("fp8_block", gate_up, down, gate_up_scale, down_scale)


def fused_experts_fp8_block(
    hidden_states, gate_up, gate_up_scale, down, down_scale,
    topk_weights, topk_ids, num_experts, activation="silu",
    apply_router_weight_on_input=False, shared: ops.ExpertBank | None = None,
):
    """Prefill W8A8 (reference ``:16-29`` -> ``fp8_blockscale_moe.py:218-256``);
    ``num_experts`` rows of the banks take part (position == expert id)."""
    assert not apply_router_weight_on_input
    assert activation == "silu"
    bank = _bank(gate_up[:num_experts], gate_up_scale[:num_experts], down[:num_experts], down_scale[:num_experts])
    return ops.experts_prefill(hidden_states, topk_weights, topk_ids, bank, shared=shared)


def fused_experts_decode_fp8_block(
    hidden_states, gate_up, gate_up_scale, down, down_scale,
    topk_weights, topk_ids, activation="silu", apply_router_weight_on_input=False,
    shared: ops.ExpertBank | None = None,
):
    """Decode W8A16 (reference ``:32-44`` -> ``fp8_blockscale_moe.py:99-123``)."""
    assert not apply_router_weight_on_input
    assert activation == "silu"
    return ops.experts_decode(hidden_states, topk_weights, topk_ids,
                              _bank(gate_up, gate_up_scale, down, down_scale), shared=shared)


__all__ = ["fused_experts_fp8_block", "fused_experts_decode_fp8_block"]
