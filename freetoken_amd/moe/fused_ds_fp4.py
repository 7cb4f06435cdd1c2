"""Row-major MXFP4 ("ds_fp4") routed experts (reference ``moe/fused_ds_fp4.py``):
packed e2m1 [S, N, K/2] (low nibble = even k) with e8m0 scales [S, N, K/32].

Decode keeps bf16 activations (W4A16, the layout's own GEMV numerics,
``kernel/triton/dsv4/fused_moe.py:15-16``); the DeepSeek-V4 specific FP8
activation round trip of the reference's decode (``:119,127``) is not applied.
Prefill FP8-round-trips both GEMM inputs with per-128 power-of-two scales, as
``routed_experts_fp4_prefill`` does (``:181-235``), and runs them on the
MX-scaled FP8 x FP4 MFMA.  ``swiglu_limit`` > 0 clamps the SwiGLU inputs,
``silu(min(gate, L)) * clamp(up, -L, L)`` on the bf16 gate and up values
(``fused_swiglu``, ``kernel/triton/dsv4/fused_moe.py:121-141``), in the gate/up
epilogue of both regimes; 0 (or None) leaves them unclamped.
"""

from __future__ import annotations

import torch

from .. import ops


def _bank(gu_p, gu_s, dn_p, dn_s, swiglu_limit) -> ops.ExpertBank:
    lim = float(swiglu_limit or 0.0)
    if not lim >= 0.0 or lim == float("inf"):
        raise ValueError(f"swiglu_limit must be finite and >= 0, got {swiglu_limit!r}")
    return ops.ExpertBank("mxfp4", gu_p, dn_p, gu_s.view(torch.uint8), dn_s.view(torch.uint8), swiglu_limit=lim)


def routed_experts_fp4(
    x: torch.Tensor,
    slots: torch.Tensor,
    topk_weights: torch.Tensor,
    gate_up_packed: torch.Tensor,
    gate_up_scale: torch.Tensor,
    down_packed: torch.Tensor,
    down_scale: torch.Tensor,
    swiglu_limit: float = 0.0,
    shared: ops.ExpertBank | None = None,
) -> torch.Tensor:
    """Decode: routed output summed over the top-k routes (+ shared expert)."""
    return ops.experts_decode(x, topk_weights, slots,
                              _bank(gate_up_packed, gate_up_scale, down_packed, down_scale, swiglu_limit),
                              shared=shared)


def routed_experts_fp4_prefill(
    x: torch.Tensor,
    slots: torch.Tensor,
    topk_weights: torch.Tensor,
    gate_up_packed: torch.Tensor,
    gate_up_scale: torch.Tensor,
    down_packed: torch.Tensor,
    down_scale: torch.Tensor,
    swiglu_limit: float,
    num_rows: int,
    shared: ops.ExpertBank | None = None,
) -> torch.Tensor:
    """Prefill: grouped MX-scaled MFMA over the first ``num_rows`` bank rows."""
    bank = _bank(gate_up_packed[:num_rows], gate_up_scale[:num_rows], down_packed[:num_rows], down_scale[:num_rows],
                 swiglu_limit)
    return ops.experts_prefill(x, topk_weights, slots, bank, shared=shared)


__all__ = ["routed_experts_fp4", "routed_experts_fp4_prefill"]
