"""The MoE-layer module interface of FreeToken (``layers/moe.py``), backed by
the gfx950 kernels: drop-in for ``MoELayer``, ``OffloadMoELayer`` and
``make_moe_layer``.

Differences from the reference, all additive:
  * ``weight_format`` also accepts ``"ds_fp4"`` (row-major MXFP4 resident banks);
  * an optional ``shared_expert`` (``ops.ExpertBank`` with one row) is added to
    the routed output inside the expert kernels, replacing the model block's
    separate ``out + shared_experts(x)`` (``models/glm4_moe/moe.py:81-82``);
  * FP8 block scales are held as float32 (the reference allocates bf16, which
    converts exactly);
  * ``swiglu_limit`` (set through ``make_moe_layer``'s ``extra_attrs``, as the
    reference's engine does) clamps the SwiGLU of the ds_fp4 experts in both
    regimes (``layers/moe.py:473,550-573``).
TP is 1 (one GPU): ``_maybe_all_reduce`` is the identity.
"""

from __future__ import annotations

from typing import TYPE_CHECKING, Tuple

import torch

from .. import ops
from ..core import get_global_ctx, has_global_ctx
from ..moe import is_offload_moe_backend
from ..moe.fused import GROUPED_MIN_ROUTES, fused_experts_impl, fused_topk
from ..moe.offload_cache import bank_from_views

if TYPE_CHECKING:
    from ..moe.offload_cache import ExpertSlotCache

TopK = Tuple[torch.Tensor, torch.Tensor]

FP8 = torch.float8_e4m3fn


def _is_prefill(num_routes: int) -> bool:
    if has_global_ctx():
        ctx = get_global_ctx()
        if ctx._batch is not None:
            return ctx.batch.is_prefill
    return num_routes >= GROUPED_MIN_ROUTES


class MoELayer:
    def __init__(
        self,
        num_experts: int,
        top_k: int,
        hidden_size: int,
        intermediate_size: int,
        renormalize: bool = True,
        activation: str = "silu",
        apply_router_weight_on_input: bool = False,
        allocate_experts: bool = True,
        weight_format: str = "bf16",
        device: torch.device | str | None = None,
    ):
        self.num_experts = num_experts
        self.top_k = top_k
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.tp_size = 1
        self.renormalize = renormalize
        self.activation = activation
        self.apply_router_weight_on_input = apply_router_weight_on_input
        self.weight_format = weight_format
        self.shared_expert: ops.ExpertBank | None = None
        self.swiglu_limit: float | None = None
        if device is None:
            device = torch.device("cuda", torch.cuda.current_device()) if torch.cuda.is_available() else "cpu"
        self.device = torch.device(device)
        if allocate_experts:
            self._alloc_resident_experts(intermediate_size)

    def _alloc_resident_experts(self, inter: int) -> None:
        n, h, dev = self.num_experts, self.hidden_size, self.device
        if self.weight_format == "fp8_block":
            blk = 128
            self.gate_up_proj = torch.empty(n, 2 * inter, h, dtype=FP8, device=dev)
            self.gate_up_scale_inv = torch.empty(n, 2 * inter // blk, h // blk, dtype=torch.float32, device=dev)
            self.down_proj = torch.empty(n, h, inter, dtype=FP8, device=dev)
            self.down_scale_inv = torch.empty(n, h // blk, inter // blk, dtype=torch.float32, device=dev)
            return
        if self.weight_format == "ds_fp4":
            self.gate_up_proj = torch.empty(n, 2 * inter, h // 2, dtype=torch.uint8, device=dev)
            self.gate_up_scale = torch.empty(n, 2 * inter, h // 32, dtype=torch.uint8, device=dev)
            self.down_proj = torch.empty(n, h, inter // 2, dtype=torch.uint8, device=dev)
            self.down_scale = torch.empty(n, h, inter // 32, dtype=torch.uint8, device=dev)
            return
        assert self.weight_format == "bf16", f"no resident expert allocation for weight_format {self.weight_format!r}"
        self.gate_up_proj = torch.empty(n, 2 * inter, h, dtype=torch.bfloat16, device=dev)
        self.down_proj = torch.empty(n, h, inter, dtype=torch.bfloat16, device=dev)

    def bank(self) -> ops.ExpertBank:
        if self.weight_format == "fp8_block":
            return ops.ExpertBank("fp8_block", self.gate_up_proj, self.down_proj, self.gate_up_scale_inv,
                                  self.down_scale_inv)
        if self.weight_format == "ds_fp4":
            return ops.ExpertBank("mxfp4", self.gate_up_proj, self.down_proj, self.gate_up_scale, self.down_scale,
                                  swiglu_limit=float(self.swiglu_limit or 0.0))
        return ops.ExpertBank("bf16", self.gate_up_proj, self.down_proj)

    def _maybe_all_reduce(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return hidden_states

    def _run_experts(self, hidden_states, topk_weights, topk_ids) -> torch.Tensor:
        return fused_experts_impl(hidden_states, self.gate_up_proj, self.down_proj, topk_weights, topk_ids,
                                  self.activation, apply_router_weight_on_input=self.apply_router_weight_on_input)

    def _resident_gemm(self, hidden_states, topk_weights, topk_ids) -> torch.Tensor:
        """Format and phase dispatch (reference ``layers/moe.py:116-145``)."""
        prefill = _is_prefill(topk_ids.numel())
        if self.weight_format == "bf16" and self.shared_expert is None:
            if prefill:
                return self._run_experts(hidden_states, topk_weights, topk_ids)
            return ops.experts_decode(hidden_states, topk_weights, topk_ids, self.bank(),
                                      activation=self.activation,
                                      apply_router_weight_on_input=self.apply_router_weight_on_input)
        assert not self.apply_router_weight_on_input or self.weight_format == "bf16"
        fn = ops.experts_prefill if prefill else ops.experts_decode
        return fn(hidden_states, topk_weights, topk_ids, self.bank(), shared=self.shared_expert,
                  activation=self.activation)

    def routed_forward(self, hidden_states: torch.Tensor, topk_weights: torch.Tensor,
                       topk_ids: torch.Tensor) -> torch.Tensor:
        """Experts for an externally computed routing (reference ``:147-164``)."""
        return self._maybe_all_reduce(self._resident_gemm(hidden_states, topk_weights, topk_ids))

    def forward(self, hidden_states: torch.Tensor, router_logits: torch.Tensor | None = None):
        """Softmax routing + experts (reference ``:166-194``)."""
        if self.weight_format == "bf16" and self.shared_expert is None and has_global_ctx() \
                and get_global_ctx().moe_backend is not None:
            ctx = get_global_ctx()
            out = ctx.moe_backend.forward(
                hidden_states=hidden_states, w1=self.gate_up_proj, w2=self.down_proj,
                gating_output=router_logits, topk=self.top_k, renormalize=self.renormalize,
                activation=self.activation, apply_router_weight_on_input=self.apply_router_weight_on_input,
            )
            return self._maybe_all_reduce(out)
        if not _is_prefill(hidden_states.shape[0] * self.top_k) and router_logits is not None:
            # decode: router and experts in one call (router + permutation in one
            # launch for small batches)
            assert not self.apply_router_weight_on_input or self.weight_format == "bf16"
            y, _, _ = ops.experts_decode_routed(hidden_states, router_logits,
                                                ops.Router("softmax", self.top_k, self.renormalize), self.bank(),
                                                shared=self.shared_expert, activation=self.activation,
                                                apply_router_weight_on_input=self.apply_router_weight_on_input)
            return self._maybe_all_reduce(y)
        topk_weights, topk_ids = fused_topk(hidden_states, router_logits, self.top_k, self.renormalize)
        return self._maybe_all_reduce(self._resident_gemm(hidden_states, topk_weights, topk_ids))


class OffloadMoELayer(MoELayer):
    """Experts served from an expert-slot cache (reference ``:197-584``).

    Decode rewrites routed expert ids to slot ids (``ensure_experts``) and runs
    the format kernel over the slot banks; non-resident experts are reported as
    misses and skipped.  Prefill reads the first ``num_experts`` rows of the
    banks (position == expert id, the materialised-layer convention).
    """

    def __init__(self, layer_id: int, num_experts: int, top_k: int, hidden_size: int, intermediate_size: int,
                 renormalize: bool = True, activation: str = "silu", apply_router_weight_on_input: bool = False,
                 device: torch.device | str | None = None):
        super().__init__(num_experts=num_experts, top_k=top_k, hidden_size=hidden_size,
                         intermediate_size=intermediate_size, renormalize=renormalize, activation=activation,
                         apply_router_weight_on_input=apply_router_weight_on_input, allocate_experts=False,
                         device=device)
        self.layer_id = layer_id
        self.offload_cache: ExpertSlotCache | None = None

    def _views_bank(self, views) -> ops.ExpertBank:
        return bank_from_views(self.offload_cache.quant_format, views, self.swiglu_limit)

    def forward(self, hidden_states: torch.Tensor, router_logits: torch.Tensor | None = None):
        topk_weights, topk_ids = fused_topk(hidden_states, router_logits, self.top_k, self.renormalize)
        return self.routed_forward(hidden_states, topk_weights, topk_ids)

    def routed_forward(self, hidden_states: torch.Tensor, topk_weights: torch.Tensor,
                       topk_ids: torch.Tensor) -> torch.Tensor:
        if _is_prefill(topk_ids.numel()):
            out = self._prefill_routed(hidden_states, topk_weights, topk_ids)
        else:
            out = self._decode_routed(hidden_states, topk_weights, topk_ids)
        return self._maybe_all_reduce(out)

    def _decode_routed(self, hidden_states, topk_weights, topk_ids) -> torch.Tensor:
        cache = self.offload_cache
        assert cache is not None
        if cache.is_cpu_layer(self.layer_id):
            return self._decode_cpu(cache, hidden_states, topk_weights, topk_ids)
        if cache.decode_target == "hybrid":
            return self._decode_hybrid(cache, hidden_states, topk_weights, topk_ids)
        if cache.sources:
            # on-demand load (layers/moe.py:288-320): admit the missing experts,
            # gather them over PCIe, then compute on the slots
            cache.ensure_experts(self.layer_id, topk_ids)
            cache.copy_missing()
            return ops.experts_decode(hidden_states, topk_weights, topk_ids, self._views_bank(cache.bank_views()),
                                      shared=self.shared_expert, activation=self.activation)
        # ensure_experts without admission (expert ids -> slot ids, in place)
        # fused into the decode call; misses are skipped and counted
        table, stats = cache.slot_lookup(self.layer_id, topk_ids)
        return ops.experts_decode(hidden_states, topk_weights, topk_ids, self._views_bank(cache.bank_views()),
                                  shared=self.shared_expert, activation=self.activation, slot_for_id=table,
                                  stats=stats)

    def _decode_hybrid(self, cache, hidden_states, topk_weights, topk_ids) -> torch.Tensor:
        """Hybrid decode (reference ``:325-372``): the admission fetches at most
        the cache's cap of this step's misses and lists the others, by expert
        id, for the CPU; the CPU job starts before the PCIe gather and the GPU
        experts, and the two partials are added at the end.  Each route is
        computed once: the GPU skips the -1 slots, the CPU the -1 ids."""
        dec = cache.cpu_executor
        assert dec is not None, "hybrid decode needs cache.set_cpu_executor"
        cpu_ids = torch.empty_like(topk_ids)
        cache.ensure_experts_hybrid(self.layer_id, topk_ids, cpu_ids=cpu_ids)
        pending = dec.decode_submit(self.layer_id, hidden_states, topk_weights, cpu_ids)
        cache.copy_missing()
        gpu = ops.experts_decode(hidden_states, topk_weights, topk_ids, self._views_bank(cache.bank_views()),
                                 shared=self.shared_expert, activation=self.activation)
        return gpu + dec.decode_sync(pending)

    def _decode_cpu(self, cache, hidden_states, topk_weights, topk_ids) -> torch.Tensor:
        """A layer decoded on the CPU executor from its host banks (reference
        ``:307-310``); the slot cache is not touched.  A shared expert runs on
        the GPU meanwhile."""
        dec = cache.cpu_executor
        assert dec is not None, "CPU layers need cache.set_cpu_executor"
        pending = dec.decode_submit(self.layer_id, hidden_states, topk_weights, topk_ids)
        if self.shared_expert is None:
            return dec.decode_sync(pending)
        shared = ops.experts_decode(hidden_states, topk_weights, torch.full_like(topk_ids, -1),
                                    self._views_bank(cache.bank_views()), shared=self.shared_expert,
                                    activation=self.activation)
        return shared + dec.decode_sync(pending)

    def _prefill_routed(self, hidden_states, topk_weights, topk_ids) -> torch.Tensor:
        """Prefill movement (reference ``:374-423``): with the double buffer,
        layer l+1's host copy is started behind this layer's GEMMs; with host
        sources and no overlap, the layer is materialized at slot == expert id
        and gathered first; otherwise the first E slots are taken to hold the
        layer.  In all cases position == expert id, so the ids pass unmapped."""
        cache = self.offload_cache
        assert cache is not None
        if cache.prefill_overlap:
            if self.layer_id == 0:
                cache.begin_prefill()
            cache.prefetch_prefill_layer(self.layer_id)
            cache.prefetch_prefill_layer(self.layer_id + 1)
            bank = self._views_bank(cache.wait_prefill_layer(self.layer_id))
            out = ops.experts_prefill(hidden_states, topk_weights, topk_ids, bank, shared=self.shared_expert,
                                      activation=self.activation)
            cache.release_prefill_layer(self.layer_id)
            return out
        if cache.sources:
            cache.materialize_layer(self.layer_id)
            cache.copy_missing()
        bank = self._views_bank(cache.bank_views(self.num_experts))
        return ops.experts_prefill(hidden_states, topk_weights, topk_ids, bank, shared=self.shared_expert,
                                   activation=self.activation)


def make_moe_layer(
    config,
    *,
    layer_id: int | None = None,
    activation: str = "silu",
    weight_format: str = "bf16",
    renormalize: bool | None = None,
    apply_router_weight_on_input: bool = False,
    num_experts: int | None = None,
    top_k: int | None = None,
    hidden_size: int | None = None,
    intermediate_size: int | None = None,
    resident_cls: type[MoELayer] | None = None,
    offload_cls: type[OffloadMoELayer] | None = None,
    extra_attrs: dict | None = None,
) -> MoELayer:
    """Construction seam (reference ``layers/moe.py:587-636``): offload family ->
    ``OffloadMoELayer``, else ``MoELayer``; geometry from ``config``."""
    offload = is_offload_moe_backend(getattr(config, "moe_backend", "fused"))
    layer_cls = (offload_cls or OffloadMoELayer) if offload else (resident_cls or MoELayer)
    kwargs = dict(
        num_experts=num_experts if num_experts is not None else config.num_experts,
        top_k=top_k if top_k is not None else config.num_experts_per_tok,
        hidden_size=hidden_size if hidden_size is not None else config.hidden_size,
        intermediate_size=intermediate_size if intermediate_size is not None else config.moe_intermediate_size,
        renormalize=renormalize if renormalize is not None else config.norm_topk_prob,
        activation=activation,
        apply_router_weight_on_input=apply_router_weight_on_input,
    )
    if offload:
        assert layer_id is not None, "offload MoE backends need the layer_id"
        kwargs["layer_id"] = layer_id
    else:
        kwargs["weight_format"] = weight_format
    layer = layer_cls(**kwargs)
    for name, value in (extra_attrs or {}).items():
        setattr(layer, name, value)
    return layer


__all__ = ["MoELayer", "OffloadMoELayer", "make_moe_layer", "TopK"]
