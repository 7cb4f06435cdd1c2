"""Torch-tensor wrappers over the C ABI (device memory and streams only).

Each wrapper validates dtypes/shapes like the reference's asserts, hands raw
device pointers and the current HIP stream to ``libftmoe.so`` and returns
torch tensors.  There is no CPU path: tensors must live on a ROCm device.
"""

from __future__ import annotations

import ctypes
import math
import os
import weakref
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import check, lib


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("ftmoe ops take device (ROCm) tensors; no CPU fallback exists")
        if t is not None and not t.is_contiguous():
            raise ValueError("ftmoe ops take contiguous tensors")


# --------------------------------------------------------------------------- routing


def route_softmax_topk(logits: torch.Tensor, topk: int, renormalize: bool):
    """Softmax top-k router (``fused_topk`` contract): returns (w fp32, ids int32)."""
    _require_gpu(logits)
    if logits.dtype == torch.float32:
        dt = _lib.DTYPE_F32
    elif logits.dtype == torch.bfloat16:
        dt = _lib.DTYPE_BF16
    else:
        logits = logits.float()
        dt = _lib.DTYPE_F32
    m, e = logits.shape
    w = torch.empty((m, topk), dtype=torch.float32, device=logits.device)
    ids = torch.empty((m, topk), dtype=torch.int32, device=logits.device)
    check(
        lib().ftmoe_route_softmax_topk(_ptr(logits), dt, m, e, topk, int(renormalize), _ptr(w), _ptr(ids),
                                       _stream(logits.device)),
        "route_softmax_topk",
    )
    return w, ids


def route_grouped_sigmoid(logits: torch.Tensor, bias: torch.Tensor | None, n_group: int, topk_group: int,
                          topk: int, renormalize: bool, scale: float):
    """DeepSeek-V3 grouped sigmoid router: returns (w fp32, ids int32)."""
    logits = logits.float().contiguous()
    if bias is not None:
        bias = bias.float().contiguous()
    _require_gpu(logits, bias)
    m, e = logits.shape
    w = torch.empty((m, topk), dtype=torch.float32, device=logits.device)
    ids = torch.empty((m, topk), dtype=torch.int32, device=logits.device)
    check(
        lib().ftmoe_route_grouped_sigmoid(_ptr(logits), _ptr(bias), m, e, n_group, topk_group, topk,
                                          int(renormalize), float(scale), _ptr(w), _ptr(ids),
                                          _stream(logits.device)),
        "route_grouped_sigmoid",
    )
    return w, ids


# --------------------------------------------------------------------------- align / slots


def align_sizes(numel: int, num_experts: int, block_size: int) -> tuple[int, int]:
    mp, mb = ctypes.c_int(), ctypes.c_int()
    lib().ftmoe_align_sizes(numel, num_experts, block_size, ctypes.byref(mp), ctypes.byref(mb))
    return mp.value, mb.value


def align(topk_ids: torch.Tensor, block_size: int, num_experts: int):
    """moe_align_block_size with the canonical stable order."""
    if topk_ids.dtype != torch.int32:
        raise ValueError("topk_ids must be int32")
    _require_gpu(topk_ids)
    numel = topk_ids.numel()
    mp, mb = align_sizes(numel, num_experts, block_size)
    dev = topk_ids.device
    sorted_ids = torch.empty((mp,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty((mb,), dtype=torch.int32, device=dev)
    ntpp = torch.empty((1,), dtype=torch.int32, device=dev)
    check(
        lib().ftmoe_align(_ptr(topk_ids), numel, num_experts, block_size, _ptr(sorted_ids), _ptr(expert_ids),
                          _ptr(ntpp), _stream(dev)),
        "align",
    )
    return sorted_ids, expert_ids, ntpp


def slot_map(topk_ids: torch.Tensor, slot_for_id: torch.Tensor, out: torch.Tensor | None = None,
             miss_mask: torch.Tensor | None = None, stats: torch.Tensor | None = None) -> torch.Tensor:
    """Expert id -> cache slot (-1 = not resident); ``out`` may be ``topk_ids``."""
    if topk_ids.dtype != torch.int32 or slot_for_id.dtype != torch.int32:
        raise ValueError("topk_ids and slot_for_id must be int32")
    _require_gpu(topk_ids, slot_for_id, out, miss_mask, stats)
    if out is None:
        out = torch.empty_like(topk_ids)
    if stats is not None and stats.dtype != torch.int64:
        raise ValueError("stats must be int64[4]")
    check(
        lib().ftmoe_slot_map(_ptr(topk_ids), topk_ids.numel(), _ptr(slot_for_id), slot_for_id.numel(), _ptr(out),
                             _ptr(miss_mask), _ptr(stats), _stream(topk_ids.device)),
        "slot_map",
    )
    return out


def route_histogram(topk_ids: torch.Tensor, freq: torch.Tensor) -> torch.Tensor:
    """freq[e] += count of e in ``topk_ids`` (int32; ids outside [0, len(freq))
    skipped); ``freq`` int64 [E] accumulates on the device (see ftmoe_route_histogram)."""
    if topk_ids.dtype != torch.int32 or freq.dtype != torch.int64:
        raise ValueError("topk_ids must be int32 and freq int64")
    _require_gpu(topk_ids, freq)
    check(lib().ftmoe_route_histogram(_ptr(topk_ids), topk_ids.numel(), freq.numel(), _ptr(freq),
                                      _stream(topk_ids.device)), "route_histogram")
    return freq


def lru_ensure(expert_ids: torch.Tensor, layer_id: int, slot_for_id: torch.Tensor, id_of_slot: torch.Tensor,
               usage: torch.Tensor, step: torch.Tensor, evict_slots: torch.Tensor, src_indices: torch.Tensor,
               num_indices: torch.Tensor, num_missing: torch.Tensor, recency: torch.Tensor | None = None,
               max_fetch: int = -1, stats: torch.Tensor | None = None, fetch_fraction: float | None = 0.0,
               cpu_ids: torch.Tensor | None = None, unserved: torch.Tensor | None = None) -> torch.Tensor:
    """LRU admission of a call's experts into the slot cache; ``expert_ids``
    (int32) are rewritten to slots in place (see ftmoe_lru_ensure).
    ``slot_for_id`` [L, E] int32, ``id_of_slot`` [S] int32, ``usage`` [S] and
    ``step`` [1] int64; ``recency`` (int64 [E] of this layer) selects the
    most-recent-first miss order.  ``fetch_fraction`` > 0 replaces the
    ``max_fetch`` cap with the bandwidth-matched share of the misses, in Q16
    as the reference rounds it (moe/offload_kernels.py:58); ``cpu_ids``
    (int32, shaped like ``expert_ids``) receives the unfetched misses' expert
    ids and -1 elsewhere.  At most as many misses are admitted as there are
    slots that hold no expert of this call; ``unserved`` (int64 [1]) accumulates
    the misses left without a slot for that reason.  A ``fetch_fraction`` of
    None (no measured rates) means the fixed ``max_fetch`` cap."""
    frac_q16 = 0 if fetch_fraction is None else min(1 << 16, max(0, round(fetch_fraction * (1 << 16))))
    i32 = (expert_ids, slot_for_id, id_of_slot, evict_slots, src_indices, num_indices, num_missing)
    if cpu_ids is not None and (cpu_ids.dtype != torch.int32 or cpu_ids.shape != expert_ids.shape
                                or not cpu_ids.is_contiguous()):
        raise ValueError("cpu_ids must be contiguous int32 shaped like expert_ids")
    if any(t.dtype != torch.int32 for t in i32):
        raise ValueError("ids, tables, evict/src lists and counts must be int32")
    if usage.dtype != torch.int64 or step.dtype != torch.int64 or (recency is not None and recency.dtype != torch.int64):
        raise ValueError("usage, step and recency must be int64")
    if stats is not None and stats.dtype != torch.int64:
        raise ValueError("stats must be int64[4]")
    if unserved is not None and unserved.dtype != torch.int64:
        raise ValueError("unserved must be int64[1]")
    _require_gpu(*i32, usage, step, recency, stats, cpu_ids, unserved)
    if not expert_ids.is_contiguous():
        raise ValueError("expert_ids must be contiguous")
    num_layers, num_experts = slot_for_id.shape
    if recency is not None and recency.numel() != num_experts:
        raise ValueError("recency must hold one entry per expert of the layer")
    check(
        lib().ftmoe_lru_ensure(_ptr(expert_ids), expert_ids.numel(), layer_id, num_layers, num_experts,
                               _ptr(slot_for_id), _ptr(id_of_slot), _ptr(usage), _ptr(step), id_of_slot.numel(),
                               _ptr(recency), max_fetch, frac_q16, _ptr(evict_slots), _ptr(src_indices),
                               min(evict_slots.numel(), src_indices.numel()), _ptr(num_indices), _ptr(num_missing),
                               _ptr(cpu_ids), _ptr(stats), _ptr(unserved), _stream(expert_ids.device)),
        "lru_ensure",
    )
    return expert_ids


def alloc_pinned_tensor(*shape: int, dtype: torch.dtype) -> torch.Tensor:
    """Exact-size pinned host tensor (hipHostMalloc; reference
    ``kernel/pinned.py:42-45``), freed when its last view is gone.  torch's
    ``pin_memory`` rounds each allocation up to a power of two."""
    nbytes = math.prod(shape) * torch.empty((), dtype=dtype).element_size()
    ptr = ctypes.c_void_p()
    check(lib().ftmoe_host_alloc(nbytes, ctypes.byref(ptr)), "host_alloc")
    addr = ptr.value
    raw = (ctypes.c_uint8 * max(nbytes, 1)).from_address(addr)
    # freed with its last view; not at interpreter exit, where the HIP runtime may be gone first
    weakref.finalize(raw, lib().ftmoe_host_free, addr).atexit = False
    return torch.from_numpy(np.frombuffer(raw, dtype=np.uint8))[:nbytes].view(dtype).view(shape)


def materialize_layer(layer_id: int, slot_for_id: torch.Tensor, id_of_slot: torch.Tensor, usage: torch.Tensor,
                      step: torch.Tensor, evict_slots: torch.Tensor, src_indices: torch.Tensor,
                      num_indices: torch.Tensor) -> None:
    """Places every expert of ``layer_id`` at slot == expert id and stages the
    whole layer for ``fetch_experts`` (see ftmoe_materialize_layer)."""
    num_layers, num_experts = slot_for_id.shape
    if evict_slots.numel() < num_experts or src_indices.numel() < num_experts:
        raise ValueError("evict_slots / src_indices must hold num_experts entries")
    for t in (slot_for_id, id_of_slot, evict_slots, src_indices, num_indices):
        if t.dtype != torch.int32:
            raise ValueError("tables, lists and count must be int32")
    if usage.dtype != torch.int64 or step.dtype != torch.int64:
        raise ValueError("usage and step must be int64")
    _require_gpu(slot_for_id, id_of_slot, usage, step, evict_slots, src_indices, num_indices)
    check(lib().ftmoe_materialize_layer(layer_id, num_layers, num_experts, _ptr(slot_for_id), _ptr(id_of_slot),
                                        _ptr(usage), _ptr(step), id_of_slot.numel(), _ptr(evict_slots),
                                        _ptr(src_indices), _ptr(num_indices), _stream(slot_for_id.device)),
          "materialize_layer")


def release_slots(slot_begin: int, slot_end: int, slot_for_id: torch.Tensor, id_of_slot: torch.Tensor,
                  usage: torch.Tensor) -> None:
    """Empties slots [slot_begin, slot_end) and unmaps their experts (see
    ftmoe_release_slots)."""
    num_layers, num_experts = slot_for_id.shape
    if slot_for_id.dtype != torch.int32 or id_of_slot.dtype != torch.int32 or usage.dtype != torch.int64:
        raise ValueError("slot tables int32, usage int64")
    _require_gpu(slot_for_id, id_of_slot, usage)
    check(lib().ftmoe_release_slots(slot_begin, slot_end, num_layers, num_experts, _ptr(slot_for_id),
                                    _ptr(id_of_slot), _ptr(usage), id_of_slot.numel(), _stream(slot_for_id.device)),
          "release_slots")


def fetch_experts(host_rows, slot_banks, evict_slots: torch.Tensor, src_indices: torch.Tensor,
                  num_indices: torch.Tensor, max_entries: int | None = None) -> None:
    """Copies the admitted experts' rows from pinned host tensors (one per
    bank, ``[E, ...]`` of one layer) into the slot banks (``[S, ...]`` on the
    device), for the first ``num_indices`` entries (see ftmoe_fetch_experts).
    A source may also be a device tensor (device-to-device gather)."""
    if len(host_rows) != len(slot_banks) or not host_rows:
        raise ValueError("one host tensor per slot bank")
    _require_gpu(evict_slots, src_indices, num_indices, *slot_banks)
    banks = (_lib.FtmoeFetchBank * len(host_rows))()
    for b, (h, d) in enumerate(zip(host_rows, slot_banks)):
        if not h.is_contiguous() or (h.device.type == "cpu" and not h.is_pinned()):
            raise ValueError("sources must be contiguous: pinned CPU tensors or device tensors")
        if not d.is_contiguous():
            raise ValueError("slot banks must be contiguous")
        row = h[0].numel() * h.element_size()
        if row != d[0].numel() * d.element_size():
            raise ValueError(f"bank {b}: host row {row} B != slot row {d[0].numel() * d.element_size()} B")
        banks[b] = _lib.FtmoeFetchBank(h.data_ptr(), d.data_ptr(), row)
    n = min(evict_slots.numel(), src_indices.numel()) if max_entries is None else max_entries
    check(
        lib().ftmoe_fetch_experts(banks, len(host_rows), _ptr(evict_slots), _ptr(src_indices), _ptr(num_indices), n,
                                  _stream(evict_slots.device)),
        "fetch_experts",
    )


def prefill_hit_compact(slot_row: torch.Tensor, threshold: int, dst_base: int, dst_rows: torch.Tensor,
                        src_rows: torch.Tensor, num_hits: torch.Tensor) -> None:
    """Lists the experts of one layer resident at slots >= ``threshold`` as
    (buffer row ``dst_base + e``, slot) entries for a device-to-device gather
    (see ftmoe_prefill_hit_compact)."""
    for t in (slot_row, dst_rows, src_rows, num_hits):
        if t.dtype != torch.int32:
            raise ValueError("slot row, lists and count must be int32")
    _require_gpu(slot_row, dst_rows, src_rows, num_hits)
    n = slot_row.numel()
    if dst_rows.numel() < n or src_rows.numel() < n:
        raise ValueError("dst_rows / src_rows must hold one entry per expert")
    check(lib().ftmoe_prefill_hit_compact(_ptr(slot_row), n, threshold, dst_base, _ptr(dst_rows), _ptr(src_rows),
                                          _ptr(num_hits), _stream(slot_row.device)), "prefill_hit_compact")


def act_quant_fp8(x: torch.Tensor, mode: int = 0):
    """Per-token per-128 FP8 quantisation of bf16 rows: mode 0 -> float32 scales
    (amax/448), mode 1 -> uint8 e8m0 power-of-two scale codes."""
    if x.dtype != torch.bfloat16:
        raise ValueError("x must be bfloat16")
    _require_gpu(x)
    rows, k = x.shape
    q = torch.empty((rows, k), dtype=torch.uint8, device=x.device)
    sdt = torch.float32 if mode == 0 else torch.uint8
    s = torch.empty((rows, k // 128), dtype=sdt, device=x.device)
    check(lib().ftmoe_act_quant_fp8(_ptr(x), rows, k, mode, _ptr(q), _ptr(s), _stream(x.device)), "act_quant_fp8")
    return q, s


# --------------------------------------------------------------------------- expert banks

_FORMATS = {"bf16": _lib.FMT_BF16, "fp8_block": _lib.FMT_FP8_B128, "mxfp4": _lib.FMT_MXFP4}


@dataclass
class ExpertBank:
    """Device tensors of one expert bank (see ftmoe_bank in include/ftmoe.h).

    fmt "bf16": gate_up [S,2I,H] bf16, down [S,H,I] bf16.
    fmt "fp8_block": e4m3 (float8_e4m3fn or uint8) gate_up/down with float32
    (or bf16, converted once) 128x128 block scales.
    fmt "mxfp4": uint8 packed [S,2I,H/2] / [S,H,I/2] with uint8 e8m0 scales
    [S,2I,H/32] / [S,H,I/32].
    ``swiglu_limit`` > 0 makes the activation the clamped SwiGLU
    ``silu(min(gate, L)) * clamp(up, -L, L)`` (DeepSeek-V4's experts,
    ``moe/fused_ds_fp4.py:105-124``); 0 leaves it unclamped.
    """

    fmt: str
    gate_up: torch.Tensor
    down: torch.Tensor
    gate_up_scale: torch.Tensor | None = None
    down_scale: torch.Tensor | None = None
    swiglu_limit: float = 0.0

    def __post_init__(self):
        if self.fmt not in _FORMATS:
            raise ValueError(f"unknown expert format {self.fmt!r}")
        if self.fmt == "fp8_block":
            for name in ("gate_up_scale", "down_scale"):
                s = getattr(self, name)
                if s is None:
                    raise ValueError(f"fp8_block bank needs {name}")
                if s.dtype != torch.float32:
                    setattr(self, name, s.float().contiguous())
        if self.fmt == "bf16" and self.gate_up.dtype != torch.bfloat16:
            raise ValueError("bf16 bank weights must be torch.bfloat16")

    @property
    def num_rows(self) -> int:
        return self.gate_up.shape[0]

    @property
    def hidden(self) -> int:
        return self.down.shape[1]

    @property
    def inter(self) -> int:
        return self.gate_up.shape[1] // 2

    def host_cstruct(self) -> _lib.FtmoeBank:
        """The bank as ftmoe_bank with host pointers (the CPU executor's banks:
        contiguous CPU tensors, pinned when the stream-ordered path reads them)."""
        for t in (self.gate_up, self.down, self.gate_up_scale, self.down_scale):
            if t is not None and (t.device.type != "cpu" or not t.is_contiguous()):
                raise ValueError("host banks are contiguous CPU tensors")
        return _lib.FtmoeBank(
            _FORMATS[self.fmt], self.num_rows, self.hidden, self.inter,
            self.gate_up.data_ptr(), _ptr(self.gate_up_scale), self.down.data_ptr(), _ptr(self.down_scale),
            float(self.swiglu_limit or 0.0),
        )

    def cstruct(self) -> _lib.FtmoeBank:
        _require_gpu(self.gate_up, self.down, self.gate_up_scale, self.down_scale)
        return _lib.FtmoeBank(
            _FORMATS[self.fmt], self.num_rows, self.hidden, self.inter,
            _ptr(self.gate_up), _ptr(self.gate_up_scale), _ptr(self.down), _ptr(self.down_scale),
            float(self.swiglu_limit or 0.0),
        )


class _Workspace:
    """Per-device scratch buffer, grown on demand (never during graph capture:
    size it with a warm-up call at the largest batch first).

    A captured graph keeps the raw address of the buffer it was captured
    with.  A buffer handed to a capture is therefore never given back to the
    allocator when a later, larger eager call (a prefill after the decode
    graphs were captured) grows the workspace: it is retired and kept, so
    replays of those graphs still write memory they own.  ``release_retired``
    frees the retired buffers once the graphs that used them are gone."""

    def __init__(self):
        self.buf: dict[int, torch.Tensor] = {}
        self.captured: dict[int, bool] = {}
        self.retired: dict[int, list[torch.Tensor]] = {}

    def get(self, device: torch.device, nbytes: int) -> torch.Tensor:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        cur = self.buf.get(idx)
        capturing = torch.cuda.is_current_stream_capturing()
        if cur is None or cur.numel() < nbytes:
            if capturing:
                raise RuntimeError("ftmoe workspace must be sized before graph capture (run one eager call)")
            if cur is not None and self.captured.get(idx):
                self.retired.setdefault(idx, []).append(cur)
            cur = torch.empty((max(nbytes, 1 << 20),), dtype=torch.uint8, device=device)
            self.buf[idx] = cur
            self.captured[idx] = False
        if capturing:
            self.captured[idx] = True
        return cur

    def release_retired(self, device: torch.device | None = None) -> None:
        for idx in ([device.index] if device is not None else list(self.retired)):
            self.retired.pop(idx, None)


_WS = _Workspace()


def release_retired_workspaces(device: torch.device | None = None) -> None:
    """Frees workspace buffers superseded after a graph capture used them; call
    only once every graph captured with them has been destroyed."""
    _WS.release_retired(device)


def experts_decode(x: torch.Tensor, topk_w: torch.Tensor, topk_ids: torch.Tensor, bank: ExpertBank,
                   shared: ExpertBank | None = None, activation: str = "silu",
                   apply_router_weight_on_input: bool = False, out: torch.Tensor | None = None,
                   slot_for_id: torch.Tensor | None = None, miss_mask: torch.Tensor | None = None,
                   stats: torch.Tensor | None = None) -> torch.Tensor:
    """Decode-regime experts (+ optional shared expert) for a precomputed routing.

    With ``slot_for_id`` the bank rows are expert-cache slots and ``topk_ids``
    holds expert ids: they are rewritten to slot ids in place (as ``slot_map``,
    with the optional ``miss_mask`` and accumulated ``stats``) by the same call.
    """
    if x.dtype != torch.bfloat16:
        raise ValueError("hidden_states must be bfloat16")
    if topk_w.dtype != torch.float32 or topk_ids.dtype != torch.int32:
        raise ValueError("topk_weights must be float32 and topk_ids int32")
    if topk_w.shape != topk_ids.shape:
        raise ValueError("topk shape mismatch")
    if activation not in _lib.ACT:
        raise ValueError(f"Unsupported activation: {activation}")
    _require_gpu(x, topk_w, topk_ids)
    m, k = topk_ids.shape
    if x.shape[0] != m:
        raise ValueError("Number of tokens mismatch")
    b = bank.cstruct()
    sb = shared.cstruct() if shared is not None else None
    bp = ctypes.byref(b)
    sp = ctypes.byref(sb) if sb is not None else None
    nbytes = lib().ftmoe_experts_decode_workspace(m, k, bp, sp)
    ws = _WS.get(x.device, nbytes)
    y = out if out is not None else torch.empty_like(x)
    if slot_for_id is None:
        check(
            lib().ftmoe_experts_decode(_ptr(x), m, k, _ptr(topk_w), _ptr(topk_ids), bp, sp, _lib.ACT[activation],
                                       int(apply_router_weight_on_input), _ptr(y), _ptr(ws), ws.numel(),
                                       _stream(x.device)),
            "experts_decode",
        )
        return y
    if slot_for_id.dtype != torch.int32:
        raise ValueError("slot_for_id must be int32")
    if stats is not None and stats.dtype != torch.int64:
        raise ValueError("stats must be int64[4]")
    _require_gpu(slot_for_id, miss_mask, stats)
    check(
        lib().ftmoe_experts_decode_cached(_ptr(x), m, k, _ptr(topk_w), _ptr(topk_ids), _ptr(slot_for_id),
                                          slot_for_id.numel(), _ptr(topk_ids), _ptr(miss_mask), _ptr(stats), bp, sp,
                                          _lib.ACT[activation], int(apply_router_weight_on_input), _ptr(y), _ptr(ws),
                                          ws.numel(), _stream(x.device)),
        "experts_decode_cached",
    )
    return y


@dataclass
class Router:
    """A router for ``experts_decode_routed``: ``"softmax"`` (``fused_topk``) or
    ``"grouped_sigmoid"`` (DeepSeek-V3 ``_route``: bias, groups, scaling)."""

    kind: str
    top_k: int
    renormalize: bool = True
    bias: torch.Tensor | None = None
    n_group: int = 1
    topk_group: int = 1
    scale: float = 1.0


def experts_decode_routed(x: torch.Tensor, logits: torch.Tensor, router: Router, bank: ExpertBank,
                          shared: ExpertBank | None = None, activation: str = "silu",
                          apply_router_weight_on_input: bool = False, out: torch.Tensor | None = None,
                          slot_for_id: torch.Tensor | None = None, miss_mask: torch.Tensor | None = None,
                          stats: torch.Tensor | None = None, topk_w: torch.Tensor | None = None,
                          topk_ids: torch.Tensor | None = None):
    """Router logits -> decode output in one call (router + ``experts_decode``);
    returns (y, topk_w, topk_ids), the ids rewritten to slots when ``slot_for_id``
    is given.  For up to 16 tokens and 64 routes the router and the permutation
    share one launch."""
    if x.dtype != torch.bfloat16:
        raise ValueError("hidden_states must be bfloat16")
    if activation not in _lib.ACT:
        raise ValueError(f"Unsupported activation: {activation}")
    if router.kind == "softmax":
        kind = _lib.ROUTER_SOFTMAX_TOPK
        if logits.dtype == torch.bfloat16:
            dt = _lib.DTYPE_BF16
        else:
            logits, dt = logits.float(), _lib.DTYPE_F32
    elif router.kind == "grouped_sigmoid":
        kind, logits, dt = _lib.ROUTER_GROUPED_SIGMOID, logits.float(), _lib.DTYPE_F32
    else:
        raise ValueError(f"Unsupported router: {router.kind}")
    bias = router.bias.float().contiguous() if router.bias is not None else None
    logits = logits.contiguous()
    _require_gpu(x, logits, bias)
    m, e = logits.shape
    if x.shape[0] != m:
        raise ValueError("Number of tokens mismatch")
    k = router.top_k
    w = topk_w if topk_w is not None else torch.empty((m, k), dtype=torch.float32, device=x.device)
    ids = topk_ids if topk_ids is not None else torch.empty((m, k), dtype=torch.int32, device=x.device)
    _require_gpu(w, ids)
    r = _lib.FtmoeRouter(kind, logits.data_ptr(), dt, e, int(router.renormalize), _ptr(bias), router.n_group,
                         router.topk_group, float(router.scale))
    b = bank.cstruct()
    sb = shared.cstruct() if shared is not None else None
    bp = ctypes.byref(b)
    sp = ctypes.byref(sb) if sb is not None else None
    nbytes = lib().ftmoe_experts_decode_workspace(m, k, bp, sp)
    ws = _WS.get(x.device, nbytes)
    y = out if out is not None else torch.empty_like(x)
    if slot_for_id is not None:
        if slot_for_id.dtype != torch.int32:
            raise ValueError("slot_for_id must be int32")
        if stats is not None and stats.dtype != torch.int64:
            raise ValueError("stats must be int64[4]")
        _require_gpu(slot_for_id, miss_mask, stats)
    check(
        lib().ftmoe_experts_decode_routed(_ptr(x), m, k, ctypes.byref(r), _ptr(w), _ptr(ids), _ptr(slot_for_id),
                                          slot_for_id.numel() if slot_for_id is not None else 0,
                                          _ptr(ids) if slot_for_id is not None else None, _ptr(miss_mask),
                                          _ptr(stats), bp, sp, _lib.ACT[activation],
                                          int(apply_router_weight_on_input), _ptr(y), _ptr(ws), ws.numel(),
                                          _stream(x.device)),
        "experts_decode_routed",
    )
    return y, w, ids


def experts_prefill(x: torch.Tensor, topk_w: torch.Tensor, topk_ids: torch.Tensor, bank: ExpertBank,
                    shared: ExpertBank | None = None, activation: str = "silu",
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """Prefill-regime experts (grouped GEMMs on MFMA) for a precomputed routing."""
    if x.dtype != torch.bfloat16:
        raise ValueError("hidden_states must be bfloat16")
    if topk_w.dtype != torch.float32 or topk_ids.dtype != torch.int32:
        raise ValueError("topk_weights must be float32 and topk_ids int32")
    if topk_w.shape != topk_ids.shape:
        raise ValueError("topk shape mismatch")
    if activation not in _lib.ACT:
        raise ValueError(f"Unsupported activation: {activation}")
    _require_gpu(x, topk_w, topk_ids)
    m, k = topk_ids.shape
    if x.shape[0] != m:
        raise ValueError("Number of tokens mismatch")
    b = bank.cstruct()
    sb = shared.cstruct() if shared is not None else None
    bp = ctypes.byref(b)
    sp = ctypes.byref(sb) if sb is not None else None
    nbytes = lib().ftmoe_experts_prefill_workspace(m, k, bp, sp)
    ws = _WS.get(x.device, nbytes)
    y = out if out is not None else torch.empty_like(x)
    check(
        lib().ftmoe_experts_prefill(_ptr(x), m, k, _ptr(topk_w), _ptr(topk_ids), bp, sp, _lib.ACT[activation],
                                    _ptr(y), _ptr(ws), ws.numel(), _stream(x.device)),
        "experts_prefill",
    )
    return y


# --------------------------------------------------------------------------- CPU executor


# executors whose jobs were captured into graphs that may still replay: kept
# for the life of the process rather than freed under those graphs
_KEPT_EXECUTORS: list = []


class CpuExecutor:
    """Host-side expert executor of the hybrid decode (ftmoe_cpu_executor):
    ``run`` computes synchronously; ``submit`` / ``wait`` order the job on a
    stream (host-function nodes) so that GPU work queued between them overlaps
    it.  Inputs and outputs are host tensors (pinned for the stream path).

    A watchdog (``watchdog_s``, default ``FTMOE_CPU_WATCHDOG_S`` or 10 s)
    fails a job whose wait sees no progress of the pool for that long, so a
    stalled pool cannot block a stream for ever; the executor is then
    unhealthy and ``raise_if_unhealthy`` raises (the reference's flag
    watchdog and ``raise_if_unhealthy``, moe/cpu_executor.py:602-656)."""

    def __init__(self, threads: int = 0, watchdog_s: float | None = None):
        if threads <= 0:  # the process's CPU share (OMP_NUM_THREADS when set, else the affinity
            # mask) less one CPU for the thread that enqueues the GPU's share and the stream's host functions
            share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or len(os.sched_getaffinity(0))
            threads = max(1, share - 1)
        self.threads = threads
        self._h = lib().ftmoe_cpu_executor_create(threads)
        if not self._h:
            raise RuntimeError("ftmoe_cpu_executor_create failed")
        if watchdog_s is not None:
            self.set_watchdog(watchdog_s)

    @property
    def isa(self) -> str:
        return lib().ftmoe_cpu_executor_isa(self._h).decode()

    def set_watchdog(self, seconds: float) -> None:
        """Seconds without progress before a waited-for job fails (0: never)."""
        lib().ftmoe_cpu_executor_set_watchdog(self._h, int(round(seconds * 1000)))

    def hold(self, on: bool) -> None:
        """Keeps the pool from starting jobs while ``on`` (maintenance; tests of the watchdog)."""
        lib().ftmoe_cpu_executor_hold(self._h, int(bool(on)))

    def stall(self, on: bool) -> None:
        """While ``on``, the driver takes its next job and stalls inside it, as a
        wedged pool would (tests of the watchdog and of ``close``)."""
        lib().ftmoe_cpu_executor_hold(self._h, 2 if on else 0)

    def set_handshake(self, mode: str) -> bool:
        """``"flags"``: stream memory operations (a ready flag the stream raises,
        a done flag it waits on; no host-function round trip), taken when a
        functional probe on this device passes; ``"host"``: host functions.
        Returns whether the flags are in use."""
        if mode not in ("flags", "host"):
            raise ValueError(f"unknown handshake {mode!r}")
        rc = lib().ftmoe_cpu_executor_set_handshake(self._h, 1 if mode == "flags" else 0)
        if rc not in (_lib.FTMOE_OK, _lib.FTMOE_ERR_UNSUPPORTED):
            check(rc, "cpu_executor_set_handshake")
        return rc == _lib.FTMOE_OK and mode == "flags"

    @property
    def handshake(self) -> str:
        """"host", "flags" (eager calls) or "flags+graphs" (captured calls too)."""
        return {0: "host", 1: "flags", 2: "flags+graphs"}[lib().ftmoe_cpu_executor_handshake(self._h)]

    @property
    def healthy(self) -> bool:
        return lib().ftmoe_cpu_executor_healthy(self._h) == _lib.FTMOE_OK

    def raise_if_unhealthy(self) -> None:
        """Raises once the watchdog has fired: outputs of the failed jobs were
        never written and the executor must be replaced."""
        if self._h and not self.healthy:
            raise RuntimeError("CPU expert executor watchdog fired: a job saw no progress of the pool within "
                               "the watchdog period; its outputs were not computed. Replace the executor.")

    def close(self, graphs_released: bool = False) -> None:
        """Frees the executor once the host functions queued on streams have run
        (the device is synchronised first).  While jobs captured into graphs
        exist the executor is kept alive instead, unless ``graphs_released``
        says those graphs are destroyed: a replay would touch a freed executor.
        A pool wedged inside a job the watchdog abandoned cannot be joined: its
        executor is kept too, and ``close`` returns at once."""
        if not self._h:
            return
        if torch.cuda.is_available() and torch.cuda.is_initialized():
            torch.cuda.synchronize()
        rc = lib().ftmoe_cpu_executor_destroy(self._h, int(graphs_released))
        if rc == _lib.FTMOE_ERR_BUSY:
            _KEPT_EXECUTORS.append(self._h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _check(x, w, ids, y):
        for t in (x, w, ids, y):
            if t.device.type != "cpu" or not t.is_contiguous():
                raise ValueError("CPU executor tensors are contiguous host tensors")
        if x.dtype != torch.bfloat16 or y.dtype != torch.bfloat16 or w.dtype != torch.float32 or ids.dtype != torch.int32:
            raise ValueError("x, y bf16; w float32; ids int32")
        if w.shape != ids.shape or x.shape[0] != ids.shape[0] or y.shape != x.shape:
            raise ValueError("shape mismatch")

    def run(self, bank: ExpertBank, x, w, ids, y=None, activation: str = "silu"):
        y = y if y is not None else torch.empty_like(x)
        self._check(x, w, ids, y)
        b = bank.host_cstruct()
        m, k = ids.shape
        check(lib().ftmoe_cpu_experts(self._h, ctypes.byref(b), x.data_ptr(), w.data_ptr(), ids.data_ptr(), m, k,
                                      _lib.ACT[activation], y.data_ptr()), "cpu_experts")
        return y

    def submit(self, bank: ExpertBank, x, w, ids, y, activation: str = "silu", device=None):
        """Enqueues the job on the current stream of ``device``; returns a handle for ``wait``."""
        self._check(x, w, ids, y)
        b = bank.host_cstruct()
        m, k = ids.shape
        job = ctypes.c_void_p()
        check(lib().ftmoe_cpu_experts_submit(self._h, ctypes.byref(b), x.data_ptr(), w.data_ptr(), ids.data_ptr(),
                                             m, k, _lib.ACT[activation], y.data_ptr(), _stream(device),
                                             ctypes.byref(job)), "cpu_experts_submit")
        return job

    def wait(self, job, device=None) -> None:
        check(lib().ftmoe_cpu_experts_wait(self._h, job, _stream(device)), "cpu_experts_wait")
