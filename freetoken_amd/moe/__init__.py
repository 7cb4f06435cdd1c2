"""MoE backend registry (reference ``moe/__init__.py:16-65``).

``"fused"`` (and its alias ``"mi355x"``) is the resident-expert backend backed
by the gfx950 kernels; ``"offload"`` marks the expert-cache path whose work is
done by ``OffloadMoELayer`` (``moe/offload.py`` of the reference); ``"cpu"``
and ``"hybrid"`` are the offload family's decode placements whose CPU share
runs on the host executor (``moe/cpu_offload.py`` of the reference).
"""

from __future__ import annotations

from typing import Callable, Dict

from .base import BaseMoeBackend


class Registry:
    def __init__(self, name: str):
        self.name = name
        self._items: Dict[str, Callable[[], BaseMoeBackend]] = {}

    def register(self, key: str):
        def deco(fn):
            assert key not in self._items, f"{self.name} {key!r} registered twice"
            self._items[key] = fn
            return fn

        return deco

    def __getitem__(self, key: str):
        if key not in self._items:
            raise KeyError(f"unknown {self.name} {key!r}; supported: {sorted(self._items)}")
        return self._items[key]

    def __contains__(self, key: str) -> bool:
        return key in self._items

    def keys(self):
        return self._items.keys()


SUPPORTED_MOE_BACKENDS = Registry("MoE Backend")

OFFLOAD_MOE_BACKENDS = frozenset({"offload", "cpu", "hybrid"})


def is_offload_moe_backend(backend: str) -> bool:
    return backend in OFFLOAD_MOE_BACKENDS


@SUPPORTED_MOE_BACKENDS.register("fused")
def create_fused_moe_backend():
    from .fused import FusedMoe

    return FusedMoe()


@SUPPORTED_MOE_BACKENDS.register("mi355x")
def create_mi355x_moe_backend():
    from .fused import FusedMoe

    return FusedMoe()


@SUPPORTED_MOE_BACKENDS.register("offload")
def create_offload_moe_backend():
    from .offload import OffloadMoeBackend

    return OffloadMoeBackend()


@SUPPORTED_MOE_BACKENDS.register("cpu")
def create_cpu_moe_backend():
    from .offload import CpuOffloadMoeBackend

    return CpuOffloadMoeBackend()


@SUPPORTED_MOE_BACKENDS.register("hybrid")
def create_hybrid_moe_backend():
    from .offload import HybridMoeBackend

    return HybridMoeBackend()


def create_moe_backend(backend: str) -> BaseMoeBackend:
    return SUPPORTED_MOE_BACKENDS[backend]()


__all__ = [
    "BaseMoeBackend",
    "create_moe_backend",
    "SUPPORTED_MOE_BACKENDS",
    "OFFLOAD_MOE_BACKENDS",
    "is_offload_moe_backend",
]
