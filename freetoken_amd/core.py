"""Minimal forward context: the phase flag and MoE backend the layer reads.

Mirrors the parts of FreeToken's ``core.py`` the MoE layer touches
(``Batch.is_prefill``/``is_decode``, ``core.py:151-158``; ``Context.moe_backend``
/ ``moe_offload_cache`` and the global-context accessors, ``core.py:168-207``).
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass, field
from typing import Any


@dataclass
class Batch:
    phase: str = "decode"  # "prefill" | "decode"

    @property
    def is_prefill(self) -> bool:
        return self.phase == "prefill"

    @property
    def is_decode(self) -> bool:
        return self.phase == "decode"


@dataclass
class Context:
    moe_backend: Any = None
    moe_offload_cache: Any = None
    _batch: Batch | None = field(default=None, init=False)

    @property
    def batch(self) -> Batch:
        assert self._batch is not None, "No active batch in context"
        return self._batch

    @contextmanager
    def forward_batch(self, batch: Batch):
        assert self._batch is None, "Nested forward_batch is not allowed"
        try:
            self._batch = batch
            yield
        finally:
            self._batch = None


_GLOBAL_CTX: Context | None = None


def set_global_ctx(ctx: Context | None) -> None:
    """Install (or, with None, clear) the process-wide context."""
    global _GLOBAL_CTX
    assert ctx is None or _GLOBAL_CTX is None, "Global context is already set"
    _GLOBAL_CTX = ctx


def get_global_ctx() -> Context:
    assert _GLOBAL_CTX is not None, "Global context is not set"
    return _GLOBAL_CTX


def has_global_ctx() -> bool:
    return _GLOBAL_CTX is not None


@contextmanager
def moe_phase(phase: str, backend: str = "fused"):
    """Convenience for tests and benchmarks: a global context with the given
    MoE backend and an active batch of the given phase."""
    from .moe import create_moe_backend

    owned = not has_global_ctx()
    if owned:
        set_global_ctx(Context(moe_backend=create_moe_backend(backend)))
    ctx = get_global_ctx()
    try:
        with ctx.forward_batch(Batch(phase=phase)):
            yield ctx
    finally:
        if owned:
            set_global_ctx(None)
