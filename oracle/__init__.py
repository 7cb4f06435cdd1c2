"""CPU oracle for the fused MoE-layer hot path -- TEST INFRASTRUCTURE ONLY.

This package is a plain-numpy restatement of FreeToken's MoE-layer algorithm
(router top-k, moe_align_block_size, the bf16 / FP8-128x128 / MXFP4 expert
math with the reference's rounding points, the weighted combine, the shared
expert and the expert-cache slot lookup).  Each function cites the reference
file:line it restates (paths relative to ``python/freetoken/`` of the
reference tree).

It is the *checker*: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it.  The product path
(``freetoken_amd``) never imports it and fails loudly when its HIP library
is missing.

Pinning status of every function is recorded in its docstring; functions
whose only check would be a restatement of the same formula say
"parity unpinned".
"""

from . import numerics, routing, align, experts, slots  # noqa: F401
