"""Router top-k restatements (softmax and grouped sigmoid).

Canonical tie rule (both routers): rank by value descending; among equal
values the LOWER expert index wins.  This is the rule of the reference's one
explicit-tie router, ``gpt_oss_routing_kernel``
(``kernel/triton/mxfp4_moe.py:288-331``: sort of packed ``key<<32 | index``).
-0.0 is canonicalised to +0.0 before ranking, so ranking equals IEEE float
comparison on every non-NaN input.

Pins (tests/test_oracle_routing.py):
  * the known-answer routing of ``tests/moe/test_fused_moe.py:42-58``;
  * brute force over every k-subset on tiny inputs (the selected set
    maximises the value sum and is lexicographically smallest on ties);
  * weights against the closed form softmax in float64;
  * hand-built grouped-router cases with exact ties between experts and
    between groups, all-equal groups and a bias that flips the selection.
"""

from __future__ import annotations

import numpy as np

from .numerics import F32, sigmoid_det


def _rank_desc(v: np.ndarray) -> np.ndarray:
    """Row-wise indices sorted by value descending, ties -> lower index."""
    v = np.asarray(v, dtype=np.float32) + F32(0.0)  # -0.0 -> +0.0
    return np.argsort(-v, axis=-1, kind="stable")


def softmax_topk(logits, topk: int, renormalize: bool):
    """``fused_topk`` (``moe/fused.py:38-85``; torch fallback ``:16-35``).

    Selection is on the fp32 logits (``:67``).  With ``renormalize`` the k
    weights are the softmax over the selected logits (``apply_softmax`` over the
    top-k, ``:68-75``), mathematically equal to softmax-all + renorm
    (``:27-30``).  Without it the weights are the softmax over all experts.
    Returns (weights float32 [M,k], ids int32 [M,k]) in rank order.
    """
    lg = np.asarray(logits, dtype=np.float32)
    order = _rank_desc(lg)[:, :topk]
    sel = np.take_along_axis(lg, order, axis=1).astype(np.float64)
    if renormalize:
        e = np.exp(sel - sel.max(axis=1, keepdims=True))
        w = e / e.sum(axis=1, keepdims=True)
    else:
        full = lg.astype(np.float64)
        mx = full.max(axis=1, keepdims=True)
        denom = np.exp(full - mx).sum(axis=1, keepdims=True)
        w = np.exp(sel - mx) / denom
    return w.astype(np.float32), order.astype(np.int32)


def grouped_sigmoid_topk(
    logits,
    bias,
    n_group: int,
    topk_group: int,
    topk: int,
    renormalize: bool,
    scale: float,
):
    """DeepSeek-V3 ``noaux_tc`` router, ``Glm4MoeSparseBlock._route`` /
    ``_group_limited`` (``models/glm4_moe/moe.py:53-75``).

    s = sigmoid(l) (deterministic float32 sigmoid, see numerics.sigmoid_det);
    c = s + bias (selection only); group score = top1 + top2 of c in the
    group; keep ``topk_group`` groups; experts of other groups -> -inf; top-k of
    c; w = s[ids]; optional renorm w / (sum + 1e-20); times ``scale``.
    Returns (weights float32 [M,k], ids int32 [M,k]) in rank order.
    """
    lg = np.asarray(logits, dtype=np.float32)
    m, e = lg.shape
    s = sigmoid_det(lg)
    c = s if bias is None else (s + np.asarray(bias, dtype=np.float32)[None, :]).astype(np.float32)
    if n_group > 1:
        per = e // n_group
        cg = c.reshape(m, n_group, per)
        top2 = -np.sort(-cg, axis=-1)[..., :2]
        gscore = (top2[..., 0] + top2[..., 1]).astype(np.float32)
        gsel = _rank_desc(gscore)[:, :topk_group]
        gmask = np.zeros((m, n_group), dtype=bool)
        np.put_along_axis(gmask, gsel, True, axis=1)
        emask = np.repeat(gmask, per, axis=1)
        c = np.where(emask, c, np.float32(-np.inf)).astype(np.float32)
    ids = _rank_desc(c)[:, :topk]
    w = np.take_along_axis(s, ids, axis=1).astype(np.float32)
    if renormalize:
        tot = np.zeros((m, 1), dtype=np.float32)
        for j in range(topk):
            tot = (tot + w[:, j : j + 1]).astype(np.float32)
        w = (w / (tot + F32(1e-20))).astype(np.float32)
    w = (w * F32(scale)).astype(np.float32)
    return w, ids.astype(np.int32)
