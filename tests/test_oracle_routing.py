"""Pins of oracle/routing.py: reference known answers, brute force over
subsets, closed-form weights and hand-built grouped-router cases."""

import itertools

import numpy as np

from oracle import routing as R
from oracle import synth
from oracle.numerics import sigmoid_det


def test_reference_kat():
    # tests/moe/test_fused_moe.py:42-58 of the reference
    lg = np.float32([[4.0, 1.0, -1.0, 2.0], [0.5, 3.0, 2.0, -2.0]])
    w, ids = R.softmax_topk(lg, 2, True)
    assert ids.tolist() == [[0, 3], [1, 2]]
    sel = np.float64([[4.0, 2.0], [3.0, 2.0]])
    ref = np.exp(sel) / np.exp(sel).sum(1, keepdims=True)
    np.testing.assert_allclose(w, ref, rtol=1e-6)


def _brute_topk(row, k):
    """Best k-subset by value sum; among equal sums the lexicographically
    smallest index set; returned in rank order (value desc, index asc)."""
    best = None
    for sub in itertools.combinations(range(len(row)), k):
        s = sum(float(row[i]) for i in sub)
        if best is None or s > best[0]:
            best = (s, sub)
    chosen = sorted(best[1], key=lambda i: (-float(row[i]), i))
    return chosen


def test_brute_force_selection_with_ties():
    rng = np.random.default_rng(0)
    for _ in range(300):
        e = int(rng.integers(3, 8))
        k = int(rng.integers(1, e))
        row = rng.integers(-3, 3, e).astype(np.float32)  # many ties
        _, ids = R.softmax_topk(row[None], k, True)
        assert ids[0].tolist() == _brute_topk(row, k), (row, k)


def test_negative_zero_ties_positive_zero():
    lg = np.float32([[-0.0, 0.0, -1.0]])
    _, ids = R.softmax_topk(lg, 2, True)
    assert ids.tolist() == [[0, 1]]


def test_weights_closed_form():
    rng = np.random.default_rng(1)
    lg = rng.standard_normal((50, 128)).astype(np.float32)
    w, ids = R.softmax_topk(lg, 8, False)
    full = np.exp(lg.astype(np.float64) - lg.max(1, keepdims=True))
    full /= full.sum(1, keepdims=True)
    np.testing.assert_allclose(w, np.take_along_axis(full, ids.astype(np.int64), 1), rtol=1e-6)
    w2, ids2 = R.softmax_topk(lg, 8, True)
    assert np.array_equal(ids, ids2)
    np.testing.assert_allclose(w2.sum(1), 1.0, rtol=1e-6)


def _grouped_loops(lg, bias, n_group, topk_group, k, renorm, scale):
    """Independent restatement with explicit loops (no argsort)."""
    m, e = lg.shape
    per = e // n_group
    s = sigmoid_det(lg)
    c = s + (bias if bias is not None else np.float32(0))
    out_w, out_i = [], []
    for r in range(m):
        gs = []
        for g in range(n_group):
            vals = sorted((float(v) for v in c[r, g * per:(g + 1) * per]), reverse=True)
            gs.append(float(np.float32(vals[0]) + np.float32(vals[1])))
        kept = []
        for _ in range(topk_group):
            best = max((gs[g], -g) for g in range(n_group) if g not in kept)
            kept.append(-best[1])
        cand = [i for i in range(e) if i // per in kept]
        chosen = []
        for _ in range(k):
            best = max((float(c[r, i]), -i) for i in cand if i not in chosen)
            chosen.append(-best[1])
        wv = [np.float32(s[r, i]) for i in chosen]
        if renorm:
            tot = np.float32(0)
            for v in wv:
                tot = np.float32(tot + v)
            wv = [np.float32(v / np.float32(tot + np.float32(1e-20))) for v in wv]
        out_w.append([np.float32(v * np.float32(scale)) for v in wv])
        out_i.append(chosen)
    return np.array(out_w, dtype=np.float32), np.array(out_i, dtype=np.int32)


def test_grouped_against_loops():
    rng = np.random.default_rng(2)
    lg = synth.tied_logits(rng, 40, 64, bf16=True)
    bias = synth.normal(rng, (64,), 0.1)
    for b in (None, bias):
        w, ids = R.grouped_sigmoid_topk(lg, b, 8, 4, 8, True, 2.5)
        w2, ids2 = _grouped_loops(lg, b, 8, 4, 8, True, 2.5)
        assert np.array_equal(ids, ids2)
        assert np.array_equal(w, w2)


def test_grouped_hand_cases():
    E = 64
    lg = np.zeros((3, E), dtype=np.float32)
    # all equal -> groups 0..3, experts 0..7 in index order
    w, ids = R.grouped_sigmoid_topk(lg, None, 8, 4, 8, True, 2.5)
    assert ids[0].tolist() == list(range(8))
    np.testing.assert_allclose(w[0], 2.5 / 8, rtol=1e-6)
    # a bias flips the selection into group 7 (selection only: w stays s-based)
    bias = np.zeros(E, dtype=np.float32)
    bias[63] = 5.0
    w, ids = R.grouped_sigmoid_topk(lg, bias, 8, 4, 8, True, 2.5)
    assert ids[0, 0] == 63 and set(ids[0, 1:].tolist()) <= set(range(32)) | {63}
    # group ties: every group has the same score -> lowest four groups
    lg2 = np.tile(np.arange(8, dtype=np.float32), 8)[None]
    _, ids = R.grouped_sigmoid_topk(lg2, None, 8, 4, 8, False, 1.0)
    assert sorted(set(int(i) // 8 for i in ids[0])) == [0, 1, 2, 3]
    # within-group top-2 uses duplicates: two equal maxima make the group win
    lg3 = np.zeros((1, E), dtype=np.float32)
    lg3[0, 56] = lg3[0, 57] = 2.0
    lg3[0, 0] = 3.0
    _, ids = R.grouped_sigmoid_topk(lg3, None, 8, 1, 2, True, 1.0)
    assert ids[0].tolist() == [56, 57]


def test_det_sigmoid_selection_matches_torch_sigmoid():
    """The grouped router's selection with the deterministic sigmoid against the
    same router on torch's float32 sigmoid (the reference's ``logits.sigmoid()``,
    models/glm4_moe/moe.py:66), on C4-distributed logits (N(0,1), bias N(0,0.1)):
    the two sigmoids differ by at most a few ulp, and the selected expert sets
    agree on every row (over 1M rows of C4 and of C5 logits, 3 rows ranked
    two near-tied experts in the other order and none chose another expert)."""
    import torch

    from oracle import routing

    rng = np.random.default_rng(2025)
    M, E = 100_000, 256
    lg = synth.normal(rng, (M, E))
    bias = synth.normal(rng, (E,), 0.1)
    w1, i1 = routing.grouped_sigmoid_topk(lg, bias, 8, 4, 8, True, 2.5)
    saved = routing.sigmoid_det
    routing.sigmoid_det = lambda x: torch.sigmoid(torch.from_numpy(np.asarray(x, np.float32))).numpy()
    try:
        w2, i2 = routing.grouped_sigmoid_topk(lg, bias, 8, 4, 8, True, 2.5)
    finally:
        routing.sigmoid_det = saved
    assert (np.sort(i1, 1) == np.sort(i2, 1)).all()
    assert (i1 != i2).any(1).mean() <= 1e-4
    np.testing.assert_allclose(w1, w2, rtol=1e-5, atol=1e-6)
