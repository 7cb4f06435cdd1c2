"""Pins of oracle/align.py: the reference's docstring KAT, a loop-based
construction and structural invariants."""

import numpy as np
import pytest

from oracle import align as A


def test_docstring_kat():
    # moe/fused.py:113-126 of the reference
    s, e, n = A.moe_align_block_size(np.array([[2, 3, 4], [1, 2, 4], [1, 3, 4], [1, 2, 3]]), 4, 4)
    assert s[:16].tolist() == [3, 6, 9, 12, 0, 4, 10, 12, 1, 7, 11, 12, 2, 5, 8, 12]
    assert n.tolist() == [16]
    assert e[:4].tolist() == [1, 2, 3, 4]
    assert len(s) == 12 + 5 * 3  # numel + (E+1)*(BM-1)


def _loops(ids, bs, E):
    eff = E + 1
    buckets = [[] for _ in range(eff)]
    for i, e in enumerate(ids):
        if 0 <= e < eff:
            buckets[e].append(i)
    out, eids = [], []
    for e, b in enumerate(buckets):
        if not b:
            continue
        pad = -(-len(b) // bs) * bs
        out += b + [len(ids)] * (pad - len(b))
        eids += [e] * (pad // bs)
    return out, eids


@pytest.mark.parametrize("seed", range(20))
def test_against_loops(seed):
    rng = np.random.default_rng(seed)
    E = int(rng.integers(1, 40))
    bs = int(rng.integers(1, 9))
    n = int(rng.integers(0, 300))
    ids = rng.integers(-2, E + 3, n).astype(np.int32)
    s, e, ntpp = A.moe_align_block_size(ids, bs, E)
    ref_s, ref_e = _loops(ids.tolist(), bs, E)
    assert ntpp[0] == len(ref_s)
    assert s[: len(ref_s)].tolist() == ref_s
    assert np.all(s[len(ref_s):] == n)
    assert e[: len(ref_e)].tolist() == ref_e
    assert np.all(e[len(ref_e):] == -1)
    mp, mb = A.buffer_sizes(n, E, bs)
    assert len(s) == mp and len(e) == mb and ntpp[0] <= mp


def test_segments():
    ids = np.array([[3, 1], [1, -1], [7, 3]], dtype=np.int32)
    ex, st, ct, routes = A.expert_segments(ids, 5)  # 7 is out of range
    assert ex.tolist() == [1, 3] and ct.tolist() == [2, 2] and st.tolist() == [0, 2]
    assert routes.tolist() == [1, 2, 0, 5]  # flat routes of expert 1, then expert 3
