"""Correctness at the sizes the bench times.

The bench's own workloads (``bench.py``: ``prefill_workload`` for C5,
``DecodeLayer`` for C2, C3 and C4), built and run at full size on the GPU, then checked
against the oracle on a sample of tokens.  Token rows are independent in both
regimes (the activation quantisation is per token and per route row, the
combine per token), so the oracle runs only the sampled tokens and the experts
they route to.  The sample always holds the first and the last tokens of the
hottest expert (its first and last M blocks), the tokens around its first
block boundary, and random tokens while the experts they add stay within a
budget; routing ids and slot ids are compared bit for bit for every token.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
import oracle
from oracle.experts import Bank
from freetoken_amd import ops

from _helpers import to_np
from conftest import COS_TOL, MAX_REL_TOL, cosine, max_rel

pytestmark = pytest.mark.gpu


def _oracle_bank(bank: ops.ExpertBank, rows) -> Bank:
    """Rows of a device bank as an oracle bank (host copies of those rows only)."""
    idx = torch.as_tensor(np.asarray(rows, dtype=np.int64), device=bank.gate_up.device)

    def sel(t):
        return t.index_select(0, idx).contiguous().cpu()

    if bank.fmt == "bf16":
        return Bank("bf16", sel(bank.gate_up).float().numpy(), sel(bank.down).float().numpy())
    gu, dn = sel(bank.gate_up).view(torch.uint8).numpy(), sel(bank.down).view(torch.uint8).numpy()
    gs, ds = sel(bank.gate_up_scale).numpy(), sel(bank.down_scale).numpy()
    return Bank("fp8" if bank.fmt == "fp8_block" else "mxfp4", gu, dn, gs, ds)


def _sample(ids: np.ndarray, rows: int, budget: int, n: int, block: int, seed: int) -> np.ndarray:
    """Tokens to check: the hottest row's first two and last two tokens and the
    two around its first M-block boundary, then random tokens while the rows
    they touch stay within ``budget``."""
    M, k = ids.shape
    flat = ids.reshape(-1)
    valid = (flat >= 0) & (flat < rows)
    counts = np.bincount(flat[valid], minlength=rows)
    hot = int(counts.argmax())
    hot_tokens = np.nonzero(flat == hot)[0] // k  # ascending flat route index: the kernel's stable order
    must = [hot_tokens[0], hot_tokens[min(1, len(hot_tokens) - 1)], hot_tokens[-2], hot_tokens[-1]]
    if len(hot_tokens) > block:
        must += [hot_tokens[block - 1], hot_tokens[block]]
    chosen, union = [], set()
    for t in must:
        if t not in chosen:
            chosen.append(int(t))
            union |= {int(e) for e in ids[t] if 0 <= e < rows}
    for t in np.random.default_rng(seed).permutation(M):
        if len(chosen) >= n:
            break
        new = {int(e) for e in ids[t] if 0 <= e < rows} - union
        if int(t) not in chosen and len(union | new) <= budget:
            chosen.append(int(t))
            union |= new
    return np.array(sorted(chosen), dtype=np.int64)


def _check_rows(y: torch.Tensor, sample, x, w, ids, bank, shared, regime: str, rows: int, what):
    """y[sample] against the oracle layer on those tokens and the rows they touch."""
    ids_s = ids[sample]
    used = np.unique(ids_s[(ids_s >= 0) & (ids_s < rows)])
    remap = np.full(rows + 1, -1, dtype=np.int32)
    remap[used] = np.arange(used.size, dtype=np.int32)
    local = np.where((ids_s >= 0) & (ids_s < rows), remap[np.clip(ids_s, 0, rows)], -1).astype(np.int32)
    sub = _oracle_bank(bank, used)
    sh = _oracle_bank(shared, [0]) if shared is not None else None
    y_ref = oracle.experts.moe_layer(regime, x[sample], w[sample], local, sub, sh)
    got = to_np(y)[sample]
    assert max_rel(got, y_ref) <= MAX_REL_TOL, (what, max_rel(got, y_ref))
    assert cosine(got, y_ref) >= COS_TOL, (what, cosine(got, y_ref))
    return used.size


@pytest.mark.parametrize("fmt", ["fp8_block", "mxfp4"])
def test_c5_prefill_full_size_sampled(dev, fmt):
    """C5: 8192 tokens, 256 experts (H 7168, I 2048) + shared expert, Zipf(1.1)
    skew -- the hottest expert holds thousands of routes, so tens of M blocks of
    one expert travel the persistent GEMM walk."""
    gen = torch.Generator(device=dev).manual_seed(4321)
    wl = bench.prefill_workload(fmt, gen, dev)
    c = bench.C4
    y = ops.experts_prefill(wl["x"], wl["w"], wl["ids"], wl["bank"], shared=wl["shared"])
    # a second call gives the same bytes: every workgroup walks about twenty
    # tiles, so the ring's stage reuse across tiles, the next tile's copies in
    # flight during an epilogue and the epilogue's staging in the freed stage
    # all run many times here
    y2 = ops.experts_prefill(wl["x"], wl["w"], wl["ids"], wl["bank"], shared=wl["shared"])
    torch.cuda.synchronize()
    assert torch.equal(y, y2), ("C5", fmt, "repeat differs")
    del y2
    logits, bias = to_np(wl["logits"]), to_np(wl["bias"])
    w_ref, ids_ref = oracle.routing.grouped_sigmoid_topk(logits, bias, 8, 4, c["k"], True, 2.5)
    ids = to_np(wl["ids"])
    np.testing.assert_array_equal(ids, ids_ref)
    np.testing.assert_allclose(to_np(wl["w"]), w_ref, rtol=1e-6, atol=1e-7)
    counts = np.bincount(ids.reshape(-1), minlength=c["E"])
    assert counts.max() > 4 * 256, counts.max()  # the skew the test is about
    sample = _sample(ids, c["E"], budget=32, n=16, block=256, seed=1)
    x = to_np(wl["x"])
    n_used = _check_rows(y, sample, x, w_ref, ids, wl["bank"], wl["shared"], "prefill", c["E"], ("C5", fmt))
    print(f"C5 {fmt}: {sample.size} tokens over {n_used} experts checked", flush=True)


_LAYERS: dict = {}


@pytest.fixture(scope="module")
def decode_layers():
    """The bench's decode layers, built once per module on first use."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device")
    yield _LAYERS
    _LAYERS.clear()
    torch.cuda.empty_cache()


def _layer(name: str, dev):
    if name not in _LAYERS:
        for other in list(_LAYERS):  # one layer at a time on the device
            del _LAYERS[other]
        torch.cuda.empty_cache()
        cfg = {"c2": bench.C2, "c3": bench.C3, "c4": bench.C4}[name]
        gen = torch.Generator(device=dev).manual_seed({"c2": 97, "c3": 98, "c4": 99}[name])
        _LAYERS[name] = (bench.DecodeLayer(cfg, dev, gen), gen)
    return _LAYERS[name]


def _oracle_routing(layer, logits: np.ndarray):
    c = layer.cfg
    if c["router"] == "softmax":
        return oracle.routing.softmax_topk(logits, c["k"], True)
    return oracle.routing.grouped_sigmoid_topk(logits, to_np(layer.bias), c["n_group"], c["topk_group"], c["k"],
                                               True, c["scale"])


# (layer, batch): every batch the bench times.  C4 (1-4 run the router and
# the shared expert's gate_up in one launch; 64 is the headline; 192 and 256
# the wide segments), C2 (128 FP8 experts, softmax router) and C3 (160 MXFP4
# experts, bf16 shared expert)
DECODE_POINTS = [("c4", 1), ("c4", 2), ("c4", 4), ("c4", 8), ("c4", 16), ("c4", 32), ("c4", 64), ("c4", 128),
                 ("c4", 192), ("c4", 256), ("c2", 1), ("c2", 8), ("c2", 32), ("c2", 64), ("c3", 1), ("c3", 8),
                 ("c3", 32), ("c3", 64)]


@pytest.mark.parametrize("name,M", DECODE_POINTS, ids=[f"{n}_b{m}" for n, m in DECODE_POINTS])
def test_decode_full_size_sampled(dev, decode_layers, name, M):
    """The bench's decode layers through the routed entry point (router, slot
    lookup, experts, combine) at the benched batches: routing weights, slot ids
    and slot-lookup counters against the oracle for every token, the output on
    a sample of tokens."""
    layer, gen = _layer(name, dev)
    c = layer.cfg
    logits = torch.randn((M, c["E"]), generator=gen, device=dev)
    x = torch.randn((M, c["H"]), generator=gen, device=dev).to(torch.bfloat16)
    stats = torch.zeros(4, dtype=torch.int64, device=dev)
    y, w, slots = ops.experts_decode_routed(x, logits, layer.router, layer.bank, shared=layer.shared,
                                            slot_for_id=layer.table, stats=stats)
    torch.cuda.synchronize()
    w_ref, ids_ref = _oracle_routing(layer, to_np(logits))
    np.testing.assert_allclose(to_np(w), w_ref, rtol=1e-6, atol=1e-7)
    slots_ref, _, stats_ref = oracle.slots.slot_map(ids_ref, to_np(layer.table))
    np.testing.assert_array_equal(to_np(slots), slots_ref)
    np.testing.assert_array_equal(to_np(stats), stats_ref)
    assert (slots_ref >= 0).sum() >= min(M, 2), "routes should hit the resident slots"
    if M <= 4:
        sample = np.arange(M, dtype=np.int64)
    else:
        sample = _sample(slots_ref, c["slots"], budget=24, n=16, block=32, seed=M)
    n_used = _check_rows(y, sample, to_np(x), w_ref, slots_ref, layer.bank, layer.shared, "decode", c["slots"],
                         (name, M))
    print(f"{name} b={M}: {sample.size} tokens over {n_used} slots checked", flush=True)
