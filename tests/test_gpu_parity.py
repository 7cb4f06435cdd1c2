"""GPU parity of the HIP path against the CPU oracle (bit-exact routing and
permutation; bf16 outputs within max-rel 2e-2 and cosine >= 0.9995)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from oracle import synth
from oracle.numerics import bf16_round
from freetoken_amd import ops

from _helpers import bf16_dev, code_bank, sub_bank, to_device_bank, to_np
from conftest import COS_TOL, MAX_REL_TOL, cosine, max_rel

pytestmark = pytest.mark.gpu


# ----------------------------------------------------------------- routing


@pytest.mark.parametrize("E,k", [(16, 2), (128, 8), (160, 8), (256, 8), (1024, 6)])
@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("bf16", [True, False])
def test_softmax_topk_exact(dev, E, k, renorm, bf16):
    rng = np.random.default_rng(E * 10 + k)
    lg = synth.tied_logits(rng, 67, E, bf16=bf16)
    w_ref, ids_ref = oracle.routing.softmax_topk(lg, k, renorm)
    t = torch.from_numpy(lg).to(dev)
    t = t.to(torch.bfloat16) if bf16 else t
    w, ids = ops.route_softmax_topk(t, k, renorm)
    np.testing.assert_array_equal(to_np(ids), ids_ref)
    np.testing.assert_allclose(to_np(w), w_ref, rtol=2e-6, atol=1e-7)


def test_softmax_topk_reference_kat(dev):
    # tests/moe/test_fused_moe.py:42-58 of the reference
    lg = torch.tensor([[4.0, 1.0, -1.0, 2.0], [0.5, 3.0, 2.0, -2.0]], device=dev, dtype=torch.bfloat16)
    w, ids = ops.route_softmax_topk(lg, 2, True)
    ref_l, ref_i = torch.topk(lg.float().cpu(), 2, dim=-1)
    np.testing.assert_array_equal(to_np(ids), ref_i.numpy())
    np.testing.assert_allclose(to_np(w), torch.softmax(ref_l, -1).numpy(), rtol=2e-4, atol=2e-4)


@pytest.mark.parametrize("M", [1, 7, 64, 256, 8192])
@pytest.mark.parametrize("with_bias", [True, False])
def test_grouped_sigmoid_exact(dev, M, with_bias):
    rng = np.random.default_rng(M + (7 if with_bias else 0))
    E = 256
    lg = synth.tied_logits(rng, M, E, bf16=False) + synth.zipf_bias(rng, E)[None, :]
    bias = synth.normal(rng, (E,), 0.1) if with_bias else None
    w_ref, ids_ref = oracle.routing.grouped_sigmoid_topk(lg, bias, 8, 4, 8, True, 2.5)
    tb = None if bias is None else torch.from_numpy(bias).to(dev)
    w, ids = ops.route_grouped_sigmoid(torch.from_numpy(lg).to(dev), tb, 8, 4, 8, True, 2.5)
    np.testing.assert_array_equal(to_np(ids), ids_ref)
    np.testing.assert_allclose(to_np(w), w_ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("E,n_group,topk_group,k", [
    (64, 32, 8, 8), (128, 16, 4, 8), (256, 16, 4, 8), (256, 8, 4, 8), (128, 2, 1, 8), (320, 5, 2, 8),
    (1024, 64, 8, 16),  # group sizes 2..64, a power of two dividing the wave: lane-block butterflies
    (96, 8, 4, 8), (160, 5, 2, 8), (40, 4, 2, 4),  # other group sizes or E: the LDS scan
])
def test_grouped_sigmoid_group_shapes(dev, E, n_group, topk_group, k):
    rng = np.random.default_rng(E * 131 + n_group)
    lg = synth.tied_logits(rng, 33, E, bf16=False)
    lg[0] = 0.25  # every group and expert tied
    bias = synth.normal(rng, (E,), 0.05)
    for b in (None, bias):
        w_ref, ids_ref = oracle.routing.grouped_sigmoid_topk(lg, b, n_group, topk_group, k, True, 2.5)
        tb = None if b is None else torch.from_numpy(b).to(dev)
        w, ids = ops.route_grouped_sigmoid(torch.from_numpy(lg).to(dev), tb, n_group, topk_group, k, True, 2.5)
        np.testing.assert_array_equal(to_np(ids), ids_ref)
        np.testing.assert_allclose(to_np(w), w_ref, rtol=1e-6, atol=1e-7)


def test_grouped_sigmoid_ties_and_flips(dev):
    E, G = 64, 8
    lg = np.zeros((4, E), dtype=np.float32)  # all equal: lowest groups, lowest experts
    lg[1, :] = 1.0
    lg[1, 40:48] = 3.0  # group 5 dominates
    lg[2] = np.tile(np.arange(8, dtype=np.float32), 8)  # every group ties
    bias = np.zeros(E, dtype=np.float32)
    bias[63] = 5.0  # flips selection to expert 63 in row 3
    for b in (None, bias):
        w_ref, ids_ref = oracle.routing.grouped_sigmoid_topk(lg, b, G, 4, 8, True, 2.5)
        tb = None if b is None else torch.from_numpy(b).to(dev)
        w, ids = ops.route_grouped_sigmoid(torch.from_numpy(lg).to(dev), tb, G, 4, 8, True, 2.5)
        np.testing.assert_array_equal(to_np(ids), ids_ref)
        np.testing.assert_allclose(to_np(w), w_ref, rtol=1e-6, atol=1e-7)


# ----------------------------------------------------------------- align / slots


@pytest.mark.parametrize(
    "numel,E,bs",
    [(0, 8, 4), (12, 4, 4), (8, 256, 1), (64, 128, 16), (512, 256, 64), (2048, 256, 16), (1000, 1023, 8),
     (65536, 256, 64), (73728, 257, 128)],
)
def test_align_exact(dev, numel, E, bs):
    rng = np.random.default_rng(numel + E)
    ids = rng.integers(-1, E + 2, size=numel).astype(np.int32)  # includes skips, the sentinel bucket, junk
    s_ref, e_ref, n_ref = oracle.align.moe_align_block_size(ids, bs, E)
    s, e, n = ops.align(torch.from_numpy(ids).to(dev), bs, E)
    np.testing.assert_array_equal(to_np(n), n_ref)
    np.testing.assert_array_equal(to_np(s), s_ref)
    np.testing.assert_array_equal(to_np(e), e_ref)


def test_align_docstring_kat(dev):
    ids = torch.tensor([[2, 3, 4], [1, 2, 4], [1, 3, 4], [1, 2, 3]], dtype=torch.int32, device=dev)
    s, e, n = ops.align(ids, 4, 4)
    assert to_np(s)[:16].tolist() == [3, 6, 9, 12, 0, 4, 10, 12, 1, 7, 11, 12, 2, 5, 8, 12]
    assert int(to_np(n)[0]) == 16
    assert to_np(e)[:4].tolist() == [1, 2, 3, 4]


def test_slot_map_exact(dev):
    rng = np.random.default_rng(3)
    E, S = 256, 64
    table = np.full(E, -1, dtype=np.int32)
    res = rng.choice(E, S, replace=False)
    table[res] = rng.permutation(S)
    ids = rng.integers(-2, E + 3, size=(64, 8)).astype(np.int32)
    slots_ref, miss_ref, stats_ref = oracle.slots.slot_map(ids, table)
    t_ids = torch.from_numpy(ids).to(dev)
    miss = torch.empty(ids.shape, dtype=torch.uint8, device=dev)
    stats = torch.zeros(4, dtype=torch.int64, device=dev)
    out = ops.slot_map(t_ids, torch.from_numpy(table).to(dev), miss_mask=miss, stats=stats)
    np.testing.assert_array_equal(to_np(out), slots_ref)
    np.testing.assert_array_equal(to_np(miss), miss_ref)
    np.testing.assert_array_equal(to_np(stats), stats_ref)
    ops.slot_map(t_ids, torch.from_numpy(table).to(dev), out=t_ids, stats=stats)  # in place, accumulate
    np.testing.assert_array_equal(to_np(t_ids), slots_ref)
    np.testing.assert_array_equal(to_np(stats), 2 * stats_ref)


# ----------------------------------------------------------------- decode experts

# (name, routed fmt, rows, H, I, k, shared fmt or None, shared I)
DECODE_CASES = [
    ("c1_bf16", "bf16", 16, 1024, 512, 2, None, 0),
    ("c2_fp8_reduced", "fp8", 24, 2048, 768, 8, None, 0),
    ("c3_mxfp4_reduced", "mxfp4", 20, 1280, 384, 8, "bf16", 384),
    ("c4_fp8_reduced", "fp8", 16, 1024, 256, 8, "fp8", 256),
]


def _decode_case(name, fmt, rows, H, I, k, sfmt, sI, M, seed=0):
    rng = np.random.default_rng(seed + M)
    bank = synth.make_bank(fmt, rows, H, I, rng)
    shared = synth.make_bank(sfmt, 1, H, sI, rng) if sfmt else None
    x = synth.activations(rng, M, H)
    ids = np.stack([rng.choice(rows, k, replace=False) for _ in range(M)]).astype(np.int32)
    w = rng.random((M, k), dtype=np.float32)
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    return bank, shared, x, w, ids


@pytest.mark.parametrize("case", DECODE_CASES, ids=[c[0] for c in DECODE_CASES])
@pytest.mark.parametrize("M", [1, 4, 33, 64, 160])
def test_decode_parity(dev, case, M):
    """M = 64 and 160 put 25-80 routes on every expert: segments are cut into
    pieces of at most 32 routes and the shared expert into pieces of 32 tokens."""
    name, fmt, rows, H, I, k, sfmt, sI = case
    bank, shared, x, w, ids = _decode_case(*case, M)
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, shared)
    y = ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                           to_device_bank(bank, dev), to_device_bank(shared, dev) if shared else None)
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL, (name, M, max_rel(got, y_ref))
    assert cosine(got, y_ref) >= COS_TOL, (name, M, cosine(got, y_ref))


# Full-size C4 and C3 matrices on a few experts: long K loops through the
# weight rings (steady rounds and tails of every ring depth), two route chunks
# at M = 40 (40 routes per expert: pieces of 32 and 8).
FULL_SHAPE_CASES = [
    ("c4_fp8_full_shape", "fp8", 10, 7168, 2048, 8, "fp8", 2048),
    ("c3_mxfp4_full_shape", "mxfp4", 10, 5120, 1536, 8, "bf16", 1536),
]
_full_banks: dict = {}


@pytest.mark.parametrize("case", FULL_SHAPE_CASES, ids=[c[0] for c in FULL_SHAPE_CASES])
@pytest.mark.parametrize("M", [4, 40])
def test_decode_parity_full_shapes(dev, case, M):
    name, fmt, rows, H, I, k, sfmt, sI = case
    if name not in _full_banks:
        rng = np.random.default_rng(77)
        bank = code_bank(fmt, rows, H, I, rng)
        shared = code_bank(sfmt, 1, H, sI, rng) if sfmt != "bf16" else synth.make_bank("bf16", 1, H, sI, rng)
        _full_banks.clear()
        _full_banks[name] = (bank, shared, to_device_bank(bank, dev), to_device_bank(shared, dev))
    bank, shared, dbank, dshared = _full_banks[name]
    rng = np.random.default_rng(M)
    x = synth.activations(rng, M, H)
    ids = np.stack([rng.choice(rows, k, replace=False) for _ in range(M)]).astype(np.int32)
    w = rng.random((M, k), dtype=np.float32)
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, shared)
    y = ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev), dbank, dshared)
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL, (name, M, max_rel(got, y_ref))
    assert cosine(got, y_ref) >= COS_TOL, (name, M, cosine(got, y_ref))


# MXFP4 decode by shape: the gate_up stage's LDS code table (H a multiple of
# 512: 2, 4, 6 or 8 K steps of 256 split over the 4 waves, so at H = 512 two
# waves have no step and at H = 1536 the waves have 1 or 2) and the down
# stage's codes in registers (I a multiple of 256 up to 2048: 1, 2, 3 and 8 K
# steps; I = 2304, 9 steps, takes the per-step code loads), with one or two
# route chunks per pass and several passes or segments per expert (M = 200:
# 67 routes per expert).
MX_SHAPE_CASES = [(512, 256), (1024, 768), (1536, 512), (2048, 2048), (512, 2304)]


@pytest.mark.parametrize("H,I", MX_SHAPE_CASES, ids=[f"H{h}_I{i}" for h, i in MX_SHAPE_CASES])
@pytest.mark.parametrize("M", [1, 24, 90, 200])
def test_decode_mxfp4_code_paths(dev, H, I, M):
    bank, shared, x, w, ids = _decode_case("mx", "mxfp4", 12, H, I, 4, "bf16", I, M, seed=3)
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, shared)
    y = ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                           to_device_bank(bank, dev), to_device_bank(shared, dev))
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL, (H, I, M, max_rel(got, y_ref))
    assert cosine(got, y_ref) >= COS_TOL, (H, I, M, cosine(got, y_ref))


def test_decode_skips_and_weight_on_input(dev):
    bank, shared, x, w, ids = _decode_case(*DECODE_CASES[0], 8, seed=5)
    ids[0, 1] = -1
    ids[3, 0] = 99  # out of range: skipped
    for on_input in (False, True):
        y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, None, weight_on_input=on_input)
        y = ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                               to_device_bank(bank, dev), None, apply_router_weight_on_input=on_input)
        got = to_np(y)
        assert max_rel(got, y_ref) <= MAX_REL_TOL
        assert cosine(got, y_ref) >= COS_TOL


@pytest.mark.parametrize("batch_size", [1, 2, 4, 8, 16, 24])
def test_decode_noncontiguous_slots_recipe(dev, batch_size):
    """Recipe of the reference's tests/moe/test_fused_moe.py:61-98 (37 cache
    slots, fixed non-contiguous slot ids, top-8), at a 128-multiple geometry."""
    rng = np.random.default_rng(42 + batch_size)
    bank = synth.make_bank("bf16", 37, 256, 128, rng, std=0.5)
    x = bf16_round(0.5 * rng.standard_normal((batch_size, 256)).astype(np.float32))
    w = rng.random((batch_size, 8), dtype=np.float32)
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    ids = np.tile(np.array([31, 4, 18, 0, 29, 7, 35, 12], dtype=np.int32), (batch_size, 1))
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank)
    y = ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                           to_device_bank(bank, dev))
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL
    assert cosine(got, y_ref) >= COS_TOL


def test_decode_deterministic(dev):
    bank, shared, x, w, ids = _decode_case(*DECODE_CASES[3], 64, seed=9)
    args = (bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
            to_device_bank(bank, dev), to_device_bank(shared, dev))
    a = ops.experts_decode(*args).clone()
    b = ops.experts_decode(*args)
    assert torch.equal(a, b)


@pytest.mark.parametrize("M", [1, 16, 64])
def test_decode_cached_matches_slot_map_then_decode(dev, M):
    """ftmoe_experts_decode_cached (slot lookup inside the decode permutation)
    equals slot_map followed by experts_decode: slot ids, miss mask and
    counters exactly, the output bit for bit; out-of-range ids included."""
    rng = np.random.default_rng(23 + M)
    E, S, H, I = 64, 16, 1024, 256
    full = synth.make_bank("fp8", E, H, I, rng)
    shared = synth.make_bank("fp8", 1, H, I, rng)
    resident = np.sort(rng.choice(E, S, replace=False))
    table = np.full(E, -1, dtype=np.int32)
    table[resident] = np.arange(S, dtype=np.int32)
    ids = np.stack([rng.choice(E, 8, replace=False) for _ in range(M)]).astype(np.int32)
    ids[0, 0] = -1
    if M > 1:
        ids[1, 3] = E + 5
    w = rng.random((M, 8), dtype=np.float32)
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    x = bf16_dev(synth.activations(rng, M, H), dev)
    bank, sh = to_device_bank(full, dev, resident), to_device_bank(shared, dev)
    t_table, t_w = torch.from_numpy(table).to(dev), torch.from_numpy(w).to(dev)

    ids_a = torch.from_numpy(ids).to(dev)
    miss_a = torch.empty(ids.shape, dtype=torch.uint8, device=dev)
    stats_a = torch.zeros(4, dtype=torch.int64, device=dev)
    ops.slot_map(ids_a, t_table, out=ids_a, miss_mask=miss_a, stats=stats_a)
    y_a = ops.experts_decode(x, t_w, ids_a, bank, sh)

    ids_b = torch.from_numpy(ids).to(dev)
    miss_b = torch.empty(ids.shape, dtype=torch.uint8, device=dev)
    stats_b = torch.zeros(4, dtype=torch.int64, device=dev)
    y_b = ops.experts_decode(x, t_w, ids_b, bank, sh, slot_for_id=t_table, miss_mask=miss_b, stats=stats_b)

    slots_ref, miss_ref, stats_ref = oracle.slots.slot_map(ids, table)
    np.testing.assert_array_equal(to_np(ids_b), slots_ref)
    np.testing.assert_array_equal(to_np(miss_b), miss_ref)
    np.testing.assert_array_equal(to_np(stats_b), stats_ref)
    np.testing.assert_array_equal(to_np(stats_a), stats_ref)
    assert torch.equal(y_a, y_b)


def test_decode_slot_cache_misses(dev):
    """C4-style expert cache: routing over 64 experts, 16 resident slots; the
    non-resident routes are reported and excluded."""
    rng = np.random.default_rng(11)
    E, S, H, I, M = 64, 16, 1024, 256, 16
    full = synth.make_bank("fp8", E, H, I, rng)
    shared = synth.make_bank("fp8", 1, H, I, rng)
    resident = np.sort(rng.choice(E, S, replace=False))
    table = np.full(E, -1, dtype=np.int32)
    table[resident] = np.arange(S, dtype=np.int32)
    lg = synth.normal(rng, (M, E))
    bias = synth.normal(rng, (E,), 0.05)
    w_ref, ids_ref = oracle.routing.grouped_sigmoid_topk(lg, bias, 8, 4, 8, True, 2.5)
    slots_ref, miss_ref, stats_ref = oracle.slots.slot_map(ids_ref, table)
    x = synth.activations(rng, M, H)
    y_ref = oracle.experts.moe_layer("decode", x, w_ref, slots_ref, sub_bank(full, resident), shared)

    w, ids = ops.route_grouped_sigmoid(torch.from_numpy(lg).to(dev), torch.from_numpy(bias).to(dev), 8, 4, 8,
                                       True, 2.5)
    stats = torch.zeros(4, dtype=torch.int64, device=dev)
    slots = ops.slot_map(ids, torch.from_numpy(table).to(dev), stats=stats)
    y = ops.experts_decode(bf16_dev(x, dev), w, slots, to_device_bank(full, dev, resident),
                           to_device_bank(shared, dev))
    np.testing.assert_array_equal(to_np(slots), slots_ref)
    np.testing.assert_array_equal(to_np(stats), stats_ref)
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL
    assert cosine(got, y_ref) >= COS_TOL


@pytest.mark.parametrize("M", [4, 40, 256])
def test_decode_large_slot_bank(dev, M):
    """Decode over a 1664-slot bank (40 layers x 256 experts, the cache size of
    the reference's tests/moe/test_offload.py:379-404).  Above 1023 rows the
    permutation of more than 64 routes takes the sort-based align (M = 40: 320
    routes, M = 256: 2048 routes); M = 4 takes the one-wave align.  Both entry
    points: plain slot ids, and expert ids looked up in the permutation with
    the miss counters."""
    rng = np.random.default_rng(1664 + M)
    S, E, H, I, k = 1664, 2048, 256, 128, 8
    bank = code_bank("fp8", S, H, I, rng)
    dbank = to_device_bank(bank, dev)
    table = np.full(E, -1, dtype=np.int32)
    resident = rng.choice(E, S - 64, replace=False)
    table[resident] = rng.permutation(S)[: S - 64].astype(np.int32)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
    w = rng.random((M, k), dtype=np.float32)
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    x = synth.activations(rng, M, H)
    slots_ref, miss_ref, stats_ref = oracle.slots.slot_map(ids, table)
    y_ref = oracle.experts.moe_layer("decode", x, w, slots_ref, bank)
    xd, wd = bf16_dev(x, dev), torch.from_numpy(w).to(dev)

    y_a = ops.experts_decode(xd, wd, torch.from_numpy(slots_ref).to(dev), dbank)
    ids_b = torch.from_numpy(ids).to(dev)
    miss_b = torch.empty(ids.shape, dtype=torch.uint8, device=dev)
    stats_b = torch.zeros(4, dtype=torch.int64, device=dev)
    y_b = ops.experts_decode(xd, wd, ids_b, dbank, slot_for_id=torch.from_numpy(table).to(dev), miss_mask=miss_b,
                             stats=stats_b)
    np.testing.assert_array_equal(to_np(ids_b), slots_ref)
    np.testing.assert_array_equal(to_np(miss_b), miss_ref)
    np.testing.assert_array_equal(to_np(stats_b), stats_ref)
    for y in (y_a, y_b):
        got = to_np(y)
        assert max_rel(got, y_ref) <= MAX_REL_TOL, (M, max_rel(got, y_ref))
        assert cosine(got, y_ref) >= COS_TOL, (M, cosine(got, y_ref))
    assert torch.equal(y_a, y_b)


def test_decode_large_bank_matches_small_bank(dev):
    """The sort-based align (bank of 2048 rows) and the counting align (the
    same touched experts as a 1000-row bank) give bit-identical outputs."""
    rng = np.random.default_rng(5)
    H, I, k, M = 256, 128, 8, 48
    small = code_bank("fp8", 1000, H, I, rng)
    big = code_bank("fp8", 2048, H, I, rng)
    for name in ("gate_up", "down", "gate_up_scale", "down_scale"):
        getattr(big, name)[:1000] = getattr(small, name)
    ids = np.stack([rng.choice(1000, k, replace=False) for _ in range(M)]).astype(np.int32)
    ids[0, :3] = ids[1, :3]  # shared experts across tokens
    w = rng.random((M, k), dtype=np.float32)
    xd, wd, idd = bf16_dev(synth.activations(rng, M, H), dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev)
    y_small = ops.experts_decode(xd, wd, idd, to_device_bank(small, dev)).clone()
    y_big = ops.experts_decode(xd, wd, idd, to_device_bank(big, dev))
    assert torch.equal(y_small, y_big)


@pytest.mark.parametrize("with_shared", [False, True])
@pytest.mark.parametrize("M", [1, 5])
def test_decode_all_routes_skipped(dev, M, with_shared):
    """Every route skipped (ids -1 or beyond the bank): the output is exactly
    zero without a shared expert and exactly the shared expert's with one --
    the folded combine has no routed arrivals to wait for."""
    rng = np.random.default_rng(91 + M)
    E, H, I, k = 8, 512, 256, 4
    bank = synth.make_bank("fp8", E, H, I, rng)
    shared = synth.make_bank("fp8", 1, H, I, rng) if with_shared else None
    x = synth.activations(rng, M, H)
    ids = np.full((M, k), -1, dtype=np.int32)
    ids[:, 1] = E + 3
    w = np.full((M, k), 0.25, dtype=np.float32)
    y = ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                           to_device_bank(bank, dev), to_device_bank(shared, dev) if shared else None)
    got = to_np(y)
    if not with_shared:
        assert not got.any()
    else:
        ref = oracle.experts.moe_layer("decode", x, w, ids, bank, shared)
        assert max_rel(got, ref) <= MAX_REL_TOL and cosine(got, ref) >= COS_TOL


def test_empty_batch_through_ops(dev):
    """Zero tokens (as a serving step with no requests hands over): every
    router and expert call returns empty outputs without an error, and the
    next non-empty call is unaffected."""
    rng = np.random.default_rng(17)
    E, H, I, k = 8, 512, 256, 4
    bank = to_device_bank(synth.make_bank("fp8", E, H, I, rng), dev)
    shared = to_device_bank(synth.make_bank("fp8", 1, H, I, rng), dev)
    x0 = torch.empty((0, H), dtype=torch.bfloat16, device=dev)
    logits0 = torch.empty((0, E), dtype=torch.float32, device=dev)
    w0, ids0 = ops.route_softmax_topk(logits0, k, True)
    assert w0.shape == (0, k) and ids0.shape == (0, k)
    w1, ids1 = ops.route_grouped_sigmoid(logits0, None, 2, 1, k, True, 2.5)
    assert w1.shape == (0, k) and ids1.shape == (0, k)
    assert ops.experts_decode(x0, w0, ids0, bank, shared).shape == (0, H)
    assert ops.experts_prefill(x0, w0, ids0, bank, shared).shape == (0, H)
    slots = torch.arange(E, dtype=torch.int32, device=dev)
    assert ops.experts_decode(x0, w0, ids0, bank, None, slot_for_id=slots).shape == (0, H)
    for router in (ops.Router("softmax", k), ops.Router("grouped_sigmoid", k, n_group=2, topk_group=1, scale=2.5)):
        y, w, ids = ops.experts_decode_routed(x0, logits0, router, bank, shared)
        assert y.shape == (0, H) and w.shape == (0, k) and ids.shape == (0, k)
    torch.cuda.synchronize(dev)
    b, s, x, w, ids = _decode_case("empty_then", "fp8", E, H, I, k, "fp8", I, 3, seed=17)
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, b, s)
    got = to_np(ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                                   to_device_bank(b, dev), to_device_bank(s, dev)))
    assert max_rel(got, y_ref) <= MAX_REL_TOL and cosine(got, y_ref) >= COS_TOL


# The gelu forms of the *_and_mul epilogue (reference kernel/triton/activation.py:
# 99-109): the decode epilogue evaluates the activation per value with the
# runtime kind; bf16, FP8 and MXFP4 (with its bf16 shared expert) at one token
# and at 33 (several route chunks).
ACT_DECODE_CASES = [c for c in DECODE_CASES if c[0] in ("c1_bf16", "c2_fp8_reduced", "c3_mxfp4_reduced")]


@pytest.mark.parametrize("activation", ["gelu", "gelu_tanh"])
@pytest.mark.parametrize("case", ACT_DECODE_CASES, ids=[c[0] for c in ACT_DECODE_CASES])
@pytest.mark.parametrize("M", [1, 33])
def test_decode_activation_variants(dev, case, M, activation):
    name, fmt, rows, H, I, k, sfmt, sI = case
    bank, shared, x, w, ids = _decode_case(*case, M, seed=7)
    y_ref = oracle.experts.moe_layer("decode", x, w, ids, bank, shared, activation=activation)
    y = ops.experts_decode(bf16_dev(x, dev), torch.from_numpy(w).to(dev), torch.from_numpy(ids).to(dev),
                           to_device_bank(bank, dev), to_device_bank(shared, dev) if shared else None,
                           activation=activation)
    got = to_np(y)
    assert max_rel(got, y_ref) <= MAX_REL_TOL, (name, M, activation, max_rel(got, y_ref))
    assert cosine(got, y_ref) >= COS_TOL, (name, M, activation, cosine(got, y_ref))
    # and the activation is really applied: SiLU gives a different layer
    y_silu = oracle.experts.moe_layer("decode", x, w, ids, bank, shared)
    assert max_rel(y_silu, y_ref) > 4 * MAX_REL_TOL
