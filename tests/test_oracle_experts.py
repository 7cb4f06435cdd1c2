"""Pins of oracle/experts.py and oracle/slots.py."""

import numpy as np
import torch

from oracle import experts as X
from oracle import slots as S
from oracle import synth
from oracle.numerics import bf16_round, e4m3_decode, silu_f32

from conftest import cosine, max_rel


def _reference_loop(x, w1, w2, tw, ids):
    """The reference's fp32 per-route loop (tests/moe/test_fused_moe.py:14-39)."""
    out = np.zeros(x.shape, dtype=np.float32)
    for t in range(x.shape[0]):
        for r in range(ids.shape[1]):
            e = int(ids[t, r])
            gu = w1[e] @ x[t]
            i = gu.shape[0] // 2
            act = silu_f32(gu[:i]) * gu[i:]
            out[t] += (w2[e] @ act) * tw[t, r]
    return bf16_round(out)


def test_bf16_layer_matches_reference_loop():
    rng = np.random.default_rng(0)
    bank = synth.make_bank("bf16", 12, 256, 128, rng, std=0.1)
    x = synth.activations(rng, 6, 256)
    ids = np.stack([rng.choice(12, 4, replace=False) for _ in range(6)]).astype(np.int32)
    w = rng.random((6, 4)).astype(np.float32)
    y = X.moe_layer("decode", x, w, ids, bank)
    ref = _reference_loop(x, bank.gate_up, bank.down, w, ids)
    assert max_rel(y, ref) < 1e-2 and cosine(y, ref) > 0.9999


def test_fp8_w8a16_equals_dequantised_product():
    rng = np.random.default_rng(1)
    w = synth.normal(rng, (256, 384), 0.02)
    q, s = X.quantize_fp8_block(w)
    x = synth.activations(rng, 5, 384)
    got = X._gemm_w16("fp8", x, q, s)
    ref = x.astype(np.float64) @ X.dequant_fp8_block(q, s).astype(np.float64).T
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-6)


def test_fp8_block_quant_error_bound():
    rng = np.random.default_rng(2)
    w = synth.normal(rng, (256, 256), 0.02)
    q, s = X.quantize_fp8_block(w)
    err = np.abs(X.dequant_fp8_block(q, s) - w)
    # e4m3 relative step is 2^-3 -> half-step error <= 2^-4 * |w| (normals), plus
    # subnormal quantum 2^-9 * s
    bound = np.maximum(np.abs(w) * 2.0 ** -4, np.repeat(np.repeat(s, 128, 0), 128, 1) * 2.0 ** -10)
    assert np.all(err <= bound * 1.0001)
    assert np.all(np.abs(X.dequant_fp8_block(q, s)).max() <= np.abs(w).max() * 1.0001)


def test_mxfp4_quant_scale_and_error():
    rng = np.random.default_rng(3)
    w = synth.normal(rng, (64, 256), 0.02)
    p, sc = X.quantize_mxfp4(w)
    d = X.dequant_mxfp4(p, sc)
    scale = np.exp2(sc.astype(np.float64) - 127)
    blocks = np.abs(w).reshape(64, 8, 32).max(-1)
    assert np.all(blocks / scale <= 6.0) and np.all(blocks / scale > 3.0)  # smallest pow2 fitting
    # error at most half of the largest grid step (2) times the scale
    assert np.all(np.abs(d - w).reshape(64, 8, 32) <= scale[..., None] * 1.0 + 1e-12)


def test_per_token_group_quant_matches_torch():
    rng = np.random.default_rng(4)
    x = synth.activations(rng, 9, 256)
    q, s = X.per_token_group_quant_fp8(x)
    g = x.reshape(9, 2, 128)
    np.testing.assert_array_equal(s, (np.abs(g).max(-1) / np.float32(448)).astype(np.float32))
    ref = torch.from_numpy(np.clip(g / s[..., None], -448, 448).astype(np.float32).reshape(9, 256))
    ref = ref.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(q, ref)


def test_act_roundtrip_ue8m0_power_of_two():
    rng = np.random.default_rng(5)
    x = synth.activations(rng, 4, 256) * 3
    q, codes = X.act_quant_ue8m0(x)
    amax = np.abs(x.reshape(4, 2, 128)).max(-1)
    sc = np.exp2(codes.astype(np.float64) - 127)
    assert np.all(amax / sc <= 448) and np.all(amax / sc > 224)
    rt = X.act_roundtrip_ue8m0(x)
    np.testing.assert_array_equal(rt.reshape(4, 2, 128),
                                  bf16_round(e4m3_decode(q).reshape(4, 2, 128) * sc[..., None].astype(np.float32)))


def test_identity_expert_reduces_to_swiglu():
    h = 128
    eye = np.eye(h, dtype=np.float32)
    bank = X.Bank("bf16", np.concatenate([eye, eye])[None], eye[None])
    rng = np.random.default_rng(6)
    x = synth.activations(rng, 3, h)
    y = X.moe_layer("decode", x, np.ones((3, 1), np.float32), np.zeros((3, 1), np.int32), bank)
    np.testing.assert_array_equal(y, bf16_round(bf16_round(silu_f32(x) * x)))


def test_linearity_in_router_weight():
    rng = np.random.default_rng(7)
    bank = synth.make_bank("fp8", 6, 256, 128, rng)
    x = synth.activations(rng, 4, 256)
    ids = np.stack([rng.choice(6, 2, replace=False) for _ in range(4)]).astype(np.int32)
    w = rng.random((4, 2)).astype(np.float32)
    y1 = X.moe_layer("decode", x, w, ids, bank)
    y2 = X.moe_layer("decode", x, 2 * w, ids, bank)
    np.testing.assert_allclose(y2, 2 * y1, rtol=2 ** -7, atol=1e-6)


def test_skipped_routes_contribute_nothing():
    rng = np.random.default_rng(8)
    bank = synth.make_bank("bf16", 4, 128, 128, rng)
    x = synth.activations(rng, 2, 128)
    ids = np.array([[0, -1], [7, 2]], dtype=np.int32)
    w = np.ones((2, 2), np.float32)
    y = X.moe_layer("decode", x, w, ids, bank)
    y0 = X.moe_layer("decode", x[:1], w[:1, :1], ids[:1, :1], bank)
    np.testing.assert_array_equal(y[0], y0[0])


def test_slot_map_closed_form():
    table = np.array([2, -1, 0, -1, 1], dtype=np.int32)
    ids = np.array([[0, 1], [4, 9], [-1, 1]], dtype=np.int32)
    slots, miss, stats = S.slot_map(ids, table)
    assert slots.tolist() == [[2, -1], [1, -1], [-1, -1]]
    assert miss.tolist() == [[0, 1], [0, 0], [0, 1]]
    assert stats.tolist() == [3, 1, 1, 2]  # active {0,1,4}, missing {1}, calls, missed routes
    # identity table: no misses, slots == ids
    ident = np.arange(8, dtype=np.int32)
    ids2 = np.array([[0, 7, 3]], dtype=np.int32)
    s2, m2, st2 = S.slot_map(ids2, ident)
    assert s2.tolist() == ids2.tolist() and m2.sum() == 0 and st2[1] == 0


def test_cpu_executor_restatement_matches_oracle():
    """Two independent CPU implementations of the decode math agree: the numpy
    oracle and the C++ restatement of the reference's CPU executor
    (tolerance of the reference's CPU-vs-GPU check, tests/moe/test_cpu_moe.py:40-75)."""
    from oracle.cpu_moe import CpuMoe
    from oracle.numerics import bf16_bits

    rng = np.random.default_rng(9)
    for fmt, (E, H, I, k, M) in (("bf16", (16, 1024, 512, 4, 5)), ("mxfp4", (8, 512, 256, 2, 4))):
        bank = synth.make_bank(fmt, E, H, I, rng, std=0.1)
        x = synth.activations(rng, M, H)
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
        w = rng.random((M, k)).astype(np.float32)
        y_ref = X.moe_layer("decode", x, w, ids, bank)
        cpu = CpuMoe(H, I, k, E, fmt, cpus=[0, 1])
        if fmt == "bf16":
            cpu.set_bank(bf16_bits(bank.gate_up), bf16_bits(bank.down))
        else:
            cpu.set_bank(bank.gate_up, bank.down, bank.gate_up_scale, bank.down_scale)
        y = (cpu.run(bf16_bits(x), w, ids).astype(np.uint32) << 16).view(np.float32)
        cpu.close()
        assert max_rel(y, y_ref) < 2e-2 and cosine(y, y_ref) > 0.9995, fmt


def test_swiglu_clamp_special_cases():
    """The clamped SwiGLU (limit L): the gate is capped from above only, the up
    value clamped on both sides; values inside [-L, L] pass unchanged; L = 0 is
    the plain SwiGLU.  Expected values from float64 closed forms."""
    import math

    def silu64(v):
        return v / (1.0 + math.exp(-v))

    L = 7.0
    g = np.array([20.0, -20.0, 3.0, 7.0, 6.5, -3.0], np.float32)
    u = np.array([10.0, -10.0, -2.0, 8.0, -9.0, 7.5], np.float32)
    want = [silu64(7.0) * 7.0, silu64(-20.0) * -7.0, silu64(3.0) * -2.0, silu64(7.0) * 7.0, silu64(6.5) * -7.0,
            silu64(-3.0) * 7.0]
    got = X.swiglu("silu", g, u, L)
    np.testing.assert_allclose(got, np.array(want), rtol=2e-6, atol=1e-30)
    plain = X.swiglu("silu", g, u, 0.0)
    np.testing.assert_allclose(plain, [silu64(float(a)) * float(b) for a, b in zip(g, u)], rtol=2e-6, atol=1e-30)
    # a limit above every |value| changes nothing, bit for bit
    np.testing.assert_array_equal(X.swiglu("silu", g, u, 1e30), plain)


def test_identity_expert_with_clamped_swiglu():
    """gate = x, up = 2x through identity weights: the layer reduces to
    bf16(bf16(silu(min(x, L)) * clamp(2x, -L, L))), which fails if the clamp
    is applied to the wrong half or before the bf16 rounding of gate and up is
    lost; the router weight scales the down output after it."""
    h = 128
    eye = np.eye(h, dtype=np.float32)
    rng = np.random.default_rng(61)
    x = bf16_round(synth.activations(rng, 3, h) * np.float32(4.0))
    for L in (0.0, 1.5, 7.0):
        bank = X.Bank("bf16", np.concatenate([eye, 2 * eye])[None], eye[None], swiglu_limit=L)
        y = X.moe_layer("decode", x, np.ones((3, 1), np.float32), np.zeros((3, 1), np.int32), bank)
        g, u = x.astype(np.float64), 2.0 * x.astype(np.float64)
        if L > 0:
            g, u = np.minimum(g, L), np.clip(u, -L, L)
        act = bf16_round((g / (1.0 + np.exp(-g)) * u).astype(np.float32))
        np.testing.assert_allclose(y, bf16_round(act), rtol=2 ** -7, atol=0)
        if L == 1.5:
            assert (np.abs(2 * x) > L).mean() > 0.3  # the clamp binds on many values
