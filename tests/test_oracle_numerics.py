"""Pins of oracle/numerics.py against independent implementations (torch's
casts) and closed forms."""

import math

import numpy as np
import torch

from oracle import numerics as N


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 7,
        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.389e38, 1e-40, -1e-41, np.inf, -np.inf],
                 dtype=np.float32),
        # exact ties at the bf16 rounding point, both parities
        (np.arange(1, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32),
    ])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ref.view(np.uint32), N.bf16_round(x).view(np.uint32))
    assert np.isnan(N.bf16_round(np.array([np.nan], dtype=np.float32)))[0]


def test_e4m3_decode_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = N.e4m3_decode(codes)
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(got))
    assert np.array_equal(ref[~nan], got[~nan])
    assert N.E4M3_VALUES[0x7E] == 448.0 and N.E4M3_VALUES[1] == 2.0 ** -9


def test_e4m3_encode_matches_torch_on_grid_and_midpoints():
    vals = N.E4M3_VALUES[:127].astype(np.float64)
    mids = (vals[1:] + vals[:-1]) / 2
    rng = np.random.default_rng(1)
    x = np.concatenate([vals, mids, -vals, -mids, mids + 1e-9, mids - 1e-9,
                        rng.standard_normal(100000) * 40]).astype(np.float32)
    x = np.clip(x, -448, 448)
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ref, N.e4m3_encode(x))


def test_e4m3_encode_saturates():
    assert N.e4m3_decode(N.e4m3_encode(np.float32([1e6, -1e6, 460.0])))[:3].tolist() == [448.0, -448.0, 448.0]


def test_e2m1_table_and_ties():
    assert N.E2M1_VALUES.tolist()[:8] == [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    assert np.all(N.E2M1_VALUES[8:] == -N.E2M1_VALUES[:8])
    grid = np.float32([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    assert np.array_equal(N.e2m1_decode(N.e2m1_encode(grid)), grid)
    # ties-to-even on the grid (kernel/triton/dsv4/fp8_linear.py:148-169)
    probes = np.float32([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 7.0, -0.75, -3.5])
    expect = [0.0, 1.0, 1.0, 2.0, 2.0, 4.0, 4.0, 6.0, -1.0, -4.0]
    assert N.e2m1_decode(N.e2m1_encode(probes)).tolist() == expect
    # brute-force nearest with even tie break on random values
    rng = np.random.default_rng(2)
    x = (rng.random(20000) * 6.5).astype(np.float32)
    got = N.e2m1_decode(N.e2m1_encode(x))
    d = np.abs(x[:, None] - grid[None, :])
    best = d.min(1)
    assert np.all(np.abs(got - x) == best)


def test_pack_roundtrip():
    rng = np.random.default_rng(3)
    c = rng.integers(0, 16, (5, 64)).astype(np.uint8)
    p = N.pack_nibbles(c)
    assert p.shape == (5, 32)
    assert np.array_equal(p[:, 0] & 0xF, c[:, 0]) and np.array_equal(p[:, 0] >> 4, c[:, 1])
    assert np.array_equal(N.unpack_nibbles(p), c)


def test_log2_ceil_closed_form():
    rng = np.random.default_rng(4)
    v = np.concatenate([np.exp2(rng.integers(-60, 60, 500).astype(np.float64)),
                        rng.random(5000) * 1e3 + 1e-6]).astype(np.float32)
    expect = np.array([math.ceil(math.log2(float(t))) if t > 0 else 0 for t in v])
    # exact powers of two: log2 is exact
    assert np.array_equal(N.log2_ceil(v), expect)


def test_sigmoid_det_accuracy_and_monotone():
    x = np.linspace(-30, 30, 600001).astype(np.float32)
    s = N.sigmoid_det(x)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(s - ref) / ulp) <= 4.0
    assert np.all(np.diff(s) >= 0)
    assert N.sigmoid_det(np.float32([0.0]))[0] == 0.5
    e = N.exp_det(np.linspace(-80, 80, 10001).astype(np.float32))
    er = np.exp(np.linspace(-80, 80, 10001).astype(np.float32).astype(np.float64))
    assert np.max(np.abs(e - er) / er) < 5e-7


def test_gelu_pins():
    """The erf gelu of the oracle (reference kernel/triton/activation.py:108-109)
    against closed forms: gelu(x) = x Phi(x), so gelu(1) = Phi(1) and
    gelu(-1) = Phi(1) - 1 (math.erf in float64); gelu(x) - gelu(-x) = x; the
    saturated tails.  A 1/sqrt(2) written as sqrt(2), or a dropped 1/2, fails
    the first two."""
    phi1 = 0.5 * (1.0 + math.erf(1.0 / math.sqrt(2.0)))
    g = N.gelu_f32(np.array([1.0, -1.0, 10.0, -10.0, 0.0], np.float32)).astype(np.float64)
    assert abs(g[0] - phi1) <= 1e-7 and abs(g[1] - (phi1 - 1.0)) <= 1e-7
    assert g[2] == 10.0 and abs(g[3]) < 1e-20 and g[4] == 0.0
    x = np.linspace(-6, 6, 4001, dtype=np.float32)
    d = N.gelu_f32(x).astype(np.float64) - N.gelu_f32(-x).astype(np.float64)
    assert np.abs(d - x).max() <= 4 * np.spacing(np.float32(6.0))


def test_gelu_tanh_pins():
    """The tanh form (reference kernel/triton/activation.py:99-101): odd part
    gelu_tanh(x) - gelu_tanh(-x) = x, its value at 1 from the float64 closed
    form, and its known distance to the erf form (at most 4.8e-4 absolute on
    [-6, 6]; a 0.044715 coefficient left out moves it to 3.4e-2)."""
    u = math.sqrt(2.0 / math.pi) * (1.0 + 0.044715)
    t1 = 0.5 * (1.0 + math.tanh(u))
    assert abs(float(N.gelu_tanh_f32(np.array([1.0], np.float32))[0]) - t1) <= 1e-7
    x = np.linspace(-6, 6, 4001, dtype=np.float32)
    d = N.gelu_tanh_f32(x).astype(np.float64) - N.gelu_tanh_f32(-x).astype(np.float64)
    assert np.abs(d - x).max() <= 4 * np.spacing(np.float32(6.0))
    gap = np.abs(N.gelu_tanh_f32(x).astype(np.float64) - N.gelu_f32(x).astype(np.float64)).max()
    assert 1e-4 < gap <= 4.8e-4, gap


def test_act_f32_dispatch():
    x = np.linspace(-3, 3, 13, dtype=np.float32)
    np.testing.assert_array_equal(N.act_f32("silu", x), N.silu_f32(x))
    np.testing.assert_array_equal(N.act_f32("gelu", x), N.gelu_f32(x))
    np.testing.assert_array_equal(N.act_f32("gelu_tanh", x), N.gelu_tanh_f32(x))
    try:
        N.act_f32("swigluoai", x)
    except ValueError:
        pass
    else:
        raise AssertionError("unknown activation accepted")
