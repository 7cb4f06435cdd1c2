"""Independent pins of the oracle's prefill GEMMs (CPU).

The oracle's W8A8 fold (``oracle/experts.py: _gemm_w8a8``, restating
``kernel/triton/fp8_blockscale_moe.py:177-189``: ``acc += dot(a, w) * a_s * w_s``
per 128-deep K block after ``per_token_group_quant_fp8``,
``fp8_block_linear.py:38-82``) and its MXFP4 prefill composition (``_gemm`` for
"mxfp4", restating ``routed_experts_fp4_prefill``, ``moe/fused_ds_fp4.py:181-235``:
FP8 round trip of both GEMM inputs with a per-128 power-of-two scale,
``dsv4/fp8_linear.py:107-195``, times the dequantised e2m1 weights) are checked
here against things that do not share their code:

* the product of independently dequantised operands in float64 (torch's
  ``float8_e4m3fn`` cast for the activation codes and the weight codes, a
  fresh e2m1 table and ``math.ldexp`` for MXFP4, ``math.frexp`` for the
  power-of-two scale exponent);
* exact scale equivariance: multiplying one activation group or one weight
  scale block by 2^j leaves every code unchanged and multiplies exactly the
  contributions it owns by 2^j;
* the FP8 activation-quantisation error bound against the unquantised
  product, and the layer's prefill-vs-decode bound on the same banks;
* a per-element brute-force loop on a 2 x 256 x 256 case.

``test_checks_reject_planted_mistakes`` plants a missing activation scale, a
transposed weight-scale table and a shifted K-block index in copies of the
fold (on the CPU) and requires every check above to reject each of them.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import experts as X
from oracle import synth
from oracle.numerics import bf16_round, e4m3_decode, silu_f32

from conftest import cosine, max_rel

BLK = 128

# ---------------------------------------------------------------------------- independent primitives


def _torch_e4m3(v) -> np.ndarray:
    """float64 values of torch's RNE cast to float8_e4m3fn (saturating inputs are pre-clamped)."""
    t = torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32))
    return t.to(torch.float8_e4m3fn).to(torch.float64).numpy()


def _codes_e4m3(q) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(q, dtype=np.uint8)).view(torch.float8_e4m3fn).to(torch.float64).numpy()


def _act_fp8_dequant(x) -> np.ndarray:
    """per_token_group_quant_fp8 then dequant: s = max(amax, 1e-10)/448 in
    float32, q = e4m3(clamp(x/s)), value q*s (float64)."""
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    g = x.reshape(m, k // BLK, BLK)
    s = (np.maximum(np.abs(g).max(-1), np.float32(1e-10)) / np.float32(448.0)).astype(np.float32)
    q = _torch_e4m3(np.clip(g / s[..., None], -448.0, 448.0))
    return (q * s[..., None].astype(np.float64)).reshape(m, k)


def _w_fp8_dequant(q, s) -> np.ndarray:
    n, k = q.shape
    return _codes_e4m3(q) * np.repeat(np.repeat(np.asarray(s, np.float64), BLK, 0), BLK, 1)[:n, :k]


_E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]  # magnitudes of codes 0..7; bit 3 is the sign


def _w_mxfp4_dequant(packed, sc) -> np.ndarray:
    """W[n, k] = e2m1(nibble) * 2^(sc[n, k/32] - 127), low nibble = even k."""
    packed = np.asarray(packed, np.uint8)
    n, kh = packed.shape
    out = np.empty((n, 2 * kh), np.float64)
    for half, nib in ((0, packed & 0xF), (1, packed >> 4)):
        mag = np.asarray(_E2M1, np.float64)[nib & 7]
        out[:, half::2] = np.where(nib & 8, -mag, mag)
    scale = np.vectorize(lambda c: math.ldexp(1.0, int(c) - 127))(np.asarray(sc, np.int64)).astype(np.float64)
    return out * np.repeat(scale, 32, 1)


def _pow2_ceil_exp(v: float) -> int:
    """ceil(log2(v)) for v > 0 from frexp: v = m * 2^e with m in [0.5, 1)."""
    m, e = math.frexp(v)
    return e - 1 if m == 0.5 else e


def _act_ue8m0_roundtrip(x) -> np.ndarray:
    """act_quant_fp8_roundtrip (block 128): amax = max(amax, 1e-4),
    e = ceil(log2(amax * (1/448))), bf16(e4m3(x / 2^e) * 2^e) (float64 values)."""
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    g = x.reshape(m, k // BLK, BLK)
    amax = np.maximum(np.abs(g).max(-1), np.float32(1e-4)).astype(np.float32)
    e = np.vectorize(lambda a: _pow2_ceil_exp(float(np.float32(a) * np.float32(1.0 / 448.0))))(amax)
    sc = np.vectorize(lambda j: math.ldexp(1.0, int(j)))(e)
    q = _torch_e4m3(np.clip(g / sc[..., None], -448.0, 448.0))
    v = torch.from_numpy((q * sc[..., None]).astype(np.float32)).to(torch.bfloat16).to(torch.float64).numpy()
    return v.reshape(m, k)


def _bf16(v) -> np.ndarray:
    return torch.from_numpy(np.asarray(v, np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


# ---------------------------------------------------------------------------- the oracle's fold and planted mistakes


def _fold(x, w, s, *, act_scale=True, transpose_s=False, kb_shift=0):
    """A copy of the block fold ``acc += (xq.wq) * a_s[row, kb] * w_s[nb, kb]``
    with optional planted mistakes (only the checks' own tests use them)."""
    xq, xs = X.per_token_group_quant_fp8(x)
    n, k = w.shape
    nkb = k // BLK
    s = np.asarray(s, np.float32)
    if transpose_s:  # the table read with the other axis' strides
        s = np.ascontiguousarray(s.T).reshape(s.shape)
    xd, wd = e4m3_decode(xq), e4m3_decode(w)
    acc = np.zeros((x.shape[0], n), np.float32)
    for kb in range(nkb):
        sl = slice(kb * BLK, (kb + 1) * BLK)
        part = xd[:, sl] @ wd[:, sl].T
        if act_scale:
            part = part * xs[:, kb][:, None]
        acc = (acc + part * np.repeat(s[:, (kb + kb_shift) % nkb], BLK)[None, :]).astype(np.float32)
    return acc


def _fp8_case(seed: int, m: int = 6, n: int = 256, k: int = 256):
    """FP8 weights whose 128x128 blocks have very different scales (x 1, 4, 1/8, 16),
    so a scale read from the wrong block changes the result."""
    rng = np.random.default_rng(seed)
    w = synth.normal(rng, (n, k), 0.02)
    mult = np.array([[1.0, 4.0, 0.125, 16.0][(i + 2 * j) % 4] for i in range(n // BLK) for j in range(k // BLK)],
                    np.float32).reshape(n // BLK, k // BLK)
    w = w * np.repeat(np.repeat(mult, BLK, 0), BLK, 1)
    q, s = X.quantize_fp8_block(w)
    x = synth.activations(rng, m, k)
    x[:, :BLK] *= np.float32(8.0)  # activation groups of different magnitude
    return x, q, s


# ---------------------------------------------------------------------------- checks (each returns a reason or None)


def _check_dequant_product(fn, x, q, s):
    """(i) fn(x, q, s) == float64 product of torch-dequantised operands, to fp32 accumulation error."""
    ref = _act_fp8_dequant(x) @ _w_fp8_dequant(q, s).T
    mag = np.abs(_act_fp8_dequant(x)) @ np.abs(_w_fp8_dequant(q, s)).T
    err = np.abs(fn(x, q, s).astype(np.float64) - ref)
    return None if np.all(err <= 1e-5 * mag + 1e-30) else f"dequant product: max err/mag {float((err / (mag + 1e-30)).max()):.3g}"


def _check_quant_bound(fn, x, q, s):
    """(i') |fn - x.W| <= sum_k (2^-4 |x_k| + 2^-10 a_s) |W_nk| (e4m3 half-step, normal and subnormal)."""
    wd = _w_fp8_dequant(q, s)
    m, k = x.shape
    a_s = np.repeat(np.abs(x.reshape(m, k // BLK, BLK)).max(-1) / 448.0, BLK, 1)
    bound = (2.0 ** -4 * np.abs(x.astype(np.float64)) + 2.0 ** -10 * a_s) @ np.abs(wd).T
    err = np.abs(fn(x, q, s).astype(np.float64) - x.astype(np.float64) @ wd.T)
    return None if np.all(err <= bound * (1 + 1e-5) + 1e-30) else "act-quant error bound exceeded"


def _check_equivariance(fn, x, q, s):
    """(ii) One activation group scaled by 2^j scales its contribution by 2^j exactly; one weight
    scale block (nb, kb) scaled by 2^j scales rows nb of group kb's contribution by 2^j and leaves
    the other rows bit-identical."""
    m, k = x.shape
    n = q.shape[0]
    for g in range(k // BLK):
        xg = np.zeros_like(x)
        xg[:, g * BLK:(g + 1) * BLK] = x[:, g * BLK:(g + 1) * BLK]
        y0 = fn(xg, q, s)
        for j in (-3, 5):
            if not np.array_equal(fn((xg * np.float32(2.0 ** j)).astype(np.float32), q, s), y0 * np.float32(2.0 ** j)):
                return f"activation group {g} scaled by 2^{j}"
        for nb in range(n // BLK):
            s2 = s.copy()
            s2[nb, g] *= np.float32(8.0)
            y1 = fn(xg, q, s2)
            rows = slice(nb * BLK, (nb + 1) * BLK)
            others = np.ones(n, bool)
            others[rows] = False
            if not (np.array_equal(y1[:, rows], y0[:, rows] * np.float32(8.0))
                    and np.array_equal(y1[:, others], y0[:, others])):
                return f"weight scale block ({nb}, {g})"
    return None


def _check_brute_force(fn):
    """(iv) per-element loop on M=2, N=256, K=256 (2 x 2 scale blocks): sum over k of
    e4m3(x/a_s)*a_s * e4m3(W)*w_s, accumulated in float64 with plain Python floats."""
    x, q, s = _fp8_case(11, m=2, n=256, k=256)
    got = fn(x, q, s)
    wv = _codes_e4m3(q)
    for r in range(2):
        a_s = [max(float(np.abs(x[r, g * BLK:(g + 1) * BLK]).max()), 1e-10) for g in range(2)]
        a_s = [float(np.float32(a) / np.float32(448.0)) for a in a_s]
        xv = [float(_torch_e4m3(np.clip(np.float32(x[r, kk]) / np.float32(a_s[kk // BLK]), -448, 448).reshape(1))[0])
              * a_s[kk // BLK] for kk in range(256)]
        for nn in range(256):
            acc = 0.0
            mag = 0.0
            for kk in range(256):
                t = xv[kk] * float(wv[nn, kk]) * float(s[nn // BLK, kk // BLK])
                acc += t
                mag += abs(t)
            if abs(float(got[r, nn]) - acc) > 1e-5 * mag + 1e-30:
                return f"element ({r}, {nn})"
    return None


# ---------------------------------------------------------------------------- tests: W8A8


def test_w8a8_equals_dequantised_product():
    for seed in (0, 1):
        x, q, s = _fp8_case(seed, n=256, k=384)
        assert _check_dequant_product(X._gemm_w8a8, x, q, s) is None


def test_w8a8_within_activation_quantisation_bound():
    x, q, s = _fp8_case(2, n=384, k=256)
    assert _check_quant_bound(X._gemm_w8a8, x, q, s) is None


def test_w8a8_scale_equivariance():
    x, q, s = _fp8_case(3)
    assert _check_equivariance(X._gemm_w8a8, x, q, s) is None


def test_w8a8_brute_force_loop():
    assert _check_brute_force(X._gemm_w8a8) is None


def test_checks_reject_planted_mistakes():
    """Every check accepts the oracle's fold and rejects each planted mistake."""
    x, q, s = _fp8_case(4)
    mutants = {
        "missing a_s": lambda x, q, s: _fold(x, q, s, act_scale=False),
        "transposed w_s": lambda x, q, s: _fold(x, q, s, transpose_s=True),
        "wrong K block": lambda x, q, s: _fold(x, q, s, kb_shift=1),
    }
    checks = {
        "dequant product": lambda fn: _check_dequant_product(fn, x, q, s),
        "quant bound": lambda fn: _check_quant_bound(fn, x, q, s),
        "equivariance": lambda fn: _check_equivariance(fn, x, q, s),
        "brute force": _check_brute_force,
        "layer prefill vs decode": _layer_prefill_vs_decode_reason,
    }
    for cname, check in checks.items():
        assert check(X._gemm_w8a8) is None, cname
        assert check(lambda x, q, s: _fold(x, q, s)) is None, cname
        for mname, mutant in mutants.items():
            assert check(mutant) is not None, f"{cname} accepts {mname}"


# ---------------------------------------------------------------------------- tests: layer, prefill vs decode


def _layer_prefill_vs_decode_reason(fold=None):
    """(iii) The FP8 layer in the prefill regime (W8A8) stays within the activation-quantisation
    error of the decode regime (W8A16) on the same bank.  Two GEMMs with e4m3 inputs (2^-4
    relative half-step) put the honest fold at max-rel 0.04-0.055 and cosine ~0.999 over seeds;
    the planted mistakes land at cosine <= 0.45.  Bound: max-rel <= 0.1, cosine >= 0.997."""
    rng = np.random.default_rng(21)
    E, H, I, k, M = 6, 256, 256, 2, 12
    bank = synth.make_bank("fp8", E, H, I, rng)
    # block-scale spread, so that a scale from the wrong block is visible
    bank.gate_up_scale = (bank.gate_up_scale * np.float32(4.0) ** rng.integers(-2, 3, bank.gate_up_scale.shape)).astype(np.float32)
    bank.down_scale = (bank.down_scale * np.float32(4.0) ** rng.integers(-2, 3, bank.down_scale.shape)).astype(np.float32)
    x = synth.activations(rng, M, H)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
    w = rng.random((M, k)).astype(np.float32)
    dec = X.moe_layer("decode", x, w, ids, bank)
    saved = X._gemm_w8a8
    try:
        if fold is not None:
            X._gemm_w8a8 = fold
        with np.errstate(over="ignore"):  # a planted mistake can blow the activations up
            pre = X.moe_layer("prefill", x, w, ids, bank)
    finally:
        X._gemm_w8a8 = saved
    rel, cos = max_rel(pre, dec), cosine(pre, dec)
    return None if rel <= 0.1 and cos >= 0.997 else f"prefill vs decode: max-rel {rel:.3g}, cos {cos:.6f}"


def test_fp8_layer_prefill_vs_decode():
    assert _layer_prefill_vs_decode_reason() is None


def test_mxfp4_layer_prefill_vs_decode():
    rng = np.random.default_rng(22)
    E, H, I, k, M = 6, 256, 256, 2, 12
    bank = synth.make_bank("mxfp4", E, H, I, rng)
    shared = synth.make_bank("mxfp4", 1, H, I, rng)
    x = synth.activations(rng, M, H)
    ids = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
    w = rng.random((M, k)).astype(np.float32)
    dec = X.moe_layer("decode", x, w, ids, bank, shared)
    pre = X.moe_layer("prefill", x, w, ids, bank, shared)
    assert max_rel(pre, dec) <= 0.1 and cosine(pre, dec) >= 0.997


# ---------------------------------------------------------------------------- tests: MXFP4 prefill GEMM


def _mx_case(seed: int, m: int = 5, n: int = 64, k: int = 256):
    rng = np.random.default_rng(seed)
    w = synth.normal(rng, (n, k), 0.02)
    packed, sc = X.quantize_mxfp4(w)
    sc = (sc.astype(np.int32) + rng.integers(-3, 4, sc.shape)).astype(np.uint8)  # spread the block scales
    x = synth.activations(rng, m, k)
    x[:, BLK:] *= np.float32(0.01)
    return x, packed, sc


def test_mxfp4_prefill_gemm_equals_dequantised_product():
    """The oracle's MXFP4 prefill product == (independent FP8 power-of-two round trip of x)
    . (independent e2m1 x e8m0 dequant of W), to fp32 accumulation error."""
    for seed in (0, 1):
        x, packed, sc = _mx_case(seed)
        got = X._gemm("prefill", "mxfp4", x, packed, sc).astype(np.float64)
        xa = _act_ue8m0_roundtrip(x)
        wd = _w_mxfp4_dequant(packed, sc)
        ref, mag = xa @ wd.T, np.abs(xa) @ np.abs(wd).T
        assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-30)


def test_mxfp4_prefill_gemm_scale_equivariance():
    """Scaling one 128-group of x by 2^j scales its contribution by 2^j exactly (power-of-two
    activation scale); raising one e8m0 weight code by 3 scales exactly that 32-block's
    contribution to that row by 8."""
    x, packed, sc = _mx_case(2, m=3, n=16, k=256)
    gemm = lambda x_, sc_: X._gemm("prefill", "mxfp4", x_, packed, sc_)  # noqa: E731
    for g in range(2):
        xg = np.zeros_like(x)
        xg[:, g * BLK:(g + 1) * BLK] = x[:, g * BLK:(g + 1) * BLK]
        y0 = gemm(xg, sc)
        assert np.array_equal(gemm((xg * np.float32(16.0)).astype(np.float32), sc), y0 * np.float32(16.0))
        # one 32-block of K inside group g, one weight row
        x32 = np.zeros_like(x)
        x32[:, g * BLK + 32:g * BLK + 64] = x[:, g * BLK + 32:g * BLK + 64]
        x32[:, g * BLK] = x[:, g * BLK]  # a second block keeps the group's amax unchanged
        base = gemm(x32, sc)
        sc2 = sc.copy()
        sc2[5, g * 4 + 1] += 3
        y1 = gemm(x32, sc2)
        only = gemm(np.where(np.arange(x.shape[1]) == g * BLK, x32, 0).astype(np.float32), sc)
        # row 5 = 8 * (block contribution) + (the other block's contribution)
        np.testing.assert_allclose(y1[:, 5], 8 * (base[:, 5] - only[:, 5]) + only[:, 5], rtol=1e-6, atol=1e-9)
        assert np.array_equal(np.delete(y1, 5, axis=1), np.delete(base, 5, axis=1))


# ---------------------------------------------------------------------------- tests: whole prefill layer vs an independent loop


def _loop_layer(regime_fmt: str, x, tw, ids, bank, shared=None):
    """The reference's prefill layer per route, from independently dequantised operands
    (float64 products) with its bf16 rounding points (ic1, act, per-route ic3, the
    fp32 route sum, the shared add): ``fused_experts_fp8_blockscale`` / ``routed_experts_fp4_prefill``."""
    fp8 = regime_fmt == "fp8"

    def deq(which, e, b):
        if fp8:
            return _w_fp8_dequant(b.gate_up[e] if which == 0 else b.down[e],
                                  b.gate_up_scale[e] if which == 0 else b.down_scale[e])
        return _w_mxfp4_dequant(b.gate_up[e] if which == 0 else b.down[e],
                                b.gate_up_scale[e] if which == 0 else b.down_scale[e])

    act_in = _act_fp8_dequant if fp8 else _act_ue8m0_roundtrip

    def mlp(b, e, rows, rw):
        g = _bf16((act_in(rows) @ deq(0, e, b).T).astype(np.float32))
        inter = g.shape[1] // 2
        gt = torch.from_numpy(g[:, :inter])
        a = _bf16((torch.nn.functional.silu(gt) * torch.from_numpy(g[:, inter:])).numpy())
        d = (act_in(a) @ deq(1, e, b).T).astype(np.float32)
        if rw is not None:
            d = (d * rw[:, None]).astype(np.float32)
        return _bf16(d)

    x = _bf16(x)
    m, k = ids.shape
    y = np.zeros_like(x)
    for t in range(m):
        acc = np.zeros(x.shape[1], np.float32)
        for r in range(k):
            acc = (acc + mlp(bank, int(ids[t, r]), x[t:t + 1], tw[t, r:r + 1])[0]).astype(np.float32)
        y[t] = _bf16(acc)
    if shared is not None:
        y = _bf16(y + mlp(shared, 0, x, None))
    return y


def test_prefill_layer_matches_independent_loop():
    rng = np.random.default_rng(31)
    E, H, I, k, M = 5, 256, 256, 2, 7
    for fmt in ("fp8", "mxfp4"):
        bank = synth.make_bank(fmt, E, H, I, rng)
        shared = synth.make_bank(fmt, 1, H, I, rng)
        x = synth.activations(rng, M, H)
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int32)
        w = rng.random((M, k)).astype(np.float32)
        got = X.moe_layer("prefill", x, w, ids, bank, shared)
        ref = _loop_layer(fmt, x, w, ids, bank, shared)
        # float32 vs float64 accumulation can move a bf16 rounding (and then an fp8 code) by a step
        assert max_rel(got, ref) <= 2e-2 and cosine(got, ref) >= 0.9999, fmt
        assert np.mean(got == ref) > 0.9, fmt


def test_silu_of_oracle_matches_torch():
    g = np.linspace(-20, 20, 4001, dtype=np.float32)
    ref = torch.nn.functional.silu(torch.from_numpy(g)).numpy()
    np.testing.assert_allclose(silu_f32(g), ref, rtol=2e-6, atol=1e-7)
    assert np.array_equal(bf16_round(g), _bf16(g))
