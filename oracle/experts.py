"""Expert math of the MoE layer, with the reference's rounding points.

Weight layouts (``layers/moe.py:60-92``; ``kernel/triton/dsv4/fused_moe.py:10-14``):
  gate_up [S, 2I, H] (gate rows [0,I), up rows [I,2I)), down [S, H, I];
  fp8 block:  e4m3 codes + float32 scales [S, 2I/128, H/128] / [S, H/128, I/128];
  mxfp4:      packed [S, N, K/2] (low nibble = even k) + e8m0 codes [S, N, K/32];
  bf16:       float32 arrays holding bf16 values.

Rounding points restated (all others are float32):
  ic1 = bf16(gate_up GEMM)                 fp8_blockscale_moe.py:115-116, fused.py:379-394
  ic2 = bf16(silu(gate) * up)              kernel/triton/activation.py:91-112
  ic3 = bf16(down GEMM * router weight)    fp8_blockscale_moe.py:72-75,119-120
  y   = bf16(sum_r ic3, r = 0..k-1, fp32)  kernel/triton/fused_moe.py:142-153
  shared expert: bf16(down(bf16(silu*up)));  block output y = bf16(routed + shared)
                                           models/glm4_moe/moe.py:81-82
Decode W8A16 (bf16 activations, ``_decode_fp8_moe_kernel``, :23-75):
  acc[n] = sum_kb (sum_{k in kb} w[n,k] x[k]) * s[n/128, kb]
Prefill W8A8 (``_prefill_fp8_moe_kernel``, :131-197 + ``per_token_group_quant_fp8``,
fp8_block_linear.py:38-82): acc = sum_kb (xq.wq) * a_s[row,kb] * w_s[nb,kb].
MXFP4 decode (``_decode_dsfp4_moe_kernel``, dsv4/fused_moe.py:40-118) keeps bf16
activations; MXFP4 prefill (``_prefill_dsfp4_moe_kernel``, :168-270, driven by
``routed_experts_fp4_prefill``, moe/fused_ds_fp4.py:181-235) FP8-round-trips both
GEMM inputs with a per-128 power-of-two scale (``act_quant_fp8_roundtrip``,
dsv4/fp8_linear.py:107-195).

The shared expert of the FP8 layer runs W8A16 in decode for every batch size
(the reference's dense ``block_fp8_linear`` uses W8A16 only at M == 1,
fp8_block_linear.py:240-259) and W8A8 in prefill.

Pins (tests/test_oracle_experts.py): the float32 per-route loop of
``tests/moe/test_fused_moe.py:14-39`` on bf16 weights; dequantised-weight
equivalence (fp8 block path == bf16 path on the dequantised weights, up to
the documented rounding points); linearity in the router weights; a single
expert with identity-like weights reducing to silu(x)*x; and the C++ CPU
executor restatement (oracle/cpu_moe) on identical banks.
Prefill pins (tests/test_oracle_prefill.py): ``_gemm_w8a8`` and the MXFP4
prefill product against float64 products of independently dequantised
operands (torch's e4m3 cast, a separate e2m1 table, frexp exponents); exact
power-of-two equivariance per activation group and per weight scale block;
the e4m3 activation-quantisation error bound; a per-element brute-force loop;
the layer's prefill-vs-decode bound on FP8 and MXFP4 banks; a per-route loop
of the whole prefill layer; each check rejects a missing activation scale, a
transposed weight-scale table and a shifted K-block index.
"""

from __future__ import annotations

import numpy as np

from .numerics import (
    F32,
    bf16_round,
    e2m1_decode,
    e2m1_encode,
    e4m3_decode,
    e4m3_encode,
    log2_ceil,
    pack_nibbles,
    act_f32,
    unpack_nibbles,
)

BLK = 128

# --------------------------------------------------------------------------- quantizers


def quantize_fp8_block(w):
    """128x128 block FP8 with absmax-derived fp32 scales (synthetic weight
    generation for the FP8 configs): s = amax/448, q = e4m3(clamp(w/s, +-448)).
    Dequant is ``q * s`` (``kernel/triton/fp8_block_linear.py:262-271``)."""
    w = np.asarray(w, dtype=np.float32)
    *lead, n, k = w.shape
    blocks = w.reshape(*lead, n // BLK, BLK, k // BLK, BLK)
    amax = np.abs(blocks).max(axis=(-3, -1))
    s = (np.maximum(amax, F32(1e-12)) / F32(448.0)).astype(np.float32)
    q = e4m3_encode(np.clip(blocks / s[..., :, None, :, None], -448.0, 448.0).astype(np.float32))
    return q.reshape(*lead, n, k), s


def dequant_fp8_block(q, s):
    q = np.asarray(q)
    *lead, n, k = q.shape
    w = e4m3_decode(q).reshape(*lead, n // BLK, BLK, k // BLK, BLK)
    return (w * np.asarray(s, dtype=np.float32)[..., :, None, :, None]).reshape(*lead, n, k)


def quantize_mxfp4(w):
    """e2m1 with an e8m0 scale per 32 K: scale = 2^ceil(log2(amax/6)), so no
    element saturates; codes = e2m1(w / scale).  Returns (packed [.., N, K/2],
    scale codes [.., N, K/32])."""
    w = np.asarray(w, dtype=np.float32)
    *lead, n, k = w.shape
    blocks = w.reshape(*lead, n, k // 32, 32)
    amax = np.abs(blocks).max(axis=-1)
    e = np.where(amax > 0, log2_ceil(np.maximum(amax, F32(1e-30)) / F32(6.0)), 0)
    e = np.clip(e, -127, 127).astype(np.int32)
    codes = e2m1_encode((blocks / np.exp2(e.astype(np.float64))[..., None]).astype(np.float32))
    return pack_nibbles(codes.reshape(*lead, n, k)), (e + 127).astype(np.uint8)


def dequant_mxfp4(packed, scales):
    """``dequant_mxfp4_blocks`` (``moe/fused_mxfp4.py:28-72``) on the row-major
    ds_fp4 layout: W[n,k] = E2M1[code] * 2^(scale[n, k/32] - 127)."""
    codes = unpack_nibbles(packed)
    *lead, n, k = codes.shape
    v = e2m1_decode(codes).reshape(*lead, n, k // 32, 32)
    sc = np.exp2(np.asarray(scales, dtype=np.float64) - 127.0).astype(np.float32)
    return (v * sc[..., None]).reshape(*lead, n, k).astype(np.float32)


def per_token_group_quant_fp8(x, block: int = BLK):
    """``per_token_group_quant_fp8`` (``kernel/triton/fp8_block_linear.py:38-82``):
    s = max(amax, 1e-10)/448 per row per 128-group, q = e4m3(clamp(x/s, +-448))."""
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    g = x.reshape(m, k // block, block)
    amax = np.maximum(np.abs(g).max(axis=-1), F32(1e-10)).astype(np.float32)
    s = (amax / F32(448.0)).astype(np.float32)
    q = e4m3_encode(np.clip((g / s[..., None]).astype(np.float32), -448.0, 448.0))
    return q.reshape(m, k), s


def act_quant_ue8m0(x, block: int = BLK):
    """DSV4 ``act_quant`` with a power-of-two scale (``dsv4/fp8_linear.py:54-80``):
    amax = max(amax, 1e-4); e = ceil(log2(amax * (1/448))); q = e4m3(clamp(x/2^e)).
    Returns (codes [M,K], e8m0 scale codes [M,K/block])."""
    x = np.asarray(x, dtype=np.float32)
    m, k = x.shape
    g = x.reshape(m, k // block, block)
    amax = np.maximum(np.abs(g).max(axis=-1), F32(1e-4)).astype(np.float32)
    e = log2_ceil((amax * F32(1.0 / 448.0)).astype(np.float32))
    q = e4m3_encode(np.clip((g / np.exp2(e.astype(np.float64))[..., None]).astype(np.float32), -448.0, 448.0))
    return q.reshape(m, k), (e + 127).astype(np.uint8)


def act_roundtrip_ue8m0(x, block: int = BLK):
    """``act_quant_fp8_roundtrip`` (``dsv4/fp8_linear.py:180-195``): bf16(q * 2^e)."""
    q, codes = act_quant_ue8m0(x, block)
    m, k = q.shape
    v = e4m3_decode(q).reshape(m, k // block, block) * np.exp2(codes.astype(np.float64) - 127.0)[..., None]
    return bf16_round(v.reshape(m, k).astype(np.float32))


# --------------------------------------------------------------------------- GEMMs


class Bank:
    """One expert bank (routed experts or the shared expert, S = 1).
    ``swiglu_limit`` > 0: the bank's experts use the clamped SwiGLU
    (``swiglu``)."""

    def __init__(self, fmt: str, gate_up, down, gate_up_scale=None, down_scale=None, swiglu_limit: float = 0.0):
        assert fmt in ("bf16", "fp8", "mxfp4"), fmt
        self.fmt = fmt
        self.gate_up = gate_up
        self.down = down
        self.gate_up_scale = gate_up_scale
        self.down_scale = down_scale
        self.swiglu_limit = float(swiglu_limit)

    def weights(self, which: str, e: int):
        w = self.gate_up if which == "gate_up" else self.down
        s = self.gate_up_scale if which == "gate_up" else self.down_scale
        return w[e], (None if s is None else s[e])


def _gemm_w16(fmt, x, w, s):
    """y[r, n] = sum_k W[n,k] x[r,k] with bf16 activations (W8A16 / W4A16 / bf16)."""
    x = np.asarray(x, dtype=np.float32)
    if fmt == "bf16":
        return x @ np.asarray(w, dtype=np.float32).T
    if fmt == "mxfp4":
        return x @ dequant_mxfp4(w, s).T
    n, k = w.shape
    wd = e4m3_decode(w)
    acc = np.zeros((x.shape[0], n), dtype=np.float32)
    for kb in range(k // BLK):
        sl = slice(kb * BLK, (kb + 1) * BLK)
        part = x[:, sl] @ wd[:, sl].T
        acc = (acc + part * np.repeat(s[:, kb], BLK)[None, :]).astype(np.float32)
    return acc


def _gemm_w8a8(x, w, s):
    """W8A8 block GEMM: sum_kb (xq.wq) * a_s[row,kb] * w_s[nb,kb]
    (``fp8_blockscale_moe.py:177-189``)."""
    xq, xs = per_token_group_quant_fp8(x)
    n, k = w.shape
    xd = e4m3_decode(xq)
    wd = e4m3_decode(w)
    acc = np.zeros((x.shape[0], n), dtype=np.float32)
    for kb in range(k // BLK):
        sl = slice(kb * BLK, (kb + 1) * BLK)
        part = (xd[:, sl] @ wd[:, sl].T) * xs[:, kb][:, None]
        acc = (acc + part * np.repeat(s[:, kb], BLK)[None, :]).astype(np.float32)
    return acc


def _gemm(regime: str, fmt: str, x, w, s):
    if regime == "decode" or fmt == "bf16":
        return _gemm_w16(fmt, x, w, s)
    if fmt == "fp8":
        return _gemm_w8a8(x, w, s)
    # mxfp4 prefill: FP8 round-tripped activations x dequantised MXFP4 weights
    return act_roundtrip_ue8m0(x) @ dequant_mxfp4(w, s).T


def swiglu(activation: str, g, u, limit: float = 0.0):
    """float32 act(g) * u of the bf16 gate and up values.  With ``limit`` L > 0
    the DeepSeek-V4 clamped form: act(min(g, L)) * clamp(u, -L, L)
    (``_swiglu_kernel``, ``kernel/triton/dsv4/fused_moe.py:121-141``, used by
    ``routed_experts_fp4`` / ``routed_experts_fp4_prefill``,
    ``moe/fused_ds_fp4.py:124,226``; the CPU pass ``cpu_moe_ext.cpp:1769-1781``).
    The gate is capped from above only."""
    g = np.asarray(g, dtype=np.float32)
    u = np.asarray(u, dtype=np.float32)
    if limit > 0:
        lim = F32(limit)
        g = np.minimum(g, lim)
        u = np.minimum(np.maximum(u, -lim), lim)
    return (act_f32(activation, g) * u).astype(np.float32)


def expert_mlp(regime: str, bank: Bank, e: int, x_rows, route_w=None, weight_on_input: bool = False,
               activation: str = "silu"):
    """One expert on a set of rows: bf16(down(bf16(act(g)*u)) * w), act = silu
    unless ``activation`` names gelu or gelu_tanh (``kernel/triton/activation.py:68-112``),
    clamped as ``swiglu`` when the bank has a ``swiglu_limit``.

    With ``weight_on_input`` the router weight scales the gate_up output before
    its bf16 rounding instead of the down output (``MUL_ROUTED_WEIGHT`` on the
    first GEMM, ``moe/fused.py:302-331``)."""
    w1, s1 = bank.weights("gate_up", e)
    w2, s2 = bank.weights("down", e)
    g = _gemm(regime, bank.fmt, x_rows, w1, s1)
    if route_w is not None and weight_on_input:
        g = (g * np.asarray(route_w, dtype=np.float32)[:, None]).astype(np.float32)
    g = bf16_round(g)
    inter = g.shape[1] // 2
    act = bf16_round(swiglu(activation, g[:, :inter], g[:, inter:], bank.swiglu_limit))
    d = _gemm(regime, bank.fmt, act, w2, s2)
    if route_w is not None and not weight_on_input:
        d = (d * np.asarray(route_w, dtype=np.float32)[:, None]).astype(np.float32)
    return bf16_round(d)


def moe_layer(regime: str, x, topk_w, topk_ids, bank: Bank, shared: Bank | None = None,
              weight_on_input: bool = False, activation: str = "silu"):
    """Full MoE layer for a precomputed routing (``routed_forward``; ids index
    bank rows, ids < 0 or >= S are skipped and contribute nothing).

    Returns y (float32 holding bf16 values) [M, H]."""
    x = bf16_round(x)
    m, k = topk_ids.shape
    s_rows = (bank.gate_up.shape[0])
    h = x.shape[1]
    ic3 = np.zeros((m, k, h), dtype=np.float32)
    ids = np.asarray(topk_ids, dtype=np.int32)
    for e in np.unique(ids[(ids >= 0) & (ids < s_rows)]):
        t, r = np.nonzero(ids == e)
        ic3[t, r] = expert_mlp(regime, bank, int(e), x[t], topk_w[t, r], weight_on_input, activation)
    acc = np.zeros((m, h), dtype=np.float32)
    for r in range(k):
        acc = (acc + ic3[:, r]).astype(np.float32)
    y = bf16_round(acc)
    if shared is not None:
        sh = expert_mlp(regime, shared, 0, x, activation=activation)
        y = bf16_round(y + sh)
    return y
