"""Number formats and scalar functions used by the MoE-layer oracle.

All arithmetic is numpy float32 (IEEE round-to-nearest-even per operation)
unless a docstring says otherwise.

Pins (tests/test_oracle_numerics.py):
  * ``bf16_round``  -- against torch's bfloat16 cast on CPU (an independent
    implementation) over random, edge and tie values.
  * ``e4m3_encode`` -- against torch.float8_e4m3fn (CPU) on all finite values
    and every midpoint between neighbouring codes; decode against the closed
    form of the OCP e4m3fn format.
  * ``e2m1_*``      -- the 16-entry table of ``moe/fused_mxfp4.py:47-68`` and
    the tie rule of ``kernel/triton/dsv4/fp8_linear.py:148-169`` (probe values
    0.75->1, 1.75->2, 3.5->4 documented there).
  * ``log2_ceil``   -- closed form ``ceil(log2(v))`` against math.frexp.
  * ``sigmoid_det`` -- against float64 ``1/(1+exp(-x))`` (<= 4 ulp) and
    monotonicity; its bit pattern is a *definition* shared with the HIP code.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32

# --------------------------------------------------------------------------- bf16


def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (RNE), returned as float32.

    Same rounding as the reference CPU executor's ``f32_to_bf16``
    (``kernel/csrc/cpu_moe/cpu_moe_ext.cpp:61-68``) and as every ``.to(bfloat16)``
    store in the Triton kernels.  NaN stays NaN.
    """
    a = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = out.copy()
        out[nan] = np.nan
    return out


def bf16_bits(x) -> np.ndarray:
    """uint16 bit patterns of ``bf16_round(x)``."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# --------------------------------------------------------------------------- e4m3 (OCP fn)

E4M3_MAX = 448.0


def _e4m3_table() -> np.ndarray:
    """Values of the 256 OCP e4m3fn codes (bias 7, no inf, 0x7f/0xff = NaN)."""
    vals = np.zeros(256, dtype=np.float64)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            vals[c] = np.nan
        elif e == 0:
            vals[c] = s * (m / 8.0) * 2.0 ** -6
        else:
            vals[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return vals


E4M3_VALUES = _e4m3_table().astype(np.float32)
_E4M3_POS = E4M3_VALUES[:127].astype(np.float64)  # codes 0..126, ascending, 0..448


def e4m3_decode(codes) -> np.ndarray:
    return E4M3_VALUES[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(x) -> np.ndarray:
    """float32 -> e4m3fn code, round-to-nearest-even, saturating at +-448.

    Callers in the reference clamp to +-448 before the cast
    (``kernel/triton/fp8_block_linear.py:55``), so saturation and the cast agree
    on every input they produce.
    """
    a = np.asarray(x, dtype=np.float32).astype(np.float64)
    sign = np.signbit(a)
    m = np.minimum(np.abs(a), E4M3_MAX)
    hi = np.searchsorted(_E4M3_POS, m, side="left")  # first value >= m
    hi = np.clip(hi, 0, 126)
    lo = np.clip(hi - 1, 0, 126)
    dlo = m - _E4M3_POS[lo]
    dhi = _E4M3_POS[hi] - m
    pick_hi = (dhi < dlo) | ((dhi == dlo) & ((hi & 1) == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(m == _E4M3_POS[hi], hi, code).astype(np.uint8)
    return np.where(sign, code | 0x80, code).astype(np.uint8)


def e4m3_round(x) -> np.ndarray:
    return e4m3_decode(e4m3_encode(x))


# --------------------------------------------------------------------------- e2m1 / e8m0

E2M1_VALUES = np.array(
    [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0],
    dtype=np.float32,
)  # moe/fused_mxfp4.py:47-68 (low nibble first, code 8..15 negative)


def e2m1_decode(codes) -> np.ndarray:
    return E2M1_VALUES[np.asarray(codes, dtype=np.uint8) & 0xF]


def e2m1_encode(x) -> np.ndarray:
    """float32 -> e2m1 code, RNE on the grid magnitudes, saturating at 6.

    Tie rule of ``kernel/triton/dsv4/fp8_linear.py:148-169``: 0.25->0, 0.75->1,
    1.25->1, 1.75->2, 2.5->2, 3.5->4, 5->4.
    """
    a = np.asarray(x, dtype=np.float32)
    m = np.abs(a)
    code = np.select(
        [m <= 0.25, m < 0.75, m <= 1.25, m < 1.75, m <= 2.5, m < 3.5, m <= 5.0],
        [0, 1, 2, 3, 4, 5, 6],
        default=7,
    ).astype(np.uint8)
    return np.where(np.signbit(a), code | 8, code).astype(np.uint8)


def e8m0_decode(codes) -> np.ndarray:
    """e8m0 code -> 2^(code-127) (``moe/fused_mxfp4.py:70``)."""
    return np.exp2(np.asarray(codes, dtype=np.float64) - 127.0).astype(np.float32)


def log2_ceil(v) -> np.ndarray:
    """Exact ceil(log2(v)) for positive normal float32 v via the IEEE fields
    (``kernel/triton/dsv4/fp8_linear.py:45-51``)."""
    b = np.asarray(v, dtype=np.float32).view(np.uint32)
    exp = ((b >> 23) & 0xFF).astype(np.int32)
    man = (b & 0x7FFFFF).astype(np.int32)
    return exp - 127 + (man != 0).astype(np.int32)


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """[..., K] 4-bit codes -> [..., K/2] bytes, low nibble = even k
    (``kernel/triton/dsv4/fused_moe.py:10-13``)."""
    c = np.asarray(codes, dtype=np.uint8)
    return (c[..., 0::2] | (c[..., 1::2] << 4)).astype(np.uint8)


def unpack_nibbles(packed: np.ndarray) -> np.ndarray:
    p = np.asarray(packed, dtype=np.uint8)
    out = np.empty(p.shape[:-1] + (p.shape[-1] * 2,), dtype=np.uint8)
    out[..., 0::2] = p & 0xF
    out[..., 1::2] = p >> 4
    return out


# --------------------------------------------------------------------------- sigmoid

# Deterministic float32 sigmoid shared bit-for-bit with the HIP router
# (freetoken_amd/csrc/ftmoe_common.h: det_sigmoid).  Selection in the grouped
# router compares sigmoid(logit)+bias, so both sides must produce identical
# bits; a library expf would not.  Method: Cody-Waite range reduction
# y = n*ln2 + r, |r| <= ln2/2, degree-6 Taylor polynomial in Horner form, then
# an exact ldexp.  Every step is a single IEEE float32 operation (no FMA).
_LOG2E = F32(float.fromhex("0x1.715476p+0"))
_LN2_HI = F32(float.fromhex("0x1.62e4p-1"))  # 0.693145751953125: 16 significant bits, n*LN2_HI exact
_LN2_LO = F32(float.fromhex("0x1.7f7d1cp-20"))
_C = [
    F32(float.fromhex("0x1.6c16c2p-10")),  # ~1/720
    F32(float.fromhex("0x1.111112p-7")),  # ~1/120
    F32(float.fromhex("0x1.555556p-5")),  # ~1/24
    F32(float.fromhex("0x1.555556p-3")),  # ~1/6
    F32(0.5),
    F32(1.0),
    F32(1.0),
]


def exp_det(y) -> np.ndarray:
    y = np.clip(np.asarray(y, dtype=np.float32), F32(-87.0), F32(87.0)).astype(np.float32)
    n = np.rint(y * _LOG2E).astype(np.float32)
    r = (y - n * _LN2_HI).astype(np.float32)
    r = (r - n * _LN2_LO).astype(np.float32)
    p = np.full_like(r, _C[0])
    for c in _C[1:]:
        p = (p * r + c).astype(np.float32)
    return np.ldexp(p, n.astype(np.int32)).astype(np.float32)


def sigmoid_det(x) -> np.ndarray:
    e = exp_det(-np.asarray(x, dtype=np.float32))
    return (F32(1.0) / (F32(1.0) + e)).astype(np.float32)


def gelu_f32(g) -> np.ndarray:
    """gelu(g) = g/2 (1 + erf(g / sqrt 2)) in float32 (``kernel/triton/activation.py:108-109``,
    the erf form of gelu_and_mul); erf evaluated in float64 and rounded."""
    from scipy.special import erf

    g = np.asarray(g, dtype=np.float32)
    e = erf(g.astype(np.float64) * 0.7071067811865476).astype(np.float32)
    return (F32(0.5) * g * (F32(1.0) + e)).astype(np.float32)


def gelu_tanh_f32(g) -> np.ndarray:
    """gelu_tanh(g) = g/2 (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))) in float32
    (``kernel/triton/activation.py:99-101``, gelu_tanh_and_mul); tanh evaluated in
    float64 and rounded (the reference's tanh.approx is not reproduced)."""
    g = np.asarray(g, dtype=np.float32)
    inner = (F32(0.7978845608028654) * (g + F32(0.044715) * g * g * g)).astype(np.float32)
    t = np.tanh(inner.astype(np.float64)).astype(np.float32)
    return (F32(0.5) * g * (F32(1.0) + t)).astype(np.float32)


def act_f32(kind: str, g) -> np.ndarray:
    """The activation of an *_and_mul epilogue by name: silu, gelu or gelu_tanh."""
    if kind == "silu":
        return silu_f32(g)
    if kind == "gelu":
        return gelu_f32(g)
    if kind == "gelu_tanh":
        return gelu_tanh_f32(g)
    raise ValueError(f"Unsupported activation: {kind}")


def silu_f32(g) -> np.ndarray:
    """silu(g) = g / (1 + e^-g) in float32 (``kernel/triton/activation.py:96-98``);
    the exponential is not bit-reproducible across implementations, so every
    use of it is compared under tolerance."""
    g = np.asarray(g, dtype=np.float32)
    return (g / (F32(1.0) + np.exp(-g.astype(np.float64)).astype(np.float32))).astype(np.float32)
