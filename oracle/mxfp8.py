"""MXFP8 oracle: block-32 E4M3FN codes + E8M0 scales, SWIZZLE_32_4_4, dequant GEMM.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Integer/bit work in numpy.

Reference: src/models/ops/mxfp8_quant.py:15-74 (padding, E8M0 rule, CPU quantizer),
src/models/ops/mxfp8_kernels.py:15-27 (E8M0 rule, swizzle address), :87-110 (fused
prenorm producer), :62-84 (activation producer), src/models/ops/mxfp8_linear.py:83-90
(scaled GEMM + crop + bias), tests/test_paper_stack_mxfp8_ops.py:14-26 (dequant oracle).
"""
from __future__ import annotations

import math

import numpy as np


def pad128(n: int) -> int:
    return -(-n // 128) * 128


# ---------------------------------------------------------------- E4M3FN (bit level) ----

def e4m3fn_encode(v: np.ndarray) -> np.ndarray:
    """fp32 -> E4M3FN byte, round-to-nearest-even (|v| <= 448 expected).

    Independent integer restatement of the OCP E4M3FN format: bias 7, subnormals
    m/8 * 2^-6, no infinities. Used by the reference through torch's
    `.to(torch.float8_e4m3fn)` (mxfp8_quant.py:71-72).
    """
    v = np.ascontiguousarray(v, dtype=np.float32)
    if v.size > _CHUNK:
        flat = v.reshape(-1)
        return np.concatenate([_encode(flat[i:i + _CHUNK]) for i in range(0, flat.size, _CHUNK)]
                              ).reshape(v.shape)
    return _encode(v)


_CHUNK = 1 << 18


def _encode(v: np.ndarray) -> np.ndarray:
    bits = v.view(np.uint32).astype(np.int64)
    sign = (bits >> 31) & 1
    exp = (bits >> 23) & 0xFF
    man = (bits & 0x7FFFFF) | np.where(exp > 0, 0x800000, 0)
    unbiased = exp - 127
    # Number of fp32 mantissa bits dropped: 20 for normal E4M3 outputs, more below 2^-6.
    shift = np.where(unbiased >= -6, 20, 14 - unbiased)
    shift = np.minimum(shift, 40)
    q = man >> shift
    rem = man & ((np.int64(1) << shift) - 1)
    half = np.int64(1) << (shift - 1)
    up = (rem > half) | ((rem == half) & ((q & 1) == 1))
    q = q + up
    normal = unbiased >= -6
    # normal: q in [8, 16]; q == 16 carries into the exponent
    e_field = np.where(q >= 16, unbiased + 8, unbiased + 7)
    m_field = np.where(q >= 16, 0, q - 8)
    code_normal = (e_field << 3) | m_field
    # subnormal: q in units of 2^-9 in [0, 8]; 8 is exactly the smallest normal (code 8)
    code = np.where(normal, code_normal, q)
    code = np.where(exp == 0, 0, code)  # fp32 zero / denormal -> (signed) zero
    return (code | (sign << 7)).astype(np.uint8)


def e4m3fn_decode(codes: np.ndarray) -> np.ndarray:
    c = codes.astype(np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    val = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e - 7))
    val = np.where((e == 15) & (m == 7), np.nan, val)
    return (sign * val).astype(np.float64)


# ------------------------------------------------------------------------ E8M0 rule ----

def e8m0_exponent(amax: np.ndarray) -> np.ndarray:
    """Unbiased scale exponent of fp32 block maxima (mxfp8_quant.py:65-69)."""
    bits = np.ascontiguousarray(amax, dtype=np.float32).view(np.uint32).astype(np.int64)
    biased = (bits >> 23) & 0xFF
    e0 = biased - 135
    thr = (((e0 + 135) << 23) | 0x600000).astype(np.uint32).view(np.float32)
    e = e0 + (np.asarray(amax, dtype=np.float32) > thr)
    return np.maximum(e, -127)


def e8m0_exponent_closed_form(amax: np.ndarray) -> np.ndarray:
    """max(ceil(log2(amax / 448)), -127), and -127 for amax == 0 (exact in float64)."""
    a = np.asarray(amax, dtype=np.float64)
    with np.errstate(divide="ignore"):
        e = np.where(a > 0, np.ceil(np.log2(np.where(a > 0, a, 1.0) / 448.0)), -127)
    return np.maximum(e, -127).astype(np.int64)


# ------------------------------------------------------------------------- swizzle ----

def swizzle_offset(r: np.ndarray, c: np.ndarray, kp: int) -> np.ndarray:
    """Flat SWIZZLE_32_4_4 byte offset of natural scale (row r, K-block c) (mxfp8_kernels.py:25-27)."""
    r = np.asarray(r, dtype=np.int64)
    c = np.asarray(c, dtype=np.int64)
    return ((r // 128) * (kp // 128) + c // 4) * 512 + (r % 32) * 16 + ((r % 128) // 32) * 4 + c % 4


def swizzle(natural: np.ndarray) -> np.ndarray:
    rp, blocks = natural.shape
    out = np.zeros(rp * blocks, dtype=np.uint8)
    r, c = np.meshgrid(np.arange(rp), np.arange(blocks), indexing="ij")
    out[swizzle_offset(r, c, blocks * 32)] = natural
    return out


def unswizzle(flat: np.ndarray, rp: int, kp: int) -> np.ndarray:
    r, c = np.meshgrid(np.arange(rp), np.arange(kp // 32), indexing="ij")
    return np.asarray(flat)[swizzle_offset(r, c, kp)]


# ----------------------------------------------------------------------- quantizer ----

def quantize(x: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """fp32-representable [R, K] -> (codes [RP,KP] u8, natural scales [RP,KP/32] u8, flat swizzled).

    Reference: mxfp8_quant.py:40-74 / mxfp8_kernels.py:31-46. Padding is zero (scale byte 0).
    """
    codes, natural = quantize_natural(x)
    return codes, natural, swizzle(natural)


def quantize_natural(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """quantize() without the swizzled copy: (codes [RP,KP], natural scales [RP,KP/32])."""
    x = np.asarray(x, dtype=np.float32)
    r, k = x.shape
    rp, kp = pad128(r), pad128(k)
    full = np.zeros((rp, kp), dtype=np.float32)
    full[:r, :k] = x
    blocks = full.reshape(rp, kp // 32, 32)
    amax = np.abs(blocks).max(axis=-1)
    e = e8m0_exponent(amax)
    inv = ((127 - e) << 23).astype(np.uint32).view(np.float32)
    scaled = (blocks * inv[..., None]).astype(np.float32)
    codes = e4m3fn_encode(scaled).reshape(rp, kp)
    natural = (e + 127).astype(np.uint8)
    return codes, natural


_DECODE = None


def dequant(codes: np.ndarray, natural: np.ndarray) -> np.ndarray:
    global _DECODE
    if _DECODE is None:
        _DECODE = e4m3fn_decode(np.arange(256))
    rp, kp = codes.shape
    vals = _DECODE[codes].reshape(rp, kp // 32, 32)
    return (vals * np.exp2(natural.astype(np.float64) - 127)[..., None]).reshape(rp, kp)


# ---------------------------------------------------------------------------- bf16 ----

def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32/fp64 -> nearest-even bf16 value, returned as float32."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    b = f.view(np.uint32).astype(np.uint64)
    rounded = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    nan = np.isnan(f)
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out).astype(np.float32)


def bf16_from_bits(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint32) << 16).view(np.float32)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


# ------------------------------------------------------------------------------ GEMM ----

def gemm(a_codes, a_natural, w_codes, w_natural, rows: int, n: int, bias=None) -> np.ndarray:
    """bf16 result of the block-scaled GEMM (mxfp8_linear.py:83-90) from exact dequantized
    operands, float64 accumulation: crop [rows, N], round to bf16, + bias rounded again."""
    a = dequant(a_codes[:rows], a_natural[:rows])
    w = dequant(w_codes[:n], w_natural[:n])
    y = bf16_round(a @ w.T)
    if bias is not None:
        y = bf16_round(y.astype(np.float32) + np.asarray(bias, dtype=np.float32)[None, :])
    return y


def gemm_magnitude(a_codes, a_natural, w_codes, w_natural, rows: int, n: int) -> np.ndarray:
    """|A| @ |W|^T of the dequantized operands: the scale of the accumulation error."""
    a = np.abs(dequant(a_codes[:rows], a_natural[:rows]))
    w = np.abs(dequant(w_codes[:n], w_natural[:n]))
    return a @ w.T


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |x| (normal range)."""
    e = np.floor(np.log2(np.maximum(np.abs(np.asarray(x, dtype=np.float64)), 2.0 ** -126)))
    return 2.0 ** (e - 7)


# The scaled fp8 MFMA accumulates with less than fp32 precision: on gfx950 the
# measured error of one v_mfma_scale_f32_16x16x128_f8f6f4 is ~1.5e-4 of sum|a*w|.
# GEMM checks therefore bound |gpu - oracle| by one bf16 ulp plus this fraction of |A||W|^T.
MFMA_ACCUMULATION_BOUND = 2.0 ** -11


# ------------------------------------------------------------------------ producers ----

def prenorm(x, weight, eps, scale, shift, indices, return_magnitude=False):
    """bf16 value of the fused RMSNorm + AdaLN producer (mxfp8_kernels.py:87-110).

    fp32 arithmetic with one rounding per operation, as the reference evaluates it
    (Triton, enable_fp_fusion=False): inv = rsqrt(sum(x^2)/K + eps),
    ((x * inv) * w) * (1 + scale[i]) + shift[i], then one bf16 rounding. The sum of squares
    is formed in float64 and rounded once (its fp32 summation order is not specified).
    With return_magnitude, also returns |((x*inv)*w)*(1+scale)| + |shift|, the scale of
    the last addition (where cancellation can amplify an fp32 rounding of inv).
    """
    f = np.float32
    x = np.asarray(x, dtype=np.float32)
    ss = (x.astype(np.float64) ** 2).sum(axis=1, keepdims=True).astype(f)
    v = (ss / f(x.shape[1])).astype(f) + f(eps)
    inv = (1.0 / np.sqrt(v.astype(np.float64))).astype(f)
    sc = np.asarray(scale, dtype=f)[indices]
    sh = np.asarray(shift, dtype=f)[indices]
    t = (x * inv) * np.asarray(weight, dtype=f)
    u = t * (f(1.0) + sc)
    y = bf16_round(u + sh)
    if return_magnitude:
        return y, np.abs(u) + np.abs(sh)
    return y


def gelu_tanh(x) -> np.ndarray:
    """torch GELU(approximate='tanh'), evaluated in fp32 as torch does (opmath float), then
    rounded to bf16. fp32 matters in the negative tail, where 1 + tanh(u) cancels."""
    x = np.asarray(x, dtype=np.float32)
    beta = np.float32(math.sqrt(2.0 / math.pi))
    inner = beta * (x + np.float32(0.044715) * (x * x * x))
    return bf16_round(np.float32(0.5) * x * (np.float32(1.0) + np.tanh(inner)))


def swiglu(x) -> np.ndarray:
    """a * silu(g) for x = [a | g] in float64, rounded to bf16 (mxfp8_kernels.py:62-64)."""
    x = np.asarray(x, dtype=np.float64)
    k = x.shape[1] // 2
    a, g = x[:, :k], x[:, k:]
    return bf16_round(a * (g / (1.0 + np.exp(-g))))
