"""MXFP8 (block-32 E4M3FN + E8M0) operators with the reference's call signatures.

Mirrors src/models/ops/mxfp8_quant.py, mxfp8_kernels.py and mxfp8_linear.py: same
names, argument meaning, padded layouts, SWIZZLE_32_4_4 scale bytes and error
behaviour. Device work runs in libvdnmi.so (hand-written gfx950 kernels); there is no
Triton, no scaled_mm and no fallback: a device or build problem raises RuntimeError.
"""
from __future__ import annotations

import math

import numpy as np
import torch
from torch import nn

from . import _lib

SUPPORTED_ROLES = {
    "q": "attn.orig.to_q",
    "k": "attn.orig.to_k",
    "v": "attn.orig.to_v",
    "softmax_out": "attn.orig.to_out.0",
    "linear_out": "attn.to_out_linear",
    "ff_up": "ff.net.0.proj",
    "ff_down": "ff.net.2",
}

ACT_GELU_TANH = 1
ACT_SWIGLU = 2


# --------------------------------------------------------------------------------------
# layout helpers (mxfp8_quant.py:15-37)
# --------------------------------------------------------------------------------------

def padded_shape(rows: int, k: int) -> tuple[int, int]:
    if rows < 0 or k <= 0:
        raise ValueError("rows must be nonnegative and K positive")
    return (-(-rows // 128) * 128, -(-k // 128) * 128)


def scale_numel(rows: int, k: int) -> int:
    rp, kp = padded_shape(rows, k)
    return rp * (kp // 32)


def require_finite(x: torch.Tensor, name: str) -> None:
    if not bool(torch.isfinite(x).all()):
        raise ValueError(f"nonfinite MXFP8 {name}")


def _swizzle_index(rows: int, blocks: int) -> torch.Tensor:
    """Flat SWIZZLE_32_4_4 position of every natural (row, K-block) scale, [rows, blocks]."""
    r = torch.arange(rows, dtype=torch.int64)[:, None]
    c = torch.arange(blocks, dtype=torch.int64)[None, :]
    tile = (r // 128) * (blocks // 4) + c // 4
    return tile * 512 + (r % 32) * 16 + ((r % 128) // 32) * 4 + c % 4


def swizzle_scales(scales: torch.Tensor) -> torch.Tensor:
    """Natural padded [rows, K/32] bytes -> flat SWIZZLE_32_4_4 bytes."""
    r, c = scales.shape
    if scales.dtype != torch.uint8 or r % 128 or c % 4:
        raise ValueError("expected uint8 scales padded to 128 rows and 4 columns")
    out = torch.empty(r * c, dtype=torch.uint8, device=scales.device)
    out[_swizzle_index(r, c).reshape(-1).to(scales.device)] = scales.reshape(-1)
    return out


def _e8m0_exponent(amax: torch.Tensor) -> torch.Tensor:
    """Unbiased E8M0 exponent of fp32 block maxima, the bit rule of mxfp8_quant.py:65-69."""
    biased = (amax.view(torch.int32) >> 23) & 0xFF
    limit = ((biased << 23) | 0x600000).view(torch.float32)  # 1.75 * 2^(biased - 127)
    return torch.clamp(biased - 135 + (amax > limit).to(torch.int32), min=-127)


def quantize_cpu(x: torch.Tensor, *, chunk_rows: int = 128) -> tuple[torch.Tensor, torch.Tensor]:
    """CPU weight preparation (mxfp8_quant.py:40-74): padded codes + swizzled scales.

    Temporaries are bounded by `chunk_rows` rows of fp32. Meta tensors return
    correctly shaped buffers without reading data. Padding is exact zero.
    """
    if x.ndim != 2 or x.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise ValueError("expected a floating 2D weight")
    if x.device.type not in ("cpu", "meta"):
        raise ValueError("weights must be converted on CPU before distribution")
    if type(chunk_rows) is not int or chunk_rows <= 0:
        raise ValueError("chunk_rows must be a positive integer")
    r, k = x.shape
    rp, kp = padded_shape(r, k)
    data = torch.zeros((rp, kp), dtype=torch.uint8, device=x.device)
    natural = torch.zeros((rp, kp // 32), dtype=torch.uint8, device=x.device)
    if x.is_meta:
        return data, natural.reshape(-1)
    for lo in range(0, r, chunk_rows):
        hi = min(r, lo + chunk_rows)
        block = torch.zeros((hi - lo, kp), dtype=torch.float32)
        block[:, :k] = x[lo:hi].detach().float()
        require_finite(block, "weight")
        block = block.view(hi - lo, kp // 32, 32)
        exponent = _e8m0_exponent(block.abs().amax(dim=-1))
        pow2 = ((127 - exponent) << 23).view(torch.float32)
        codes = (block * pow2.unsqueeze(-1)).to(torch.float8_e4m3fn).view(torch.uint8)
        data[lo:hi] = codes.view(hi - lo, kp)
        natural[lo:hi] = (exponent + 127).to(torch.uint8)
    return data, swizzle_scales(natural)


# --------------------------------------------------------------------------------------
# device producers (mxfp8_kernels.py:31-58, 62-84, 87-139)
# --------------------------------------------------------------------------------------

def _unit_inner(x: torch.Tensor) -> bool:
    """Unit innermost stride where it matters (empty and width-1 tensors have no K stride)."""
    return x.stride(-1) == 1 or x.numel() == 0 or x.shape[-1] == 1


def _check_activation(x: torch.Tensor, what: str = "activation") -> None:
    if x.ndim != 2 or x.dtype != torch.bfloat16 or x.device.type != "cuda":
        raise ValueError(f"expected CUDA BF16 [rows,K] {what}")
    if not _unit_inner(x):
        raise ValueError(f"{what} K dimension must be contiguous")


def _row_stride(x: torch.Tensor, width: int) -> int:
    return x.stride(0) if x.shape[0] > 1 else max(x.stride(0), width)


def _new_outputs(x: torch.Tensor, rows: int, k: int):
    rp, kp = padded_shape(rows, k)
    q = torch.empty((rp, kp), dtype=torch.uint8, device=x.device)
    s = torch.empty(scale_numel(rows, k), dtype=torch.uint8, device=x.device)
    flag = torch.zeros(1, dtype=torch.int32, device=x.device)
    return q, s, flag


def empty_activation(rows: int, k: int, device):
    """Codes [RP, KP] and flat swizzled scales for an MXFP8 activation that fused producers
    (vdn_window_attention_mxfp8, vdn_vda_readout_mxfp8) fill chunk by chunk. The padding rows
    rows .. RP-1 are zeroed here (codes 0, scale bytes 0), as the quantize producer leaves
    them; every real row must then be written by the producers."""
    rp, kp = padded_shape(rows, k)
    q = torch.empty((rp, kp), dtype=torch.uint8, device=device)
    s = torch.empty(scale_numel(rows, k), dtype=torch.uint8, device=device)
    if rp > rows:
        q[rows:].zero_()
        # the scales of a 128-row block are one contiguous run of KP/128 x 512 bytes
        s[(rows // 128) * (kp // 128) * 512:].zero_()
    return q, s


def mxfp8_destination(dest, rows: int, heads: int, device):
    """Validates (codes, scales, chunk0) for a producer writing chunks chunk0 .. chunk0+heads-1
    of rows [0, rows)."""
    codes, scales, chunk0 = dest
    if (codes.dtype != torch.uint8 or scales.dtype != torch.uint8 or codes.ndim != 2
            or not codes.is_contiguous() or not scales.is_contiguous()
            or codes.device != device or scales.device != device):
        raise ValueError("MXFP8 destination must be contiguous uint8 codes [RP, KP] and scales "
                         "on the producer's device")
    rp, kp = codes.shape
    if rp % 128 or kp % 128 or rp < rows or scales.numel() != rp * kp // 32:
        raise ValueError("MXFP8 destination must be padded to 128 rows/columns with "
                         "RP * KP / 32 scale bytes")
    if isinstance(chunk0, bool) or not isinstance(chunk0, int) or chunk0 < 0 \
            or (chunk0 + heads) * 128 > kp:
        raise ValueError("chunk0 must leave room for one 128-column chunk per head")
    return codes, scales, chunk0


def launch_quantize(x: torch.Tensor):
    """bf16 [R,K] -> (codes u8 [RP,KP], flat swizzled scales u8). No finite check."""
    q, s, _ = _quantize(x)
    return q, s


def _quantize(x: torch.Tensor):
    _check_activation(x)
    r, k = x.shape
    q, s, flag = _new_outputs(x, r, k)
    if r:
        _lib.call("vdn_mxfp8_quantize", x.data_ptr(), r, k, _row_stride(x, k), q.data_ptr(),
                  s.data_ptr(), flag.data_ptr(), _lib.stream(x.device))
    return q, s, flag


def quantize_activation(x: torch.Tensor, *, check_finite: bool = True):
    """Fused pad + block-32 quantization + swizzle (mxfp8_quant.py:77-90).

    Finite checking is fail-closed by default: a nonfinite input raises
    ValueError("nonfinite MXFP8 activation") after one host synchronisation.
    """
    if x.ndim != 2 or x.dtype != torch.bfloat16 or x.device.type != "cuda":
        raise ValueError("expected CUDA BF16 [rows,K] activation")
    if not _unit_inner(x):
        raise ValueError("activation K dimension must be contiguous")
    q, s, flag = _quantize(x)
    if check_finite and int(flag.item()) != 0:
        raise ValueError("nonfinite MXFP8 activation")
    return q, s


def _act_quantize(x: torch.Tensor, k: int, act: int):
    r = x.shape[0]
    q, s, flag = _new_outputs(x, r, k)
    rp, kp = q.shape
    # one flag per (16-row, 256-column) tile, the reference producer's program grid
    finite = torch.ones(-(-rp // 16) * -(-kp // 256), dtype=torch.bool, device=x.device)
    if r:
        _lib.call("vdn_mxfp8_act_quantize", x.data_ptr(), r, k, _row_stride(x, x.shape[1]), act,
                  q.data_ptr(), s.data_ptr(), flag.data_ptr(), finite.data_ptr(),
                  _lib.stream(x.device))
    return q, s, finite


def launch_swiglu_quantize(x: torch.Tensor):
    """[R, 2K] -> MXFP8 of bf16(a * silu(g)), a = x[:, :K], g = x[:, K:] (mxfp8_kernels.py:113-124).

    Returns (codes, scales, finite): `finite` is bool [ceil(RP/16) * ceil(KP/256)], one flag
    per (16-row, 256-column) tile of the output, False where the tile's a, g or activation
    holds a nonfinite value (the reference producer's FINITE, one per program).
    """
    _check_activation(x)
    if x.shape[1] % 2:
        raise ValueError("SwiGLU input width must be even")
    return _act_quantize(x, x.shape[1] // 2, ACT_SWIGLU)


def launch_gelu_quantize(x: torch.Tensor):
    """[R, K] -> MXFP8 of bf16(gelu_tanh(x)); the GELU-tanh FFN's fused producer."""
    _check_activation(x)
    return _act_quantize(x, x.shape[1], ACT_GELU_TANH)


def launch_prenorm_quantize(x, weight, eps, scale, shift, indices, *, write_bf16):
    """RMSNorm(x; weight, eps) * (1 + scale[idx]) + shift[idx] -> bf16 -> MXFP8.

    Returns (bf16 [R,K] or None, codes, scales, finite bool [RP]) like
    mxfp8_kernels.py:127-139. Arithmetic is fp32 with a single bf16 rounding.
    """
    _check_activation(x)
    r, k = x.shape
    if weight.shape != (k,) or weight.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("weight must be [K] bf16 or fp32")
    for name, t in (("scale", scale), ("shift", shift)):
        if t.ndim != 2 or t.shape[1] != k or t.stride(-1) != 1:
            raise ValueError(f"{name} must be a [rows, K] table with contiguous K")
        if t.dtype not in (torch.bfloat16, torch.float32) or t.device != x.device:
            raise ValueError(f"{name} must be bf16/fp32 on the activation device")
    if scale.dtype != shift.dtype:
        raise ValueError("scale and shift must share a dtype")
    if indices.shape != (r,):
        raise ValueError("indices must be [rows]")
    if r and not math.isfinite(float(eps)):
        raise ValueError("eps must be finite")
    weight = weight.contiguous()
    indices = indices.to(device=x.device, dtype=torch.int64).contiguous()
    rp, kp = padded_shape(r, k)
    q = torch.empty((rp, kp), dtype=torch.uint8, device=x.device)
    s = torch.empty(scale_numel(r, k), dtype=torch.uint8, device=x.device)
    y = torch.empty((r, k), dtype=torch.bfloat16, device=x.device) if write_bf16 else None
    finite = torch.empty(rp, dtype=torch.bool, device=x.device)
    if r:
        flags = (1 if weight.dtype == torch.float32 else 0) | (2 if scale.dtype == torch.float32 else 0)
        _lib.call("vdn_mxfp8_prenorm_quantize", x.data_ptr(), r, k, _row_stride(x, k),
                  weight.data_ptr(), float(eps), scale.data_ptr(), scale.stride(0),
                  shift.data_ptr(), shift.stride(0), indices.data_ptr(), flags,
                  _lib.ptr(y), q.data_ptr(), s.data_ptr(), finite.data_ptr(),
                  _lib.stream(x.device))
    return y, q, s, finite


# --------------------------------------------------------------------------------------
# block-scaled GEMM (mxfp8_linear.py:36-142)
# --------------------------------------------------------------------------------------

def _matrix_arg(t, rows, n, name, device):
    if t is None:
        return None, 0
    if (t.dtype != torch.bfloat16 or t.ndim != 2 or t.shape[0] < rows or t.shape[1] != n
            or (t.shape[1] > 1 and t.stride(-1) != 1)):
        raise ValueError(f"{name} must be bf16 [rows, N] with contiguous N")
    if t.device != device:
        raise ValueError(f"{name} must be on the activation's device")
    if rows > 1 and t.stride(0) < n:
        raise ValueError(f"{name} rows overlap (row stride below N)")
    return t.data_ptr(), (t.stride(0) if rows > 1 else n)


def _row_starts(t, rows, n):
    """Element addresses (bf16 units) of the first element of each of `rows` rows."""
    stride = t.stride(0) if rows > 1 else n
    return t.data_ptr() // 2 + stride * np.arange(rows, dtype=np.int64)


def _check_alias(out, other, rows, n, name):
    """`out` may be exactly `other` (same address and row stride: each element is read and
    written by one lane) or share no element with it (for example the interleaved column
    halves of one buffer); a partial overlap would read values the kernel has already
    overwritten."""
    if other is None or rows == 0:
        return
    if out.data_ptr() == other.data_ptr() and (rows == 1 or out.stride(0) == other.stride(0)):
        return
    a, b = _row_starts(out, rows, n), _row_starts(other, rows, n)
    if a[-1] + n <= b[0] or b[-1] + n <= a[0]:
        return
    # rows of each view are disjoint and ascending: a row of `out` meets a row of `other`
    # when the first `other` row starting after a - n starts before a + n
    first = np.searchsorted(b, a - n + 1)
    hit = first < rows
    if np.any(b[np.minimum(first, rows - 1)][hit] < a[hit] + n):
        raise ValueError(f"out overlaps {name} without being the same view")


def _check_operand(t, rows, kp, what):
    if t.dtype != torch.uint8 or t.ndim != 2 or not t.is_contiguous():
        raise ValueError(f"{what} codes must be contiguous uint8 [rows, KP]")
    if t.shape[0] % 128 or t.shape[1] % 128 or t.shape[1] != kp or t.shape[0] < rows:
        raise ValueError(f"{what} codes must be padded to 128 rows and K")


def _check_scales(s, rows, kp, device, what):
    if s.dtype != torch.uint8 or not s.is_contiguous() or s.device != device:
        raise ValueError(f"{what} scales must be contiguous uint8 on the activation's device")
    if s.numel() != rows * (kp // 32):
        raise ValueError(f"{what} scales must hold RP * KP / 32 bytes")


def _nonfinite_flag(nonfinite, check_finite, device):
    """The device word a launch ORs 1 into on a nonfinite value: the caller's `nonfinite`
    (int32 [1], never read here, so no host sync), else a fresh zero when check_finite."""
    if nonfinite is not None:
        if (nonfinite.dtype != torch.int32 or nonfinite.numel() != 1 or
                nonfinite.device != device or not nonfinite.is_contiguous()):
            raise ValueError("nonfinite must be a contiguous int32 [1] tensor on the operands' device")
        return nonfinite
    return torch.zeros(1, dtype=torch.int32, device=device) if check_finite else None


def mxfp8_gemm(data, scales, weight_data, weight_scale, n, *, rows=None, bias=None, out=None,
               accumulate=False, addend=None, residual=None, gate=None, check_finite=False,
               nonfinite=None):
    """y[rows, n] = dequant(data) @ dequant(weight_data).T in bf16, then (each step rounded
    to bf16) + bias, addend + y, residual + gate * y.

    accumulate=True adds into `out` (addend = out), as `out += linear(x)`; `residual` /
    `gate` ([n]) fuse the block's gated residual `hidden + gate * branch`. `nonfinite`
    (int32 [1] on the device) becomes nonzero when an output is inf/NaN, with no host sync.
    """
    if data.device.type != "cuda":
        raise RuntimeError("native MXFP8 requires a HIP device; no fallback")
    dev = data.device
    if data.ndim != 2 or weight_data.ndim != 2:
        raise ValueError("MXFP8 codes must be 2D [rows, KP]")
    mp, kp = data.shape
    np_, kpw = weight_data.shape
    if kp != kpw:
        raise ValueError("activation and weight padded K differ")
    if weight_data.device != dev:
        raise ValueError("weight codes must be on the activation's device")
    _check_operand(data, 0, kp, "activation")
    _check_operand(weight_data, n, kp, "weight")
    _check_scales(scales, mp, kp, dev, "activation")
    _check_scales(weight_scale, np_, kp, dev, "weight")
    rows = mp if rows is None else rows
    if not 0 <= rows <= mp or not 0 < n <= np_:
        raise ValueError("rows and N must lie within the padded operands")
    if out is None:
        out = torch.empty((rows, n), dtype=torch.bfloat16, device=dev)
    elif out.shape != (rows, n) or out.dtype != torch.bfloat16 or (n > 1 and out.stride(-1) != 1):
        raise ValueError("out must be bf16 [rows, N] with contiguous N")
    elif out.device != dev:
        raise ValueError("out must be on the activation's device")
    elif rows > 1 and out.stride(0) < n:
        raise ValueError("out rows overlap (row stride below N)")
    if bias is not None:
        if bias.dtype != torch.bfloat16 or bias.shape != (n,) or bias.device != dev:
            raise ValueError("bias must be bf16 [N] on the activation's device")
        bias = bias.contiguous()
    if accumulate:
        if addend is not None:
            raise ValueError("accumulate and addend are exclusive")
        addend = out
    if gate is not None:
        if residual is None:
            raise ValueError("a gate needs a residual")
        gate = gate.reshape(-1)
        if gate.shape != (n,) or gate.dtype != torch.bfloat16 or gate.device != dev:
            raise ValueError("gate must be bf16 [N] on the activation's device")
        gate = gate.contiguous()
    add_ptr, ld_add = _matrix_arg(addend, rows, n, "addend", dev)
    res_ptr, ld_res = _matrix_arg(residual, rows, n, "residual", dev)
    _check_alias(out, addend, rows, n, "addend")
    _check_alias(out, residual, rows, n, "residual")
    flag = _nonfinite_flag(nonfinite, check_finite, dev)
    if rows:
        _lib.call("vdn_mxfp8_gemm", data.data_ptr(), scales.data_ptr(), mp,
                  weight_data.data_ptr(), weight_scale.data_ptr(), np_, kp, _lib.ptr(bias),
                  add_ptr, ld_add, res_ptr, ld_res, _lib.ptr(gate), out.data_ptr(), rows, n,
                  out.stride(0) if rows > 1 else n, _lib.ptr(flag), _lib.stream(data.device))
    if check_finite and int(flag.item()) != 0:
        raise ValueError("nonfinite MXFP8 result")
    return out


def interleave_swiglu(weight: torch.Tensor, bias: torch.Tensor | None = None):
    """[a | g] rows of a SwiGLU up projection ([2F, K], bias [2F]) -> the layout of the fused
    SwiGLU producer: each half padded to pad128(F) rows with zeros, then 128-row blocks
    interleaved a0, g0, a1, g1, ... ([2 pad128(F), K]); the bias likewise."""
    if weight.shape[0] % 2:
        raise ValueError("a SwiGLU up projection has an even number of rows")
    f = weight.shape[0] // 2
    fp = -(-f // 128) * 128

    def arrange(t):
        a, g = t[:f], t[f:]
        pad = (0, 0) * (t.ndim - 1) + (0, fp - f)
        a, g = torch.nn.functional.pad(a, pad), torch.nn.functional.pad(g, pad)
        rest = t.shape[1:]
        return torch.stack((a.reshape(fp // 128, 128, *rest), g.reshape(fp // 128, 128, *rest)),
                           dim=1).reshape(2 * fp, *rest)
    return arrange(weight), None if bias is None else arrange(bias)


def _gemm_swiglu_quantize(data, scales, weight_data, weight_scale, n, rows, bias, check_finite,
                          nonfinite):
    mp, kp = data.shape
    np_ = weight_data.shape[0]
    kp_out = -(-n // 128) * 128
    if np_ != 2 * kp_out:
        raise ValueError("SwiGLU takes the interleave_swiglu weight (2 pad128(n) rows)")
    rows = mp if rows is None else rows
    if mp < 1024 or np_ < 1024:
        # small problems: the GEMM's bf16 [a0 g0 a1 g1 ...] output, regrouped as [a | g], then
        # the stand-alone SwiGLU producer (the fused hand-over is in the persistent kernel)
        y = mxfp8_gemm(data, scales, weight_data, weight_scale, np_, rows=rows, bias=bias,
                       check_finite=check_finite, nonfinite=nonfinite)
        y = y.view(rows, kp_out // 128, 2, 128).transpose(1, 2).reshape(rows, 2, kp_out)
        q, s, fin = launch_swiglu_quantize(y[:, :, :n].reshape(rows, 2 * n))
        if nonfinite is not None:
            nonfinite.bitwise_or_((~fin.all()).to(torch.int32))
        if q.shape[0] != mp:
            q2 = torch.zeros((mp, kp_out), dtype=torch.uint8, device=data.device)
            s2 = torch.zeros(mp * kp_out // 32, dtype=torch.uint8, device=data.device)
            q2[:q.shape[0]] = q
            s2[:s.numel()] = s
            q, s = q2, s2
        return q, s
    q = torch.empty((mp, kp_out), dtype=torch.uint8, device=data.device)
    s = torch.empty(mp * kp_out // 32, dtype=torch.uint8, device=data.device)
    flag = _nonfinite_flag(nonfinite, check_finite, data.device)
    if rows:
        _lib.call("vdn_mxfp8_gemm_act_quantize", data.data_ptr(), scales.data_ptr(), mp,
                  weight_data.data_ptr(), weight_scale.data_ptr(), np_, kp, _lib.ptr(bias), 2,
                  q.data_ptr(), s.data_ptr(), rows, n, _lib.ptr(flag), _lib.stream(data.device))
    else:
        q.zero_()
        s.zero_()
    if check_finite and int(flag.item()) != 0:
        raise ValueError("nonfinite MXFP8 activation")
    return q, s


def mxfp8_gemm_act_quantize(data, scales, weight_data, weight_scale, n, *, rows=None, bias=None,
                            act="gelu_tanh", check_finite=False, nonfinite=None):
    """MXFP8 codes/scales of act(bf16(dequant(data) @ dequant(weight)ᵀ + bias)) for the next
    projection, produced in the GEMM epilogue. Bit-identical to mxfp8_gemm followed by
    launch_gelu_quantize (act "gelu_tanh"), launch_quantize (act None) or, for act "swiglu"
    over a weight from interleave_swiglu (n = the SwiGLU width), launch_swiglu_quantize of
    the [a | g] output. `nonfinite` (int32 [1] on the device) becomes nonzero on an inf/NaN
    activation, with no host sync.
    Returns (codes u8 [RP, pad128(n)], flat swizzled scales u8)."""
    mp, kp = data.shape
    np_, kpw = weight_data.shape
    if kp != kpw:
        raise ValueError("activation and weight padded K differ")
    if act not in ("gelu_tanh", "swiglu", None):
        raise ValueError("act must be 'gelu_tanh', 'swiglu' or None")
    if act == "swiglu":
        return _gemm_swiglu_quantize(data, scales, weight_data, weight_scale, n, rows, bias,
                                     check_finite, nonfinite)
    rows = mp if rows is None else rows
    kp_out = -(-n // 128) * 128
    q = torch.empty((mp, kp_out), dtype=torch.uint8, device=data.device)
    s = torch.empty(mp * kp_out // 32, dtype=torch.uint8, device=data.device)
    flag = _nonfinite_flag(nonfinite, check_finite, data.device)
    if rows:
        _lib.call("vdn_mxfp8_gemm_act_quantize", data.data_ptr(), scales.data_ptr(), mp,
                  weight_data.data_ptr(), weight_scale.data_ptr(), np_, kp, _lib.ptr(bias),
                  1 if act == "gelu_tanh" else 0, q.data_ptr(), s.data_ptr(), rows, n,
                  _lib.ptr(flag), _lib.stream(data.device))
    else:
        q.zero_()
        s.zero_()
    if check_finite and int(flag.item()) != 0:
        raise ValueError("nonfinite MXFP8 activation")
    return q, s


class MXFP8Linear(nn.Module):
    """Inference-only effective weight as two uint8 buffers (mxfp8_linear.py:36-102).

    There is no .weight attribute on purpose. A CPU weight is converted with
    quantize_cpu (the reference's weight preparation); a CUDA bf16 weight is converted
    on device by the same producer kernel activations use (identical bytes).
    """

    def __init__(self, linear: nn.Linear, *, chunk_rows=128, check_finite=True):
        super().__init__()
        if type(check_finite) is not bool:
            raise ValueError("check_finite must be a bool")
        if type(linear) is not nn.Linear:
            raise TypeError("MXFP8 requires an ordinary merged nn.Linear")
        self.in_features, self.out_features = linear.in_features, linear.out_features
        self.check_finite = check_finite
        w = linear.weight.detach()
        if w.device.type == "cuda" and w.dtype == torch.bfloat16:
            data, scales = quantize_activation(w.contiguous(), check_finite=True)
        else:
            data, scales = quantize_cpu(w, chunk_rows=chunk_rows)
        if linear.bias is not None and not linear.bias.is_meta:
            require_finite(linear.bias, "bias")
        self.register_buffer("weight_data", data)
        self.register_buffer("weight_scale", scales)
        self.register_parameter("bias", None if linear.bias is None else
                                nn.Parameter(linear.bias.detach(), requires_grad=False))
        self.eval()

    @torch.no_grad()
    def forward_quantized(self, data, scales, *, rows=None, out_dtype=torch.bfloat16, out=None,
                          accumulate=False, addend=None, residual=None, gate=None,
                          nonfinite=None):
        """Consume padded uint8 codes and swizzled scales, return cropped bf16 [rows, N].
        `nonfinite` (int32 [1] on the device): set nonzero on an inf/NaN output, no host sync."""
        if self.training or out_dtype != torch.bfloat16:
            raise ValueError("MXFP8 supports eval BF16 output only")
        if data.device.type != "cuda":
            raise RuntimeError("native MXFP8 requires a HIP device; no fallback")
        tensors = (data, scales, self.weight_data, self.weight_scale)
        if any(t.dtype != torch.uint8 or not t.is_contiguous() or t.device != data.device
               for t in tensors):
            raise ValueError("MXFP8 data/scales must be contiguous uint8 on the same CUDA device")
        np_, kp = padded_shape(self.out_features, self.in_features)
        if data.ndim != 2 or data.shape[1] != kp or data.shape[0] % 128:
            raise ValueError("invalid padded activation shape")
        if self.weight_data.shape != (np_, kp) or self.weight_scale.shape != (scale_numel(np_, kp),):
            raise ValueError("invalid compressed weight layout")
        if scales.shape != (scale_numel(data.shape[0], kp),):
            raise ValueError("invalid activation scale layout")
        if self.check_finite and (bool(((data & 127) == 127).any()) or bool((scales == 255).any())):
            raise ValueError("nonfinite MXFP8 prepared activation")
        rows = data.shape[0] if rows is None else rows
        if not 0 <= rows <= data.shape[0]:
            raise ValueError("invalid output row count")
        if rows == 0 and out is None:
            return torch.empty((0, self.out_features), device=data.device, dtype=out_dtype)
        bias = None
        if self.bias is not None:
            bias = self.bias.to(device=data.device, dtype=torch.bfloat16).contiguous()
        return mxfp8_gemm(data, scales, self.weight_data, self.weight_scale, self.out_features,
                          rows=rows, bias=bias, out=out, accumulate=accumulate, addend=addend,
                          residual=residual, gate=gate, check_finite=self.check_finite,
                          nonfinite=nonfinite)

    @classmethod
    def swiglu_up(cls, linear: nn.Linear, *, chunk_rows=128, check_finite=True):
        """The up projection of a SwiGLU FFN (rows [a | g], mxfp8_kernels.py:62-64) stored in
        the fused SwiGLU producer's layout (interleave_swiglu). forward_act_quantized(
        act="swiglu") then returns the MXFP8 activation a * silu(g), of width
        linear.out_features // 2; forward_quantized returns the GEMM in that layout."""
        if type(linear) is not nn.Linear:
            raise TypeError("MXFP8 requires an ordinary merged nn.Linear")
        w, b = interleave_swiglu(linear.weight.detach(),
                                 None if linear.bias is None else linear.bias.detach())
        inter = nn.Linear(w.shape[1], w.shape[0], bias=b is not None, dtype=w.dtype,
                          device=w.device)
        with torch.no_grad():
            inter.weight.copy_(w)
            if b is not None:
                inter.bias.copy_(b)
        module = cls(inter, chunk_rows=chunk_rows, check_finite=check_finite)
        module.swiglu_width = linear.out_features // 2
        return module

    @torch.no_grad()
    def forward_act_quantized(self, data, scales, *, rows=None, act="gelu_tanh", nonfinite=None):
        """Consume MXFP8 input and return the MXFP8 codes/scales of act(bf16 output): the
        producer of the next projection fused into this GEMM's epilogue. act "swiglu" needs a
        module built by swiglu_up."""
        if data.device.type != "cuda":
            raise RuntimeError("native MXFP8 requires a HIP device; no fallback")
        np_, kp = padded_shape(self.out_features, self.in_features)
        if data.ndim != 2 or data.shape[1] != kp or data.shape[0] % 128 or data.dtype != torch.uint8:
            raise ValueError("invalid padded activation shape")
        if scales.shape != (scale_numel(data.shape[0], kp),):
            raise ValueError("invalid activation scale layout")
        bias = None
        if self.bias is not None:
            bias = self.bias.to(device=data.device, dtype=torch.bfloat16).contiguous()
        n = self.out_features
        if act == "swiglu":
            n = getattr(self, "swiglu_width", None)
            if n is None:
                raise ValueError("act 'swiglu' needs the interleaved weight of swiglu_up")
        return mxfp8_gemm_act_quantize(data, scales, self.weight_data, self.weight_scale,
                                       n, rows=rows, bias=bias, act=act,
                                       check_finite=self.check_finite, nonfinite=nonfinite)

    @torch.no_grad()
    def forward(self, x):
        if x.ndim < 2 or x.shape[-1] != self.in_features or x.requires_grad:
            raise ValueError("MXFP8 expects inference activation [...,in_features]")
        rows = math.prod(x.shape[:-1])
        data, scales = quantize_activation(x.reshape(rows, self.in_features).contiguous(),
                                           check_finite=self.check_finite)
        return self.forward_quantized(data, scales, rows=rows).reshape(*x.shape[:-1],
                                                                       self.out_features)


def projection_features(module):
    if not isinstance(module, (nn.Linear, MXFP8Linear)):
        raise TypeError("unsupported projection module")
    return module.in_features, module.out_features


def project(module, x):
    projection_features(module)
    return module(x)


def project_to_out(to_out, x):
    if isinstance(to_out, (nn.ModuleList, nn.Sequential, list, tuple)):
        if len(to_out) != 2:
            raise ValueError("expected projection/dropout pair")
        return to_out[1](project(to_out[0], x))
    return project(to_out, x)


def project_qkv(projections, x):
    """One activation quantization shared by Q, K and V (mxfp8_linear.py:127-142)."""
    if len(projections) != 3:
        raise ValueError("expected Q, K, V")
    native = [isinstance(p, MXFP8Linear) for p in projections]
    if any(native) and not all(native):
        raise ValueError("mixed QKV precision is not supported")
    if not any(native):
        return tuple(project(p, x) for p in projections)
    if x.requires_grad or any(p.in_features != x.shape[-1] for p in projections):
        raise ValueError("invalid inference QKV input")
    rows = math.prod(x.shape[:-1])
    data, scales = quantize_activation(x.reshape(rows, x.shape[-1]).contiguous(),
                                       check_finite=any(p.check_finite for p in projections))
    return tuple(p.forward_quantized(data, scales, rows=rows).reshape(*x.shape[:-1], p.out_features)
                 for p in projections)


def convert_linear_to_mxfp8(model, *, enabled=False, chunk_rows=128, check_finite=True):
    """Default-off seven-role conversion of every transformer block (mxfp8_linear.py:145-180)."""
    if type(enabled) is not bool or type(check_finite) is not bool:
        raise ValueError("enabled and check_finite must be booleans")
    if not enabled:
        return []
    if model.training:
        raise ValueError("convert an eval model after effective-weight merging")
    uses = {}
    for _, parameter in model.named_parameters(remove_duplicate=False):
        uses[id(parameter)] = uses.get(id(parameter), 0) + 1
    targets, seen = [], set()
    for index, block in enumerate(model.transformer_blocks):
        for role, suffix in SUPPORTED_ROLES.items():
            child = block.get_submodule(suffix)
            if type(child) is not nn.Linear or child.weight.device.type not in ("cpu", "meta"):
                raise ValueError(f"{index}:{role} requires a merged CPU/meta nn.Linear")
            if id(child.weight) in seen or uses[id(child.weight)] != 1:
                raise ValueError("tied MXFP8 target weights are unsupported")
            seen.add(id(child.weight))
            parent, name = suffix.rsplit(".", 1)
            targets.append((index, role, block.get_submodule(parent), name, suffix))
    records = []
    for index, role, parent, name, suffix in targets:
        child = getattr(parent, name)
        records.append(dict(block=index, role=role, module=f"transformer_blocks.{index}.{suffix}",
                            in_features=child.in_features, out_features=child.out_features))
        setattr(parent, name, MXFP8Linear(child, chunk_rows=chunk_rows, check_finite=check_finite))
    return records
