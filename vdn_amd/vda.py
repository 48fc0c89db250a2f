"""VDA (frame-wise delta-rule linear attention) operators with the reference's signatures.

Mirrors src/models/linear_attention/paper_stack.py (paper_prepare, paper_statistics,
BoundaryPlan / paper_boundary_plan, paper_boundary_scan, paper_gather, paper_readout),
paper_factor.py (paper_delta_factors) and paper_sglang.py (vdn_linear_epilogue). Every
device step runs in libvdnmi.so; there is no eager or Triton fallback.

Two fused entry points have no single reference counterpart but compute exactly what the
reference chain computes, without the intermediate frame-major copies:
  statistics_from_projections  paper_prepare(k), paper_prepare(v) + paper_statistics
  linear_readout               paper_prepare(q) + q @ stateᵀ + vdn_linear_epilogue
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from functools import lru_cache

import torch
from torch import nn

from . import _lib
from .mxfp8 import mxfp8_destination

HEAD_DIM = 128
# Head dims the branch accepts. The kernels work on 128-wide rows; a smaller head dim runs
# with its channels zero-padded to 128, which is exact: SiLU(0) = 0 and zeros add nothing to
# the L2 norms, to A = Kᵀ diag(β) K and B = (vβ)ᵀ K (whose padded rows and columns are zero,
# so (I + A)⁻¹ is block diagonal with an identity block), to the scans and gathers (the
# state's padded rows and columns stay zero), and to the readout, whose RMSNorm takes its
# mean over the true head dim.
HEAD_DIMS = (16, 32, 64, 128)


def _check_head_dim(d):
    if d not in HEAD_DIMS:
        raise ValueError(f"head_dim must be one of {HEAD_DIMS}, got {d}")


def _pad_channels(x, value=0.0):
    """[..., d] -> [..., 128] with `value` in the added channels (x itself when d = 128)."""
    d = x.shape[-1]
    if d == HEAD_DIM:
        return x
    out = x.new_full((*x.shape[:-1], HEAD_DIM), value)
    out[..., :d] = x
    return out


def _pad_square(x):
    """[..., d, d] -> [..., 128, 128] zero-padded (x itself when d = 128)."""
    d = x.shape[-1]
    if d == HEAD_DIM:
        return x
    out = x.new_zeros((*x.shape[:-2], HEAD_DIM, HEAD_DIM))
    out[..., :d, :d] = x
    return out


def _cuda(t, name, dtype=None):
    if not isinstance(t, torch.Tensor) or not t.is_cuda or (dtype is not None and t.dtype != dtype):
        raise ValueError(f"{name} must be CUDA {dtype or 'floating point'}")
    if t.requires_grad:
        raise ValueError(f"{name}: paper stack is inference only")


def _stream(t):
    return _lib.stream(t.device)


# -------------------------------------------------------------------- prepare ----

class LinearAttentionSepConv(nn.Module):
    """The linear branch's separable short conv on the projections named in `projs`
    (features.py:133-196): per projection a depthwise 5x5 spatial Conv2d `{proj}_sp` and a
    depthwise 5-tap temporal Conv1d `{proj}_tm`, both bias-free, initialised N(0, 1/25) and
    N(0, 1/5) as the reference does. Parameter names and shapes match, so a reference
    state dict loads. The convolution itself runs in vdn_vda_conv_prepare (paper_prepare)."""

    KERNEL = 5

    def __init__(self, channels, projs=("k", "v")):
        super().__init__()
        self.projs = tuple(projs)
        k = self.KERNEL
        for name in self.projs:
            sp = nn.Conv2d(channels, channels, k, padding=k // 2, groups=channels, bias=False)
            nn.init.normal_(sp.weight, std=(k * k) ** -0.5)
            tm = nn.Conv1d(channels, channels, k, padding=k // 2, groups=channels, bias=False)
            nn.init.normal_(tm.weight, std=k ** -0.5)
            setattr(self, f"{name}_sp", sp)
            setattr(self, f"{name}_tm", tm)

    def weights(self, proj, dtype):
        """(w_sp [C, 25], w_tm [C, 5]) in `dtype`, contiguous (the temporal weight is cast to
        the activation dtype as in spatial(), features.py:193-195)."""
        w_sp = getattr(self, f"{proj}_sp").weight
        w_tm = getattr(self, f"{proj}_tm").weight
        c = w_sp.shape[0]
        return (w_sp.detach().reshape(c, 25).to(dtype).contiguous(),
                w_tm.detach().reshape(c, 5).to(dtype).contiguous())


def _conv_prepare(tokens, frames, spatial, l2norm, conv, proj, frame_size):
    if frame_size is None or frame_size[0] * frame_size[1] != spatial:
        raise ValueError("convolution requires the exact spatial frame_size")
    if tokens.dtype != torch.bfloat16:
        raise NotImplementedError("the gfx950 short-conv kernel takes bf16 tokens")
    n, h, d = tokens.shape
    w_sp, w_tm = conv.weights(proj, tokens.dtype)
    if w_sp.shape != (h * d, 25) or w_tm.shape != (h * d, 5):
        raise ValueError(f"{proj} conv has {w_sp.shape[0]} channels, tokens {h * d}")
    if w_sp.device != tokens.device:
        raise ValueError("conv weights must be on the tokens' device")
    if tokens.stride(-1) != 1 or tokens.stride(0) % 8 or tokens.stride(1) % 8 or tokens.data_ptr() % 16:
        tokens = tokens.contiguous()
    out = torch.empty((frames, h, spatial, d), dtype=tokens.dtype, device=tokens.device)
    _lib.call("vdn_vda_conv_prepare", tokens.data_ptr(), h, tokens.stride(0), tokens.stride(1),
              frames, int(frame_size[0]), int(frame_size[1]), w_sp.data_ptr(), w_tm.data_ptr(),
              int(bool(l2norm)), out.data_ptr(), _stream(tokens))
    return out


def paper_prepare(tokens, *, frames, spatial, l2norm, conv=None, proj=None, frame_size=None):
    """Raw [F*S, H, D] -> contiguous [F, H, S, D]: SiLU (+ L2 over D) (paper_stack.py:30-48).
    With a LinearAttentionSepConv listing `proj`, the spatial and temporal convolutions run
    first, fused into the same kernel (bf16 tokens; frame_size = (H_f, W_f))."""
    _cuda(tokens, "tokens")
    if tokens.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("paper_prepare supports BF16/FP32")
    if tokens.ndim != 3 or tokens.shape[0] != frames * spatial or min(frames, spatial) < 1:
        raise ValueError("tokens must be [frames*spatial, heads, dim] with positive sizes")
    n, h, d = tokens.shape
    _check_head_dim(d)
    if conv is not None and proj in getattr(conv, "projs", ()):
        if d != HEAD_DIM:
            raise NotImplementedError("the gfx950 short-conv kernel takes head_dim 128")
        return _conv_prepare(tokens, frames, spatial, l2norm, conv, proj, frame_size)
    if d != HEAD_DIM:
        out = paper_prepare(_pad_channels(tokens), frames=frames, spatial=spatial, l2norm=l2norm)
        return out[..., :d].contiguous()
    if tokens.stride(-1) != 1:
        tokens = tokens.contiguous()
    out = torch.empty((frames, h, spatial, d), dtype=tokens.dtype, device=tokens.device)
    _lib.call("vdn_vda_prepare", tokens.data_ptr(), n, h, tokens.stride(0), tokens.stride(1),
              frames, spatial, int(bool(l2norm)), int(tokens.dtype == torch.float32),
              out.data_ptr(), _stream(tokens))
    return out


# ----------------------------------------------------------------- statistics ----

def _stats_call(k, k_strides, v, v_strides, beta, b_strides, frames, heads, spatial, activate,
                a=None, b=None):
    if a is None:
        a = torch.empty((frames, heads, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=k.device)
        b = torch.empty_like(a)
    _lib.call("vdn_vda_statistics", k.data_ptr(), *k_strides, v.data_ptr(), *v_strides,
              beta.data_ptr(), *b_strides, int(beta.dtype == torch.float32), frames, heads,
              spatial, activate, a.data_ptr(), b.data_ptr(), _stream(k))
    return a, b


def paper_statistics(key, value, beta):
    """Joint A/B statistics of prepared [F,H,S,D] K/V and [F,H,S] beta (paper_stack.py:86-110).

    A = (Kᵀ diag(β) K + transpose)/2 in fp32-grade arithmetic; B = bf16(bf16(v·β)ᵀ k) for
    bf16 K/V. Both returned as fp32 [F,H,D,D].
    """
    for name, t in (("key", key), ("value", value), ("beta", beta)):
        _cuda(t, name)
    if (key.ndim != 4 or value.shape != key.shape or beta.shape != key.shape[:-1]
            or value.dtype != key.dtype or key.dtype not in (torch.bfloat16, torch.float32)
            or beta.dtype not in (torch.bfloat16, torch.float32)
            or any(t.device != key.device or not t.is_contiguous() for t in (value, beta, key))):
        raise ValueError("joint statistics require contiguous compatible F,H,S,D inputs")
    f, h, s, d = key.shape
    if min(f, h, s) < 1 or d not in (16, 32, 64, 128):
        raise ValueError("positive F,H,S and D in 16,32,64,128 required")
    if key.dtype != torch.bfloat16:
        raise NotImplementedError("the gfx950 statistics kernel takes bf16 K/V")
    if d != HEAD_DIM:
        a, b = paper_statistics(_pad_channels(key), _pad_channels(value), beta)
        return a[..., :d, :d].contiguous(), b[..., :d, :d].contiguous()
    ks = (h * s * d, s * d, d)
    bs = (h * s, s, 1)
    return _stats_call(key, ks, value, ks, beta, bs, f, h, s, 0)


def statistics_from_projections(k_raw, v_raw, beta, frames, spatial, a=None, b=None):
    """A/B statistics straight from raw token-major projections.

    k_raw, v_raw: [F*S, H, D] bf16 views (any row/head stride, unit channel stride), the
    pre-activation K/V of the shared QKV projection; beta: [F*S, H]. Equivalent to
    paper_statistics(paper_prepare(k, l2norm=True), paper_prepare(v, l2norm=False), beta
    reshaped to [F,H,S]); `a`/`b` may be preallocated [F,H,D,D] fp32 outputs.
    """
    for name, t in (("k_raw", k_raw), ("v_raw", v_raw), ("beta", beta)):
        _cuda(t, name)
    n, h, d = k_raw.shape
    if (v_raw.shape != k_raw.shape or d != HEAD_DIM or n != frames * spatial
            or beta.shape != (n, h) or k_raw.dtype != torch.bfloat16 or v_raw.dtype != torch.bfloat16
            or k_raw.stride(-1) != 1 or v_raw.stride(-1) != 1):
        raise ValueError("expected bf16 [frames*spatial, H, 128] projections and [F*S, H] beta")
    ks = (spatial * k_raw.stride(0), k_raw.stride(1), k_raw.stride(0))
    vs = (spatial * v_raw.stride(0), v_raw.stride(1), v_raw.stride(0))
    bs = (spatial * beta.stride(0), beta.stride(1), beta.stride(0))
    return _stats_call(k_raw, ks, v_raw, vs, beta, bs, frames, h, spatial, 1, a, b)


# -------------------------------------------------------------------- factors ----

def _check_factor_tensor(t, name):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.dtype != torch.float32:
        raise TypeError(f"{name} must have dtype float32, got {t.dtype}")
    if not t.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor")
    if t.layout != torch.strided or not t.is_contiguous():
        raise ValueError(f"{name} must have contiguous strided storage")
    if t.requires_grad:
        raise ValueError(f"{name} requires_grad is unsupported by this inference-only kernel")


def _aligned(t):
    return t if t.data_ptr() % 16 == 0 else t.clone()


def paper_delta_factors(A, B, alpha=None):
    """(diag(alpha) @ inv(I + A), B @ inv(I + A)) for [..., 128, 128] fp32 (paper_factor.py:133-186)."""
    _check_factor_tensor(A, "A")
    _check_factor_tensor(B, "B")
    if A.ndim < 2 or A.shape[-2:] != (HEAD_DIM, HEAD_DIM):
        raise ValueError("A must have shape [..., 128, 128]")
    if B.shape != A.shape:
        raise ValueError("B shape must exactly equal A shape")
    if B.device != A.device:
        raise ValueError("A and B must be on the same CUDA device")
    if alpha is not None:
        _check_factor_tensor(alpha, "alpha")
        if alpha.shape != A.shape[:-1]:
            raise ValueError("alpha must have exact shape [..., 128] matching A")
        if alpha.device != A.device:
            raise ValueError("alpha must be on the same CUDA device as A")
    transition, injection = torch.empty_like(A), torch.empty_like(B)
    if A.numel() == 0:
        return transition, injection
    n = A.numel() // (HEAD_DIM * HEAD_DIM)
    A, B = _aligned(A), _aligned(B)
    al = None if alpha is None else _aligned(alpha)
    _lib.call("vdn_vda_factors", A.data_ptr(), B.data_ptr(), _lib.ptr(al), n,
              transition.data_ptr(), injection.data_ptr(), _stream(A))
    return transition, injection


# ------------------------------------------------------------- boundary plan ----

@dataclass(frozen=True)
class BoundaryPlan:
    frames: int
    cuts: tuple
    starts: torch.Tensor
    ends: torch.Tensor
    before: torch.Tensor
    after: torch.Tensor
    has_before: torch.Tensor
    has_after: torch.Tensor
    bridge_before: torch.Tensor
    bridge_after: torch.Tensor

    @property
    def chunks(self):
        return len(self.cuts) - 1


@lru_cache(maxsize=64)
def _boundary_plan(bounds, frames, chunk_size, device):
    """Compact boundary plan (paper_stack.py:131-154): chunk cut points are every window edge
    plus splits every `chunk_size` frames between edges; each frame reads the prefix bank of
    the chunk ending at its window start and the suffix bank of the chunk starting after it."""
    if frames < 1 or len(bounds) != frames or chunk_size < 1:
        raise ValueError("positive frames/chunk_size and one bound per frame required")
    edges = {0, frames}
    for f, (lo, hi) in enumerate(bounds):
        if not lo <= f <= hi:
            raise ValueError("each inclusive window must contain its query frame")
        edges.add(max(0, lo))
        edges.add(min(frames, hi + 1))
    ordered = sorted(edges)
    cuts = set(ordered)
    for a, b in zip(ordered[:-1], ordered[1:]):
        cuts.update(range(a + chunk_size, b, chunk_size))
    cuts = tuple(sorted(cuts))
    index = {x: i for i, x in enumerate(cuts)}
    last_chunk = len(cuts) - 2

    def i32(values):
        return torch.tensor(values, dtype=torch.int32, device=device)

    return BoundaryPlan(
        frames, cuts, i32(cuts[:-1]), i32(cuts[1:]),
        i32([max(0, index[max(0, lo)] - 1) for lo, _ in bounds]),
        i32([min(last_chunk, index[min(frames, hi + 1)]) for _, hi in bounds]),
        i32([int(lo > 0) for lo, _ in bounds]),
        i32([int(hi + 1 < frames) for _, hi in bounds]),
        i32([max(0, lo) for lo, _ in bounds]),
        i32([min(frames, hi + 1) for _, hi in bounds]))


def paper_boundary_plan(bounds, frames, device, chunk_size=8):
    return _boundary_plan(tuple(tuple(int(x) for x in b) for b in bounds), int(frames),
                          int(chunk_size), str(device))


# ----------------------------------------------------------------------- scan ----

def paper_boundary_scan(transitions, injections, plan, text_state=None):
    """Chunk composition, then both directional scans: bank [2, C, H, D, D] fp32
    (paper_stack.py:202-236). bank[0, c] is the forward state after chunk c; bank[1, c] the
    reverse state after chunk c (i.e. covering frames cuts[c]..F-1)."""
    _cuda(transitions, "transitions", torch.float32)
    _cuda(injections, "injections", torch.float32)
    if (transitions.ndim != 4 or transitions.shape != injections.shape
            or transitions.device != injections.device
            or not transitions.is_contiguous() or not injections.is_contiguous()):
        raise ValueError("matching contiguous FP32 [F,H,D,D] factors required")
    f, h, d, dk = transitions.shape
    if f != plan.frames or d != dk or d not in (16, 32, 64, 128) or h < 1:
        raise ValueError("factor geometry incompatible with boundary plan")
    if plan.starts.device != transitions.device:
        raise ValueError("plan and factors must share a device")
    if text_state is not None:
        _cuda(text_state, "text_state", torch.float32)
        if text_state.shape != (h, d, d) or text_state.device != transitions.device:
            raise ValueError("text_state must be head-local H,D,D")
        text_state = text_state.contiguous()
    if d != HEAD_DIM:
        bank = paper_boundary_scan(_pad_square(transitions), _pad_square(injections), plan,
                                   None if text_state is None else _pad_square(text_state))
        return bank[..., :d, :d].contiguous()
    shape = (2, plan.chunks, h, d, d)
    bank = transitions.new_empty(shape)
    stream = _stream(transitions)
    if plan.chunks == f:
        # every chunk is one frame: both directions scan the frame factors themselves
        _lib.call("vdn_vda_scan", transitions.data_ptr(), injections.data_ptr(),
                  _lib.ptr(text_state), plan.chunks, h, 0, bank.data_ptr(), stream)
        return bank
    ct = transitions.new_empty(shape)
    ci = transitions.new_empty(shape)
    _lib.call("vdn_vda_compose", transitions.data_ptr(), injections.data_ptr(), h,
              plan.starts.data_ptr(), plan.ends.data_ptr(), plan.chunks, ct.data_ptr(),
              ci.data_ptr(), stream)
    _lib.call("vdn_vda_scan", ct.data_ptr(), ci.data_ptr(), _lib.ptr(text_state), plan.chunks,
              h, 1, bank.data_ptr(), stream)
    return bank


# --------------------------------------------------------------------- gather ----

def paper_gather(bank, alpha, plan, text_state=None, out_dtype=torch.bfloat16, bridge=True):
    """Alpha-bridged boundary gather [F, H, D, D] (paper_stack.py:239-263)."""
    _cuda(bank, "bank", torch.float32)
    _cuda(alpha, "alpha", torch.float32)
    if bank.ndim != 5 or bank.shape[:2] != (2, plan.chunks):
        raise ValueError("bank must be [2,chunks,H,D,D]")
    _, _, h, d, dk = bank.shape
    if (d != dk or alpha.shape != (plan.frames, h, d) or not bank.is_contiguous()
            or alpha.device != bank.device or plan.starts.device != bank.device
            or out_dtype not in (torch.bfloat16, torch.float32)):
        raise ValueError("gather geometry/device/dtype mismatch")
    if text_state is not None:
        _cuda(text_state, "text_state", torch.float32)
        if text_state.shape != (h, d, d) or text_state.device != bank.device:
            raise ValueError("text_state geometry/device mismatch")
        text_state = text_state.contiguous()
    if d != HEAD_DIM:
        _check_head_dim(d)
        out = paper_gather(_pad_square(bank), _pad_channels(alpha, 1.0), plan,
                           None if text_state is None else _pad_square(text_state), out_dtype,
                           bridge)
        return out[..., :d, :d].contiguous()
    alpha = alpha.contiguous()
    stream = _stream(bank)
    logp = None
    if bridge:
        logp = torch.empty((plan.frames + 1, h, d), dtype=torch.float32, device=bank.device)
        _lib.call("vdn_vda_log_prefix", alpha.data_ptr(), plan.frames, h, logp.data_ptr(), stream)
    out = torch.empty((plan.frames, h, d, d), device=bank.device, dtype=out_dtype)
    _lib.call("vdn_vda_gather", bank[0].data_ptr(), bank[1].data_ptr(), _lib.ptr(logp),
              _lib.ptr(text_state), plan.before.data_ptr(), plan.after.data_ptr(),
              plan.has_before.data_ptr(), plan.has_after.data_ptr(),
              plan.bridge_before.data_ptr(), plan.bridge_after.data_ptr(), plan.frames, h,
              int(bool(bridge)), int(out_dtype == torch.float32), out.data_ptr(), stream)
    return out


# ------------------------------------------------------------ readout / norm ----

def _weight_flag(w):
    if w.dtype not in (torch.bfloat16, torch.float32) or w.shape != (HEAD_DIM,):
        raise ValueError("norm weight must be [head_dim] bf16 or fp32")
    return int(w.dtype == torch.float32)


def _norm_weight(norm_weight, d, device):
    """The norm weight as the kernels read it: [128] on `device`, zero past the head dim (so
    the padded output channels are zero)."""
    w = norm_weight.to(device=device)
    if w.shape != (d,):
        raise ValueError("norm weight must be [head_dim] bf16 or fp32")
    return _pad_channels(w).contiguous()


def vdn_linear_epilogue(readout, norm_weight, gate, eps):
    """readout [F,H,S,D] bf16, gate [F*S,H,D] -> RMSNorm(d)·w·gate as [F*S, H*D] bf16
    (paper_sglang.py:406-437)."""
    _cuda(readout, "readout", torch.bfloat16)
    f, h, s, d = readout.shape
    _check_head_dim(d)
    gate = gate.reshape(f * s, h, d).to(readout.dtype)
    w = _norm_weight(norm_weight, d, readout.device)
    readout = _pad_channels(readout).contiguous()
    gate = _pad_channels(gate)
    if gate.stride(-1) != 1:
        gate = gate.contiguous()
    out = torch.empty((f * s, h * HEAD_DIM), dtype=readout.dtype, device=readout.device)
    gs = (s * gate.stride(0), gate.stride(1), gate.stride(0))
    os_ = (s * out.stride(0), HEAD_DIM, out.stride(0))
    _lib.call("vdn_vda_epilogue", readout.data_ptr(), w.data_ptr(), _weight_flag(w), float(eps),
              gate.data_ptr(), *gs, out.data_ptr(), *os_, d, f, h, s, _stream(readout))
    if d != HEAD_DIM:
        out = out.view(f * s, h, HEAD_DIM)[..., :d].reshape(f * s, h * d)
    return out


@dataclass(frozen=True)
class OutputGateProjection:
    """The linear branch's low-rank output gate as its operands, for the readout to form in
    its kernel: gate = sigmoid(up(down)) = bf16(sigmoid(bf16(down · up_weightᵀ + up_bias)))
    (OutputGate.forward, src/models/attention_gates.py:52-55). down [F*S, 128] bf16 (any row
    stride, unit column stride) is the bottleneck projection down(x); up_weight [H*128, 128]
    and up_bias [H*128] bf16 are the up Linear's parameters."""
    down: torch.Tensor
    up_weight: torch.Tensor
    up_bias: torch.Tensor


def _gate_projection(gp, n, h, device):
    down, w, b = gp.down, gp.up_weight, gp.up_bias
    for t, name in ((down, "down"), (w, "up_weight"), (b, "up_bias")):
        _cuda(t, name, torch.bfloat16)
        if t.device != device:
            raise ValueError(f"{name} must be on the q device")
    if down.shape != (n, HEAD_DIM):
        raise ValueError("down must be [F*S, 128]")
    if down.stride(-1) != 1 or down.stride(0) % 8 or down.data_ptr() % 16:
        down = down.contiguous()  # the kernel reads 16-byte aligned rows
    if w.shape != (h * HEAD_DIM, HEAD_DIM) or b.shape != (h * HEAD_DIM,):
        raise ValueError("up_weight must be [H*128, 128] and up_bias [H*128]")
    return down, w.contiguous(), b.contiguous()


def _q_view(q, frames, spatial):
    """(q, (frame, head, token) strides) of token-major raw q [F*S, H, D] (any row / head
    stride) or frame-major prepared q [F, H, S, D]; unit channel stride, 16-byte rows."""
    if q.ndim == 4:
        if q.shape[0] != frames or q.shape[2] != spatial:
            raise ValueError("readout geometry mismatch")
        strides = (q.stride(0), q.stride(1), q.stride(2))
    elif q.ndim == 3 and q.shape[0] == frames * spatial:
        strides = (spatial * q.stride(0), q.stride(1), q.stride(0))
    else:
        raise ValueError("readout geometry mismatch")
    if q.stride(-1) != 1:
        raise ValueError("readout geometry mismatch")
    return q, strides


def linear_readout(q, state, norm_weight, gate, eps, frames, spatial, *, activate_q=True,
                   out=None, out_mxfp8=None, head_dim=HEAD_DIM):
    """Fused q activation + readout + epilogue.

    q: raw [F*S, H, D] bf16 (any row/head stride), or prepared q (token-major, or frame-major
    [F, H, S, D] from paper_prepare) with activate_q=False;
    state: [F, H, D, D] bf16 from paper_gather; gate [F*S, H, D] bf16, or an
    OutputGateProjection, which the kernel turns into that gate itself.
    Returns (or writes into `out`) [F*S, H*D] bf16 = RMSNorm(bf16(q'·stateᵀ))·w·gate.
    D may be 16, 32, 64 or 128 (a smaller D runs zero-padded to 128 with an explicit gate
    and a bf16 destination). `head_dim` is internal: with 128-wide operands whose channels
    past it are zero, it sets the norm's mean to that many channels.
    `out_mxfp8` = (codes, scales, chunk0) instead quantizes the result in the kernel: head h of
    row r becomes chunk chunk0 + h of row r of an MXFP8 activation (empty_activation),
    byte-identical to quantize_activation of the bf16 result; returns None then.
    """
    _cuda(q, "q", torch.bfloat16)
    _cuda(state, "state", torch.bfloat16)
    q, qs = _q_view(q, frames, spatial)
    n, h, d = frames * spatial, q.shape[-3] if q.ndim == 4 else q.shape[1], q.shape[-1]
    if d not in HEAD_DIMS or state.shape != (frames, h, d, d):
        raise ValueError("readout geometry mismatch")
    if d != HEAD_DIM:
        return _padded_readout(q, state, norm_weight, gate, eps, frames, spatial, activate_q,
                               out, out_mxfp8)
    if isinstance(gate, OutputGateProjection):
        return _gated_readout(q, state, norm_weight, gate, eps, frames, spatial, activate_q,
                              out, out_mxfp8)
    _cuda(gate, "gate", torch.bfloat16)
    if gate.shape != (n, h, d) or gate.stride(-1) != 1:
        raise ValueError("readout geometry mismatch")
    state = state.contiguous()
    w = norm_weight.to(device=q.device).contiguous()
    gs = (spatial * gate.stride(0), gate.stride(1), gate.stride(0))
    if out_mxfp8 is not None:
        if out is not None:
            raise ValueError("out_mxfp8 excludes out")
        codes, scales, chunk0 = mxfp8_destination(out_mxfp8, n, h, q.device)
        _lib.call("vdn_vda_readout_mxfp8", q.data_ptr(), *qs, int(bool(activate_q)),
                  state.data_ptr(), w.data_ptr(), _weight_flag(w), float(eps), gate.data_ptr(),
                  *gs, codes.data_ptr(), scales.data_ptr(), codes.shape[1], chunk0, frames, h,
                  spatial, _stream(q))
        return None
    if out is None:
        out = torch.empty((n, h * d), dtype=torch.bfloat16, device=q.device)
    elif out.shape != (n, h * d) or out.stride(-1) != 1 or out.dtype != torch.bfloat16:
        raise ValueError("out must be bf16 [F*S, H*D]")
    os_ = (spatial * out.stride(0), d, out.stride(0))
    _lib.call("vdn_vda_readout", q.data_ptr(), *qs, int(bool(activate_q)), state.data_ptr(),
              w.data_ptr(), _weight_flag(w), float(eps), gate.data_ptr(), *gs, out.data_ptr(),
              *os_, head_dim, frames, h, spatial, _stream(q))
    return out


def _padded_readout(q, state, norm_weight, gate, eps, frames, spatial, activate_q, out,
                    out_mxfp8):
    """linear_readout at head_dim d < 128: q, state, gate and the norm weight zero-padded to
    the kernel's 128 channels, the norm's mean over d, the output's first d channels kept."""
    n, h, d = frames * spatial, state.shape[1], state.shape[-1]
    if isinstance(gate, OutputGateProjection) or out_mxfp8 is not None:
        raise ValueError("the formed output gate and the MXFP8 destination take head_dim 128")
    _cuda(gate, "gate", torch.bfloat16)
    if gate.shape != (n, h, d):
        raise ValueError("readout geometry mismatch")
    if out is not None and (out.shape != (n, h * d) or out.dtype != torch.bfloat16):
        raise ValueError("out must be bf16 [F*S, H*D]")
    w = _norm_weight(norm_weight, d, q.device)
    full = linear_readout(_pad_channels(q), _pad_square(state), w, _pad_channels(gate), eps,
                          frames, spatial, activate_q=activate_q, head_dim=d)
    full = full.view(n, h, HEAD_DIM)[..., :d].reshape(n, h * d)
    if out is None:
        return full
    out.copy_(full)
    return out


def _gated_readout(q, state, norm_weight, gp, eps, frames, spatial, activate_q, out, out_mxfp8):
    q, qs = _q_view(q, frames, spatial)
    n, h, d = frames * spatial, state.shape[1], HEAD_DIM
    down, up_w, up_b = _gate_projection(gp, n, h, q.device)
    state = state.contiguous()
    w = norm_weight.to(device=q.device).contiguous()
    common = (q.data_ptr(), *qs, int(bool(activate_q)), state.data_ptr(), w.data_ptr(),
              _weight_flag(w), float(eps), down.data_ptr(), down.stride(0), up_w.data_ptr(),
              up_b.data_ptr())
    if out_mxfp8 is not None:
        if out is not None:
            raise ValueError("out_mxfp8 excludes out")
        codes, scales, chunk0 = mxfp8_destination(out_mxfp8, n, h, q.device)
        _lib.call("vdn_vda_readout_gated", *common, None, 0, 0, 0, codes.data_ptr(),
                  scales.data_ptr(), codes.shape[1], chunk0, frames, h, spatial, _stream(q))
        return None
    if out is None:
        out = torch.empty((n, h * d), dtype=torch.bfloat16, device=q.device)
    elif out.shape != (n, h * d) or out.stride(-1) != 1 or out.dtype != torch.bfloat16:
        raise ValueError("out must be bf16 [F*S, H*D]")
    _lib.call("vdn_vda_readout_gated", *common, out.data_ptr(), spatial * out.stride(0), d,
              out.stride(0), None, None, 0, 0, frames, h, spatial, _stream(q))
    return out


# ---------------------------------------------------------------- orchestration ----

def vda_forward(q_raw, k_raw, v_raw, beta, gate, alpha, bounds, num_frames, tokens_per_frame,
                norm_weight, eps, *, chunk_size=8, bridge=True, text=None, out=None,
                out_mxfp8=None, conv=None, frame_size=None, _head_dim=HEAD_DIM):
    """The paper VDA branch body on raw projections (paper_stack.py:266-318).

    q_raw/k_raw/v_raw: [F*S, H, 128] bf16 raw projections; beta [F*S, H]; gate [F*S, H, 128]
    or an OutputGateProjection; alpha [F, H, 128] fp32. `text` = (tk_raw, tv_raw, text_beta)
    adds the prompt's virtual frame (its factors share the batch; half its injection seeds
    both scans). `conv` (a LinearAttentionSepConv, frame_size = (H_f, W_f)) convolves the
    projections it lists before their activation; the prompt's tokens are not convolved.
    `out` / `out_mxfp8` as in linear_readout.
    A head dim of 16, 32 or 64 (the reference's eager body, delta_rule.py:45-60) runs with
    every operand's channels zero-padded to 128 (alpha padded with ones), which is exact; it
    takes an explicit gate, a bf16 destination and no short conv.
    """
    d = q_raw.shape[-1]
    if d != HEAD_DIM:
        _check_head_dim(d)
        n, h = q_raw.shape[:2]
        if (k_raw.shape[-1] != d or v_raw.shape[-1] != d or alpha.shape[-1] != d
                or (not isinstance(gate, OutputGateProjection) and gate.shape[-1] != d)):
            raise ValueError("q, k, v, gate and alpha must share the head dim")
        if isinstance(gate, OutputGateProjection) or out_mxfp8 is not None or conv is not None:
            raise ValueError("head_dim < 128 takes an explicit gate, a bf16 destination and no "
                             "short conv")
        if out is not None and (out.shape != (n, h * d) or out.dtype != torch.bfloat16):
            raise ValueError("out must be bf16 [F*S, H*D]")
        if text is not None:
            text = (_pad_channels(text[0]), _pad_channels(text[1]), text[2])
        w = _norm_weight(norm_weight, d, q_raw.device)
        full = vda_forward(_pad_channels(q_raw), _pad_channels(k_raw), _pad_channels(v_raw),
                           beta, _pad_channels(gate), _pad_channels(alpha, 1.0).contiguous(),
                           bounds, num_frames, tokens_per_frame, w, eps, chunk_size=chunk_size,
                           bridge=bridge, text=text, _head_dim=d)
        full = full.view(n, h, HEAD_DIM)[..., :d].reshape(n, h * d)
        if out is None:
            return full
        out.copy_(full)
        return out
    f, s = num_frames, tokens_per_frame
    h = q_raw.shape[1]
    device = q_raw.device
    extra = 1 if text is not None else 0
    a = torch.empty((f + extra, h, HEAD_DIM, HEAD_DIM), dtype=torch.float32, device=device)
    b = torch.empty_like(a)
    projs = getattr(conv, "projs", ()) if conv is not None else ()
    if "k" in projs or "v" in projs:
        kp = paper_prepare(k_raw, frames=f, spatial=s, l2norm=True, conv=conv, proj="k",
                           frame_size=frame_size)
        vp = paper_prepare(v_raw, frames=f, spatial=s, l2norm=False, conv=conv, proj="v",
                           frame_size=frame_size)
        bs = (s * beta.stride(0), beta.stride(1), beta.stride(0))
        ks = (h * s * HEAD_DIM, s * HEAD_DIM, HEAD_DIM)
        _stats_call(kp, ks, vp, ks, beta, bs, f, h, s, 0, a[extra:], b[extra:])
        del kp, vp
    else:
        statistics_from_projections(k_raw, v_raw, beta, f, s, a[extra:], b[extra:])
    if text is not None:
        tk, tv, tb = text
        statistics_from_projections(tk, tv, tb, 1, tk.shape[0], a[:1], b[:1])
        factor_alpha = torch.cat((torch.ones_like(alpha[:1]), alpha))
    else:
        factor_alpha = alpha
    transitions, injections = paper_delta_factors(a, b, factor_alpha.contiguous())
    del a, b
    seed = None
    if text is not None:
        seed = injections[0] * 0.5
        transitions, injections = transitions[1:], injections[1:]
    plan = paper_boundary_plan(bounds, f, device, chunk_size)
    bank = paper_boundary_scan(transitions, injections, plan, seed)
    del transitions, injections
    state = paper_gather(bank, alpha, plan, seed, torch.bfloat16, bridge)
    del bank
    if "q" in projs:
        q = paper_prepare(q_raw, frames=f, spatial=s, l2norm=True, conv=conv, proj="q",
                          frame_size=frame_size)
        return linear_readout(q, state, norm_weight, gate, eps, f, s, activate_q=False, out=out,
                              out_mxfp8=out_mxfp8)
    return linear_readout(q_raw, state, norm_weight, gate, eps, f, s, out=out,
                          out_mxfp8=out_mxfp8, head_dim=_head_dim)


def paper_readout(branch, xv, num_frames, tokens_per_frame, bounds, qkv_raw, frame_size=None,
                  text_x=None, text_qkv_raw=None, heads=None, beta=None, gate=None,
                  frame_mean=None, text_beta=None):
    """Branch body with the reference signature (paper_stack.py:266-318). `branch` supplies
    beta_proj, alpha, output_gate, norm, bridge and paper_vda_chunk_size."""
    conv = getattr(branch, "short_conv", None)
    q, k, v = qkv_raw
    h = q.shape[1]
    if beta is None:
        beta = torch.sigmoid(branch.beta_proj(xv))
    if frame_mean is None:
        frame_mean = xv.view(num_frames, tokens_per_frame, -1).mean(1, dtype=torch.float32)
    alpha = branch.alpha(frame_mean, heads=heads).float().contiguous()
    text = None
    if text_x is not None or text_beta is not None:
        if text_qkv_raw is None or text_qkv_raw[1].shape[0] < 1:
            raise ValueError("prompt inputs require nonempty text QKV")
        if text_beta is None:
            text_beta = torch.sigmoid(branch.beta_proj(text_x))
        text = (text_qkv_raw[1], text_qkv_raw[2], text_beta.reshape(-1, h))
    d = q.shape[-1]
    if gate is None:
        gate = _output_gate(branch.output_gate, xv, h, d)
    else:
        gate = gate.reshape(-1, h, d)
    return vda_forward(q, k, v, beta.reshape(-1, h), gate, alpha, bounds,
                       num_frames, tokens_per_frame, branch.norm.weight, branch.norm.eps,
                       chunk_size=branch.paper_vda_chunk_size, bridge=branch.bridge == "alpha",
                       text=text, conv=conv, frame_size=frame_size)


def _output_gate(module, xv, heads, head_dim=HEAD_DIM):
    """OutputGate(xv) of the linear branch: a bottleneck-128 gate in bf16 goes to the readout
    kernel as its projection operands (only down(xv) is formed here); any other gate is
    evaluated by the module itself."""
    down, up = getattr(module, "down", None), getattr(module, "up", None)
    if (head_dim == HEAD_DIM and down is not None and up is not None
            and down.out_features == HEAD_DIM
            and up.in_features == HEAD_DIM and up.out_features == heads * HEAD_DIM
            and up.bias is not None and xv.dtype == torch.bfloat16
            and all(p.dtype == torch.bfloat16 for p in (down.weight, up.weight, up.bias))):
        return OutputGateProjection(down(xv), up.weight, up.bias)
    return module(xv).reshape(-1, heads, head_dim)
