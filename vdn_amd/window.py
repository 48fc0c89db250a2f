"""Frame-window softmax attention and QK RMSNorm + RoPE with the reference's signatures.

Mirrors src/models/sequence_layout.py (SequenceLayout), softmax_attention/window.py
(window_bounds), paper_window.py (prepare_paper_window_plan, paper_window_attention),
paper_qk_rope.py (paper_qk_rmsnorm_rope) and kernels.py (apply_softmax_gate). Device work
runs in libvdnmi.so. The plan keeps the reference's groups, passes and budget errors; the
gfx950 kernel consumes an interval form of the same visible sets (query blocks of <= 128
rows, each with <= 8 contiguous key intervals), so it never gathers K/V.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from functools import cached_property
from numbers import Real

import torch

from . import _lib
from .mxfp8 import mxfp8_destination

BLOCK_M = 256
MAX_INTERVALS = 8


@dataclass(frozen=True)
class SequenceLayout:
    """Packed-row geometry (sequence_layout.py:10-116)."""
    seq_len: int
    video_start: int
    num_frames: int
    tokens_per_frame: int
    frame_height: int = 0
    frame_width: int = 0
    text_start: int = 0
    text_len: int = 0

    @property
    def video_end(self):
        return self.video_start + self.num_frames * self.tokens_per_frame

    @property
    def text_range(self):
        if not self.text_len:
            raise ValueError("this layout carries no text rows")
        return self.text_start, self.text_start + self.text_len

    @property
    def frame_size(self):
        if not (self.frame_height and self.frame_width):
            raise ValueError("this layout carries no spatial grid")
        if self.frame_height * self.frame_width != self.tokens_per_frame:
            raise ValueError("grid does not match tokens/frame")
        return self.frame_height, self.frame_width

    def global_index(self, device):
        idx = torch.arange(self.seq_len, device=device)
        return torch.cat([idx[:self.video_start], idx[self.video_end:]])


def window_bounds(num_frames, radius, chunk=0):
    """Per-frame inclusive window [lo, hi], unclamped (window.py:26-52)."""
    if chunk <= 0:
        return [(t - radius, t + radius) for t in range(num_frames)]
    return [(((t // chunk) - radius) * chunk, ((t // chunk) + radius + 1) * chunk - 1)
            for t in range(num_frames)]


# --------------------------------------------------------------------------- plan ----
#
# The plan is built from row *units* in row order: the non-video rows before the video,
# each video frame, and the non-video rows after it. What a query row sees is a subset of
# units (all of them for non-video rows and row-anchor frames; for frame t the non-video
# rows, the frames of its clamped window and the column-anchor frames), and a run of
# adjacent visible units is one contiguous key interval. The kernel takes, per group of
# query rows with one visible set, at most MAX_INTERVALS such intervals, and walks K and V
# in place: nothing is gathered, so the plan allocates no index tensors on the device.
# The reference's pass structure (budgeted varlen passes over gathered rows) is kept as a
# lazily built host-side view with the same groups, budgets and errors.


@dataclass(frozen=True)
class VisibleGroup:
    """Query rows (ranges) that see exactly the key rows `key_ranges` (sorted, disjoint)."""
    query_ranges: tuple
    key_ranges: tuple


@dataclass(frozen=True)
class PackedPass:
    """One budgeted pass of the reference's plan (paper_window.py:60-70): groups, their
    concatenated query / key row indices (int64), cumulative segment lengths (int32) and the
    longest segments. Host tensors: the gfx950 kernel reads the interval form instead."""
    groups: tuple
    query_rows: torch.Tensor
    key_rows: torch.Tensor | None
    cu_q: torch.Tensor
    cu_k: torch.Tensor
    max_q: int
    max_k: int
    dense: bool


@dataclass(frozen=True)
class DevicePlan:
    """Interval form for the gfx950 kernel: blocks int32 [nb, 3] (q0, range end, group),
    intervals int32 [ng, 8, 2], counts int32 [ng]."""
    blocks: torch.Tensor
    intervals: torch.Tensor
    counts: torch.Tensor
    nblocks: int


def _rows(ranges):
    return sum(b - a for a, b in ranges)


def _cut(ranges, size):
    """The concatenation of `ranges` (in order) cut into consecutive pieces of `size` rows
    (the last may be shorter); each piece is a tuple of ranges."""
    pieces, piece, room = [], [], size
    for a, b in ranges:
        while a < b:
            step = min(room, b - a)
            piece.append((a, a + step))
            a, room = a + step, room - step
            if room == 0:
                pieces.append(tuple(piece))
                piece, room = [], size
    return pieces + ([tuple(piece)] if piece else [])


def _join(ranges):
    """Sorted ranges with touching neighbours joined (inputs never overlap)."""
    joined = []
    for a, b in sorted(r for r in ranges if r[0] < r[1]):
        if joined and joined[-1][1] == a:
            joined[-1] = (joined[-1][0], b)
        else:
            joined.append((a, b))
    return tuple(joined)


@dataclass(frozen=True)
class PaperWindowPlan:
    """Visible-set plan of one request (paper_window.py:72-84). `groups` holds one entry per
    run of consecutive video frames with the same visible set, `dense_rows` the query rows
    that see every row; `device_plan` is what the kernel reads."""
    layout: SequenceLayout
    bounds: tuple
    anchor_frames: str
    max_gather_rows: int
    max_query_rows: int
    device: torch.device
    dense_rows: tuple = ()
    groups: tuple = ()
    device_plan: DevicePlan = field(default=None, compare=False)

    @cached_property
    def passes(self):
        """The reference's budgeted passes: each chunk of at most max_query_rows dense rows
        is a pass of its own; the groups' query rows, cut into chunks of at most
        max_query_rows, are packed in order, a new pass starting before a chunk that would
        take the pass over max_query_rows queries or max_gather_rows keys."""
        seq = self.layout.seq_len
        out = [_packed((VisibleGroup(chunk, ((0, seq),)),), dense=True)
               for chunk in _cut(self.dense_rows, self.max_query_rows)]
        open_pass, nq, nk = [], 0, 0
        for group in self.groups:
            keys = _rows(group.key_ranges)
            for chunk in _cut(group.query_ranges, self.max_query_rows):
                q = _rows(chunk)
                if open_pass and (nq + q > self.max_query_rows or nk + keys > self.max_gather_rows):
                    out.append(_packed(tuple(open_pass)))
                    open_pass, nq, nk = [], 0, 0
                open_pass.append(VisibleGroup(chunk, group.key_ranges))
                nq, nk = nq + q, nk + keys
        if open_pass:
            out.append(_packed(tuple(open_pass)))
        return tuple(out)

    @property
    def peak_gather_rows(self):
        """Largest number of key rows a non-dense pass of the reference gathers."""
        return max((_rows(r for g in p.groups for r in g.key_ranges)
                    for p in self.passes if not p.dense), default=0)


def _packed(groups, dense=False):
    def index(ranges):
        return torch.cat([torch.arange(a, b, dtype=torch.long) for a, b in ranges])

    def offsets(lengths):
        return torch.tensor([0, *lengths], dtype=torch.int64).cumsum(0).to(torch.int32)

    q_len = [_rows(g.query_ranges) for g in groups]
    k_len = [_rows(g.key_ranges) for g in groups]
    return PackedPass(groups, index(r for g in groups for r in g.query_ranges),
                      None if dense else index(r for g in groups for r in g.key_ranges),
                      offsets(q_len), offsets(k_len), max(q_len), max(k_len), dense)


def _device_plan(sets, device):
    """Kernel form of [(query ranges, key intervals)]: every query range cut into blocks of
    BLOCK_M rows, each naming its range end and its set; one transfer to the device."""
    nsets = max(len(sets), 1)
    intervals = torch.zeros(nsets, MAX_INTERVALS, 2, dtype=torch.int32)
    counts = torch.zeros(nsets, dtype=torch.int32)
    blocks = []
    for index, (query_ranges, keys) in enumerate(sets):
        if len(keys) > MAX_INTERVALS:
            raise ValueError(f"a visible set needs {len(keys)} key intervals; the kernel "
                             f"takes at most {MAX_INTERVALS}")
        if keys:
            intervals[index, :len(keys)] = torch.tensor(keys, dtype=torch.int32)
        counts[index] = len(keys)
        blocks += [(q0, b, index) for a, b in query_ranges for q0 in range(a, b, BLOCK_M)]
    block_t = torch.tensor(blocks or [(0, 0, 0)], dtype=torch.int32)
    # one host buffer, one copy: [blocks | intervals | counts]
    flat = torch.cat((block_t.reshape(-1), intervals.reshape(-1), counts)).to(device)
    nb, ni = block_t.numel(), intervals.numel()
    return DevicePlan(flat[:nb].view(-1, 3), flat[nb:nb + ni].view(nsets, MAX_INTERVALS, 2),
                      flat[nb + ni:], len(blocks))


def _check_plan_arguments(layout, bounds, anchor_frames, max_gather_rows, max_query_rows):
    """The reference's argument contract and messages (paper_window.py:103-115)."""
    if not isinstance(layout, SequenceLayout):
        raise TypeError("layout must be SequenceLayout")
    geometry = (layout.seq_len, layout.video_start, layout.num_frames, layout.tokens_per_frame)
    if any(type(x) is not int for x in geometry):
        raise ValueError("invalid used-row/video geometry")
    seq, start, frames, per_frame = geometry
    if seq <= 0 or frames < 0 or per_frame <= 0 or start < 0 or start + frames * per_frame > seq:
        raise ValueError("invalid used-row/video geometry")
    if anchor_frames not in ("none", "rows", "columns", "both"):
        raise ValueError("anchor_frames must be none, rows, columns, or both")
    if any(type(x) is not int or x <= 0 for x in (max_gather_rows, max_query_rows)):
        raise ValueError("row budgets must be positive integers")
    bounds = tuple(tuple(b) for b in bounds)
    well_formed = all(len(b) == 2 and type(b[0]) is int and type(b[1]) is int and b[0] <= b[1]
                      for b in bounds)
    if len(bounds) != frames or not well_formed:
        raise ValueError("one ordered integer bound pair required per video frame")
    return bounds


def prepare_paper_window_plan(layout: SequenceLayout, bounds, anchor_frames="none", *,
                              device="cpu", max_gather_rows=65_536, max_query_rows=8_192):
    """Plan of each query row's visible key rows (the contract of paper_window.py:86-168:
    inclusive frame bounds clamped to the video, non-video rows seen by and seeing every
    row, anchor frames 0 and F-1 as rows and/or columns, a visible set over
    max_gather_rows refused, the same errors), in the kernel's interval form."""
    bounds = _check_plan_arguments(layout, bounds, anchor_frames, max_gather_rows,
                                   max_query_rows)
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    seq, start, frames, per_frame = (layout.seq_len, layout.video_start, layout.num_frames,
                                     layout.tokens_per_frame)
    end = start + frames * per_frame
    # units in row order: (first row, end row, frame or -1 for non-video rows)
    units = ([(0, start, -1)] if start else []) + \
        [(start + t * per_frame, start + (t + 1) * per_frame, t) for t in range(frames)] + \
        ([(end, seq, -1)] if end < seq else [])
    edge = {0, frames - 1} if frames else set()
    row_anchor = edge if anchor_frames in ("rows", "both") else set()
    col_anchor = edge if anchor_frames in ("columns", "both") else set()

    def keys_of(t):
        lo, hi = max(0, bounds[t][0]), min(frames - 1, bounds[t][1])
        return _join((a, b) for a, b, u in units
                     if u < 0 or lo <= u <= hi or u in col_anchor)

    everything = ((0, seq),)
    frame_keys = [everything if t in row_anchor else keys_of(t) for t in range(frames)]
    dense = [(a, b) for a, b, u in units if u < 0 or frame_keys[u] == everything]
    groups = []
    for t, keys in enumerate(frame_keys):
        if keys == everything:
            continue
        if not keys:
            raise ValueError(f"video frame {t} has no visible keys")
        if _rows(keys) > max_gather_rows:
            raise ValueError(f"visible set requires {_rows(keys)} gather rows, "
                             f"budget={max_gather_rows}; increase max_gather_rows")
        rows = (start + t * per_frame, start + (t + 1) * per_frame)
        # consecutive frames with one visible set share a group (one run of query rows)
        if groups and groups[-1][1] == keys and groups[-1][0][-1] == rows[0]:
            groups[-1][0][-1] = rows[1]
        else:
            groups.append(([rows[0], rows[1]], keys))
    dense_rows = _join(dense)
    groups = tuple(VisibleGroup(((a, b),), keys) for (a, b), keys in groups)
    sets = ([(dense_rows, everything)] if dense_rows else []) + \
        [(g.query_ranges, g.key_ranges) for g in groups]
    covered = _rows(dense_rows) + sum(_rows(g.query_ranges) for g in groups)
    if covered != seq:
        raise AssertionError(f"window plan covers {covered} of {seq} query rows")
    return PaperWindowPlan(layout, bounds, anchor_frames, max_gather_rows, max_query_rows, device,
                           dense_rows, groups, _device_plan(sets, device))


# ---------------------------------------------------------------------- attention ----

def paper_window_attention(query, key, value, plan: PaperWindowPlan, scale=None, *,
                           enabled=False, return_lse=False, nvtx=True, gate=None, out=None,
                           out_mxfp8=None):
    """[used+padding, H, D] -> fresh output of the same shape; padding rows are zero
    (paper_window.py:182-243). LSE (fp32 [rows, H], natural log) is -inf on padding.
    BF16 and FP16 activations (the output takes the activation dtype). `gate` ([rows, H] or
    [rows, H, 1]) fuses apply_softmax_gate: out = act(act(o) * gate), with the gate cast to
    the activation dtype as apply_softmax_gate does. `out` (optional [rows, H, D] view of the
    activation dtype with unit channel stride) receives the result instead of a fresh tensor,
    e.g. a column slice of a wider buffer.
    `out_mxfp8` = (codes, scales, chunk0) instead quantizes the output in the kernel: head h of
    used row r becomes chunk chunk0 + h of row r of an MXFP8 activation (empty_activation),
    byte-identical to quantize_activation of the bf16 output; returns None then."""
    if not enabled:
        raise RuntimeError("paper window attention is disabled; retain the existing caller path "
                           "or explicitly enable")
    if torch.is_grad_enabled():
        raise RuntimeError("paper window attention is inference-only; use no_grad/inference_mode")
    if not isinstance(plan, PaperWindowPlan):
        raise TypeError("plan must be prepared with prepare_paper_window_plan")
    if any(x.ndim != 3 or x.shape != query.shape or x.dtype != query.dtype
           or x.device != query.device for x in (query, key, value)):
        raise ValueError("Q/K/V must have identical [rows,H,D], dtype and device")
    if query.shape[0] < plan.layout.seq_len or query.shape[1] <= 0 or query.shape[2] not in (64, 128, 256):
        raise ValueError("invalid Q/K/V geometry or insufficient used rows")
    if query.dtype not in (torch.bfloat16, torch.float16) or any(x.stride(-1) != 1 for x in (query, key, value)):
        raise ValueError("native varlen requires BF16/FP16 and unit innermost stride")
    if not query.is_cuda or query.device != plan.device:
        raise ValueError("Q/K/V and prepared plan must be on the same CUDA device")
    scale = query.shape[-1] ** -0.5 if scale is None else float(scale)
    if not math.isfinite(scale):
        raise ValueError("scale must be finite")
    rows, h, d = query.shape
    if out_mxfp8 is not None:
        if out is not None or return_lse:
            raise ValueError("out_mxfp8 excludes out and return_lse")
        if d != 128:
            raise ValueError("out_mxfp8 holds one head per 128-column chunk: head_dim 128")
        if query.dtype != torch.bfloat16:
            raise ValueError("out_mxfp8 quantizes bf16 attention (the block's activations)")
        codes, scales, chunk0 = mxfp8_destination(out_mxfp8, plan.layout.seq_len, h,
                                                  query.device)
        if gate is not None:
            gate = _gate_rows(gate, plan.layout.seq_len, h, query.dtype)
        dp = plan.device_plan
        _lib.call("vdn_window_attention_mxfp8", query.data_ptr(), query.stride(0),
                  query.stride(1), key.data_ptr(), key.stride(0), key.stride(1),
                  value.data_ptr(), value.stride(0), value.stride(1), dp.blocks.data_ptr(),
                  dp.nblocks, dp.intervals.data_ptr(), dp.counts.data_ptr(), h, scale,
                  _lib.ptr(gate), 0 if gate is None else gate.stride(0),
                  0 if gate is None else gate.stride(1), None, 0.0, codes.data_ptr(),
                  scales.data_ptr(), codes.shape[1], chunk0, _lib.stream(query.device))
        return None
    if out is None:
        out = torch.empty((rows, h, d), dtype=query.dtype, device=query.device)
    elif (out.shape != (rows, h, d) or out.dtype != query.dtype or out.device != query.device
          or out.stride(-1) != 1):
        raise ValueError("out must be a [rows, H, D] view like the queries, unit channel stride")
    lse = torch.empty((rows, h), dtype=torch.float32, device=query.device) if return_lse else None
    used = plan.layout.seq_len
    if rows > used:
        out[used:].zero_()
        if lse is not None:
            lse[used:].fill_(-float("inf"))
    if gate is not None:
        gate = _gate_rows(gate, used, h, query.dtype)
    dp = plan.device_plan
    _lib.call("vdn_window_attention", query.data_ptr(), query.stride(0), query.stride(1),
              key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(), value.stride(0),
              value.stride(1), dp.blocks.data_ptr(), dp.nblocks, dp.intervals.data_ptr(),
              dp.counts.data_ptr(), h, d, int(query.dtype == torch.float16), scale,
              _lib.ptr(gate),
              0 if gate is None else gate.stride(0), 0 if gate is None else gate.stride(1),
              out.data_ptr(), out.stride(0), out.stride(1), _lib.ptr(lse),
              0 if lse is None else lse.stride(0), 0 if lse is None else lse.stride(1),
              _lib.stream(query.device))
    return (out, lse) if return_lse else out


def _gate_rows(gate, used, h, dtype):
    if gate.shape[0] < used or gate.numel() != gate.shape[0] * h:
        raise ValueError("gate must be [rows, H] or [rows, H, 1] covering the used rows")
    if gate.device.type != "cuda":
        raise ValueError("gate must be on the activations' device")
    gate = gate.reshape(gate.shape[0], h)
    return gate if gate.dtype == dtype else gate.to(dtype)


def apply_softmax_gate(softmax_out, gate, inference=False):
    """out * gate (bf16) flattened to [T, H*D] (softmax_attention/kernels.py:62-67); the fused
    form is paper_window_attention(..., gate=gate)."""
    return (softmax_out * gate.to(softmax_out.dtype)).reshape(softmax_out.shape[0], -1)


# ---------------------------------------------------------------- QK norm + RoPE ----

_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _validate_rope(q, k, q_weight, k_weight, eps, cos, sin, enabled, nvtx):
    if not isinstance(enabled, bool) or not isinstance(nvtx, bool):
        raise TypeError("enabled and nvtx must be bool")
    if torch.is_grad_enabled():
        raise RuntimeError("paper_qk_rmsnorm_rope is inference-only; use torch.no_grad()")
    if isinstance(eps, bool) or not isinstance(eps, Real):
        raise TypeError("eps must be a finite positive real scalar")
    if not math.isfinite(eps) or eps <= 0:
        raise ValueError("eps must be finite and positive")
    for name, value in (("q", q), ("k", k), ("q_weight", q_weight), ("k_weight", k_weight)):
        if not isinstance(value, torch.Tensor):
            raise TypeError(f"{name} must be a tensor")
        if value.layout != torch.strided:
            raise ValueError(f"{name} must have strided layout")
    if q.ndim != 3 or k.shape != q.shape:
        raise ValueError("q and k must have identical [T, H, D] shapes")
    t, h, d = q.shape
    if h <= 0 or d not in (64, 128, 256):
        raise ValueError("H must be positive and D must be 64, 128, or 256")
    if q.dtype not in _DTYPES or k.dtype != q.dtype:
        raise TypeError("q and k must share a BF16, FP16, or FP32 dtype")
    if q.device.type not in ("cpu", "cuda") or k.device != q.device:
        raise ValueError("q and k must share a CPU or CUDA device")
    for name, weight in (("q_weight", q_weight), ("k_weight", k_weight)):
        if weight.shape != (d,):
            raise ValueError(f"{name} must have shape [D], shared by every head")
        if weight.device != q.device:
            raise ValueError(f"{name} must be on the q/k device")
        if weight.dtype not in (q.dtype, torch.float32):
            raise TypeError(f"{name} must have the activation dtype or FP32")
    if (cos is None) != (sin is None):
        raise ValueError("cos and sin must both be supplied or both be None")
    if cos is not None:
        for name, table in (("cos", cos), ("sin", sin)):
            if not isinstance(table, torch.Tensor):
                raise TypeError(f"{name} must be a tensor")
            if table.layout != torch.strided or table.ndim != 2:
                raise ValueError(f"{name} must have strided shape [T, R]")
            if table.device != q.device:
                raise ValueError(f"{name} must be on the q/k device")
            if table.dtype not in _DTYPES:
                raise TypeError(f"{name} must be BF16, FP16, or FP32")
        if cos.shape != sin.shape or cos.shape[0] != t:
            raise ValueError("cos and sin must have identical [T, R] shapes")
        r = cos.shape[1]
        if r <= 0 or r > d or r % 2:
            raise ValueError("rotary width R must be positive, even, and at most D")


def paper_qk_rmsnorm_rope(q, k, q_weight, k_weight, eps=1e-6, cos=None, sin=None, *,
                          enabled=False, nvtx=True):
    """New contiguous normalized/rotated Q and K (paper_qk_rope.py:145-211) for BF16, FP16 and
    FP32 activations.

    enabled=True runs the gfx950 kernel (a HIP device is required; there is no fallback).
    enabled=False is the reference's disabled path: its eager torch ops on the tensors'
    own device (CPU or GPU), with the same rounding points (_eager_norm / _eager_rope,
    paper_qk_rope.py:82-95). Callers select it explicitly; the device path never takes it.
    """
    _validate_rope(q, k, q_weight, k_weight, eps, cos, sin, enabled, nvtx)
    if not enabled:
        qo, ko = _eager_rms(q, q_weight, eps), _eager_rms(k, k_weight, eps)
        if cos is not None:
            qo, ko = _eager_rotate(qo, cos, sin), _eager_rotate(ko, cos, sin)
        return qo, ko
    if not q.is_cuda:
        raise ValueError("enabled=True requires a HIP device")
    qo = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    ko = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    if q.shape[0] == 0:
        return qo, ko
    tables = cos is not None
    if tables:
        # the kernel reads tables of the activation dtype or fp32 (any other dtype is widened
        # to fp32 exactly; the kernel then rounds to the activation dtype, as cos.to(dtype))
        if cos.dtype not in (q.dtype, torch.float32):
            cos = cos.float()
        if sin.dtype != cos.dtype:
            sin = sin.to(cos.dtype)
    act = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}[q.dtype]
    flags = (int(q_weight.dtype == torch.float32) | (int(k_weight.dtype == torch.float32) << 1)
             | (int(tables and cos.dtype == torch.float32) << 2) | (act << 4))
    t, h, d = q.shape
    _lib.call("vdn_qk_rmsnorm_rope", q.data_ptr(), *q.stride(), k.data_ptr(), *k.stride(),
              q_weight.data_ptr(), q_weight.stride(0), k_weight.data_ptr(), k_weight.stride(0),
              float(eps), _lib.ptr(cos) if tables else None, cos.stride(0) if tables else 0,
              cos.stride(1) if tables else 0, _lib.ptr(sin) if tables else None,
              sin.stride(0) if tables else 0, sin.stride(1) if tables else 0,
              cos.shape[1] if tables else 0, flags, t, h, d, qo.data_ptr(), ko.data_ptr(),
              _lib.stream(q.device))
    return qo, ko


def _eager_rms(x, weight, eps):
    """RMSNorm over the last dim in fp32, the weight multiplied in fp32, one rounding to x's
    dtype (nn.RMSNorm's order, paper_qk_rope.py:82-87)."""
    xf = x.float()
    inv = torch.rsqrt(xf.square().mean(-1, keepdim=True) + eps)
    return ((xf * inv) * weight.float()).to(x.dtype).contiguous()


def _eager_rotate(x, cos, sin):
    """Rotate-half RoPE of the first R channels in x's dtype: each product and the sum round
    to that dtype (torch's elementwise ops on x's dtype, paper_qk_rope.py:90-95)."""
    r = cos.shape[-1]
    lo, hi = x[..., :r // 2], x[..., r // 2:r]
    c = cos.to(x.dtype)[:, None, :]
    s = sin.to(x.dtype)[:, None, :]
    turned = torch.cat((-hi, lo), dim=-1)
    return torch.cat((x[..., :r] * c + turned * s, x[..., r:]), dim=-1).contiguous()


def qk_rmsnorm(x, weight, eps=1e-6):
    """RMSNorm of one [T, H, D] bf16 operand per (token, head) row, n = bf16((x * rsqrt(mean
    x^2 + eps)) * w): the QK norm of paper_qk_rope.py:82-95 without rotary, for operands whose
    row count differs from their partner's (cross-attention queries vs context keys)."""
    if torch.is_grad_enabled():
        raise RuntimeError("qk_rmsnorm is inference-only; use torch.no_grad()")
    if (x.ndim != 3 or x.dtype != torch.bfloat16 or not x.is_cuda or x.shape[2] not in (64, 128, 256)
            or weight.shape != (x.shape[2],) or weight.dtype not in (torch.bfloat16, torch.float32)
            or weight.device != x.device):
        raise ValueError("expected CUDA bf16 [T, H, D] and a [D] bf16/fp32 weight on its device")
    if not math.isfinite(eps) or eps <= 0:
        raise ValueError("eps must be finite and positive")
    out = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    t, h, d = x.shape
    if t == 0:
        return out
    flags = int(weight.dtype == torch.float32) | 8
    _lib.call("vdn_qk_rmsnorm_rope", x.data_ptr(), *x.stride(), None, 0, 0, 0, weight.data_ptr(),
              weight.stride(0), None, 0, float(eps), None, 0, 0, None, 0, 0, 0, flags, t, h, d,
              out.data_ptr(), None, _lib.stream(x.device))
    return out


def rope_tables_3d(frames, height, width, *, dims=(44, 42, 42), theta=10000.0, device="cpu",
                   dtype=torch.float32):
    """Full-width rotate-half cos/sin tables [F*H*W, sum(dims)] for 3D positions (t, h, w).

    Pair i of the rotate-half layout pairs channel i with i + R/2 (R = sum(dims)); the R/2
    pairs are split over the axes as dims/2 each (22 t, 21 h, 21 w for 44/42/42), each axis
    using frequencies theta^(-2j/dim_axis). Column i and i + R/2 carry the same angle.
    """
    pos = torch.stack(torch.meshgrid(torch.arange(frames), torch.arange(height),
                                     torch.arange(width), indexing="ij"), -1).reshape(-1, 3)
    angles = []
    for axis, dim in enumerate(dims):
        inv = theta ** (-torch.arange(0, dim, 2, dtype=torch.float64) / dim)
        angles.append(pos[:, axis:axis + 1].double() * inv[None, :])
    half = torch.cat(angles, dim=1)
    full = torch.cat((half, half), dim=1)
    return full.cos().to(device=device, dtype=dtype), full.sin().to(device=device, dtype=dtype)
