"""Frame-window softmax and QK RMSNorm + RoPE oracle.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). torch-CPU.

Reference: src/models/softmax_attention/window.py:26-111 (window_bounds,
window_softmax_reference), paper_window.py:86-168 (visible sets), paper_qk_rope.py:82-95
(eager norm / rope with bf16 rounding points), kernels.py:62-67 (softmax gate), and the
reference tests' independent oracles (tests/test_paper_stack_attention_window.py:14-27,
121-124; tests/test_paper_stack_attention_rope.py:31-52).

Pins (tests/test_oracle_window.py):
  dense_mask      brute force per (q, k) pair, independent of interval planning; the
                  product plan reproduces it exactly
  attention_dense q = k = 0 gives the closed form mean of visible values and
                  LSE = log |visible| (test_paper_stack_attention_window.py:171-183);
                  agrees with the per-frame SDPA reference (window_softmax_reference)
  qk_rope         fp64 complex rotation bounds the unrounded variant; the reference's
                  rounding traps change > 100 elements when a rounding is dropped;
                  norm-only equals torch rms_norm with fp32 weight rounded once
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def dense_mask(seq_len, video_start, num_frames, tokens_per_frame, bounds, anchors="none"):
    """Boolean [S, S] visibility, pair by pair (test_paper_stack_attention_window.py:14-27)."""
    vs, ve = video_start, video_start + num_frames * tokens_per_frame
    q = torch.arange(seq_len)[:, None]
    k = torch.arange(seq_len)[None, :]
    glob = (q < vs) | (q >= ve) | (k < vs) | (k >= ve)
    qf = ((q - vs) // tokens_per_frame).clamp(0, max(num_frames - 1, 0))
    kf = ((k - vs) // tokens_per_frame).clamp(0, max(num_frames - 1, 0))
    lo = torch.tensor([b[0] for b in bounds] or [0])[qf]
    hi = torch.tensor([b[1] for b in bounds] or [0])[qf]
    inside = (kf >= lo) & (kf <= hi)
    if anchors in ("rows", "both"):
        inside |= (qf == 0) | (qf == num_frames - 1)
    if anchors in ("columns", "both"):
        inside |= (kf == 0) | (kf == num_frames - 1)
    return glob | inside


def attention_dense(q, k, v, mask, scale):
    """fp32 exact masked softmax attention and natural-log LSE [rows, H]
    (test_paper_stack_attention_window.py:121-124). q, k, v: [S, H, D]."""
    scores = torch.einsum("qhd,khd->hqk", q.float(), k.float()) * scale
    scores = scores.masked_fill(~mask[None], -float("inf"))
    out = torch.einsum("hqk,khd->qhd", scores.softmax(-1), v.float())
    return out, scores.logsumexp(-1).T


def window_softmax_reference(query, key, value, layout, bounds, scale, anchor_frames="none"):
    """Per-frame SDPA over each frame's window (window.py:56-111), CPU fp32 or the input
    dtype. The CPU baseline path for the window branch."""
    heads, head_dim = query.shape[1], query.shape[2]
    vs, ve = layout.video_start, layout.video_end
    nf, tpf = layout.num_frames, layout.tokens_per_frame
    gidx = layout.global_index(query.device)
    out = torch.empty_like(query)

    def sdpa(qr, kr, vr):
        o = F.scaled_dot_product_attention(qr.permute(1, 0, 2).unsqueeze(0),
                                           kr.permute(1, 0, 2).unsqueeze(0),
                                           vr.permute(1, 0, 2).unsqueeze(0), scale=scale)
        return o.squeeze(0).permute(1, 0, 2)

    if gidx.numel():
        out[gidx] = sdpa(query[gidx], key, value)
    gk, gv = key[gidx], value[gidx]
    shape = (nf, tpf, heads, head_dim)
    vq, vk, vv = query[vs:ve].view(shape), key[vs:ve].view(shape), value[vs:ve].view(shape)
    for f in range(nf):
        lo, hi = max(bounds[f][0], 0), min(bounds[f][1], nf - 1)
        if anchor_frames in ("rows", "both") and f in (0, nf - 1):
            lo, hi = 0, nf - 1
        extra = [a for a in ((0, nf - 1) if anchor_frames in ("columns", "both") else ())
                 if not lo <= a <= hi]
        wk = torch.cat([gk, vk[lo:hi + 1].reshape(-1, heads, head_dim)]
                       + [vk[a].reshape(-1, heads, head_dim) for a in extra])
        wv = torch.cat([gv, vv[lo:hi + 1].reshape(-1, heads, head_dim)]
                       + [vv[a].reshape(-1, heads, head_dim) for a in extra])
        out[vs + f * tpf: vs + (f + 1) * tpf] = sdpa(vq[f], wk, wv)
    return out


def softmax_gate(out, gate):
    """bf16(out) * bf16(gate) rounded to bf16, [T, H*D] (kernels.py:62-63)."""
    o = out.to(torch.bfloat16)
    return (o * gate.reshape(o.shape[0], o.shape[1], 1).to(torch.bfloat16)).reshape(o.shape[0], -1)


def qk_rope(x, weight, eps, cos=None, sin=None, *, round_norm=True, round_products=True):
    """fp32 QK RMSNorm + rotate-half RoPE with the bf16 rounding points of
    paper_qk_rope.py:82-95, using an indexed partner (test_paper_stack_attention_rope.py:31-52)."""
    acc = x.float()
    variance = torch.sum(acc * acc, dim=-1, keepdim=True) / x.shape[-1]
    norm = (acc * (variance + eps).rsqrt()) * weight.float()
    if round_norm:
        norm = norm.to(x.dtype).float()
    if cos is not None:
        r = cos.shape[-1]
        index = (torch.arange(r) + r // 2) % r
        sign = torch.ones(r)
        sign[:r // 2] = -1
        lhs = norm[..., :r] * cos.to(x.dtype).float()[:, None]
        rhs = norm.index_select(-1, index) * sign * sin.to(x.dtype).float()[:, None]
        if round_products:
            lhs, rhs = lhs.to(x.dtype).float(), rhs.to(x.dtype).float()
        norm = torch.cat((lhs + rhs, norm[..., r:]), dim=-1)
    return norm.to(x.dtype)


def rope_complex_fp64(n, cos, sin):
    """Rotate-half RoPE as complex multiplication in float64: pairs (i, i + R/2) are
    (re, im) and the angle is arccos-free (uses the given cos/sin columns i)."""
    r = cos.shape[-1]
    z = torch.complex(n[..., :r // 2].double(), n[..., r // 2:r].double())
    w = torch.complex(cos[:, None, :r // 2].double(), sin[:, None, :r // 2].double())
    y = z * w
    return torch.cat((y.real, y.imag, n[..., r:].double()), dim=-1)


def rope_tables_3d(frames, height, width, dims=(44, 42, 42), theta=10000.0):
    """Independent float64 restatement of the 3D rotate-half tables: angle of pair i =
    position along its axis * theta^(-2j/dim) for its j-th frequency."""
    pairs = []
    for axis, dim in enumerate(dims):
        for j in range(dim // 2):
            pairs.append((axis, theta ** (-2.0 * j / dim)))
    rows = []
    for t in range(frames):
        for y in range(height):
            for x in range(width):
                p = (t, y, x)
                rows.append([p[a] * fr for a, fr in pairs])
    half = torch.tensor(rows, dtype=torch.float64)
    full = torch.cat((half, half), dim=1)
    return full.cos(), full.sin()
