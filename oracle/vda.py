"""VDA oracle: frame-wise delta-rule linear attention (vdn_solve, bridge alpha).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). torch-CPU float64 unless stated.

Reference: src/models/linear_attention/paper_stack.py (prepare :30-48, statistics :51-110,
boundary plan :131-159, compose/scan :162-236, gather :239-263, readout :266-318),
paper_sglang.py (activation :211-283, epilogue :377-437, gather :445-501), scan.py
(frame_statistics :122-173, _run_scans :176-213, gather_linear_state :267-402),
delta_rule.py:45-60 (VdnDelta), branch.py:404-482 (eager _readout), layers.py:36-69
(FrameKDAAlpha), rms_norm.py:29-32.

Pins (tests/test_oracle_vda.py):
  factors        (I + A) T / alpha = I; J (I + A) = B; the solve form of one recurrence step
                 S' = (S diag(alpha) + B)(I + A)^-1 (delta_rule.py:32) equals S T + J
  scan/gather    explicit per-frame loops; alpha == 1 with A == 0 reduces the state to the
                 closed form sum of B over the frames outside the window; compact bank ==
                 full banks at the plan's cut points
  boundary_plan  reference KAT: F=35, chunk-5 windows -> cuts (0,4,9,...,34,35)
                 (tests/test_paper_stack_vda_ops.py:300-307)
  statistics     A symmetric, equals sum_s beta k k^T; B == bf16(bf16(v beta)^T k)
  prepare        torch SiLU / L2 over D
  short conv     torch conv2d / conv1d (groups = channels) in float64; the reference test's
                 temporal loop (test_paper_stack_vda_ops.py:43-49); a unit impulse weight
                 reduces it to prepare
  eager path     float64 restatement at relative error < 4e-3 (the reference's own
                 branch-vs-fp64 bound, test_paper_stack_vda_ops.py:208-256)
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import mxfp8 as _mx

D = 128


def bf16(x: torch.Tensor) -> torch.Tensor:
    """Round to bf16 values (kept in x's float dtype)."""
    return x.to(torch.bfloat16).to(x.dtype)


# ------------------------------------------------------------------------ geometry ----

def window_bounds(num_frames, radius, chunk=0):
    """Per-frame inclusive window [lo, hi] (window.py:26-52)."""
    if chunk <= 0:
        return [(t - radius, t + radius) for t in range(num_frames)]
    return [((t // chunk - radius) * chunk, (t // chunk + radius + 1) * chunk - 1)
            for t in range(num_frames)]


def boundary_plan(bounds, frames, chunk_size=8):
    """Python restatement of _boundary_plan (paper_stack.py:131-154)."""
    cuts = {0, frames}
    for f, (lo, hi) in enumerate(bounds):
        assert lo <= f <= hi
        cuts.update((max(0, lo), min(frames, hi + 1)))
    req = sorted(cuts)
    for a, b in zip(req[:-1], req[1:]):
        cuts.update(range(a + chunk_size, b, chunk_size))
    cuts = tuple(sorted(cuts))
    pos = {x: i for i, x in enumerate(cuts)}
    return dict(
        cuts=cuts,
        before=[max(0, pos[max(0, lo)] - 1) for lo, _ in bounds],
        after=[min(len(cuts) - 2, pos[min(frames, hi + 1)]) for _, hi in bounds],
        has_before=[lo > 0 for lo, _ in bounds],
        has_after=[hi + 1 < frames for _, hi in bounds],
    )


# ------------------------------------------------------------------------ features ----

def prepare(tokens: torch.Tensor, frames: int, spatial: int, l2norm: bool) -> torch.Tensor:
    """SiLU (+ L2 over D, clamp 1e-12 on the sum of squares) -> [F, H, S, D], float64
    (paper_sglang.py:235-238). Not rounded."""
    x = F.silu(tokens.double())
    if l2norm:
        x = x / x.square().sum(-1, keepdim=True).clamp_min(1e-12).sqrt()
    n, h, d = x.shape
    return x.reshape(frames, spatial, h, d).permute(0, 2, 1, 3).contiguous()


def short_conv_prepare(tokens: torch.Tensor, frames: int, frame_h: int, frame_w: int,
                       w_sp: torch.Tensor, w_tm: torch.Tensor, l2norm: bool,
                       round_spatial: bool = True) -> torch.Tensor:
    """paper_prepare with the separable short conv (paper_stack.py:43-47): the depthwise 5x5
    spatial conv of each frame (cross-correlation, zero padding 2, no bias;
    LinearAttentionSepConv.spatial, features.py:175-196), rounded to bf16 as the reference's
    bf16 conv2d output is (round_spatial); then the depthwise 5-tap temporal conv across
    frames, out[t] = sum_j x[t + j - 2] w_tm[:, j] with zero frames outside [0, F)
    (vdn_temporal_conv_act, paper_sglang.py:165-203; the reference test's loop,
    test_paper_stack_vda_ops.py:43-49); SiLU (+ L2 over D). tokens [F*S, H, D], token
    f*S + y*W + x; w_sp [H*D, 5, 5]; w_tm [H*D, 5]. Returns float64 [F, H, S, D], not rounded.
    Written as explicit shifted sums (no convolution routine)."""
    n, h, d = tokens.shape
    c = h * d
    x = tokens.double().reshape(frames, frame_h, frame_w, c)
    ws, wt = w_sp.double().reshape(c, 5, 5), w_tm.double().reshape(c, 5)
    xp = torch.zeros(frames, frame_h + 4, frame_w + 4, c, dtype=torch.float64)
    xp[:, 2:2 + frame_h, 2:2 + frame_w] = x
    sp = torch.zeros_like(x)
    for i in range(5):
        for j in range(5):
            sp += xp[:, i:i + frame_h, j:j + frame_w] * ws[:, i, j]
    if round_spatial:
        sp = bf16(sp.float()).double()
    tp = torch.zeros(frames + 4, frame_h, frame_w, c, dtype=torch.float64)
    tp[2:2 + frames] = sp
    y = torch.zeros_like(sp)
    for j in range(5):
        y += tp[j:j + frames] * wt[:, j]
    y = F.silu(y)
    if l2norm:
        y = y.reshape(frames, frame_h, frame_w, h, d)
        y = y / y.square().sum(-1, keepdim=True).clamp_min(1e-12).sqrt()
    return y.reshape(frames, frame_h * frame_w, h, d).permute(0, 2, 1, 3).contiguous()


# --------------------------------------------------------------------- statistics ----

def statistics(k: torch.Tensor, v: torch.Tensor, beta: torch.Tensor, bf16_b: bool = True):
    """A = K^T diag(beta) K (float64, exactly symmetric); B = bf16(bf16(v * bf16(beta))^T k)
    for the bf16 path (paper_stack.py:72-83), else (v beta)^T k. k, v: [F,H,S,D]; beta [F,H,S]."""
    k, v, beta = k.double(), v.double(), beta.double()
    A = (k * beta[..., None]).transpose(-1, -2) @ k
    if bf16_b:
        vb = bf16((v * bf16(beta)[..., None]).float()).double()
        B = bf16((vb.transpose(-1, -2) @ k).float()).double()
    else:
        B = (v * beta[..., None]).transpose(-1, -2) @ k
    return A, B


# ----------------------------------------------------------------------- factors ----

def factors(A: torch.Tensor, B: torch.Tensor, alpha: torch.Tensor | None = None):
    """T = diag(alpha) (I + A)^-1, J = B (I + A)^-1 (delta_rule.py:45-60), float64."""
    A, B = A.double(), B.double()
    eye = torch.eye(A.shape[-1], dtype=torch.float64)
    inv = torch.linalg.inv(A + eye)
    T = inv if alpha is None else alpha.double()[..., None] * inv
    return T, B @ inv


# -------------------------------------------------------------------- scan/gather ----

def scan(T: torch.Tensor, J: torch.Tensor, seed: torch.Tensor | None = None):
    """Forward prefix[f] (frames 0..f) and reverse suffix[f] (frames f..F-1) banks
    (scan.py:199-211): state = state @ T[f] + J[f] from `seed` (zero when None)."""
    T, J = T.double(), J.double()
    start = torch.zeros_like(J[0]) if seed is None else seed.double()
    prefix, suffix = [], [None] * len(T)
    state = start
    for f in range(len(T)):
        state = state @ T[f] + J[f]
        prefix.append(state)
    state = start
    for f in range(len(T) - 1, -1, -1):
        state = state @ T[f] + J[f]
        suffix[f] = state
    return torch.stack(prefix), torch.stack(suffix)


def compact_bank(prefix, suffix, cuts):
    """bank[0, c] = prefix after chunk c, bank[1, c] = suffix from chunk c's first frame."""
    fwd = prefix[torch.tensor(cuts[1:]) - 1]
    rev = suffix[list(cuts[:-1])]
    return torch.stack((fwd, rev))


def gather(prefix, suffix, alpha, bounds, seed=None, bridge=True):
    """Complement-of-window state per frame, bridged by products of alpha
    (scan.py:359-402 / the reference test oracle's product form), float64."""
    start = torch.zeros_like(prefix[0]) if seed is None else seed.double()
    frames = len(prefix)
    out = []
    for f, (lo, hi) in enumerate(bounds):
        left = prefix[lo - 1] if lo > 0 else start
        right = suffix[hi + 1] if hi + 1 < frames else start
        if bridge:
            a = alpha.double().clamp_min(1e-12)
            left = left * a[max(0, lo):f + 1].prod(0)[..., None, :]
            right = right * a[f:min(frames, hi + 1)].prod(0)[..., None, :]
        out.append(left + right)
    return torch.stack(out)


# ------------------------------------------------------------------------ readout ----

def epilogue(readout: torch.Tensor, weight: torch.Tensor, gate: torch.Tensor, eps: float):
    """RMSNorm over D * weight * gate (paper_sglang.py:398-403), float64 of bf16 inputs.
    readout [F,H,S,D] -> [F*S, H*D]."""
    r = readout.double()
    ms = r.square().mean(-1, keepdim=True)
    y = r * torch.rsqrt(ms + eps) * weight.double()
    f, h, s, d = r.shape
    return (y.permute(0, 2, 1, 3).reshape(f * s, h, d) * gate.double()).reshape(f * s, h * d)


def paper_branch(q_raw, k_raw, v_raw, beta, gate, alpha, bounds, frames, spatial, weight, eps,
                 text=None, bridge=True, chunk_size=8, conv=None, frame_size=None):
    """The paper VDA body (paper_stack.py:266-318) at float64 with the bf16 rounding points
    of the reference's bf16 path: prepared q/k/v, B, the gathered state and the readout are
    rounded to bf16; A, the factors, scans and gather run in float64.

    q_raw/k_raw/v_raw [F*S, H, D]; beta [F*S, H]; gate [F*S, H, D]; alpha [F, H, D].
    text = (tk_raw, tv_raw, text_beta [L, H]) seeds both scans with half its injection.
    conv = {proj: (w_sp [H*D, 5, 5], w_tm [H*D, 5])} convolves those projections
    (short_conv_prepare; frame_size = (H_f, W_f)).
    Returns float64 [F*S, H*D] (not rounded) and intermediates.
    """
    h = q_raw.shape[1]

    def prep(raw, proj, l2):
        if conv is not None and proj in conv:
            x = short_conv_prepare(raw, frames, *frame_size, *conv[proj], l2)
        else:
            x = prepare(raw, frames, spatial, l2)
        return bf16(x.float()).double()

    q = prep(q_raw, "q", True)
    k = prep(k_raw, "k", True)
    v = prep(v_raw, "v", False)
    b = beta.double().reshape(frames, spatial, h).permute(0, 2, 1)
    A, B = statistics(k, v, b)
    seed = None
    if text is not None:
        tk_raw, tv_raw, tb = text
        L = tk_raw.shape[0]
        tk = bf16(prepare(tk_raw, 1, L, True).float()).double()
        tv = bf16(prepare(tv_raw, 1, L, False).float()).double()
        tA, tB = statistics(tk, tv, tb.double().reshape(1, L, h).permute(0, 2, 1))
        _, tJ = factors(tA, tB)
        seed = 0.5 * tJ[0]
    T, J = factors(A, B, alpha)
    prefix, suffix = scan(T, J, seed)
    state = gather(prefix, suffix, alpha, bounds, seed, bridge)
    state = bf16(state.float()).double()
    readout = bf16((q @ state.transpose(-1, -2)).float()).double()
    out = epilogue(readout, weight, gate.reshape(frames * spatial, h, q_raw.shape[2]), eps)
    return out, dict(A=A, B=B, T=T, J=J, prefix=prefix, suffix=suffix, state=state,
                     readout=readout, seed=seed)


# --------------------------------------------------------- eager fp32 (CPU path) ----

def frame_kda_alpha(frame_mean, down_w, up_w, dt_bias, a_log, heads, head_dim):
    """alpha = exp(-exp(A_log) * softplus(up(down(mean)) + dt_bias)), fp32 (layers.py:36-69)."""
    delta = F.linear(F.linear(frame_mean.float(), down_w.float()), up_w.float()) + dt_bias.float()
    scale = torch.exp(a_log.float())[:, None]
    return torch.exp(-scale * F.softplus(delta.view(-1, heads, head_dim)))


def eager_branch_fp32(q_raw, k_raw, v_raw, beta, gate, alpha, bounds, frames, spatial, weight,
                      eps=1e-6, text_state=None):
    """The reference's eager `_readout` in fp32 on the CPU (branch.py:404-482): features
    (SiLU, F.normalize eps 1e-6 for q/k), frame_statistics with fp32 A (scan.py:144-173),
    VdnDelta Cholesky factors (delta_rule.py:45-60), _run_scans, the log-prefix gather
    (scan.py:359-402), einsum readout, RMSNorm via vector_norm (rms_norm.py:29-32), gate.

    This is the CPU baseline path at C1 (F=4, S=256, H=8, d=64) and at larger shapes.
    q_raw etc. [F*S, H, d] fp32; beta [F*S, H]; gate [F*S, H, d]; alpha [F, H, d].
    """
    h, d = q_raw.shape[1], q_raw.shape[2]
    q = F.normalize(F.silu(q_raw), dim=-1, eps=1e-6)
    k = F.normalize(F.silu(k_raw), dim=-1, eps=1e-6)
    v = F.silu(v_raw)
    shape = (frames, spatial, h, d)
    kf = k.view(shape).permute(0, 2, 1, 3)
    vf = v.view(shape).permute(0, 2, 1, 3)
    b = beta.view(frames, spatial, h).permute(0, 2, 1)
    kf32 = kf.contiguous().float()
    A = torch.matmul((kf32 * b.unsqueeze(-1).float()).transpose(-1, -2), kf32)
    A = 0.5 * (A + A.transpose(-1, -2))
    B = torch.matmul((vf * b.unsqueeze(-1)).contiguous().transpose(-1, -2), kf).float()
    eye = torch.eye(d, dtype=torch.float32).expand_as(A)
    chol = torch.linalg.cholesky(A + eye)
    linv = torch.linalg.solve_triangular(chol, eye, upper=False, left=True)
    inv = linv.transpose(-1, -2) @ linv
    T = alpha.unsqueeze(-1) * inv
    J = B @ inv
    start = torch.zeros_like(J[0]) if text_state is None else text_state
    prefix, suffix = [], [None] * frames
    state = start
    for f in range(frames):
        state = state @ T[f] + J[f]
        prefix.append(state)
    state = start
    for f in range(frames - 1, -1, -1):
        state = state @ T[f] + J[f]
        suffix[f] = state
    prefix, suffix = torch.stack(prefix), torch.stack(suffix)
    last_before = torch.tensor([lo for lo, _ in bounds]) - 1
    first_after = torch.tensor([hi for _, hi in bounds]) + 1
    before_idx, after_idx = last_before.clamp(min=0), first_after.clamp(max=frames - 1)
    has_before, has_after = last_before >= 0, first_after < frames
    sb, sa = prefix[before_idx], suffix[after_idx]
    if text_state is not None:
        sb = torch.where(has_before.view(-1, 1, 1, 1), sb, text_state)
        sa = torch.where(has_after.view(-1, 1, 1, 1), sa, text_state)
    log_alpha = torch.log(alpha.clamp_min(1e-12))
    lp = torch.cat([torch.zeros_like(log_alpha[:1]), log_alpha.cumsum(0)])
    frames_idx = torch.arange(frames)
    sb = sb * torch.exp(lp[frames_idx + 1] - lp[(last_before + 1).clamp(min=0)]).unsqueeze(2)
    sa = sa * torch.exp(lp[first_after.clamp(max=frames)] - lp[frames_idx]).unsqueeze(2)
    if text_state is not None:
        st = sb + sa
    else:
        st = sb * has_before.view(-1, 1, 1, 1) + sa * has_after.view(-1, 1, 1, 1)
    readout = torch.einsum("fhvk,fshk->fshv", st, q.view(shape)).reshape(frames * spatial, h, d)
    ms = torch.linalg.vector_norm(readout, dim=-1, keepdim=True, dtype=torch.float32).pow(2) / d
    normed = readout * torch.rsqrt(ms + eps) * weight.float()
    return (normed * gate).reshape(frames * spatial, h * d)


def eager_branch_fp64(q_raw, k_raw, v_raw, beta, gate, alpha, bounds, frames, spatial, weight,
                      eps=1e-6):
    """Independent float64 restatement of eager_branch_fp32 (solve form, product-form bridge),
    used to pin it."""
    h, d = q_raw.shape[1], q_raw.shape[2]

    def feat(x, l2):
        y = F.silu(x.double())
        return y / y.norm(dim=-1, keepdim=True).clamp_min(1e-6) if l2 else y

    q, k, v = feat(q_raw, True), feat(k_raw, True), feat(v_raw, False)
    out = torch.zeros(frames * spatial, h, d, dtype=torch.float64)
    kk = k.view(frames, spatial, h, d)
    vv = v.view(frames, spatial, h, d)
    bb = beta.double().view(frames, spatial, h)
    a = alpha.double()
    eye = torch.eye(d, dtype=torch.float64)
    for hh in range(h):
        Ms, Bs = [], []
        for f in range(frames):
            kf, vf, bf = kk[f, :, hh], vv[f, :, hh], bb[f, :, hh]
            Ms.append(eye + (kf * bf[:, None]).T @ kf)
            Bs.append((vf * bf[:, None]).T @ kf)
        pre, suf = [], [None] * frames
        s = torch.zeros(d, d, dtype=torch.float64)
        for f in range(frames):
            s = torch.linalg.solve(Ms[f], (s * a[f, hh][None, :] + Bs[f]).T).T
            pre.append(s)
        s = torch.zeros(d, d, dtype=torch.float64)
        for f in range(frames - 1, -1, -1):
            s = torch.linalg.solve(Ms[f], (s * a[f, hh][None, :] + Bs[f]).T).T
            suf[f] = s
        for f, (lo, hi) in enumerate(bounds):
            st = torch.zeros(d, d, dtype=torch.float64)
            if lo > 0:
                st = st + pre[lo - 1] * a[max(0, lo):f + 1, hh].prod(0)[None, :]
            if hi + 1 < frames:
                st = st + suf[hi + 1] * a[f:min(frames, hi + 1), hh].prod(0)[None, :]
            r = q[f * spatial:(f + 1) * spatial, hh] @ st.T
            r = r * torch.rsqrt(r.square().mean(-1, keepdim=True) + eps) * weight.double()
            out[f * spatial:(f + 1) * spatial, hh] = r * gate[f * spatial:(f + 1) * spatial, hh].double()
    return out.reshape(frames * spatial, h * d)


def bf16_np(x):
    return _mx.bf16_round(np.asarray(x, dtype=np.float32))
