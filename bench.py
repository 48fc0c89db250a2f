"""Hybrid DiT block forward at the 108k-token clip shape on one MI355X.

Workload: one block (hidden 5120, 40 heads x 128, FFN 13824 GELU-tanh, rank-64 LoRA merged into
QKV, AdaLN from a timestep embedding, frame-window softmax (+-1 frame) with 3D RoPE, VDA linear
attention, cross-attention to 512 context rows, gated residuals) over 30 latent frames of
45 x 80 = 108,000 tokens, bf16 activations, MXFP8 projections. Random-init weights N(0, 0.02),
hidden/temb/context N(0, 1), all resident in HBM before timing.

Prints one JSON line: value = the median ms per block forward over the timed steps (one event
pair per step, lower is better), the MXFP8 GEMM roofline (algorithmic FLOP / measured launch
time, HIP events on the launch stream, from separate instrumented steps), the VDA passes'
algorithmic GB/s, a per-entry-point breakdown, the caller stream's idle time per block, and the
CPU fp32 path timed on a bounded sample.

  python bench.py [--steps K] [--warmup W] [--frames F] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import sys
import time

METRIC = "ms per hybrid DiT block fwd @108k tok; MXFP8 TFLOP/s & VDA GB/s vs peak"
PEAK_MXFP8_TFLOPS = 5000.0   # dense MXFP8 / FP8 MFMA, MI355X
PEAK_BF16_TFLOPS = 2500.0    # dense bf16 MFMA, MI355X
PEAK_HBM_GBS = 8000.0        # HBM3E, MI355X
HEIGHT, WIDTH = 45, 80
D = 128

GEMMS = ("vdn_mxfp8_gemm", "vdn_mxfp8_gemm_act_quantize")
VDA_ENTRIES = ("vdn_vda_statistics", "vdn_vda_factors", "vdn_vda_compose", "vdn_vda_scan",
               "vdn_vda_log_prefix", "vdn_vda_gather", "vdn_vda_readout", "vdn_vda_readout_mxfp8",
               "vdn_vda_readout_gated")
ATTENTION = ("vdn_window_attention", "vdn_window_attention_mxfp8")
# the VDA passes bounded by HBM (the factors and the scan are latency-bound: 128x128
# eliminations and 30 serial frame steps)
VDA_HBM_BOUND = ("vdn_vda_statistics", "vdn_vda_gather", "vdn_vda_readout",
                 "vdn_vda_readout_mxfp8", "vdn_vda_readout_gated")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def padded(n):
    return -(-n // 128) * 128


def work(name, a, plans):
    """Algorithmic (flop, bytes) of one launch from its C-ABI arguments."""
    if name == "vdn_mxfp8_gemm":
        kp, rows, n = a[6], a[14], a[15]
        ops = [a[7], a[8], a[10], a[12]]  # bias, addend, residual, gate
        extra = rows * n * 2 * sum(1 for p in ops[1:3] if p is not None)
        return 2.0 * rows * n * kp, rows * kp + n * kp + (rows + n) * kp / 32 + rows * n * 2 + extra
    if name == "vdn_mxfp8_gemm_act_quantize":
        kp, rows, n = a[6], a[11], a[12]
        kp_out = padded(n)
        return 2.0 * rows * n * kp, rows * kp + n * kp + (rows + n) * kp / 32 + rows * kp_out * (1 + 1 / 32)
    if name == "vdn_mxfp8_quantize":
        rows, k = a[1], a[2]
        return 0.0, rows * k * 2 + padded(rows) * padded(k) * (1 + 1 / 32)
    if name == "vdn_mxfp8_act_quantize":
        rows, k, act = a[1], a[2], a[4]
        inner = 2 * k if act == 2 else k
        return 0.0, rows * inner * 2 + padded(rows) * padded(k) * (1 + 1 / 32)
    if name == "vdn_mxfp8_prenorm_quantize":
        rows, k, y = a[1], a[2], a[12]
        return 0.0, (rows * k * 2 * (2 if y is not None else 1) + rows * 8 + padded(rows)
                     + padded(rows) * padded(k) * (1 + 1 / 32))
    if name == "vdn_qk_rmsnorm_rope":
        flags, tokens, heads, hd, rot = a[20], a[21], a[22], a[23], a[19]
        operands = 1 if flags & 8 else 2
        tables = 0 if a[13] is None else 2 * tokens * rot * (4 if flags & 4 else 2)
        return 0.0, operands * tokens * heads * hd * 4 + tables
    if name in ("vdn_window_attention", "vdn_window_attention_mxfp8"):
        heads = a[13]
        pairs = plans.get(a[11], 0)
        return 4.0 * D * heads * pairs, 0.0
    if name == "vdn_vda_statistics":
        f, h, s, beta_f32 = a[13], a[14], a[15], a[12]
        return (4.0 * f * h * s * D * D, 2 * f * s * h * D * 2 + f * s * h * (4 if beta_f32 else 2)
                + 2 * f * h * D * D * 4)
    if name == "vdn_vda_factors":
        count = a[3]
        return 0.0, 4 * count * D * D * 4 + (count * D * 4 if a[2] is not None else 0)
    if name == "vdn_vda_compose":
        heads, chunks = a[2], a[5]
        return 0.0, 4 * chunks * heads * D * D * 4
    if name == "vdn_vda_scan":
        chunks, heads = a[3], a[4]
        return 0.0, 4 * chunks * heads * D * D * 4
    if name == "vdn_vda_log_prefix":
        f, h = a[1], a[2]
        return 0.0, 2 * f * h * D * 4
    if name == "vdn_vda_gather":
        f, h, out_f32 = a[10], a[11], a[13]
        return 0.0, 2 * f * h * D * D * 4 + f * h * D * D * (4 if out_f32 else 2)
    if name == "vdn_vda_readout":   # (..., o_ss, head_dim, frames, heads, spatial, stream)
        f, h, s = a[18], a[19], a[20]
        return 2.0 * f * s * h * D * D, 3 * f * s * h * D * 2 + f * h * D * D * 2
    if name == "vdn_vda_readout_mxfp8":   # q, gate read (bf16); codes + scales written
        f, h, s = a[17], a[18], a[19]
        return (2.0 * f * s * h * D * D,
                2 * f * s * h * D * 2 + f * s * h * D * (1 + 1 / 32) + f * h * D * D * 2)
    if name == "vdn_vda_readout_gated":   # q and the gate's down rows read; gate formed inside
        f, h, s, mx = a[21], a[22], a[23], a[17] is not None
        out = f * s * h * D * ((1 + 1 / 32) if mx else 2)
        return (4.0 * f * s * h * D * D,
                f * s * h * D * 2 + f * s * D * 2 + h * D * (D + 1) * 2 + f * h * D * D * 2 + out)
    return 0.0, 0.0


def aggregate(timer, plans, stream=None):
    """name -> [launches, ms, flop, bytes] over the timer's records (those on `stream`, a
    stream handle, if given)."""
    per = {}
    for name, a, t, handle in timer.durations():
        if stream is not None and handle != stream:
            continue
        flop, nbytes = work(name, a, plans)
        e = per.setdefault(name, [0, 0.0, 0.0, 0.0])
        e[0] += 1
        e[1] += t
        e[2] += flop
        e[3] += nbytes
    return per


def breakdown_of(per, steps):
    out = {}
    for name, (count, t, flop, nbytes) in sorted(per.items(), key=lambda kv: -kv[1][1]):
        row = dict(ms_per_step=round(t / steps, 3), launches_per_step=count // steps,
                   avg_launch_ms=round(t / count, 4))
        if flop and name in GEMMS + ATTENTION:
            row["tflops"] = round(flop / (t * 1e-3) / 1e12, 1)
        if nbytes and name not in GEMMS + ATTENTION:
            row["gbs"] = round(nbytes / (t * 1e-3) / 1e9, 1)
        out[name] = row
    return out


def short_conv_prepare(cfg, device, frames, steps):
    """The linear branch's short-conv feature prep (vdn_vda_conv_prepare) on K and V of the
    clip shape, outside the block (the block's configuration has no short conv): random
    N(0,1) K/V columns of a fused [T, 3H] projection, a random-init LinearAttentionSepConv.
    Algorithmic bytes per projection: the bf16 input read once and the bf16 output written
    once (2 x 2 B per element)."""
    if steps <= 0:
        return None
    import torch
    from vdn_amd import _lib
    from vdn_amd import vda as vv
    tokens = frames * HEIGHT * WIDTH
    hd, heads = cfg.hidden, cfg.heads
    g = torch.Generator(device=device).manual_seed(7)
    qkv = torch.randn(tokens, 3 * hd, generator=g, device=device).to(torch.bfloat16)
    torch.manual_seed(7)
    conv = vv.LinearAttentionSepConv(hd, ("k", "v")).to(torch.bfloat16).to(device)

    def run():
        for i, proj in ((1, "k"), (2, "v")):
            view = qkv[:, i * hd:(i + 1) * hd].view(tokens, heads, D)
            vv.paper_prepare(view, frames=frames, spatial=HEIGHT * WIDTH, l2norm=proj == "k",
                             conv=conv, proj=proj, frame_size=(HEIGHT, WIDTH))

    run()
    torch.cuda.synchronize()
    with _lib.LaunchTimer({"vdn_vda_conv_prepare"}) as timer:
        for _ in range(steps):
            run()
        torch.cuda.synchronize()
    times = [t for _, _, t, _ in timer.durations()]
    ms = sum(times) / len(times)
    nbytes = 2 * tokens * hd * 2
    log(f"short-conv prepare: {ms:.3f} ms per projection")
    return {"workload": f"K or V of [{tokens}, {hd}] bf16, 5x5 spatial + 5-tap temporal depthwise "
                        f"conv, SiLU (+L2), frame-major store", "ms_per_projection": round(ms, 4),
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}


def production_geometry(steps):
    """Both attention branches at the H3 production call's geometry on one GPU (random
    inputs): 37 latent frames of 28 x 36 = 1008 tokens (37,296 video rows) followed by 1,200
    global (text) rows, 56 heads x 128; a chunk-aligned window (VAE chunks of 5 frames,
    radius 1: up to 15 frames) with anchor frames 0 and 36 dense in both directions; the VDA
    branch on frames 1..35 (the anchors skipped and the bounds rebased by -1), with the K/V
    short conv, the 1,200 text rows as its virtual frame and boundary chunks of 8 frames.
    Window q/k are RMS-normalised N(0,1) rows (the QK-norm/RoPE pass is measured in the
    block)."""
    if steps <= 0:
        return None
    import torch
    import torch.nn.functional as F
    from vdn_amd import _lib
    from vdn_amd import vda as vv
    from vdn_amd import window as vw
    frames, fh, fw, heads, text = 37, 28, 36, 56, 1200
    tpf = fh * fw
    video = frames * tpf
    rows = video + text
    dev = "cuda"
    g = torch.Generator(device=dev).manual_seed(11)
    qkv = torch.randn(rows, 3, heads, D, generator=g, device=dev)
    q = F.normalize(qkv[:, 0], dim=-1).mul(D ** 0.5).bfloat16()
    k = F.normalize(qkv[:, 1], dim=-1).mul(D ** 0.5).bfloat16()
    v = qkv[:, 2].bfloat16()
    raw = torch.randn(rows, 3 * heads * D, generator=g, device=dev).bfloat16()
    del qkv
    layout = vw.SequenceLayout(rows, 0, frames, tpf, frame_height=fh, frame_width=fw,
                               text_start=video, text_len=text)
    bounds = vw.window_bounds(frames, 1, 5)
    plan = vw.prepare_paper_window_plan(layout, bounds, "both", device=dev)
    pairs = 0
    for p in plan.passes:
        for grp in p.groups:
            nq = sum(b - a for a, b in grp.query_ranges)
            nk = sum(b - a for a, b in grp.key_ranges)
            pairs += nq * nk
    # linear branch: frames 1 .. F-2, bounds rebased (branch.py:380-400)
    lf = frames - 2
    lrows = slice(tpf, (frames - 1) * tpf)
    hd = heads * D
    rq, rk, rv = (raw[lrows, i * hd:(i + 1) * hd].view(-1, heads, D) for i in range(3))
    tk, tv = (raw[video:, i * hd:(i + 1) * hd].view(-1, heads, D) for i in (1, 2))
    beta = torch.sigmoid(torch.randn(lf * tpf, heads, generator=g, device=dev)).bfloat16()
    tbeta = torch.sigmoid(torch.randn(text, heads, generator=g, device=dev)).bfloat16()
    down = torch.randn(lf * tpf, D, generator=g, device=dev).bfloat16()
    up_w = (torch.randn(hd, D, generator=g, device=dev) * 0.05).bfloat16()
    up_b = (torch.randn(hd, generator=g, device=dev) * 0.05).bfloat16()
    alpha = torch.rand(lf, heads, D, generator=g, device=dev) * 0.1 + 0.9
    lbounds = [(lo - 1, hi - 1) for lo, hi in bounds[1:-1]]
    torch.manual_seed(11)
    conv = vv.LinearAttentionSepConv(hd, ("k", "v")).to(torch.bfloat16).to(dev)
    normw = torch.ones(D, device=dev)
    gp = vv.OutputGateProjection(down, up_w, up_b)

    def run():
        vw.paper_window_attention(q, k, v, plan, enabled=True)
        vv.vda_forward(rq, rk, rv, beta, gp, alpha, lbounds, lf, tpf, normw, 1e-6,
                       chunk_size=8, text=(tk, tv, tbeta), conv=conv, frame_size=(fh, fw))

    with torch.no_grad():
        run()
        torch.cuda.synchronize()
        names = set(VDA_ENTRIES) | set(ATTENTION) | {"vdn_vda_conv_prepare"}
        with _lib.LaunchTimer(names) as timer:
            for _ in range(steps):
                run()
            torch.cuda.synchronize()
    per = {}
    for name, _, t, _ in timer.durations():
        per[name] = per.get(name, 0.0) + t / steps
    attn = sum(per.get(n, 0.0) for n in ATTENTION)
    vda = sum(t for n, t in per.items() if n not in ATTENTION)
    log(f"production geometry: window {attn:.2f} ms, VDA branch {vda:.2f} ms")
    return {"workload": (f"{frames} frames x {fh}x{fw} + {text} global rows, {heads}x{D} heads, "
                         f"window chunk 5 radius 1, anchors both; VDA on frames 1..{frames - 2} "
                         f"with K/V short conv and text state, chunk 8"),
            "window_attention_ms": round(attn, 3),
            "window_attention_tflops": round(4.0 * D * heads * pairs / (attn * 1e-3) / 1e12, 1),
            "vda_branch_ms": round(vda, 3),
            "vda_breakdown_ms": {n: round(t, 4) for n, t in sorted(per.items(), key=lambda x: -x[1])
                                 if n not in ATTENTION}}


def h3_block(steps, plans_of):
    """The block at VDN-H3's widths: hidden 5376, 56 x 128 heads (attention width 7168),
    SwiGLU FFN 14336 (up 5376 -> 28672 = [a | g], bf16, then the SwiGLU MXFP8 producer), on the
    production clip size of 37 frames x 28 x 36 = 37,296 tokens, +-1 frame window, 512
    context rows; random-init weights, synthetic inputs, one warmup block."""
    if steps <= 0:
        return None
    import torch
    from vdn_amd import _lib
    from vdn_amd import window as vw
    from vdn_amd.block import (BlockConfig, BlockWeights, HybridDiTBlock, cross_attention_plan,
                               make_inputs)
    cfg = BlockConfig(hidden=5376, heads=56, head_dim=128, ffn=14336, ffn_act="swiglu")
    frames, fh, fw = 37, 28, 36
    weights = BlockWeights.random(cfg, seed=0, device="cuda")
    block = HybridDiTBlock(cfg, weights)
    del weights
    hidden, temb, ctx, layout, rope = make_inputs(cfg, frames, fh, fw, seed=1, device="cuda")
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(frames, cfg.radius),
                                        device="cuda")
    cplan = cross_attention_plan(hidden.shape[0], ctx.shape[0], "cuda")
    plans = plans_of(plan, cplan, frames, fh * fw, hidden.shape[0], ctx.shape[0])
    with torch.no_grad():
        block(hidden, temb, ctx, layout, rope, plan, cplan)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with _lib.LaunchTimer(set(GEMMS)) as timer:
            start.record()
            for _ in range(steps):
                block(hidden, temb, ctx, layout, rope, plan, cplan)
            end.record()
            torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    # the projections on the caller's stream (the two context projections run on the side
    # stream, where an event pair also spans their wait for the attention's CUs)
    per = aggregate(timer, plans, torch.cuda.current_stream().cuda_stream)
    g = [sum(per[nm][i] for nm in GEMMS if nm in per) for i in range(4)]
    log(f"H3 widths: {ms:.2f} ms per block")
    return {"workload": f"block at hidden {cfg.hidden}, {cfg.heads}x{cfg.head_dim} heads, SwiGLU FFN "
                        f"{cfg.ffn}, {frames} frames x {fh}x{fw} = {hidden.shape[0]} tokens, "
                        f"+-1 frame window, {cfg.context} context rows",
            "ms_per_block": round(ms, 3),
            "mxfp8_gemm_tflops": round(g[2] / (g[1] * 1e-3) / 1e12, 1),
            # the FFN up projection with the SwiGLU producer in its epilogue (one launch)
            "ffn_up_swiglu_gemm_ms": round(
                per.get("vdn_mxfp8_gemm_act_quantize", [0, 0.0])[1] / steps, 3)}


def _launch_ms(timer, name):
    times = [t for n, _, t, _ in timer.durations() if n == name]
    return sum(times) / len(times) if times else float("nan")


def c2_quantize_gemm(steps):
    """MXFP8 quantize + block-scaled GEMM alone: bf16 activations [32768, 5120] ~ N(0,1)
    with 1% of the channels (51, seeded) scaled x20; weights [N, 5120] ~ N(0, 0.02) for
    N = 5120, 15360 (fused QKV), 13824 (FFN up); bf16 output. Algorithmic work: the
    quantize reads 2 B and writes 1 + 1/32 B per (padded) element; a GEMM is 2 M N K FLOP."""
    if steps <= 0:
        return None
    import torch
    from vdn_amd import _lib
    from vdn_amd import mxfp8 as vm
    m, k = 32768, 5120
    g = torch.Generator(device="cuda").manual_seed(2)
    x = torch.randn(m, k, generator=g, device="cuda")
    cols = torch.randperm(k, generator=g, device="cuda")[:k // 100]
    x[:, cols] *= 20
    x = x.to(torch.bfloat16)
    qbytes = m * k * 2 + m * k * (1 + 1 / 32)
    vm.launch_quantize(x)
    torch.cuda.synchronize()
    with _lib.LaunchTimer({"vdn_mxfp8_quantize"}) as timer:
        for _ in range(steps):
            q, s = vm.launch_quantize(x)
        torch.cuda.synchronize()
    qms = _launch_ms(timer, "vdn_mxfp8_quantize")
    out = {"workload": f"bf16 [{m}, {k}] N(0,1) with {k // 100} outlier channels x20; "
                       f"weights [N, {k}] N(0,0.02); bf16 output",
           "quantize": {"us": round(qms * 1e3, 2), "gbs": round(qbytes / (qms * 1e-3) / 1e9, 1),
                        "hbm_frac": round(qbytes / (qms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                        "target_us": 90.8}}
    del x
    for n in (5120, 15360, 13824):
        w = (torch.randn(n, k, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        wq, ws = vm.launch_quantize(w)
        del w
        y = vm.mxfp8_gemm(q, s, wq, ws, n, rows=m)
        torch.cuda.synchronize()
        with _lib.LaunchTimer({"vdn_mxfp8_gemm"}) as timer:
            for _ in range(steps):
                vm.mxfp8_gemm(q, s, wq, ws, n, rows=m, out=y)
            torch.cuda.synchronize()
        ms = _launch_ms(timer, "vdn_mxfp8_gemm")
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        out[f"gemm_n{n}"] = {"ms": round(ms, 4), "tflops": round(tf, 1),
                             "mxfp8_frac": round(tf / PEAK_MXFP8_TFLOPS, 4)}
        del wq, ws, y
    log("C2: " + ", ".join(f"{key} {v.get('ms', v.get('us'))}" for key, v in out.items()
                           if isinstance(v, dict)))
    return out


def c3_vda(steps, frames=30):
    """The VDA linear-attention branch alone at the clip shape: 30 frames x 3600 tokens, 40
    heads x 128, bf16 q, k, v ~ N(0,1) with q and k L2-normalised, beta = sigmoid(N(0,1)),
    alpha = exp(-A_h dt_c) (A ~ U(1,16) per head, dt log-uniform in [1e-3, 1e-1]), output
    gate sigmoid(N(0,1)), norm weight 1, one chunk per frame, +-1 frame window, fp32 state.
    The branch runs statistics, factors, both scans, the gather and the gated readout."""
    if steps <= 0:
        return None
    import torch
    import torch.nn.functional as F
    from vdn_amd import _lib
    from vdn_amd import vda as vv
    heads, spatial = 40, HEIGHT * WIDTH
    t = frames * spatial
    g = torch.Generator(device="cuda").manual_seed(3)

    def normal(*shape):
        return torch.randn(*shape, generator=g, device="cuda")

    q = F.normalize(normal(t, heads, D), dim=-1).to(torch.bfloat16)
    k = F.normalize(normal(t, heads, D), dim=-1).to(torch.bfloat16)
    v = normal(t, heads, D).to(torch.bfloat16)
    beta = torch.sigmoid(normal(t, heads)).to(torch.bfloat16)
    gate = torch.sigmoid(normal(t, heads, D)).to(torch.bfloat16)
    a = torch.rand(heads, generator=g, device="cuda") * 15 + 1
    dt = torch.exp(torch.rand(heads, D, generator=g, device="cuda")
                   * (math.log(0.1) - math.log(1e-3)) + math.log(1e-3))
    alpha = torch.exp(-a[:, None] * dt)[None].expand(frames, heads, D).contiguous()
    normw = torch.ones(D, device="cuda")
    bounds = [(f - 1, f + 1) for f in range(frames)]
    out = torch.empty(t, heads * D, dtype=torch.bfloat16, device="cuda")

    def run():
        vv.vda_forward(q, k, v, beta, gate, alpha, bounds, frames, spatial, normw, 1e-6,
                       chunk_size=8, out=out)

    with torch.no_grad():
        run()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with _lib.LaunchTimer(set(VDA_ENTRIES)) as timer:
            start.record()
            for _ in range(steps):
                run()
            end.record()
            torch.cuda.synchronize()
    wall = start.elapsed_time(end) / steps
    per = aggregate(timer, {})
    kern = sum(e[1] for e in per.values()) / steps
    nbytes = sum(e[3] for e in per.values()) / steps
    hb = [sum(per[n][i] for n in VDA_HBM_BOUND if n in per) for i in range(4)]
    hb_gbs = hb[3] / (hb[1] * 1e-3) / 1e9
    log(f"C3: VDA branch {wall:.3f} ms per call ({kern:.3f} ms in kernels)")
    return {"workload": f"VDA branch, {frames} frames x {spatial} tokens, {heads}x{D} heads, "
                        f"bf16 q,k,v N(0,1) (q, k L2-normalised), fp32 state",
            "ms": round(wall, 4), "kernel_ms": round(kern, 4),
            "gbs": round(nbytes / (kern * 1e-3) / 1e9, 1),
            "hbm_bound_passes": {"entries": [n for n in VDA_HBM_BOUND if n in per],
                                 "ms": round(hb[1] / steps, 4), "gbs": round(hb_gbs, 1),
                                 "hbm_frac": round(hb_gbs / PEAK_HBM_GBS, 4)},
            "passes": breakdown_of(per, steps)}


def c1_vda(steps):
    """C1, the reference's CPU-runnable case: one VDA layer at 4 frames x 16x16 tokens, 8 heads,
    head_dim 64; q, k, v ~ N(0,1) with q and k L2-normalised, beta = sigmoid(N(0,1)),
    alpha = exp(-A_h dt_c) (A ~ U(1,16), dt log-uniform in [1e-3, 1e-1]), gate and norm
    weight 1, +-1 frame window. The GPU path (bf16 operands, head dim zero-padded to the
    kernels' 128) is timed per call; beside it the reference's eager fp32 body on the host
    cores (the oracle's restatement of branch.py:404-482), whose output the GPU result is
    compared with. At this size a call is bound by its 15 launches, not by the GPU."""
    if steps <= 0:
        return None
    import torch
    import torch.nn.functional as F
    from oracle import vda as ov
    from vdn_amd import _lib
    from vdn_amd import vda as vv
    frames, spatial, heads, d = 4, 256, 8, 64
    g = torch.Generator().manual_seed(0)
    q = F.normalize(torch.randn(frames * spatial, heads, d, generator=g), dim=-1)
    k = F.normalize(torch.randn(frames * spatial, heads, d, generator=g), dim=-1)
    v = torch.randn(frames * spatial, heads, d, generator=g)
    beta = torch.sigmoid(torch.randn(frames * spatial, heads, generator=g))
    a = torch.empty(heads).uniform_(1, 16, generator=g)
    dt = torch.exp(torch.rand(heads * d, generator=g) * (math.log(0.1) - math.log(1e-3))
                   + math.log(1e-3))
    alpha = torch.exp(-a[:, None] * dt.view(heads, d)).expand(frames, heads, d).contiguous()
    gate, w = torch.ones(frames * spatial, heads, d), torch.ones(d)
    bounds = [(max(f - 1, 0), min(f + 1, frames - 1)) for f in range(frames)]
    dev = [x.cuda() for x in (q.bfloat16(), k.bfloat16(), v.bfloat16(), beta, gate.bfloat16(),
                              alpha, w)]
    reps = 10 * steps

    def run():
        return vv.vda_forward(*dev[:6], bounds, frames, spatial, dev[6], 1e-6)

    with torch.no_grad():
        out = run()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            run()
        end.record()
        torch.cuda.synchronize()
        # the layer's own kernels, apart from the zero-padding of its d = 64 operands to the
        # 128-wide kernels (torch copies) and the launch gaps
        with _lib.LaunchTimer(set(VDA_ENTRIES) | {"vdn_vda_prepare"}) as timer:
            for _ in range(reps):
                run()
            torch.cuda.synchronize()
        kernel_ms = sum(t for _, _, t, _ in timer.durations()) / reps
        launches = len(timer.durations()) // reps
    gpu_ms = start.elapsed_time(end) / reps
    threads = host_threads()
    torch.set_num_threads(threads)
    t0 = time.perf_counter()
    ref = ov.eager_branch_fp32(q, k, v, beta, gate, alpha, bounds, frames, spatial, w)
    cpu_ms = (time.perf_counter() - t0) * 1e3
    rel = float((out.float().cpu() - ref).norm() / ref.norm())
    log(f"C1: VDA layer {gpu_ms:.3f} ms on the GPU ({kernel_ms:.3f} ms in {launches} kernels), "
        f"{cpu_ms:.1f} ms eager fp32 on {threads} host threads, rel-L2 {rel:.1e}")
    return {"workload": f"VDA layer, {frames} frames x {spatial} tokens, {heads}x{d} heads",
            "ms": round(gpu_ms, 4), "tokens_per_s": round(frames * spatial / gpu_ms * 1e3),
            "kernel_ms": round(kernel_ms, 4), "kernel_launches": launches,
            "rel_l2_vs_cpu_eager_fp32": float(f"{rel:.3g}"),
            "cpu_baseline": {"ms": round(cpu_ms, 2), "cores": threads, "kind": "port",
                             "sample": "the whole layer, eager fp32 body on the host"}}


def c4_window(steps, frames=30):
    """The frame-window softmax branch alone: 30 frames x 3600 tokens, 40 heads x 128, bf16
    q, k, v ~ N(0,1)/sqrt(128); QK RMSNorm (weight 1) + 3D RoPE (t, h, w split 44/42/42,
    theta 1e4), then exact softmax over the frame and its +-1 neighbours. Algorithmic work of
    the attention: 4 d FLOP per visible (query, key) pair per head (2.336e13 FLOP)."""
    if steps <= 0:
        return None
    import torch
    from vdn_amd import _lib
    from vdn_amd import window as vw
    heads, spatial = 40, HEIGHT * WIDTH
    t = frames * spatial
    g = torch.Generator(device="cuda").manual_seed(4)
    q, k, v = ((torch.randn(t, heads, D, generator=g, device="cuda") * D ** -0.5)
               .to(torch.bfloat16) for _ in range(3))
    ones = torch.ones(D, dtype=torch.bfloat16, device="cuda")
    cos, sin = vw.rope_tables_3d(frames, HEIGHT, WIDTH, device="cuda", dtype=torch.bfloat16)
    layout = vw.SequenceLayout(t, 0, frames, spatial, frame_height=HEIGHT, frame_width=WIDTH)
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(frames, 1), device="cuda")
    pairs = visible_pairs(frames, spatial, 1)
    flop = 4.0 * D * heads * pairs

    def run():
        qo, ko = vw.paper_qk_rmsnorm_rope(q, k, ones, ones, 1e-6, cos, sin, enabled=True)
        return vw.paper_window_attention(qo, ko, v, plan, enabled=True)

    with torch.no_grad():
        run()
        torch.cuda.synchronize()
        with _lib.LaunchTimer({"vdn_qk_rmsnorm_rope", "vdn_window_attention"}) as timer:
            for _ in range(steps):
                run()
            torch.cuda.synchronize()
    rope = _launch_ms(timer, "vdn_qk_rmsnorm_rope")
    attn = _launch_ms(timer, "vdn_window_attention")
    tf = flop / (attn * 1e-3) / 1e12
    rope_bytes = 2 * t * heads * D * 4 + 2 * t * D * 2
    log(f"C4: RoPE {rope:.3f} ms, window attention {attn:.3f} ms ({tf:.0f} TFLOP/s)")
    return {"workload": f"QK RMSNorm + 3D RoPE, then +-1 frame window softmax, {frames} frames x "
                        f"{spatial} tokens, {heads}x{D} heads, bf16",
            "ms": round(rope + attn, 4), "attention_ms": round(attn, 4),
            "attention_tflops": round(tf, 1), "attention_bf16_frac": round(tf / PEAK_BF16_TFLOPS, 4),
            "attention_frac_of_mxfp8_peak": round(tf / PEAK_MXFP8_TFLOPS, 4),
            "flop": flop, "qk_rope_ms": round(rope, 4),
            "qk_rope_gbs": round(rope_bytes / (rope * 1e-3) / 1e9, 1)}


def timed_steps(step, count):
    """Runs `step` count times back to back with one event pair per step on the caller's
    stream, bracketed by device synchronisations. Returns (per-step ms, mean ms over the
    whole run: first start to last end / count)."""
    import torch
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(count)]
    torch.cuda.synchronize()
    for s, e in evs:
        s.record()
        step()
        e.record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in evs], evs[0][0].elapsed_time(evs[-1][1]) / count


def visible_pairs(frames, spatial, radius):
    """Query-key pairs per head of the +-radius frame window."""
    total = 0
    for f in range(frames):
        lo, hi = max(0, f - radius), min(frames - 1, f + radius)
        total += spatial * spatial * (hi - lo + 1)
    return total


def host_threads():
    """Host cores this process may run on (its CPU affinity; os.cpu_count() counts the
    whole machine, which a host with several GPUs shares among them)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_baseline(cfg, weights, hidden, temb, ctx, cos, sin, frames_total, sample_frames):
    """The fp32 CPU block (the oracle's eager path) on the first `sample_frames` frames,
    extrapolated linearly in frames to the full clip, on every host core available."""
    import torch
    from oracle import block as ob
    threads = host_threads()
    torch.set_num_threads(threads)
    log(f"CPU baseline on {torch.get_num_threads()} threads (os.cpu_count() = {os.cpu_count()})")
    spatial = HEIGHT * WIDTH
    t = sample_frames * spatial
    w = {k: v.cpu() for k, v in weights.tensors.items()}
    args = (w, cfg, hidden[:t].cpu(), temb.cpu(), ctx.cpu(), sample_frames, HEIGHT, WIDTH,
            cos[:t].cpu(), sin[:t].cpu())
    start = time.perf_counter()
    with torch.no_grad():
        ob.eager_block_fp32(*args)
    elapsed = time.perf_counter() - start
    return dict(value=round(elapsed * 1e3 * frames_total / sample_frames, 1), unit="ms",
                cores=torch.get_num_threads(), kind="port",
                sample=(f"fp32 eager block (torch CPU, nn.Linear-equivalent bf16->fp32 weights, "
                        f"per-frame SDPA, eager VDA) on the first {sample_frames} frames "
                        f"({t} tokens): {elapsed:.1f} s, scaled x{frames_total / sample_frames:g} "
                        f"to {frames_total} frames"))


def summarize_counters(paths, command=""):
    """Markdown table of per-dispatch means of every counter in one or more rocprofv3 --pmc
    counter_collection.csv files (one pass each), one row per kernel. FETCH_SIZE and
    WRITE_SIZE (KiB) are scaled to bytes by the factor that maps their reading for the
    calibration kernel (a torch.neg of 1 GiB into 1 GiB, --calibrate-copy) onto 1 GiB."""
    import csv
    means, names = {}, {}
    for path in paths:
        per = {}
        with open(path) as f:
            for r in csv.DictReader(f):
                key = (r["Kernel_Name"], r["Counter_Name"])
                d = r["Dispatch_Id"]
                per.setdefault(key, {})
                per[key][d] = per[key].get(d, 0.0) + float(r["Counter_Value"])
        for (kernel, counter), by_dispatch in per.items():
            means.setdefault(kernel, {})[counter] = (sum(by_dispatch.values()) / len(by_dispatch),
                                                     len(by_dispatch))
            names[counter] = True
    scale = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        cal = [v[counter][0] for k, v in means.items() if CALIBRATION_KERNEL in k and counter in v]
        if cal:
            scale[counter] = CALIBRATION_KIB / max(cal) * 1024   # KiB reading -> bytes
    counters = sorted(names)

    def short(name):
        name = name.replace("void ", "").replace("(anonymous namespace)::", "")
        return name.split("(")[0].replace("vdn::", "")[:60]

    def fmt(counter, value):
        if counter in scale:
            return f"{value * scale[counter] / 1e9:.3f} GB"
        return f"{value:.3g}"

    out = []
    if command:
        out += ["Commands (from the repository root, on one MI355X):", "", *[f"    {c}" for c in
                                                                          command.split(" ;; ")], ""]
    if scale:
        out += ["Byte counters are scaled by the calibration kernel (1 GiB read, 1 GiB written): " +
                ", ".join(f"{c} x{scale[c] / 1024:.4f}" for c in scale) + ".", ""]
    out += ["| kernel | dispatches | " + " | ".join(counters) + " |",
            "|---|---:|" + "---:|" * len(counters)]
    for kernel, vals in sorted(means.items(), key=lambda kv: kv[0]):
        if CALIBRATION_KERNEL not in kernel and not any(t in kernel for t in ("vdn::", "vda_", "mxfp8", "window_attn", "qk_rope", "prenorm")):
            continue
        n = max(v[1] for v in vals.values())
        out.append(f"| `{short(kernel)}` | {n} | " +
                   " | ".join(fmt(c, vals[c][0]) if c in vals else "" for c in counters) + " |")
    print("\n".join(out))


def summarize_trace(stats_csv, bench_log, command):
    """Markdown summary of a rocprofv3 --kernel-trace --stats run of bench.py: one row per
    kernel (calls, total, average, share) and the MXFP8 GEMM family's average launch time
    beside the one the same run's bench line reports (HIP events on the launch stream)."""
    import csv
    rows = []
    with open(stats_csv) as f:
        for r in csv.DictReader(f):
            rows.append((r["Name"], int(r["Calls"]), float(r["TotalDurationNs"]) / 1e6))
    total = sum(t for _, _, t in rows)
    line = None
    with open(bench_log) as f:
        for text in f:
            if text.startswith("{"):
                line = json.loads(text)
    gemm = [(c, t) for n, c, t in rows if GEMM_KERNEL.search(n)]
    g_calls, g_ms = sum(c for c, _ in gemm), sum(t for _, t in gemm)

    def short(name):
        name = name.replace("void ", "").replace("(anonymous namespace)::", "")
        return name.split("(")[0][:80]

    out = [f"Command (from the repository root, on one MI355X):", "", f"    {command}", "",
           f"All kernels: {total:.1f} ms over {sum(c for _, c, _ in rows)} dispatches "
           "(the whole process, input setup included).", ""]
    if line is not None:
        out += [f"The same run's bench line: {line['value']:.2f} ms per block; its MXFP8 GEMM "
                f"family averages {line['roofline']['avg_launch_ms']:.4f} ms per launch (HIP "
                f"events), the trace {g_ms / g_calls:.4f} ms ({g_calls} launches).", ""]
        small = [(c, t) for n, c, t in rows if GEMM_KERNEL.search(n) and "persistent" not in n]
        if small:
            s_calls, s_ms = sum(c for c, _ in small), sum(t for _, t in small)
            out += ["The bench line times the family in the blocks without the side stream. In "
                    "the overlapped blocks the two context projections "
                    "(`mxfp8_gemm_kernel<128, 128, ...>`) run on the side stream beside the "
                    "window attention, whose workgroups hold the CUs, so their trace durations "
                    f"stretch (average {s_ms / s_calls:.4f} ms over {s_calls} launches). The "
                    "persistent kernel alone, the family's "
                    f"{100 * (g_ms - s_ms) / g_ms:.1f}% of GEMM time, averages "
                    f"{(g_ms - s_ms) / (g_calls - s_calls):.4f} ms per launch in the trace.", ""]
    out += ["| kernel | calls | total ms | avg ms | % |", "|---|---:|---:|---:|---:|"]
    for name, calls, t in sorted(rows, key=lambda r: -r[2]):
        if t / total < 2e-4:
            continue
        out.append(f"| `{short(name)}` | {calls} | {t:.3f} | {t / calls:.4f} | "
                   f"{100 * t / total:.2f} |")
    print("\n".join(out))


TRAFFIC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "gemm_block_108k_traffic.md")
CALIBRATION_KERNEL = "neg_kernel_cuda"   # torch.neg over 2**29 bf16: 1 GiB read, 1 GiB written
CALIBRATION_KIB = float(1 << 20)


def _counter_rows(path, counter):
    """[(dispatch id, kernel name, KiB)] of one counter from a rocprofv3 --pmc CSV (a dispatch
    may span several rows; they are summed)."""
    import csv
    per = {}
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                d = int(r["Dispatch_Id"])
                name, kib = per.get(d, (r["Kernel_Name"], 0.0))
                per[d] = (name, kib + float(r["Counter_Value"]))
    return [(d, name, kib) for d, (name, kib) in per.items()]


GEMM_KERNEL = re.compile(r"mxfp8_gemm_(persistent_)?kernel")


def summarize_traffic(fetch_csv, write_csv, command=""):
    """Markdown summary of the HBM traffic per MXFP8 GEMM launch from a FETCH_SIZE pass and a
    WRITE_SIZE pass (each run with --calibrate-copy). Each counter is scaled by the factor
    that maps its reading for the calibration kernel onto the kernel's known 1 GiB.
    `command` (the passes' command lines) replaces the default ones in the summary."""
    passes = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _counter_rows(path, counter)
        # the calibration launch is the process's last negation (the block negates small
        # tensors of its own earlier)
        cal = max(((d, kib) for d, name, kib in rows if CALIBRATION_KERNEL in name), default=None)
        if cal is None:
            raise SystemExit(f"{path}: no {CALIBRATION_KERNEL} dispatch (run with --calibrate-copy)")
        gemm = sorted((d, name, kib) for d, name, kib in rows if GEMM_KERNEL.search(name))
        passes[counter] = (CALIBRATION_KIB / cal[1], gemm)
    fetch_factor, fetch = passes["FETCH_SIZE"]
    write_factor, write = passes["WRITE_SIZE"]
    if len(fetch) != len(write) or not fetch:
        raise SystemExit("the two passes hold different GEMM launches")
    total = 0.0
    lines = []
    for (d, name, fk), (_, _, wk) in zip(fetch, write):
        nbytes = (fk * fetch_factor + wk * write_factor) * 1024
        total += nbytes
        kname = GEMM_KERNEL.search(name).group(0)
        tile = name[name.index("<"):name.index(">") + 1] if "<" in name else ""
        lines.append(f"| {len(lines)} | `{kname}{tile}` | {fk * fetch_factor / 2**20:.3f} | "
                     f"{wk * write_factor / 2**20:.3f} | {nbytes / 1e9:.3f} |")
    per_launch = total / len(fetch)
    if command:
        cmd_lines = ["Commands (from the repository root, on one MI355X):", "",
                     *["    " + c.strip()
                       for c in command.replace(" ;; ", "\n").strip().splitlines()], "",
                     "    python3 bench.py --summarize-traffic "
                     f"{fetch_csv} {write_csv}", ""]
    else:
        # the profiler's output directory and file prefix of each pass, read back from the
        # CSV paths (<dir>/<prefix>_counter_collection.csv)
        def pass_args(csv_path):
            prefix = os.path.basename(csv_path).split("_counter_collection")[0]
            return f"-d {os.path.dirname(csv_path) or '.'} -o {prefix}"
        cmd_lines = [
            "Commands (from the repository root, on one MI355X; one block forward, no warmup):", "",
            f"    rocprofv3 --pmc FETCH_SIZE {pass_args(fetch_csv)} --output-format csv -- "
            "python3 bench.py --steps 1 --warmup 0 --isolated-steps 0 --no-cpu-baseline --calibrate-copy",
            f"    rocprofv3 --pmc WRITE_SIZE {pass_args(write_csv)} --output-format csv -- "
            "python3 bench.py --steps 1 --warmup 0 --isolated-steps 0 --no-cpu-baseline --calibrate-copy",
            f"    python3 bench.py --summarize-traffic {fetch_csv} {write_csv}", ""]
    out = ["# HBM traffic per MXFP8 GEMM launch, hybrid DiT block at 108,000 tokens", "",
           *cmd_lines,
           "Calibration: `torch.neg` over 2^29 bf16 values (1 GiB read, 1 GiB written) reads "
           f"FETCH_SIZE x{fetch_factor:.4f} and WRITE_SIZE x{write_factor:.4f} of its true bytes; "
           "each GEMM reading below is scaled by that factor.", "",
           "FETCH_SIZE counts L2 misses sent to the fabric. Those served by the MALL are counted too, "
           "so this is an upper bound on DRAM bytes.", "",
           "| launch | kernel | read GiB | written GiB | GB |", "|---:|---|---:|---:|---:|",
           *lines, "",
           f"bytes_per_launch: {per_launch:.0f}"]
    print("\n".join(out))


def traffic_per_launch():
    """HBM bytes per GEMM launch recorded by --summarize-traffic, or None."""
    if not os.path.exists(TRAFFIC_SUMMARY):
        return None
    with open(TRAFFIC_SUMMARY) as f:
        for line in f:
            if line.startswith("bytes_per_launch:"):
                return int(line.split(":")[1])
    return None


def calibrate_copy():
    """One elementwise kernel of known traffic (torch.neg of 2^29 bf16 values into another
    buffer: 1 GiB read, 1 GiB written) for scaling HBM byte counters."""
    import torch
    src = torch.ones(1 << 29, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    torch.neg(src, out=dst)
    torch.cuda.synchronize()
    log("negated 1 GiB into 1 GiB (calibration kernel: 1 GiB read, 1 GiB written)")


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--summarize-counters", nargs="+", metavar="CSV",
                   help="print the markdown table of per-kernel mean counters of one or more "
                        "rocprofv3 --pmc CSVs and exit")
    p.add_argument("--command", default="",
                   help="the profiling commands to quote in a summary (separated by ' ;; ')")
    p.add_argument("--summarize-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                   help="print the GEMM HBM-traffic summary of a FETCH_SIZE and a WRITE_SIZE "
                        "pass and exit")
    p.add_argument("--summarize-trace", nargs=3, metavar=("STATS_CSV", "BENCH_LOG", "COMMAND"),
                   help="print the markdown kernel-trace summary of a rocprofv3 --stats run of "
                        "bench.py (its kernel_stats.csv, its output, the command) and exit")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="after the timed steps, negate one 1 GiB bf16 buffer into another (an "
                        "elementwise kernel of known traffic for scaling HBM byte counters)")
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--frames", type=int, default=30)
    p.add_argument("--cpu-sample-frames", type=int, default=6)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--config-steps", type=int, default=5,
                   help="timed repeats of the stand-alone config measurements (C1 VDA layer "
                        "at head_dim 64, C2 quantize + GEMMs, C3 VDA branch, C4 RoPE + window "
                        "attention); 0 skips them and the other workloads beside the block "
                        "(short-conv prepare, production geometry, H3 widths)")
    p.add_argument("--configs-only", action="store_true",
                   help="run only the stand-alone config measurements (C1, C2, C3, C4 and the "
                        "short-conv prepare) and print them as one JSON line (for profiling their "
                        "kernels apart from the block)")
    p.add_argument("--breakdown-steps", type=int, default=3,
                   help="instrumented steps after the timed ones (an event pair around every "
                        "launch) for the per-kernel breakdown, the roofline and idle_ms")
    p.add_argument("--isolated-steps", type=int, default=2,
                   help="untimed-for-value steps with the VDA branch after the window attention "
                        "on one stream, for the branch kernels' and the projections' own launch "
                        "times (the roofline)")
    args = p.parse_args()
    if args.summarize_counters:
        summarize_counters(args.summarize_counters, args.command)
        return
    if args.summarize_traffic:
        summarize_traffic(*args.summarize_traffic, command=args.command)
        return
    if args.summarize_trace:
        summarize_trace(*args.summarize_trace)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the block runs whole on a single MI355X "
              "(no sharding is implemented); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from vdn_amd import _lib
    from vdn_amd import window as vw
    from vdn_amd.block import (BlockConfig, BlockWeights, HybridDiTBlock, cross_attention_plan,
                               make_inputs)
    if not torch.cuda.is_available():
        raise RuntimeError("bench.py needs a HIP device")
    _lib.load()
    cfg = BlockConfig()
    frames = args.frames
    if args.configs_only:
        steps = max(args.config_steps, 1)
        print(json.dumps({"configs": {"C1": c1_vda(steps), "C2": c2_quantize_gemm(steps),
                                      "C3": c3_vda(steps, frames),
                                      "C4": c4_window(steps, frames)},
                          "short_conv_prepare": short_conv_prepare(cfg, torch.device("cuda"),
                                                                   frames, steps)}), flush=True)
        if args.calibrate_copy:
            calibrate_copy()
        return
    spatial = HEIGHT * WIDTH
    tokens = frames * spatial
    log(f"building block weights (hidden {cfg.hidden}, ffn {cfg.ffn}) and inputs "
        f"({frames} x {HEIGHT}x{WIDTH} = {tokens} tokens)")
    weights = BlockWeights.random(cfg, seed=0, device="cuda")
    block = HybridDiTBlock(cfg, weights)
    hidden, temb, ctx, layout, (cos, sin) = make_inputs(cfg, frames, HEIGHT, WIDTH, seed=1,
                                                       device="cuda")
    plan = vw.prepare_paper_window_plan(layout, vw.window_bounds(frames, cfg.radius),
                                        device="cuda")
    cplan = cross_attention_plan(tokens, ctx.shape[0], "cuda")
    plans = {plan.device_plan.intervals.data_ptr(): visible_pairs(frames, spatial, cfg.radius),
             cplan.intervals.data_ptr(): tokens * ctx.shape[0]}

    def step():
        return block(hidden, temb, ctx, layout, (cos, sin), plan, cplan)

    for i in range(args.warmup):
        step()
        torch.cuda.synchronize()
        log(f"warmup {i + 1}/{args.warmup} done")
    # The headline: K steps back to back, one event pair per step on the caller's stream (the
    # block joins its side stream back into it), no per-launch events; value = the median.
    steps_ms, wall_ms = timed_steps(step, args.steps)
    ms = statistics.median(steps_ms)
    log(f"timed {args.steps} steps: median {ms:.2f} ms per block (mean {wall_ms:.2f}, "
        f"min {min(steps_ms):.2f}, max {max(steps_ms):.2f})")
    if args.calibrate_copy:
        calibrate_copy()

    # The per-kernel breakdown comes from separate instrumented steps (an event pair around
    # every launch). idle_ms = a step's wall time minus the sum of its caller-stream launch
    # times: what the caller's stream spends waiting (on the host, or on the side stream).
    # A side-stream entry's time in the breakdown is a wall time: its event pair also spans
    # the time the launch waits for the CUs the caller's stream holds.
    names = set(_lib.SIGNATURES)
    b_steps = max(args.breakdown_steps, 1)
    caller = torch.cuda.current_stream().cuda_stream
    with _lib.LaunchTimer(names) as timer:
        inst_ms, _ = timed_steps(step, b_steps)
    per = aggregate(timer, plans)
    breakdown = breakdown_of(per, b_steps)
    main_launch_ms = sum(v[1] for v in aggregate(timer, plans, caller).values()) / b_steps
    idle = {"ms": round(ms - main_launch_ms, 3),
            "instrumented_ms": round(statistics.median(inst_ms) - main_launch_ms, 3),
            "caller_stream_launch_ms": round(main_launch_ms, 3),
            "instrumented_step_ms": round(statistics.median(inst_ms), 3),
            "steps": b_steps}
    log(f"instrumented {b_steps} steps: caller-stream launches {main_launch_ms:.2f} ms, "
        f"idle {idle['ms']:.3f} ms per block")
    # The branch kernels again, one stream, no overlap: the VDA passes share the GPU with the
    # window attention in the timed steps above, so their launch times there are wall times
    # under contention. These steps give each branch kernel's own launch time.
    iso_steps = args.isolated_steps
    serial_ms = None
    if iso_steps > 0:
        block.overlap_vda = False
        serial_ms = statistics.median(timed_steps(step, iso_steps)[0])
        with _lib.LaunchTimer(set(VDA_ENTRIES) | set(ATTENTION) | set(GEMMS)) as iso_timer:
            timed_steps(step, iso_steps)
        block.overlap_vda = True
        iso = aggregate(iso_timer, plans)
        attn_timer = iso_timer
        log(f"isolated branch kernels timed over {iso_steps} steps; the block without the "
            f"side stream: {serial_ms:.2f} ms")
    else:   # only the overlapped times exist
        iso, iso_steps = per, b_steps
        attn_timer = timer
    # the block's projections apart, told apart by their shapes: QKV (N = 3 inner), [O | O_lin]
    # (K = 2 inner), cross-Q and cross-O (K = N = hidden, without and with the residual), the
    # context K / V rows, FFN-up (the producer entry point) and FFN-down (K = FFN width)
    inner = cfg.heads * cfg.head_dim

    def gemm_label(nm, a):
        if nm == "vdn_mxfp8_gemm_act_quantize":
            return "ffn_up"
        kp, rows, n, res = a[6], a[14], a[15], a[10] is not None
        if rows != tokens:
            return "context_kv"
        if kp == padded(2 * inner):
            return "o_cat"
        if kp == padded(cfg.ffn):
            return "ffn_down"
        if n == 3 * inner:
            return "qkv"
        return "cross_o" if res else "cross_q"

    gemm_launches = {}
    for nm, a, t, _ in attn_timer.durations():
        if nm in GEMMS:
            flop, _ = work(nm, a, plans)
            e = gemm_launches.setdefault(gemm_label(nm, a), [0, 0.0, 0.0])
            e[0] += 1
            e[1] += t
            e[2] += flop
    gemm_launches = {k: {"launches_per_step": e[0] // max(iso_steps, 1),
                         "avg_launch_ms": round(e[1] / e[0], 4),
                         "tflops": round(e[2] / (e[1] * 1e-3) / 1e12, 1),
                         "mxfp8_frac": round(e[2] / (e[1] * 1e-3) / 1e12 / PEAK_MXFP8_TFLOPS, 4)}
                     for k, e in gemm_launches.items()}
    # the block's two attention launches apart: the +-radius frame window and the
    # cross-attention to the context rows (told apart by their plans)
    attn_launches = {}
    for label, key in (("self", plan.device_plan.intervals.data_ptr()),
                       ("cross", cplan.intervals.data_ptr())):
        ts = [t for nm, a, t, _ in attn_timer.durations() if nm in ATTENTION and a[11] == key]
        if ts:
            avg = sum(ts) / len(ts)
            flop = 4.0 * D * cfg.heads * plans[key]
            attn_launches[label] = {"avg_launch_ms": round(avg, 4),
                                    "tflops": round(flop / (avg * 1e-3) / 1e12, 1),
                                    "bf16_frac": round(flop / (avg * 1e-3) / 1e12 /
                                                       PEAK_BF16_TFLOPS, 4)}
    # The GEMM family from the steps without the side stream: there every projection launches
    # on the caller's stream and runs alone (in the overlapped block the two context
    # projections queue on the side stream behind the attention's workgroups).
    g = [sum(iso[nm][i] for nm in GEMMS if nm in iso) for i in range(4)]
    gemm_tflops = g[2] / (g[1] * 1e-3) / 1e12
    vda_t = sum(iso[n][1] for n in VDA_ENTRIES if n in iso)
    vda_bytes = sum(iso[n][3] for n in VDA_ENTRIES if n in iso)
    vda_gbs = vda_bytes / (vda_t * 1e-3) / 1e9
    hb_t = sum(iso[n][1] for n in VDA_HBM_BOUND if n in iso)
    hb_bytes = sum(iso[n][3] for n in VDA_HBM_BOUND if n in iso)
    hb_gbs = hb_bytes / (hb_t * 1e-3) / 1e9
    w = [sum(iso[nm][i] for nm in ATTENTION if nm in iso) for i in range(4)]
    extra_steps = args.isolated_steps if args.config_steps > 0 else 0
    conv = short_conv_prepare(cfg, hidden.device, frames, extra_steps)
    production = production_geometry(extra_steps)
    h3 = h3_block(extra_steps,
                  lambda p, c, f, s, t, l: {p.device_plan.intervals.data_ptr():
                                            visible_pairs(f, s, cfg.radius),
                                            c.intervals.data_ptr(): t * l})
    configs = {"C1": c1_vda(args.config_steps),
               "C2": c2_quantize_gemm(args.config_steps),
               "C3": c3_vda(args.config_steps, frames),
               "C4": c4_window(args.config_steps, frames)}
    traffic = traffic_per_launch()

    result = {
        "metric": METRIC, "value": round(ms, 3), "unit": "ms", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "step_ms": {"median": round(ms, 3), "mean": round(wall_ms, 3),
                    "min": round(min(steps_ms), 3), "max": round(max(steps_ms), 3),
                    "all": [round(t, 3) for t in steps_ms]},
        "idle_ms": idle,
        "vda_side_stream": {"overlapped_ms": round(ms, 3),
                            "serial_ms": None if serial_ms is None else round(serial_ms, 3)},
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "mxfp8-e4m3 GEMMs, bf16 attention/activations, fp32 VDA state",
        "data": "synthetic: random-init weights N(0,0.02), hidden/temb/context N(0,1)",
        "config": {"workload": (f"hybrid DiT block forward, {frames} frames x {HEIGHT}x{WIDTH} = "
                                f"{tokens} tokens, hidden {cfg.hidden}, {cfg.heads}x{cfg.head_dim} "
                                f"heads, FFN {cfg.ffn} GELU-tanh, {ctx.shape[0]} context rows, "
                                f"LoRA r{cfg.lora_rank} merged, +-{cfg.radius} frame window"),
                   "tokens": tokens, "hidden": cfg.hidden, "heads": cfg.heads,
                   "head_dim": cfg.head_dim, "ffn": cfg.ffn, "context": ctx.shape[0],
                   "parallelism": "single GPU"},
        "roofline": {"kernel": "mxfp8_gemm_persistent_kernel / mxfp8_gemm_kernel (all block "
                               "projections: vdn_mxfp8_gemm and the FFN-up "
                               "vdn_mxfp8_gemm_act_quantize; launch times from the block "
                               "steps without the side stream)" if iso_steps and
                               args.isolated_steps > 0 else
                               "mxfp8_gemm_persistent_kernel / mxfp8_gemm_kernel (all block "
                               "projections: vdn_mxfp8_gemm and the FFN-up "
                               "vdn_mxfp8_gemm_act_quantize)", "bound": "mfma",
                     "achieved": round(gemm_tflops, 1), "peak": PEAK_MXFP8_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(gemm_tflops / PEAK_MXFP8_TFLOPS, 4),
                     "traffic": traffic,
                     "traffic_source": ("recorded, not measured in this run: " +
                                        os.path.relpath(TRAFFIC_SUMMARY, os.path.dirname(
                                            os.path.abspath(__file__))) +
                                        " (rocprofv3 FETCH_SIZE + WRITE_SIZE passes)")
                     if traffic is not None else None,
                     "avg_launch_ms": round(g[1] / g[0], 4),
                     "flop_per_launch": g[2] / g[0]},
        "mxfp8_tflops": round(gemm_tflops, 1),
        "vda_gbs": round(vda_gbs, 1), "vda_hbm_frac": round(vda_gbs / PEAK_HBM_GBS, 4),
        "vda_ms": round(vda_t / iso_steps, 3),
        "vda_hbm_bound_passes": {"entries": list(VDA_HBM_BOUND), "gbs": round(hb_gbs, 1),
                                 "frac": round(hb_gbs / PEAK_HBM_GBS, 4),
                                 "ms": round(hb_t / iso_steps, 3)},
        "window_attention_tflops": round(w[2] / (w[1] * 1e-3) / 1e12, 1),
        "window_attention_bf16_frac": round(w[2] / (w[1] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "window_attention_launches": attn_launches,
        "gemm_launches": gemm_launches,
        "configs": configs,
        "short_conv_prepare": conv,
        "production_geometry": production,
        "h3_widths": h3,
        "breakdown": breakdown,
        "breakdown_isolated_branches": breakdown_of(iso, iso_steps),
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        sample = min(args.cpu_sample_frames, frames)
        log(f"timing the CPU fp32 path on {sample} frames")
        result["cpu_baseline"] = cpu_baseline(cfg, weights, hidden, temb, ctx, cos, sin, frames,
                                              sample)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
